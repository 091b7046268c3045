"""GPU parity of the streaming GGUF loader: every 2D block tensor of a written file, loaded
with jk_gguf_load_weight in one chunk and in chunks of one 8-row tile (the two pinned buffers
and their events reused many times, a partial last tile), is the handle jk_weight_upload makes
of the same bytes: equal dequantized rows (and so the dequantize_row round trip, which
tests/test_gpu_parity.py holds to the oracle's GGUF dequantizers) and equal GEMM outputs."""
import numpy as np
import pytest

import jk
from gguf_writer import STR, write_gguf
from jk import synth

pytestmark = pytest.mark.gpu

SHAPES = [("blk.0.attn_q.weight", jk.Q4_K, 19, 512), ("blk.0.ffn_down.weight", jk.Q6_K, 8, 256),
          ("blk.0.attn_k.weight", jk.Q8_0, 5, 64), ("blk.0.ffn_up.weight", jk.TQ1_0, 3, 256),
          ("blk.0.ffn_gate.weight", jk.I2_S, 12, 128), ("blk.0.x.weight", jk.Q5_0, 9, 96),
          ("blk.0.y.weight", jk.Q3_K, 17, 256), ("blk.0.z.weight", jk.IQ4_NL, 33, 64),
          ("blk.0.q40.weight", jk.Q4_0, 21, 128), ("blk.0.q41.weight", jk.Q4_1, 10, 64),
          ("blk.0.q51.weight", jk.Q5_1, 11, 96), ("blk.0.q2k.weight", jk.Q2_K, 16, 512),
          ("blk.0.q5k.weight", jk.Q5_K, 7, 256), ("blk.0.tq2.weight", jk.TQ2_0, 9, 256),
          ("blk.0.big.weight", jk.Q4_K, 1000, 4096)]


def same_bits(a, b) -> bool:
    a, b = np.ascontiguousarray(a, np.float32), np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and bool(np.all((a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))))


def rows_of(torch, w):
    out = torch.empty(w.rows * w.cols, dtype=torch.float32, device="cuda")
    jk.dev_dequantize_rows(w, 0, w.rows, out, w.rows * w.cols)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def gemm_of(torch, w, m=3):
    x = torch.from_numpy(synth.activations(m * w.cols, 7)).cuda()
    need = jk.act_q8_bytes(m, w.cols)
    store = torch.zeros(need, dtype=torch.uint8, device="cuda")
    act = jk.act_q8_bind(store, need, m, w.cols)
    jk.dev_quantize_act_q8(x, m, w.cols, act)
    y = torch.empty(m * w.rows, dtype=torch.float32, device="cuda")
    jk.dev_gemm_repacked(w, act, y, m * w.rows, 0, w.rows)
    torch.cuda.synchronize()
    return y.cpu().numpy()


@pytest.mark.parametrize("chunk_bytes", [0, 1, 300 * 1024])
def test_gguf_load_matches_upload(gpu, tmp_path, chunk_bytes):
    torch = gpu
    tensors = [(n, q, [c, r], synth.gguf_weights(q, r, c, seed=r + q)) for n, q, r, c in SHAPES]
    path = tmp_path / "model.gguf"
    write_gguf(path, tensors, [("general.architecture", STR, "llama")], alignment=64)
    g = jk.GGUF(str(path))
    stream = torch.cuda.Stream()
    for name, quant, ne, data in tensors:
        w = g.load(name, stream.cuda_stream, chunk_bytes)
        ref = jk.Weight(jk.TensorView(name, quant, ne, data), ne[1], ne[0])
        assert (w.quant, w.rows, w.cols, w.device_bytes) == (quant, ne[1], ne[0], ref.device_bytes)
        assert same_bits(rows_of(torch, w), rows_of(torch, ref)), name
        assert same_bits(gemm_of(torch, w), gemm_of(torch, ref)), name
        w.free()
        ref.free()
    g.close()
