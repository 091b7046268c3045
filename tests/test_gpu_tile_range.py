"""GPU parity of load-time assembly from tile ranges: jk_weight_layout_for / jk_weight_create /
jk_weight_upload_tile_range / jk_weight_repack_tile_range / jk_weight_seal, the device form of
RepackedWeight::block_scaled_layout + repack_into_tile_range + from_tile_buffers
(repack.rs:2372, 1579, 2386).

Follows the reference's own tests: tests/wave3_prefill_gqa_and_gemm.rs:280-360 (67 x 512 weights
repacked by 4 threads over disjoint tile ranges, then every dequantized row equal to the
sequential repack) and src/repack.rs:5990-6060 (19 x 256 Q4_K split at tile 1, the GEMM of 5
tokens and every row equal). Here every format is covered, the rows are also held to the
oracle's GGUF dequantizer (the dequantize_row round trip), and the threads run on streams of
their own.
"""
import threading

import numpy as np
import pytest

import jk
import oracle as O
from jk import synth

pytestmark = pytest.mark.gpu

ALL_FORMATS = [jk.Q4_0, jk.Q4_1, jk.Q5_0, jk.Q5_1, jk.Q8_0, jk.IQ4_NL, jk.Q2_K, jk.Q3_K, jk.Q4_K, jk.Q5_K, jk.Q6_K,
               jk.TQ1_0, jk.TQ2_0, jk.I2_S]


def same_bits(a, b) -> bool:
    a, b = np.ascontiguousarray(a, np.float32), np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and bool(np.all((a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))))


def dequant_all(torch, w, rows, cols):
    out = torch.empty(rows * cols, dtype=torch.float32, device="cuda")
    jk.dev_dequantize_rows(w, 0, rows, out, rows * cols)
    torch.cuda.synchronize()
    return out.cpu().numpy().reshape(rows, cols)


def gemm_out(torch, w, rows, cols, m=5):
    i = np.arange(m * cols)
    x = torch.from_numpy(((i % 23).astype(np.float32) - 11.0) * 0.125).cuda()  # repack.rs:6040-6042
    need = jk.act_q8_bytes(m, cols)
    store = torch.zeros(need, dtype=torch.uint8, device="cuda")
    act = jk.act_q8_bind(store, need, m, cols)
    jk.dev_quantize_act_q8(x, m, cols, act)
    y = torch.empty(m * rows, dtype=torch.float32, device="cuda")
    jk.dev_gemm_repacked(w, act, y, m * rows, 0, rows)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def view_of(quant, rows, cols, seed):
    raw = synth.gguf_weights(quant, rows, cols, seed=seed)
    return jk.TensorView("w_par", quant, [cols, rows], raw), raw


@pytest.mark.parametrize("quant", ALL_FORMATS)
def test_parallel_tile_range_upload_is_bit_exact_across_4_threads(gpu, quant):
    torch = gpu
    rows, cols = 67, 512
    view, raw = view_of(quant, rows, cols, 67 + quant)
    seq = jk.Weight(view, rows, cols)
    layout = jk.block_scaled_layout(view, rows, cols)
    par = jk.Weight.create(layout)
    assert par.device_bytes == seq.device_bytes and par.gguf_bytes == seq.gguf_bytes
    n_tiles, workers = layout.n_tiles, 4
    per = -(-n_tiles // workers)
    errors = []

    def work(t0, t1):
        try:
            st = torch.cuda.Stream()
            par.repack_into_tile_range(view, t0, t1, st.cuda_stream)
        except Exception as e:  # reported by the main thread
            errors.append(e)

    threads = [threading.Thread(target=work, args=(s, min(n_tiles, s + per))) for s in range(0, n_tiles, per)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    par.seal()
    a, b = dequant_all(torch, seq, rows, cols), dequant_all(torch, par, rows, cols)
    assert same_bits(a, b)
    # the dequantize_row round trip: the GGUF block dequantizers of the oracle
    ref = np.stack([O.dequantize_tensor_row(quant, [cols, rows], raw, r, cols) for r in range(rows)])
    assert same_bits(b, ref)
    assert same_bits(gemm_out(torch, seq, rows, cols), gemm_out(torch, par, rows, cols))


@pytest.mark.parametrize("quant", [jk.Q4_K, jk.Q6_K, jk.Q3_K, jk.TQ1_0, jk.I2_S, jk.Q5_0])
def test_device_tile_ranges_in_reverse_order(gpu, quant):
    """GGUF bytes already on the device, repacked tile range by tile range from the last to the
    first (19 rows = tiles of 8, 8, 3 as in repack.rs:6000), against the whole upload; the
    GEMV of formats that have one agrees too."""
    torch = gpu
    rows, cols = 19, 512
    view, raw = view_of(quant, rows, cols, 19 + quant)
    seq = jk.Weight(view, rows, cols)
    par = jk.Weight.create(jk.block_scaled_layout(view, rows, cols))
    row_bytes = (cols // jk.BLOCK_ELEMENTS[quant]) * jk.BLOCK_BYTES[quant]
    dev = torch.from_numpy(raw[:rows * row_bytes].copy()).cuda()
    for t in (2, 1, 0):
        r0, r1 = 8 * t, min(rows, 8 * t + 8)
        par.repack_tile_range(dev[r0 * row_bytes:], (r1 - r0) * row_bytes, t, t + 1)
    par.seal()
    assert same_bits(dequant_all(torch, seq, rows, cols), dequant_all(torch, par, rows, cols))
    assert same_bits(gemm_out(torch, seq, rows, cols, 3), gemm_out(torch, par, rows, cols, 3))
    if quant in jk.GEMV_FORMATS:
        x = synth.activations(cols, 5)
        xq = O.quantize_row_q8_0(x) if quant in jk.Q8_0_ACT else O.quantize_row_q8_k(x)
        dq = torch.from_numpy(xq.view(np.uint8).reshape(-1).copy()).cuda()
        y1 = torch.empty(rows, dtype=torch.float32, device="cuda")
        y2 = torch.empty_like(y1)
        jk.dev_gemv_q8_rows(seq, dq, xq.size, y1, 0, rows)
        jk.dev_gemv_q8_rows(par, dq, xq.size, y2, 0, rows)
        torch.cuda.synchronize()
        assert same_bits(y1.cpu().numpy(), y2.cpu().numpy())


def test_unwritten_tiles_and_sealed_handles_fail_closed(gpu):
    torch = gpu
    rows, cols = 19, 256
    view, raw = view_of(jk.Q4_K, rows, cols, 3)
    layout = jk.block_scaled_layout(view, rows, cols)
    w = jk.Weight.create(layout)
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    x = torch.zeros(cols, dtype=torch.float32, device="cuda")
    with pytest.raises(jk.TensorBoundsError, match="sealed"):  # not usable before sealing
        jk.dev_gemv_q8_f32(w, x, cols, y, rows)
    with pytest.raises(jk.TensorBoundsError, match="sealed"):
        jk.dev_dequantize_rows(w, 0, 1, torch.empty(cols, dtype=torch.float32, device="cuda"), cols)
    with pytest.raises(jk.TensorBoundsError, match="exceeds n_tiles"):  # repack.rs:1588-1600
        w.repack_into_tile_range(view, 2, 4)
    with pytest.raises(jk.TensorBoundsError):
        w.repack_into_tile_range(view, 2, 1)
    w.repack_into_tile_range(view, 0, 0)  # empty range: nothing written
    w.repack_into_tile_range(view, 0, 1)
    with pytest.raises(jk.TensorBoundsError, match="never written"):  # tiles 1, 2 missing
        w.seal()
    with pytest.raises(jk.TensorBoundsError):  # the view must be the layout's tensor
        w.repack_into_tile_range(jk.TensorView("other", jk.Q4_K, [256, 18], raw[:18 * 144]), 1, 3)
    other = jk.TensorView("q6", jk.Q6_K, [256, 19], synth.gguf_weights(jk.Q6_K, rows, cols, seed=1))
    with pytest.raises(jk.TensorBoundsError):  # another format
        w.repack_into_tile_range(other, 1, 3)
    dev = torch.from_numpy(raw.copy()).cuda()
    with pytest.raises(jk.TensorBoundsError):  # byte count of the device slice
        w.repack_tile_range(dev[8 * 144:], 11 * 144 - 1, 1, 3)
    w.repack_tile_range(dev[8 * 144:], 11 * 144, 1, 3)
    w.seal()
    with pytest.raises(jk.TensorBoundsError, match="sealed"):  # immutable once sealed
        w.repack_into_tile_range(view, 0, 1)
    jk.dev_gemv_q8_f32(w, x, cols, y, rows)
    torch.cuda.synchronize()
    with pytest.raises(jk.TensorBoundsError):  # a layout that does not describe its dimensions
        bad = jk.block_scaled_layout(view, rows, cols)
        bad.device_bytes += 1
        jk.Weight.create(bad)


def test_i2_s_tile_range_keeps_the_tensor_scale(gpu):
    torch = gpu
    rows, cols = 20, 256
    view, raw = view_of(jk.I2_S, rows, cols, 9)
    seq = jk.Weight(view, rows, cols)
    layout = jk.block_scaled_layout(view, rows, cols)
    par = jk.Weight.create(layout)
    changed = raw.copy()
    changed[-32:-28] = np.frombuffer(np.float32(layout.tensor_scale * 2 + 1).tobytes(), np.uint8)
    with pytest.raises(jk.TensorBoundsError, match="trailer"):
        par.repack_into_tile_range(jk.TensorView("w", jk.I2_S, [cols, rows], changed), 0, 3)
    par.repack_into_tile_range(view, 0, 3)
    par.seal()
    a = torch.from_numpy(((np.arange(3 * cols) % 7) - 3).astype(np.int8)).cuda()
    sc = torch.tensor([0.5, 1.0, 0.25], dtype=torch.float32, device="cuda")
    y1 = torch.empty(3 * rows, dtype=torch.float32, device="cuda")
    y2 = torch.empty_like(y1)
    jk.dev_bitlinear_i8(seq, a, sc, 3, cols, y1, 3 * rows)
    jk.dev_bitlinear_i8(par, a, sc, 3, cols, y2, 3 * rows)
    torch.cuda.synchronize()
    assert same_bits(y1.cpu().numpy(), y2.cpu().numpy())
