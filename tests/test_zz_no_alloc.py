"""jk_gemv_q8_argmax_noalloc (the entry point that allocates nothing: argmax slots in a static
device array of the library) against jk_gemv_q8_argmax with a caller workspace, through the C ABI.

Two calls in a row share the static array; the second has a smaller input, so it must not read
slots left by the first. Outputs are compared bit for bit and the index with the oracle's argmax.
"""
import numpy as np
import pytest

import jk
import oracle as O
from jk import synth

pytestmark = pytest.mark.gpu


def same_bits(a, b) -> bool:
    a, b = np.ascontiguousarray(a, np.float32), np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and bool(np.all(a.view(np.uint32) == b.view(np.uint32)))


def run_both(torch, quant, rows, cols, f32, seed):
    raw = synth.gguf_weights(quant, rows, cols, seed=seed)
    w = jk.Weight(jk.TensorView("lm_head", quant, [rows, cols], raw), rows, cols)
    x = synth.activations(cols, seed + 1)
    xq = O.quantize_row_q8_0(x) if quant in jk.Q8_0_ACT else O.quantize_row_q8_k(x)
    if f32:
        xa, xb, n = None, torch.from_numpy(x).cuda(), cols
    else:
        xa, xb, n = torch.from_numpy(xq.view(np.uint8).reshape(-1).copy()).cuda(), None, xq.size
    y0 = torch.empty(rows, dtype=torch.float32, device="cuda")
    y1 = torch.full((rows,), float("nan"), dtype=torch.float32, device="cuda")
    i0 = torch.full((1,), -7, dtype=torch.int32, device="cuda")
    i1 = torch.full((1,), -7, dtype=torch.int32, device="cuda")
    ws = torch.full((jk.argmax_workspace_bytes(rows),), 0xFF, dtype=torch.uint8, device="cuda")
    jk.dev_gemv_q8_argmax(w, xa, xb, n, y0, i0, ws)
    jk.dev_gemv_q8_argmax_noalloc(w, xa, xb, n, y1, i1)
    torch.cuda.synchronize()
    ref_i = O.argmax_f32(O.gemv_q8(quant, [rows, cols], raw, xq, rows))
    print(f"no-alloc case {jk.QUANT_NAMES[quant]} {rows}x{cols} f32={f32}", flush=True)
    assert same_bits(y1.cpu().numpy(), y0.cpu().numpy())
    assert int(i1.cpu()[0]) == int(i0.cpu()[0]) == ref_i
    w.free()


@pytest.mark.parametrize("cases", [
    # fast path (Q6_K rows of 16 blocks), then a smaller looped-path launch (Q4_K, 56 blocks a row)
    [(jk.Q6_K, 32000, 4096, False), (jk.Q4_K, 300, 14336, True)],
    # many workgroup slots (131072 rows), then the global-activation path with few rows
    [(jk.Q4_0, 131072, 256, False), (jk.Q4_0, 77, 32 * 2000, False)],
    # the same shape twice with the second smaller: Q8_0, f32 activations quantized in the launch
    [(jk.Q8_0, 8200, 4096, True), (jk.Q8_0, 1000, 4096, True)],
])
def test_noalloc_matches_workspace_entry(gpu, cases):
    for k, (quant, rows, cols, f32) in enumerate(cases):
        run_both(gpu, quant, rows, cols, f32, seed=100 * k + rows % 97)


def test_noalloc_limit_and_validation(gpu):
    torch = gpu
    idx = torch.zeros(1, dtype=torch.int32, device="cuda")
    rows = (1 << 18) + 1  # one row beyond the static scratch
    raw = np.zeros(rows * 18, np.uint8)
    w = jk.Weight(jk.TensorView("big", jk.Q4_0, [rows, 32], raw), rows, 32)
    xq = torch.zeros(36, dtype=torch.uint8, device="cuda")
    with pytest.raises(jk.TensorBoundsError, match="static scratch"):
        jk.dev_gemv_q8_argmax_noalloc(w, xq, None, 1, None, idx)
    w.free()
    wi = jk.Weight(jk.TensorView("w", jk.I2_S, [4, 128], synth.gguf_weights(jk.I2_S, 4, 128, seed=1)), 4, 128)
    x = torch.zeros(256, dtype=torch.float32, device="cuda")
    with pytest.raises(jk.CapabilityMismatch):
        jk.dev_gemv_q8_argmax_noalloc(wi, None, x, 128, None, idx)
    torch.cuda.synchronize()
