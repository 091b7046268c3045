"""The oracle's restatement of the compact 4-bit GEMM (PackedNibbleMatrix::gemm_rows,
repack.rs:5181-5397) against its repacked block-scaled GEMM (execute_gemm_repacked_rows,
repack.rs:2718-3042), which the device GEMM is held to bit for bit.

The two reference paths store the same weights differently (8-row nibble tiles with a
per-format tile-scale decode, repack.rs:4414-4644 and 5044-5090, versus logical i8 rows with
per-group scales, repack.rs:1724-2103) and share the per-block accumulation
(accumulate_scaled_tile_scalar, repack.rs:3045-3093). Equal outputs on adversarial payloads --
random bytes in every field, zero / subnormal / Inf / NaN scales, odd row counts that leave a
tile's last pair without its odd row, ragged token tiles and row slices -- show the nibble
packing, unpacking and scale decode carry the same numbers into the same sums, so the device
GEMM serves the PackedNibbleMatrix entry points too. A float64 product of the dequantized
operands pins both against the mathematics.
"""
import numpy as np
import pytest

import oracle as O
from jk import synth

Q4_0, Q4_1, Q4_K, Q8_0, IQ4_NL = 2, 3, 12, 8, 20


def same_bits(a, b):
    a, b = np.ascontiguousarray(a, np.float32), np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and bool(np.all((a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))))


def activations(m, k, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((m, k)) * rng.choice([1e-3, 1.0, 30.0], (m, k))).astype(np.float32)
    x[rng.random((m, k)) < 0.01] = 0.0
    return x


SHAPES = [(13, 256, 5, 0, 13), (37, 512, 11, 3, 30), (8, 1024, 1, 0, 8), (64, 256, 17, 9, 63), (3, 768, 9, 1, 2)]


@pytest.mark.parametrize("quant", [Q4_0, Q4_1, IQ4_NL, Q4_K])
@pytest.mark.parametrize("rows,cols,m,r0,r1", SHAPES)
def test_nibble_gemm_equals_repacked_gemm(quant, rows, cols, m, r0, r1):
    raw = synth.random_weights(quant, rows, cols, seed=rows * 131 + cols + quant, specials=True)
    act = O.ActQ8(activations(m, cols, rows + m), m, cols)
    for shape in ([rows, cols], [cols, rows]):
        nib = O.nibble_gemm_rows(quant, shape, raw, rows, cols, act, r0, r1)
        rep = O.gemm_repacked(quant, shape, raw, rows, cols, act, r0, r1)
        assert same_bits(nib, rep), np.argwhere(nib.view(np.uint32) != rep.view(np.uint32))[:5]


@pytest.mark.parametrize("quant", [Q4_0, Q4_1, IQ4_NL, Q4_K])
def test_nibble_gemm_matches_float64_product(quant):
    """Finite scales, and activations the quantizer represents exactly (multiples of 2^-3 with
    each 32-element block's maximum at 127 * 2^-3, so scale, quants and block sums are exact):
    the output is the float64 product of the dequantized weights and the activations, within
    the f32 rounding of the per-block accumulation."""
    rows, cols, m = 21, 512, 6
    raw = synth.gguf_weights(quant, rows, cols, seed=quant)
    rng = np.random.default_rng(3)
    q = rng.integers(-127, 128, (m, cols))
    q[:, ::32] = 127 * rng.choice([-1, 1], (m, cols // 32))
    x = (q * 0.125).astype(np.float32)
    act = O.ActQ8(x, m, cols)
    assert np.array_equal(act.qs[:, :cols], q) and np.all(act.scales == 0.125)
    w = np.stack([O.dequantize_tensor_row(quant, [rows, cols], raw, r, cols) for r in range(rows)]).astype(np.float64)
    ref = x.astype(np.float64) @ w.T
    got = O.nibble_gemm_rows(quant, [rows, cols], raw, rows, cols, act, 0, rows).astype(np.float64)
    bound = 1e-5 * (np.abs(x).astype(np.float64) @ np.abs(w).T)
    assert np.all(np.abs(got - ref) <= bound)


def test_nibble_gemm_refuses_other_formats_and_bad_shapes():
    """validate_nibble_quant (repack.rs:4231-4236) and the shape checks of
    execute_nibble_gemm_rows (repack.rs:5188-5236)."""
    rows, cols = 8, 256
    act = O.ActQ8(activations(2, cols, 1), 2, cols)
    with pytest.raises(O.OracleError):
        O.nibble_gemm_rows(Q8_0, [rows, cols], synth.gguf_weights(Q8_0, rows, cols, seed=1), rows, cols, act, 0, rows)
    raw = synth.gguf_weights(Q4_0, rows, cols, seed=1)
    assert O.nibble_gemm_rows(Q4_0, [rows, cols], raw, rows, cols, act, 0, 0).shape == (2, 0)
    with pytest.raises(O.OracleError):
        O.nibble_gemm_rows(Q4_0, [rows, cols], raw, rows, cols, act, 3, rows + 1)
    with pytest.raises(O.OracleError):
        O.nibble_gemm_rows(Q4_0, [rows, cols], raw, rows, cols, O.ActQ8(activations(2, 512, 1), 2, 512), 0, rows)
