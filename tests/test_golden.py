"""The committed golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU checks:
 * the fixture inputs are the reference tests' LCG constructions
   (tests/wave4_quant_gemv_and_argmax.rs:31-226, restated in refgen.py);
 * the oracle reproduces every stored output bit for bit;
 * the stored outputs agree with float64 products of the dequantized operands at the
   reference's own tolerances (rel-L2 < 1e-5 for the Q8 GEMV against its dequantized Q8
   blocks, tests/wave4_quant_gemv_and_argmax.rs:397-535), and row-sliced GEMM outputs
   equal the full GEMM's (tests/test_repack_gemv_gemm.rs:750-829).
"""
import glob
import os

import numpy as np
import pytest

import oracle as O
import refgen as R

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K, TQ1_0, TQ2_0, I2_S = 2, 6, 8, 12, 13, 14, 34, 35, 36
Q4_1, Q5_1, Q2_K, Q3_K, IQ4_NL = 3, 7, 10, 11, 20
FILL = {Q4_0: R.fill_q4_0, Q8_0: R.fill_q8_0, Q4_K: R.fill_q4_k, Q6_K: R.fill_q6_k, TQ2_0: R.fill_tq2_0,
        Q5_0: R.fill_q5_0, Q5_K: R.fill_q5_k, TQ1_0: R.fill_tq1_0}
FILL.update({q: (lambda r, c, s, q=q: R.build_synthetic(q, r, c, s)) for q in (Q4_1, Q5_1, Q2_K, Q3_K, IQ4_NL)})
Q8_0_ACT = (Q4_0, Q5_0, Q8_0)
CASES = sorted(p for p in glob.glob(os.path.join(HERE, "*.npz")) if not p.endswith("quantizers.npz"))


def load(path):
    return dict(np.load(path, allow_pickle=False))


def bits_equal(a, b) -> bool:
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and bool(np.all((a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))))


def dequant_q8_blocks(quant, xq_bytes, n):
    """f64 values of the quantized activation blocks (Q8_0: f32 d + 32 i8; Q8_K: f32 d,
    256 i8, 16 i16 bsums)."""
    raw = np.asarray(xq_bytes, np.uint8)
    if quant in Q8_0_ACT:
        blk = raw.reshape(-1, 36)
        d = blk[:, :4].copy().view(np.float32)[:, 0].astype(np.float64)
        q = blk[:, 4:].view(np.int8).astype(np.float64)
    else:
        blk = raw.reshape(-1, 292)
        d = blk[:, :4].copy().view(np.float32)[:, 0].astype(np.float64)
        q = blk[:, 4:260].view(np.int8).astype(np.float64)
    return (q * d[:, None]).reshape(-1)[:n]


def test_fixtures_present():
    names = {os.path.basename(p) for p in glob.glob(os.path.join(HERE, "*.npz"))}
    assert {"q4_0.npz", "q5_0.npz", "q8_0.npz", "q4_k.npz", "q5_k.npz", "q6_k.npz", "tq1_0.npz", "tq2_0.npz",
            "i2_s.npz", "q4_1.npz", "q5_1.npz", "q2_k.npz", "q3_k.npz", "iq4_nl.npz", "quantizers.npz"} <= names


@pytest.mark.parametrize("path", CASES, ids=os.path.basename)
def test_inputs_are_the_reference_constructions(path):
    f = load(path)
    quant, rows, cols = int(f["quant"]), int(f["rows"]), int(f["cols"])
    xs = int(f["xseed"])
    assert bits_equal(f["x"], R.gen_activation(cols, xs))
    assert bits_equal(f["X"].reshape(-1), R.gen_activation(f["X"].size, xs + 1))
    if quant in FILL:
        assert np.array_equal(f["w"], FILL[quant](rows, cols, int(f["wseed"])))


@pytest.mark.parametrize("path", CASES, ids=os.path.basename)
def test_oracle_reproduces_fixture(path):
    f = load(path)
    quant, rows, cols = int(f["quant"]), int(f["rows"]), int(f["cols"])
    shape, w = [rows, cols], f["w"]
    deq = np.stack([O.dequantize_tensor_row(quant, shape, w, r, cols) for r in range(rows)])
    assert bits_equal(deq, f["deq"])
    if "xq" in f:
        xq = O.quantize_row_q8_0(f["x"]) if quant in Q8_0_ACT else O.quantize_row_q8_k(f["x"])
        assert np.array_equal(xq.view(np.uint8).reshape(-1), f["xq"])
        assert bits_equal(O.gemv_q8(quant, shape, w, xq, rows), f["y_gemv"])
    if "y_gemm" in f:
        act = O.ActQ8(f["X"], f["X"].shape[0], cols)
        assert bits_equal(O.gemm_repacked(quant, shape, w, rows, cols, act, 0, rows), f["y_gemm"])
        assert bits_equal(O.gemm_repacked(quant, shape, w, rows, cols, act, 2, 7), f["y_gemm_rows"])
    if "y_vec_f32" in f:
        assert bits_equal(O.vec_dot_f32(quant, shape, w, f["x"], rows), f["y_vec_f32"])
    if "y_bitlinear" in f:
        a, s = O.quantize_absmax_i8(f["x"])
        assert np.array_equal(a, f["act_i8"]) and bits_equal(np.float32([s]), np.float32([f["act_scale"]]))
        assert bits_equal(O.bitlinear_i8(quant, shape, w, a, s, rows), f["y_bitlinear"])


@pytest.mark.parametrize("path", CASES, ids=os.path.basename)
def test_fixture_outputs_match_float64_products(path):
    f = load(path)
    quant, rows, cols = int(f["quant"]), int(f["rows"]), int(f["cols"])
    deq = f["deq"].astype(np.float64)
    if "y_gemv" in f:
        ref = deq @ dequant_q8_blocks(quant, f["xq"], cols)
        got = f["y_gemv"].astype(np.float64)
        assert np.linalg.norm(got - ref) <= 1e-5 * np.linalg.norm(ref)
    if "y_gemm" in f:
        # per-32 activation quantization of X against the unquantized product
        ref_m = f["X"].astype(np.float64) @ deq.T
        got_m = f["y_gemm"].astype(np.float64)
        assert np.linalg.norm(got_m - ref_m) <= 2e-2 * np.linalg.norm(ref_m)
        assert bits_equal(f["y_gemm_rows"], f["y_gemm"][:, 2:7])
    if "y_vec_f32" in f:
        ref = deq @ f["x"].astype(np.float64)
        assert np.linalg.norm(f["y_vec_f32"] - ref) <= 2e-2 * np.linalg.norm(ref)
    if "y_bitlinear" in f:
        a = f["act_i8"].astype(np.float64) * float(f["act_scale"])
        ref = deq @ a
        assert np.linalg.norm(f["y_bitlinear"] - ref) <= 1e-4 * np.linalg.norm(ref)


def test_quantizer_fixture():
    f = load(os.path.join(HERE, "quantizers.npz"))
    x = f["x"]
    assert np.array_equal(O.quantize_row_q8_0(x).view(np.uint8).reshape(-1), f["q8_0"])
    assert np.array_equal(O.quantize_row_q8_k(x).view(np.uint8).reshape(-1), f["q8_k"])
    q, s = O.subln_quantize_absmax_i8(x, f["norm_w"], 1e-5)
    assert np.array_equal(q, f["subln_q"]) and bits_equal(np.float32([s]), np.float32([f["subln_scale"]]))
    clean = np.nan_to_num(x, nan=0.0, posinf=0.0, neginf=0.0)
    qa, sa = O.quantize_absmax_i8(clean)
    assert np.array_equal(qa, f["absmax_q"]) and bits_equal(np.float32([sa]), np.float32([f["absmax_scale"]]))
    # closed forms: Q8_0 scale = amax / 127 per block of the sanitized row, |q| <= 127,
    # non-finite inputs quantize to 0
    blk = f["q8_0"].reshape(-1, 36)
    d = blk[:, :4].copy().view(np.float32)[:, 0]
    q8 = blk[:, 4:].view(np.int8)
    amax = np.abs(clean.reshape(-1, 32)).max(axis=1)
    assert bits_equal(d, (amax / np.float32(127.0)).astype(np.float32))
    assert q8.reshape(-1)[3] == 0 and q8.reshape(-1)[40] == 0 and q8.reshape(-1)[77] == 0
    assert np.abs(q8.astype(np.int32)).max() <= 127
