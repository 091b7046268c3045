"""The HIP library against the committed golden fixtures (tests/golden/*.npz), bit for bit.

The fixtures hold seeded inputs of the reference tests' construction and the oracle's
outputs for them; nothing here runs the oracle. Every call goes through the C ABI: the
host tier (synchronous slice signatures) and, for the GEMM, a device weight handle.
"""
import glob
import os

import numpy as np
import pytest

import jk

pytestmark = pytest.mark.gpu

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
Q4_0, Q8_0, Q4_K, Q6_K, TQ2_0, I2_S = jk.Q4_0, jk.Q8_0, jk.Q4_K, jk.Q6_K, jk.TQ2_0, jk.I2_S
Q5_0, Q5_K, TQ1_0 = jk.Q5_0, jk.Q5_K, jk.TQ1_0
CASES = sorted(p for p in glob.glob(os.path.join(HERE, "*.npz")) if not p.endswith("quantizers.npz"))
GEMV = {Q4_0: jk.gemv_q4_0_q8_0, Q8_0: jk.gemv_q8_0_q8_0, Q4_K: jk.gemv_q4_k_q8_k, Q6_K: jk.gemv_q6_k_q8_k,
        TQ2_0: jk.gemv_tq2_0_q8_k, Q5_0: jk.gemv_q5_0_q8_0, Q5_K: jk.gemv_q5_k_q8_k, TQ1_0: jk.gemv_tq1_0_q8_k}
VEC_F32 = {Q4_0: jk.vec_dot_q4_0, Q8_0: jk.vec_dot_q8_0, Q6_K: jk.vec_dot_q6_k, Q4_K: jk.vec_dot_q4_k_m,
           I2_S: jk.vec_dot_i2_s, Q5_0: jk.vec_dot_q5_0, Q5_K: jk.vec_dot_q5_k, jk.Q4_1: jk.vec_dot_q4_1,
           jk.Q5_1: jk.vec_dot_q5_1, jk.Q2_K: jk.vec_dot_q2_k, jk.Q3_K: jk.vec_dot_q3_k, jk.IQ4_NL: jk.vec_dot_iq4_nl}


def load(path):
    return dict(np.load(path, allow_pickle=False))


def bits_equal(a, b) -> bool:
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and bool(np.all((a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))))


@pytest.mark.parametrize("path", CASES, ids=os.path.basename)
def test_golden_case(gpu, path):
    f = load(path)
    quant, rows, cols = int(f["quant"]), int(f["rows"]), int(f["cols"])
    view = jk.TensorView("golden", quant, [rows, cols], f["w"])
    for r in range(rows):
        out = np.zeros(cols, np.float32)
        jk.dequantize_tensor_row(view, r, out)
        assert bits_equal(out, f["deq"][r]), (path, "dequant row", r)
    if "xq" in f:
        xq = jk.quantize_row_q8_0(f["x"]) if quant in jk.Q8_0_ACT else jk.quantize_row_q8_k(f["x"])
        assert np.array_equal(xq.view(np.uint8).reshape(-1), f["xq"]), (path, "activation blocks")
        y = np.zeros(rows, np.float32)
        GEMV[quant](y, view, xq)
        assert bits_equal(y, f["y_gemv"]), (path, "gemv", y, f["y_gemv"])
    if "y_gemm" in f:
        w = jk.Weight(view, rows, cols)
        m = f["X"].shape[0]
        yg = np.zeros(m * rows, np.float32)
        jk.host_gemm_repacked_f32(yg, w, f["X"], m, 0, rows)
        assert bits_equal(yg.reshape(m, rows), f["y_gemm"]), (path, "gemm")
        ys = np.zeros(m * 5, np.float32)
        jk.host_gemm_repacked_f32(ys, w, f["X"], m, 2, 7)
        assert bits_equal(ys.reshape(m, 5), f["y_gemm_rows"]), (path, "gemm rows 2..7")
        w.free()
    if "y_vec_f32" in f:
        y = np.zeros(rows, np.float32)
        VEC_F32[quant](y, view, f["x"])
        assert bits_equal(y, f["y_vec_f32"]), (path, "vec_dot f32")
    if "y_bitlinear" in f:
        y = np.zeros(rows, np.float32)
        jk.bitlinear_i8(y, view, f["act_i8"], float(f["act_scale"]))
        assert bits_equal(y, f["y_bitlinear"]), (path, "bitlinear")


def test_golden_quantizers(gpu):
    torch = gpu
    f = load(os.path.join(HERE, "quantizers.npz"))
    x = f["x"]
    assert np.array_equal(jk.quantize_row_q8_0(x).view(np.uint8).reshape(-1), f["q8_0"])
    assert np.array_equal(jk.quantize_row_q8_k(x).view(np.uint8).reshape(-1), f["q8_k"])
    k = x.size
    dx = torch.from_numpy(x.copy()).cuda()
    dw = torch.from_numpy(f["norm_w"].copy()).cuda()
    dq = torch.empty(k, dtype=torch.int8, device="cuda")
    ds = torch.empty(1, dtype=torch.float32, device="cuda")
    jk.dev_subln_quantize_absmax_i8(dx, dw, 1, k, 1e-5, dq, ds)
    clean = torch.from_numpy(np.nan_to_num(x, nan=0.0, posinf=0.0, neginf=0.0)).cuda()
    dq2 = torch.empty(k, dtype=torch.int8, device="cuda")
    ds2 = torch.empty(1, dtype=torch.float32, device="cuda")
    jk.dev_quantize_absmax_i8(clean, 1, k, dq2, ds2)
    torch.cuda.synchronize()
    assert np.array_equal(dq.cpu().numpy(), f["subln_q"])
    assert bits_equal(ds.cpu().numpy(), np.float32([f["subln_scale"]]))
    assert np.array_equal(dq2.cpu().numpy(), f["absmax_q"])
    assert bits_equal(ds2.cpu().numpy(), np.float32([f["absmax_scale"]]))
