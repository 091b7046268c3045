"""The oracle's Q4_1, Q5_1, Q2_K, Q3_K and IQ4_NL functions (dequantization, f32 vec_dot and the
repacked GEMM -- the entry points the reference offers these formats on).

Known answers transcribed from the reference's tests (file:line on each), plus checks the
oracle's formulas do not share: independent numpy encoders, bit-for-bit identities with formats
pinned elsewhere (Q5_1 without high bits = Q4_1; IQ4_NL = Q8_0 holding the table values; Q3_K =
Q6_K holding the same signed scales and quants) and float64 products of the dequantized operands.
"""
import struct

import numpy as np
import pytest

import oracle as O
import refgen as R

Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q2_K, Q3_K, Q6_K, IQ4_NL = 2, 3, 6, 7, 8, 10, 11, 14, 20
BE = {Q4_1: 32, Q5_1: 32, IQ4_NL: 32, Q2_K: 256, Q3_K: 256, Q8_0: 32, Q6_K: 256}
BB = {Q4_1: 20, Q5_1: 24, IQ4_NL: 18, Q2_K: 84, Q3_K: 110, Q8_0: 34, Q6_K: 210}
KVALUES = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], np.int64)


def u16(v):
    return list(struct.pack("<H", v))


def f16(v):
    return int(np.float16(v).view(np.uint16))


def same_bits(a, b):
    a, b = np.ascontiguousarray(a, np.float32), np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and bool(np.all((a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))))


def dequant_matrix(quant, raw, rows, cols):
    return np.stack([O.dequantize_tensor_row(quant, [rows, cols], raw, r, cols) for r in range(rows)])


# ------------------------------------------------------------------ known answers
def test_wave2_block_dequant_kats():
    # src/quant.rs:2836-2906
    b = np.zeros(20, np.uint8)
    b[0:2], b[2:4], b[4:20] = u16(0x3800), u16(0xB400), 0xF0
    out = O.dequantize_row_bytes(Q4_1, b, 32)
    assert np.all(np.abs(out[:16] + 0.25) < 1e-6) and np.all(np.abs(out[16:] - 7.25) < 1e-6)
    b = np.zeros(20, np.uint8)
    b[2:4] = u16(0xB800)  # d = 0, m = -0.5: the min survives
    assert np.all(O.dequantize_row_bytes(Q4_1, b, 32) == -0.5)
    b = np.zeros(24, np.uint8)
    b[0:2], b[2:4] = u16(0x3800), u16(0x3C00)
    b[4:8] = list(struct.pack("<I", 0x00010001))
    b[8] = 0x32
    out = O.dequantize_row_bytes(Q5_1, b, 32)
    assert abs(out[0] - 10.0) < 1e-6 and abs(out[16] - 10.5) < 1e-6
    b = np.zeros(84, np.uint8)
    b[0], b[16] = (1 << 4) | 2, 0x03
    b[80:82], b[82:84] = u16(0x3C00), u16(0x3800)
    assert abs(O.dequantize_row_bytes(Q2_K, b, 256)[0] - 5.5) < 1e-6
    b = np.zeros(110, np.uint8)
    b[96:104], b[104:108], b[32] = 0x11, 0xAA, 0x03
    b[108:110] = u16(0x3800)
    assert abs(O.dequantize_row_bytes(Q3_K, b, 256)[0] + 0.5) < 1e-6
    b = np.zeros(18, np.uint8)
    b[0:2], b[2], b[3] = u16(0x3C00), 0xF0, 0x08
    out = O.dequantize_row_bytes(IQ4_NL, b, 32)
    assert (out[0], out[16], out[1], out[17]) == (-127.0, 113.0, 1.0, -127.0)


def test_iq4_nl_all_lanes_sentinel():
    # src/quant.rs:3086-3131: four blocks with scales 1.0, -0.5, -0.0 and NaN (-> 0.0)
    scales = [0x3C00, 0xB800, 0x8000, 0x7E00]
    raw = np.zeros(4 * 18, np.uint8)
    for b, s in enumerate(scales):
        raw[18 * b:18 * b + 2] = u16(s)
        for j in range(16):
            lo, hi = (j + 3 * b) & 15, (15 - j + b) & 15
            raw[18 * b + 2 + j] = (hi << 4) | lo
    out = O.dequantize_row_bytes(IQ4_NL, raw, 128)
    for b, d in enumerate((1.0, -0.5, None, None)):
        blk = raw[18 * b:18 * b + 18]
        idx = np.concatenate([blk[2:] & 15, blk[2:] >> 4])
        exp = np.zeros(32, np.float32) if d is None else (np.float32(d) * KVALUES[idx].astype(np.float32))
        assert same_bits(out[32 * b:32 * b + 32], exp)  # d == +-0 and NaN both give +0.0


def make_activations(m, k, seed):
    """tests/test_repack_gemv_gemm.rs:51-63 (xorshift64*)."""
    out = np.empty(m * k, np.float32)
    s = ((seed * 0x9E3779B97F4A7C15) | 1) & 0xFFFFFFFFFFFFFFFF
    for i in range(m * k):
        s ^= s >> 12
        s ^= (s << 25) & 0xFFFFFFFFFFFFFFFF
        s ^= s >> 27
        u = (s * 0x2545F4914F6CDD1D) & 0xFFFFFFFFFFFFFFFF
        out[i] = np.float32(np.float32(u >> 40) / np.float32(1 << 24)) * np.float32(2.0) - np.float32(1.0)
    return out.reshape(m, k)


@pytest.mark.parametrize("q_idx,quant,cols,rows,tol", [(0, Q4_1, 256, 19, 1.5e-2), (2, Q5_1, 256, 17, 1.5e-2),
                                                       (3, Q2_K, 512, 15, 2.0e-2), (4, Q3_K, 512, 19, 1.5e-2),
                                                       (5, IQ4_NL, 256, 23, 1.5e-2)])
def test_wave2_new_quants_repack_gemm(q_idx, quant, cols, rows, tol):
    # tests/test_repack_gemv_gemm.rs:919-990 (the GEMM bars and the row dequant identities), with
    # the unquantized-activation reference computed in float64 here
    raw = R.build_synthetic(quant, rows, cols, q_idx + 17)
    W = dequant_matrix(quant, raw, rows, cols)
    stride = cols // BE[quant] * BB[quant]
    for r in (0, rows // 2, rows - 1):
        assert same_bits(O.dequantize_row_bytes(quant, raw[r * stride:(r + 1) * stride], cols), W[r])
    q, sc, mn, cps = O.repack_logical(quant, [cols, rows], raw, rows, cols)
    g = 16 * cps
    rec = np.repeat(sc, g, axis=1) * q.astype(np.float32) - (np.repeat(mn, g, axis=1) if mn is not None else 0)
    assert np.max(np.abs(rec - W)) < 1e-4
    for m in (1, 5, 8, 17, 64):
        x = make_activations(m, cols, 300 + q_idx * 10 + m)
        out = O.gemm_repacked(quant, [cols, rows], raw, rows, cols, O.ActQ8(x, m, cols), 0, rows)
        ref = x.astype(np.float64) @ W.astype(np.float64).T
        cos = float((out.ravel() @ ref.ravel()) / (np.linalg.norm(out) * np.linalg.norm(ref)))
        assert cos > 0.999 and R.rel_l2(out, ref) < tol, (quant, m, cos)


# ------------------------------------------------------------------ encoders
@pytest.mark.parametrize("seed", [0, 1])
def test_q4_1_q5_1_iq4_nl_encoders(seed):
    rng = np.random.default_rng(seed)
    d, m = np.float16(rng.uniform(-1, 1)), np.float16(rng.uniform(-1, 1))
    q = rng.integers(0, 32, 32)
    blk = np.zeros(24, np.uint8)
    blk[0:2], blk[2:4] = u16(f16(d)), u16(f16(m))
    blk[4:8] = list(struct.pack("<I", sum(int(q[j] >> 4) << j for j in range(32))))
    blk[8:] = (q[:16] & 15) | ((q[16:] & 15) << 4)
    exp = np.float32(d) * q.astype(np.float32) + np.float32(m)
    assert np.array_equal(O.dequantize_row_bytes(Q5_1, blk, 32), exp)
    q4 = q & 15
    b4 = np.zeros(20, np.uint8)
    b4[0:4] = blk[0:4]
    b4[4:] = (q4[:16]) | (q4[16:] << 4)
    assert np.array_equal(O.dequantize_row_bytes(Q4_1, b4, 32), np.float32(d) * q4.astype(np.float32) + np.float32(m))
    bi = np.zeros(18, np.uint8)
    bi[0:2] = u16(f16(d))
    bi[2:] = b4[4:]
    assert np.array_equal(O.dequantize_row_bytes(IQ4_NL, bi, 32), np.float32(d) * KVALUES[q4].astype(np.float32))


def encode_q2_k(d, dmin, sc, mn, q):
    blk = np.zeros(84, np.uint8)
    blk[0:16] = sc | (mn << 4)
    for half in range(2):
        for j in range(4):
            for part in range(2):
                for l in range(16):
                    blk[16 + 32 * half + 16 * part + l] |= q[128 * half + 32 * j + 16 * part + l] << (2 * j)
    blk[80:82], blk[82:84] = u16(f16(d)), u16(f16(dmin))
    return blk


def encode_q3_k(d, sc6, q):
    """sc6: 16 six-bit scales (value - 32 is the signed scale), q: 256 quants in -4..3."""
    blk = np.zeros(110, np.uint8)
    u = q + 4  # bit 2 set <=> hmask bit set (no -4)
    for half in range(2):
        for j in range(4):
            for part in range(2):
                for l in range(16):
                    e = 128 * half + 32 * j + 16 * part + l
                    blk[32 + 32 * half + 16 * part + l] |= (u[e] & 3) << (2 * j)
                    blk[16 * part + l] |= (u[e] >> 2) << (4 * half + j)
    for i in range(8):
        blk[96 + i] = (sc6[i] & 15) | ((sc6[i + 8] & 15) << 4)
    for i in range(4):
        blk[104 + i] = sum(((sc6[i + 4 * k] >> 4) & 3) << (2 * k) for k in range(4))
    blk[108:110] = u16(f16(d))
    return blk


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_q2_k_q3_k_encoders(seed):
    rng = np.random.default_rng(seed)
    d, dmin = np.float16(rng.uniform(0.01, 1)), np.float16(rng.uniform(0.01, 1))
    sc, mn, q = rng.integers(0, 16, 16), rng.integers(0, 16, 16), rng.integers(0, 4, 256)
    out = O.dequantize_row_bytes(Q2_K, encode_q2_k(d, dmin, sc, mn, q), 256)
    g = np.arange(256) // 16
    exp = (np.float32(d) * sc[g].astype(np.float32)) * q.astype(np.float32) - np.float32(dmin) * mn[g].astype(np.float32)
    assert np.array_equal(out, exp)
    sc6, q3 = rng.integers(0, 64, 16), rng.integers(-4, 4, 256)
    out = O.dequantize_row_bytes(Q3_K, encode_q3_k(d, sc6, q3), 256)
    exp = (np.float32(d) * (sc6[g] - 32).astype(np.float32)) * q3.astype(np.float32)
    assert np.array_equal(out, exp)


# ------------------------------------------------------------------ cross-format identities
def twins(kind, rows, cols, seed):
    rng = np.random.default_rng(seed)
    if kind == "q5_1=q4_1":
        a = R.build_synthetic(Q4_1, rows, cols, seed)
        nb = rows * cols // 32
        b = np.zeros(nb * 24, np.uint8)
        for i in range(nb):
            b[24 * i:24 * i + 4] = a[20 * i:20 * i + 4]
            b[24 * i + 8:24 * i + 24] = a[20 * i + 4:20 * i + 20]
        return Q4_1, a, Q5_1, b
    if kind == "iq4_nl=q8_0":
        a = R.build_synthetic(IQ4_NL, rows, cols, seed)
        nb = rows * cols // 32
        b = np.zeros(nb * 34, np.uint8)
        for i in range(nb):
            qs = a[18 * i + 2:18 * i + 18]
            b[34 * i:34 * i + 2] = a[18 * i:18 * i + 2]
            b[34 * i + 2:34 * i + 34] = np.concatenate([KVALUES[qs & 15], KVALUES[qs >> 4]]).astype(np.int8).view(np.uint8)
        return IQ4_NL, a, Q8_0, b
    # q3_k=q6_k: the same signed 16-element scales and quants in -4..3 (d != 0)
    nb = rows * cols // 256
    a, b = [], []
    for _ in range(nb):
        d = np.float16(rng.uniform(0.01, 0.2))
        sc6, q = rng.integers(0, 64, 16), rng.integers(-4, 4, 256)
        a.append(encode_q3_k(d, sc6, q))
        u = q + 32
        blk = np.zeros(210, np.uint8)
        for h in range(2):
            for l in range(32):
                n = 128 * h
                v1, v2, v3, v4 = u[n + l], u[n + l + 32], u[n + l + 64], u[n + l + 96]
                blk[64 * h + l] = (v1 & 15) | ((v3 & 15) << 4)
                blk[64 * h + l + 32] = (v2 & 15) | ((v4 & 15) << 4)
                blk[128 + 32 * h + l] = (v1 >> 4) | ((v2 >> 4) << 2) | ((v3 >> 4) << 4) | ((v4 >> 4) << 6)
        blk[192:208] = ((sc6 - 32) & 0xFF).astype(np.uint8)
        blk[208:210] = u16(f16(d))
        b.append(blk)
    return Q3_K, np.concatenate(a), Q6_K, np.concatenate(b)


@pytest.mark.parametrize("kind", ["q5_1=q4_1", "iq4_nl=q8_0", "q3_k=q6_k"])
def test_cross_format_identities(kind):
    rows, cols = 7, 512
    qa, wa, qb, wb = twins(kind, rows, cols, 11)
    shape = [rows, cols]
    assert same_bits(dequant_matrix(qa, wa, rows, cols), dequant_matrix(qb, wb, rows, cols))
    x = R.gen_activation(cols, 9)
    assert same_bits(O.vec_dot_f32(qa, shape, wa, x, rows), O.vec_dot_f32(qb, shape, wb, x, rows))
    X = R.gen_activation(3 * cols, 10).reshape(3, cols)
    act = O.ActQ8(X, 3, cols)
    assert same_bits(O.gemm_repacked(qa, shape, wa, rows, cols, act, 0, rows),
                     O.gemm_repacked(qb, shape, wb, rows, cols, act, 0, rows))


@pytest.mark.parametrize("quant", [Q4_1, Q5_1, Q2_K, Q3_K, IQ4_NL])
def test_vec_dot_f32_vs_f64(quant):
    rows, cols = 6, 1024
    raw = R.build_synthetic(quant, rows, cols, 3)
    x = R.gen_activation(cols, 4)
    out = O.vec_dot_f32(quant, [rows, cols], raw, x, rows)
    ref = dequant_matrix(quant, raw, rows, cols).astype(np.float64) @ x.astype(np.float64)
    assert R.rel_l2(out, ref) < 1e-5


def test_more_formats_validation():
    assert O.status_of(O.vec_dot_f32, Q4_1, [1, 32], np.zeros(20, np.uint8), np.ones(32, np.float32), 1) == 0
    assert O.status_of(O.vec_dot_f32, Q4_1, [1, 32], np.zeros(19, np.uint8), np.ones(32, np.float32), 1) == 1
    assert O.status_of(O.vec_dot_f32, Q3_K, [1, 255], np.zeros(110, np.uint8), np.ones(255, np.float32), 1) == 1
    assert O.status_of(O.bitlinear_i8, Q4_1, [1, 32], np.zeros(20, np.uint8), np.zeros(32, np.int8), 1.0, 1) == 1
