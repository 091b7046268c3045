"""Pins of the oracle's Q5_0, Q5_K and TQ1_0 functions that do not depend on its own formulas.

 * block layouts: independent encoders (integer quants + scales -> GGUF bytes) decoded by
   the oracle; every TQ1_0 byte value against Python's integer base-3 digits.
 * cross-format identities, bit for bit on every entry point: Q5_K with all high bits clear
   is Q4_K; Q5_0 with all high bits set is Q8_0 holding the nibbles; TQ1_0 is TQ2_0 holding
   the same trits (the reference's own equivalence test,
   tests/test_unpack_tq1_0_and_tq2_0.rs:211-262, on every entry point).
 * GEMV / GEMM / BitLinear: float64 products of the dequantized operands at the reference's
   tolerances (tests/wave4_quant_gemv_and_argmax.rs:254-542, tests/wave3_prefill_gqa_and_gemm.rs:123-189).
"""
import numpy as np
import pytest

import oracle as O
import refgen as R

Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K, TQ1_0, TQ2_0 = 2, 6, 8, 12, 13, 14, 34, 35


def f16(v):
    return int(np.float16(v).view(np.uint16))


def put16(buf, off, bits):
    buf[off] = bits & 0xFF
    buf[off + 1] = bits >> 8


def dequant_matrix(quant, raw, rows, cols):
    return np.stack([O.dequantize_tensor_row(quant, [rows, cols], raw, r, cols) for r in range(rows)])


def same_bits(a, b):
    a, b = np.ascontiguousarray(a, np.float32), np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and bool(np.all((a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))))


# ------------------------------------------------------------------ encoders
def encode_q5_k(d, dmin, sc, mn, q):
    """GGUF Q5_K: Q4_K's header, qh[l] bit 2c (low nibble, element 64c + l) and bit 2c + 1
    (high nibble, element 64c + 32 + l), then the nibbles of chunk c at qs[32c + l]."""
    blk = np.zeros(176, np.uint8)
    put16(blk, 0, f16(d))
    put16(blk, 2, f16(dmin))
    for j in range(4):
        blk[4 + j] = sc[j] | ((sc[j + 4] >> 4) << 6)
        blk[8 + j] = mn[j] | ((mn[j + 4] >> 4) << 6)
        blk[12 + j] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    for c in range(4):
        for l in range(32):
            lo, hi = q[64 * c + l], q[64 * c + 32 + l]
            blk[48 + 32 * c + l] = (lo & 15) | ((hi & 15) << 4)
            blk[16 + l] |= ((lo >> 4) << (2 * c)) | ((hi >> 4) << (2 * c + 1))
    return blk


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_q5_k_encoder_roundtrip(seed):
    rng = np.random.default_rng(seed)
    sc, mn, q = rng.integers(0, 64, 8), rng.integers(0, 64, 8), rng.integers(0, 32, 256)
    d, dmin = np.float16(rng.uniform(0.01, 1)), np.float16(rng.uniform(0.01, 1))
    out = O.dequantize_row_bytes(Q5_K, encode_q5_k(d, dmin, sc, mn, q), 256)
    sub = np.arange(256) // 32
    exp = (np.float32(d) * sc[sub].astype(np.float32)) * q.astype(np.float32) - np.float32(dmin) * mn[sub].astype(np.float32)
    assert np.array_equal(out, exp.astype(np.float32))


def test_q5_0_encoder_roundtrip():
    """GGUF Q5_0: d, u32 qh (bit j: element j), nibbles (byte j: elements j, j + 16)."""
    rng = np.random.default_rng(3)
    for _ in range(5):
        q = rng.integers(-16, 16, 32)
        u = q + 16
        d = np.float16(rng.uniform(-1, 1))
        blk = np.zeros(22, np.uint8)
        put16(blk, 0, f16(d))
        qh = sum(int(u[j] >> 4) << j for j in range(32))
        blk[2:6] = [(qh >> (8 * i)) & 0xFF for i in range(4)]
        blk[6:] = (u[:16] & 15) | ((u[16:] & 15) << 4)
        s, t = O.unpack_q5_0_block_i8(blk)
        assert list(t) == list(q) and s == np.float32(d)
        assert np.array_equal(O.dequantize_row_bytes(Q5_0, blk, 32), np.float32(d) * q.astype(np.float32))


def test_tq1_0_every_byte_value():
    """Element 5i + j is base-3 digit j (least significant first) of byte 2 + i, minus 1, for
    all 256 byte values (243..255 included); element 255 is the lowest digit of byte 53."""
    blk = np.zeros(54, np.uint8)
    put16(blk, 0, 0x3C00)
    for val in range(256):
        exp = [(val // 3 ** j) % 3 - 1 for j in range(5)]
        for pos in (0, 26, 50):
            blk[2:] = 1  # digits 1, 0, 0, 0, 0 -> 0, -1, -1, -1, -1
            blk[2 + pos] = val
            s, t = O.unpack_tq1_0_block_i8(blk)
            assert s == 1.0 and list(t[5 * pos:5 * pos + 5]) == exp
        blk[53] = val
        assert O.unpack_tq1_0_block_i8(blk)[1][255] == val % 3 - 1


def encode_tq1_0(t, d_bits=0x3C00):
    """trits (256, values -1..1) -> one TQ1_0 block."""
    u = np.asarray(t, np.int64) + 1
    blk = np.zeros(54, np.uint8)
    put16(blk, 0, d_bits)
    blk[2:53] = (u[:255].reshape(51, 5) * np.array([1, 3, 9, 27, 81])).sum(axis=1)
    blk[53] = u[255]
    return blk


def encode_tq2_0(t, d_bits=0x3C00):
    u = (np.asarray(t, np.int64) + 1).reshape(64, 4)
    blk = np.zeros(66, np.uint8)
    put16(blk, 0, d_bits)
    blk[2:] = u[:, 0] | (u[:, 1] << 2) | (u[:, 2] << 4) | (u[:, 3] << 6)
    return blk


# ------------------------------------------------------------------ cross-format identities
def twin_q4_k_q5_k(rows, cols, seed):
    """A Q4_K matrix and the Q5_K matrix with the same header and nibbles and qh = 0."""
    q4 = R.fill_q4_k(rows, cols, seed)
    nb = rows * cols // 256
    q5 = np.zeros(nb * 176, np.uint8)
    for b in range(nb):
        q5[b * 176:b * 176 + 16] = q4[b * 144:b * 144 + 16]
        q5[b * 176 + 48:b * 176 + 176] = q4[b * 144 + 16:b * 144 + 144]
    return q4, q5


def twin_q8_0_q5_0(rows, cols, seed):
    """A Q5_0 matrix with every high bit set (q = nibble) and the Q8_0 matrix holding the nibbles."""
    q5 = R.fill_q5_0(rows, cols, seed)
    nb = rows * cols // 32
    q8 = np.zeros(nb * 34, np.uint8)
    for b in range(nb):
        q5[b * 22 + 2:b * 22 + 6] = 0xFF
        q8[b * 34:b * 34 + 2] = q5[b * 22:b * 22 + 2]
        nib = q5[b * 22 + 6:b * 22 + 22]
        q8[b * 34 + 2:b * 34 + 18] = nib & 15
        q8[b * 34 + 18:b * 34 + 34] = nib >> 4
    return q8, q5


def twin_tq2_0_tq1_0(rows, cols, seed):
    rng = np.random.default_rng(seed)
    nb = rows * cols // 256
    t = rng.integers(-1, 2, (nb, 256))
    d = [f16(v) for v in rng.uniform(-0.5, 0.5, nb)]
    d[0] = 0x7C00  # +inf -> 0.0 in both
    tq2 = np.concatenate([encode_tq2_0(t[b], d[b]) for b in range(nb)])
    tq1 = np.concatenate([encode_tq1_0(t[b], d[b]) for b in range(nb)])
    return tq2, tq1


TWINS = [(Q4_K, Q5_K, twin_q4_k_q5_k), (Q8_0, Q5_0, twin_q8_0_q5_0), (TQ2_0, TQ1_0, twin_tq2_0_tq1_0)]


@pytest.mark.parametrize("qa,qb,twin", TWINS, ids=["q5_k=q4_k", "q5_0=q8_0", "tq1_0=tq2_0"])
def test_cross_format_identities(qa, qb, twin):
    rows, cols = 9, 1024
    wa, wb = twin(rows, cols, 17)
    shape = [rows, cols]
    x = R.gen_activation(cols, 5)
    assert same_bits(dequant_matrix(qa, wa, rows, cols), dequant_matrix(qb, wb, rows, cols))
    xq = O.quantize_row_q8_0(x) if qa == Q8_0 else O.quantize_row_q8_k(x)
    assert same_bits(O.gemv_q8(qa, shape, wa, xq, rows), O.gemv_q8(qb, shape, wb, xq, rows))
    if qa != TQ2_0:
        assert same_bits(O.vec_dot_f32(qa, shape, wa, x, rows), O.vec_dot_f32(qb, shape, wb, x, rows))
    X = R.gen_activation(4 * cols, 6).reshape(4, cols)
    act = O.ActQ8(X, 4, cols)
    assert same_bits(O.gemm_repacked(qa, shape, wa, rows, cols, act, 0, rows),
                     O.gemm_repacked(qb, shape, wb, rows, cols, act, 0, rows))
    if qa in (TQ2_0, Q8_0) and qb == TQ1_0:
        a = np.random.default_rng(1).integers(-128, 128, cols).astype(np.int8)
        assert same_bits(O.bitlinear_i8(qa, shape, wa, a, 0.03, rows), O.bitlinear_i8(qb, shape, wb, a, 0.03, rows))


def test_q5_k_high_bits_add_sixteen_times_scale():
    """Setting every qh bit adds exactly 16 * d * sc to each dequantized value (before the
    min), i.e. q -> q + 16: checked on integer-valued scales where every value is exact."""
    rows, cols = 2, 512
    q4, q5 = twin_q4_k_q5_k(rows, cols, 3)
    for b in range(rows * cols // 256):
        q5[b * 176:b * 176 + 4] = [0x00, 0x3C, 0x00, 0x3C]  # d = dmin = 1.0
    hi = q5.copy()
    for b in range(rows * cols // 256):
        hi[b * 176 + 16:b * 176 + 48] = 0xFF
    lo_v, hi_v = dequant_matrix(Q5_K, q5, rows, cols), dequant_matrix(Q5_K, hi, rows, cols)
    raw = q5.reshape(-1, 176)
    for b in range(raw.shape[0]):
        s = raw[b, 4:16].astype(np.int64)
        sc = [s[j] & 63 if j < 4 else (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4) for j in range(8)]
        r, c0 = divmod(b * 256, cols)
        for g in range(8):
            diff = hi_v[r, c0 + 32 * g:c0 + 32 * g + 32] - lo_v[r, c0 + 32 * g:c0 + 32 * g + 32]
            assert np.all(diff == 16.0 * sc[g])


# ------------------------------------------------------------------ float64 products
def _deq_q8(blocks):
    return (blocks["qs"].astype(np.float32) * blocks["d"][:, None]).reshape(-1)


@pytest.mark.parametrize("k", [256, 1536, 2048, 3584, 5120])
def test_q5_k_tq1_0_gemv_vs_f64(k):
    """tests/wave4_quant_gemv_and_argmax.rs:360-542 (Q5_K, TQ1_0 arms): rel-L2 < 1e-5 against
    float64 on the dequantized Q8_K activations; < 1.5e-2 against the f32 activations."""
    rows = 5
    x = R.gen_activation(k, 700 + k)
    xq = O.quantize_row_q8_k(x)
    xd = _deq_q8(xq).astype(np.float64)
    for quant, fill, seed in ((Q5_K, R.fill_q5_k, 22), (TQ1_0, R.fill_tq1_0, 44)):
        raw = fill(rows, k, seed + k)
        out = O.gemv_q8(quant, [k, rows], raw, xq, rows)
        W = dequant_matrix(quant, raw, rows, k).astype(np.float64)
        assert R.rel_l2(out, W @ xd) < 1e-5, quant
        assert R.rel_l2(out, W @ x.astype(np.float64)) < 1.5e-2, quant
        if quant == Q5_K:
            f = O.vec_dot_f32(Q5_K, [k, rows], raw, x, rows)
            assert R.rel_l2(f, W @ x.astype(np.float64)) < 1e-5


@pytest.mark.parametrize("k,n", [(128, 1), (896, 3), (2048, 4), (4096, 17)])
def test_q5_0_gemv_vs_f64(k, n):
    """tests/wave4_quant_gemv_and_argmax.rs:254-348 (Q5_0 arm): cosine > 0.9995 against the
    f32 vec_dot, tightened to rel-L2 < 1e-5 against float64 on the dequantized activations."""
    x = R.gen_activation(k, 100 + k)
    xq = O.quantize_row_q8_0(x)
    raw = R.fill_q5_0(n, k, 300 + k + n)
    W = dequant_matrix(Q5_0, raw, n, k).astype(np.float64)
    out = O.gemv_q8(Q5_0, [k, n], raw, xq, n)
    assert R.rel_l2(out, W @ _deq_q8(xq).astype(np.float64)) < 1e-5
    f = O.vec_dot_f32(Q5_0, [k, n], raw, x, n)
    assert R.rel_l2(f, W @ x.astype(np.float64)) < 1e-5
    assert R.cosine(out, f) > 0.9995


@pytest.mark.parametrize("quant", [Q5_0, Q5_K, TQ1_0])
def test_repack_and_gemm_new_formats(quant):
    """The repacked layout reproduces the block dequantizers (w_sc * q - w_mn), and on
    lattice activations the GEMM matches a float64 GEMM of the dequantized weights."""
    from jk import synth
    rows, cols, m = 11, 512, 6
    raw = synth.random_weights(quant, rows, cols, seed=quant, specials=True)
    q, sc, mn, cps = O.repack_logical(quant, [rows, cols], raw, rows, cols)
    assert (mn is not None) == (quant == Q5_K) and cps == 2
    ws = np.repeat(sc, 32, axis=1)
    wm = np.repeat(mn, 32, axis=1) if mn is not None else np.float32(0.0)
    assert np.array_equal((ws * q.astype(np.float32) - wm).astype(np.float32), dequant_matrix(quant, raw, rows, cols))
    raw = synth.gguf_weights(quant, rows, cols, seed=quant)
    rng = np.random.default_rng(quant)
    x = rng.integers(-127, 128, size=(m, cols)).astype(np.float32)
    x[:, ::32] = 127.0
    out = O.gemm_repacked(quant, [rows, cols], raw, rows, cols, O.ActQ8(x, m, cols), 0, rows)
    ref = x.astype(np.float64) @ dequant_matrix(quant, raw, rows, cols).astype(np.float64).T
    for i in range(m):
        assert np.max(np.abs(out[i] - ref[i])) <= 1e-5 * np.linalg.norm(ref[i])


def test_bitlinear_tq1_0_vs_f64():
    from jk import synth
    rows, cols = 13, 512
    raw = synth.gguf_weights(TQ1_0, rows, cols, seed=1)
    a = np.random.default_rng(2).integers(-128, 128, cols).astype(np.int8)
    out = O.bitlinear_i8(TQ1_0, [rows, cols], raw, a, 0.0123, rows)
    W = dequant_matrix(TQ1_0, raw, rows, cols).astype(np.float64)
    assert R.rel_l2(out, W @ (a.astype(np.float64) * np.float64(np.float32(0.0123)))) < 1e-6


def test_new_format_validation():
    xq8 = O.quantize_row_q8_0(np.ones(64, np.float32))
    xqk = O.quantize_row_q8_k(np.ones(256, np.float32))
    raw5 = np.zeros(2 * 22, np.uint8)
    assert O.status_of(O.gemv_q8, Q5_0, [1, 64], raw5, xq8, 1) == 0
    assert O.status_of(O.gemv_q8, Q5_0, [1, 64], raw5[:-1], xq8, 1) == 1
    assert O.status_of(O.vec_dot_q8, Q5_0, raw5[:21], xq8[:1]) == 1
    assert O.status_of(O.vec_dot_q8, Q5_K, np.zeros(176, np.uint8), xqk) == 0
    assert O.status_of(O.vec_dot_q8, TQ1_0, np.zeros(53, np.uint8), xqk) == 1
    assert O.status_of(O.bitlinear_i8, Q5_K, [1, 256], np.zeros(176, np.uint8), np.zeros(256, np.int8), 1.0, 1) == 1
    assert O.status_of(O.bitlinear_i8, TQ1_0, [1, 256], np.zeros(54, np.uint8), np.zeros(256, np.int8), 1.0, 1) == 0
