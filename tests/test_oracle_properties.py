"""Pins of the oracle that do not depend on the oracle's own formulas.

 * f16 decode: exhaustive over all 65,536 patterns against numpy's float16 conversion.
 * block layouts: independent encoders (integer quants + scales -> GGUF bytes) whose
   decode through the oracle must return the encoded values.
 * quantizers: closed-form invariants (scale = amax / 127, round-to-nearest bound,
   extreme element at +-127, sanitization, bsums, sequential sums via np.cumsum).
 * dot / GEMV / GEMM / BitLinear: float64 matrix products of the dequantized operands,
   at the reference's own tolerances (tests/wave4_quant_gemv_and_argmax.rs:360-542,
   tests/wave3_prefill_gqa_and_gemm.rs:123-189).
"""
import numpy as np
import pytest

import oracle as O
import refgen as R

Q4_0, Q8_0, Q4_K, Q6_K, TQ2_0, I2_S = 2, 8, 12, 14, 35, 36
BE = {Q4_0: 32, Q8_0: 32, Q4_K: 256, Q6_K: 256, TQ2_0: 256, I2_S: 128}
BB = {Q4_0: 18, Q8_0: 34, Q4_K: 144, Q6_K: 210, TQ2_0: 66, I2_S: 32}


def dequant_matrix(quant, raw, rows, cols):
    """Row-by-row oracle dequantization (the weights' f32 values)."""
    out = np.zeros((rows, cols), np.float32)
    for r in range(rows):
        out[r] = O.dequantize_tensor_row(quant, [rows, cols], raw, r, cols)
    return out


# ------------------------------------------------------------------ f16
def test_f16_exhaustive_against_numpy():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([O.f16_to_f32_ieee(int(b)) for b in bits], np.float32)
    fin = np.isfinite(ref)
    assert np.array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))
    inf = np.isinf(ref)
    assert np.array_equal(got[inf], ref[inf])
    assert np.all(np.isnan(got[np.isnan(ref)]))
    fgot = np.array([O.f16_to_f32_finite(int(b)) for b in bits], np.float32)
    assert np.array_equal(fgot[fin].view(np.uint32), ref[fin].view(np.uint32))
    assert np.all(fgot[~fin] == 0.0) and not np.any(np.signbit(fgot[~fin]))


# ------------------------------------------------------------------ encoders
def f16(v):
    return int(np.float16(v).view(np.uint16))


def put16(buf, off, bits):
    buf[off] = bits & 0xFF
    buf[off + 1] = bits >> 8


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_q4_k_encoder_roundtrip(seed):
    """GGUF Q4_K: 6-bit scales/mins packed in 12 bytes, nibbles lo -> elements 64c+l,
    hi -> 64c+32+l. Encode chosen values, decode with the oracle."""
    rng = np.random.default_rng(seed)
    sc = rng.integers(0, 64, 8)
    mn = rng.integers(0, 64, 8)
    q = rng.integers(0, 16, 256)
    d, dmin = np.float16(rng.uniform(0.01, 1)), np.float16(rng.uniform(0.01, 1))
    blk = np.zeros(144, np.uint8)
    put16(blk, 0, f16(d))
    put16(blk, 2, f16(dmin))
    for j in range(4):
        blk[4 + j] = sc[j] | ((sc[j + 4] >> 4) << 6)
        blk[8 + j] = mn[j] | ((mn[j + 4] >> 4) << 6)
        blk[12 + j] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    for c in range(4):
        for l in range(32):
            blk[16 + 32 * c + l] = q[64 * c + l] | (q[64 * c + 32 + l] << 4)
    out = O.dequantize_row_bytes(Q4_K, blk, 256)
    sub = np.arange(256) // 32
    d32, m32 = np.float32(d), np.float32(dmin)
    exp = (d32 * sc[sub].astype(np.float32)) * q.astype(np.float32) - (m32 * mn[sub].astype(np.float32))
    assert np.array_equal(out, exp.astype(np.float32))


@pytest.mark.parametrize("seed", [0, 1])
def test_q6_k_encoder_roundtrip(seed):
    """GGUF Q6_K: ql low/high nibbles + qh 2-bit fields, 16 i8 scales, d at byte 208."""
    rng = np.random.default_rng(seed)
    q = rng.integers(-32, 32, 256)
    sc = rng.integers(-128, 128, 16)
    d = np.float16(rng.uniform(0.001, 0.1))
    blk = np.zeros(210, np.uint8)
    u = q + 32
    for h in range(2):
        for l in range(32):
            n = 128 * h
            v1, v2, v3, v4 = u[n + l], u[n + l + 32], u[n + l + 64], u[n + l + 96]
            blk[64 * h + l] = (v1 & 15) | ((v3 & 15) << 4)
            blk[64 * h + l + 32] = (v2 & 15) | ((v4 & 15) << 4)
            blk[128 + 32 * h + l] = (v1 >> 4) | ((v2 >> 4) << 2) | ((v3 >> 4) << 4) | ((v4 >> 4) << 6)
    blk[192:208] = (sc & 0xFF).astype(np.uint8)
    put16(blk, 208, f16(d))
    out = O.dequantize_row_bytes(Q6_K, blk, 256)
    grp = np.arange(256) // 16  # element e belongs to scale (e // 16)
    exp = (np.float32(d) * sc[grp].astype(np.float32)) * q.astype(np.float32)
    assert np.array_equal(out, exp.astype(np.float32))


def test_q4_0_q8_0_tq2_0_i2_s_encoder_roundtrip():
    rng = np.random.default_rng(5)
    d = np.float16(0.37)
    # Q4_0: q in [-8, 7]; element i < 16 low nibble of byte i, element 16 + i high nibble
    q = rng.integers(-8, 8, 32)
    blk = np.zeros(18, np.uint8)
    put16(blk, 0, f16(d))
    blk[2:] = (q[:16] + 8) | ((q[16:] + 8) << 4)
    assert np.array_equal(O.dequantize_row_bytes(Q4_0, blk, 32), np.float32(d) * q.astype(np.float32))
    # Q8_0
    q = rng.integers(-128, 128, 32)
    blk = np.zeros(34, np.uint8)
    put16(blk, 0, f16(d))
    blk[2:] = q & 0xFF
    assert np.array_equal(O.dequantize_row_bytes(Q8_0, blk, 32), np.float32(d) * q.astype(np.float32))
    # TQ2_0 crate layout: element 4i + j = bits 2j of qs[i]
    t = rng.integers(-1, 2, 256)
    blk = np.zeros(66, np.uint8)
    put16(blk, 0, f16(d))
    u = (t + 1).reshape(64, 4)
    blk[2:] = u[:, 0] | (u[:, 1] << 2) | (u[:, 2] << 4) | (u[:, 3] << 6)
    assert np.array_equal(O.dequantize_row_bytes(TQ2_0, blk, 256), np.float32(d) * t.astype(np.float32))
    # I2_S: byte g holds elements g, 32+g, 64+g, 96+g in bits 7:6, 5:4, 3:2, 1:0; f32 trailer
    t = rng.integers(-1, 2, 128)
    u = (t + 1).reshape(4, 32)
    row = np.zeros(64, np.uint8)
    row[:32] = (u[0] << 6) | (u[1] << 4) | (u[2] << 2) | u[3]
    row[32:36] = np.frombuffer(np.float32(0.75).tobytes(), np.uint8)
    assert np.array_equal(O.dequantize_row_bytes(I2_S, row, 128), np.float32(0.75) * t.astype(np.float32))


# ------------------------------------------------------------------ quantizers
def _specials(rng, n):
    x = rng.standard_normal(n).astype(np.float32) * rng.choice([1e-3, 1.0, 40.0], size=n).astype(np.float32)
    pick = rng.random(n) < 0.03
    x[pick] = rng.choice(np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 1e-40], np.float32), size=int(pick.sum()))
    return x


@pytest.mark.parametrize("seed", range(4))
def test_quantize_q8_0_and_q8_k_invariants(seed):
    rng = np.random.default_rng(seed)
    for be, fn in ((32, O.quantize_row_q8_0), (256, O.quantize_row_q8_k)):
        x = _specials(rng, be * 24)
        x[:be] = np.nan  # all-non-finite block
        x[be:2 * be] = 0.0  # all-zero block
        blocks = fn(x)
        for b, blk in enumerate(blocks):
            xb = x[b * be:(b + 1) * be]
            fin = np.isfinite(xb)
            amax = np.float32(np.max(np.abs(xb[fin]))) if fin.any() else np.float32(0)
            qs = blk["qs"].astype(np.int64)
            if amax == 0:
                assert blk["d"] == 0 and np.all(qs == 0)
                continue
            assert blk["d"] == np.float32(amax / np.float32(127.0))
            assert np.all(qs[~fin] == 0) and np.all(np.abs(qs) <= 127)
            inv = np.float32(127.0) / amax
            v = (xb[fin].astype(np.float32) * inv).astype(np.float64)
            assert np.all(np.abs(v - qs[fin]) <= 0.5 + 1e-12)  # round to nearest
            assert np.all(np.sign(qs[fin]) * np.sign(v) >= 0)
            assert 127 in np.abs(qs[fin])
            if be == 256:
                assert np.array_equal(blk["bsums"], qs.reshape(16, 16).sum(1).astype(np.int16))


@pytest.mark.parametrize("k", [32, 40, 256, 300, 4096])
def test_act_q8_invariants(k):
    rng = np.random.default_rng(k)
    m = 3
    x = _specials(rng, m * k).reshape(m, k)
    a = O.ActQ8(x, m, k)
    kp = (k + 31) // 32 * 32
    clean = np.zeros((m, kp), np.float32)
    clean[:, :k] = np.where(np.isfinite(x), x, 0.0)
    for r in range(m):
        for b in range(kp // 32):
            blk = clean[r, 32 * b:32 * b + 32]
            seq = np.cumsum(np.concatenate([[np.float32(0.0)], blk]).astype(np.float32), dtype=np.float32)[-1]
            assert a.sums[r, b].view(np.uint32) == np.float32(seq).view(np.uint32)
            amax = np.max(np.abs(blk))
            if amax < np.float32(1e-30):
                assert a.scales[r, b] == 0 and np.all(a.qs[r, 32 * b:32 * b + 32] == 0)
            else:
                assert a.scales[r, b] == np.float32(amax / np.float32(127))
                qs = a.qs[r, 32 * b:32 * b + 32].astype(np.float64)
                v = (blk * (np.float32(127) / amax)).astype(np.float64)
                assert np.all(np.abs(v - qs) <= 0.5 + 1e-12)
        for c in range(kp // 16):
            s16 = np.cumsum(clean[r, 16 * c:16 * c + 16], dtype=np.float32)[-1]
            assert a.sums16[r, c].view(np.uint32) == np.float32(s16).view(np.uint32)
        for sb in range((k + 255) // 256):
            assert a.super256[r, sb] == max(0.0, a.scales[r, 8 * sb:8 * sb + 8].max())


def test_quantize_absmax_equals_subln_when_rms_is_one():
    rng = np.random.default_rng(3)
    x = rng.choice(np.array([-1.0, 1.0], np.float32), size=2560)
    q1, s1 = O.subln_quantize_absmax_i8(x, np.ones_like(x), 0.0)
    q2, s2 = O.quantize_absmax_i8(x)
    assert np.array_equal(q1, q2) and s1 == s2 and s1 == np.float32(1.0) / np.float32(127.0)


def test_quantize_absmax_bounds():
    rng = np.random.default_rng(9)
    x = rng.standard_normal(6912).astype(np.float32)
    q, s = O.quantize_absmax_i8(x)
    assert s == np.float32(np.max(np.abs(x)) / np.float32(127))
    v = (x / np.float32(s)).astype(np.float64)
    assert np.all(np.abs(v - q) <= 0.5 + 1e-12) and np.abs(q).max() == 127


# ------------------------------------------------------------------ dots vs float64
def _deq_q8(blocks):
    return (blocks["qs"].astype(np.float32) * blocks["d"][:, None]).reshape(-1)


@pytest.mark.parametrize("k", [256, 1536, 2048, 3584, 5120])
def test_k_quant_gemv_vs_f64_on_dequantized_activations(k):
    """tests/wave4_quant_gemv_and_argmax.rs:360-542: rel-L2 < 1e-5 against a float64
    matvec of the dequantized Q8_K activations; < 1.5e-2 against the f32 activations."""
    rows = 5
    x = R.gen_activation(k, 700 + k)
    xq = O.quantize_row_q8_k(x)
    xd = _deq_q8(xq).astype(np.float64)
    for quant, fill, seed in ((Q4_K, R.fill_q4_k, 11), (Q6_K, R.fill_q6_k, 33), (TQ2_0, R.fill_tq2_0, 55)):
        raw = fill(rows, k, seed + k)
        out = O.gemv_q8(quant, [k, rows], raw, xq, rows)
        W = dequant_matrix(quant, raw, rows, k).astype(np.float64)
        assert R.rel_l2(out, W @ xd) < 1e-5, quant
        assert R.rel_l2(out, W @ x.astype(np.float64)) < 1.5e-2, quant
        if quant == Q4_K:
            f = O.vec_dot_f32(Q4_K, [k, rows], raw, x, rows)
            assert R.rel_l2(f, W @ x.astype(np.float64)) < 1e-5
        if quant == Q6_K:
            f = O.vec_dot_f32(Q6_K, [k, rows], raw, x, rows)
            assert R.rel_l2(f, W @ x.astype(np.float64)) < 1e-5


@pytest.mark.parametrize("k,n", [(128, 1), (896, 3), (2048, 4), (4096, 17)])
def test_q4_0_q8_0_gemv_vs_f64(k, n):
    """tests/wave4_quant_gemv_and_argmax.rs:253-348 (cosine > 0.9995 vs f32 vec_dot),
    tightened to rel-L2 < 1e-5 against float64 on the dequantized Q8_0 activations."""
    x = R.gen_activation(k, 100 + k)
    xq = O.quantize_row_q8_0(x)
    xd = _deq_q8(xq).astype(np.float64)
    for quant, fill in ((Q4_0, R.fill_q4_0), (Q8_0, R.fill_q8_0)):
        raw = fill(n, k, 7 + k)
        W = dequant_matrix(quant, raw, n, k).astype(np.float64)
        out = O.gemv_q8(quant, [k, n], raw, xq, n)
        assert R.rel_l2(out, W @ xd) < 1e-5
        f = O.vec_dot_f32(quant, [k, n], raw, x, n)
        assert R.rel_l2(f, W @ x.astype(np.float64)) < 1e-5
        assert R.cosine(out, f) > 0.9995


def test_single_row_vec_dot_equals_gemv_row():
    k = 1024
    x = R.gen_activation(k, 3)
    xq = O.quantize_row_q8_k(x)
    raw = R.fill_q4_k(3, k, 4)
    full = O.gemv_q8(Q4_K, [3, k], raw, xq, 3)
    row_bytes = k // 256 * 144
    for r in range(3):
        v = O.vec_dot_q8(Q4_K, raw[r * row_bytes:(r + 1) * row_bytes], xq)
        assert np.float32(v) == full[r]


def test_tail_rows_fold_from_negative_zero():
    """run_4row_chunked_gemv (quant_q8.rs:1510-1560): rows below rows/4*4 start from +0.0,
    tail rows use `.sum()` (neutral element -0.0). Blocks whose value is -0.0 expose it."""
    rows, k = 5, 64
    raw = np.zeros(rows * 2 * 18, np.uint8)
    for blk in range(rows * 2):
        put16(raw, blk * 18, f16(-0.5))
        raw[blk * 18 + 2:blk * 18 + 18] = 0x88  # every quant is 8 - 8 = 0
    xq = O.quantize_row_q8_0(np.ones(k, np.float32))
    out = O.gemv_q8(Q4_0, [rows, k], raw, xq, rows)
    assert np.all(out == 0.0)
    assert list(np.signbit(out)) == [False, False, False, False, True]


def test_repack_logical_matches_block_dequant():
    """w_sc * q - w_mn of the repacked layout reproduces the GGUF dequantizers
    (repack.rs:2529-2598 round trip)."""
    rng = np.random.default_rng(1)
    for quant in (Q4_0, Q8_0, Q4_K, Q6_K, TQ2_0, I2_S):
        rows, cols = 9, 512
        from jk import synth
        raw = synth.random_weights(quant, rows, cols, seed=quant, specials=True)
        q, sc, mn, cps = O.repack_logical(quant, [rows, cols], raw, rows, cols)
        g = 16 * cps
        ws = np.repeat(sc, g, axis=1)
        wm = np.repeat(mn, g, axis=1) if mn is not None else np.float32(0.0)
        rec = (ws * q.astype(np.float32) - wm).astype(np.float32)
        W = dequant_matrix(quant, raw, rows, cols)
        assert np.array_equal(rec, W), quant  # +0.0 == -0.0 for the zero-scale blocks
    del rng


@pytest.mark.parametrize("quant", [Q8_0, Q4_0, Q4_K, Q6_K, TQ2_0, I2_S])
def test_repacked_gemm_on_lattice_activations(quant):
    """tests/wave3_prefill_gqa_and_gemm.rs:123-189: activations exactly on the Q8 grid make
    the activation quantization lossless, so the GEMM must match a float64 GEMM of the
    dequantized weights (max-rel < 1e-3 there; 1e-5 of the row norm here)."""
    from jk import synth
    rng = np.random.default_rng(quant)
    m, rows, cols = 6, 11, 512
    x = rng.integers(-127, 128, size=(m, cols)).astype(np.float32)
    x[:, ::32] = 127.0  # every 32-block has |x| max 127 -> scale 1.0, quants == x
    raw = synth.gguf_weights(quant, rows, cols, seed=quant)
    act = O.ActQ8(x, m, cols)
    assert np.all(act.scales == 1.0) and np.array_equal(act.qs[:, :cols], x.astype(np.int8))
    out = O.gemm_repacked(quant, [rows, cols], raw, rows, cols, act, 0, rows)
    W = dequant_matrix(quant, raw, rows, cols).astype(np.float64)
    ref = x.astype(np.float64) @ W.T
    for i in range(m):
        assert np.max(np.abs(out[i] - ref[i])) <= 1e-5 * np.linalg.norm(ref[i])


def test_repacked_gemm_row_slices_are_bit_identical():
    """tests/test_repack_gemv_gemm.rs:750-829: row-sliced outputs equal the full output."""
    from jk import synth
    rows, cols, m = 37, 1024, 5
    raw = synth.gguf_weights(Q4_K, rows, cols, seed=2)
    act = O.ActQ8(synth.activations((m, cols), 3), m, cols)
    full = O.gemm_repacked(Q4_K, [rows, cols], raw, rows, cols, act, 0, rows)
    for r0, r1 in ((0, 8), (5, 21), (30, 37)):
        part = O.gemm_repacked(Q4_K, [rows, cols], raw, rows, cols, act, r0, r1)
        assert np.array_equal(part.view(np.uint32), full[:, r0:r1].view(np.uint32))


@pytest.mark.parametrize("quant", [TQ2_0, I2_S, Q8_0])
def test_bitlinear_vs_f64(quant):
    from jk import synth
    rng = np.random.default_rng(quant)
    rows, cols = 13, 512
    raw = synth.gguf_weights(quant, rows, cols, seed=quant)
    a = rng.integers(-128, 128, cols).astype(np.int8)
    out = O.bitlinear_i8(quant, [rows, cols], raw, a, 0.0123, rows)
    W = dequant_matrix(quant, raw, rows, cols).astype(np.float64)
    ref = W @ (a.astype(np.float64) * np.float64(np.float32(0.0123)))
    assert R.rel_l2(out, ref) < 1e-6


def test_oracle_validation_errors():
    raw = np.zeros(4 * 18, np.uint8)
    xq = O.quantize_row_q8_0(np.ones(32, np.float32))
    assert O.status_of(O.gemv_q8, Q4_0, [4, 32], raw, xq, 4) == 0
    assert O.status_of(O.gemv_q8, Q4_0, [4, 32], raw, xq, 3) == 1      # output length
    assert O.status_of(O.gemv_q8, Q4_0, [4, 32], raw[:-1], xq, 4) == 1  # short buffer
    assert O.status_of(O.gemv_q8, Q8_0, [4, 32], raw, xq, 4) == 1      # view is not Q8_0
    assert O.status_of(O.gemv_q8, Q4_0, [32, 4], raw, xq, 4) == 0      # GGUF orientation
    assert O.status_of(O.vec_dot_q8, Q4_0, raw[:17], xq) == 1          # row length
