"""Known-answer tests of the oracle, transcribed from the reference crate's own tests.

Each test names the reference test it transcribes (file:line). These pin the oracle's
block layouts, scale handling, sanitization and signs against values the reference
asserts; the GPU library is then compared against the oracle.
"""
import math
import struct

import numpy as np
import pytest

import oracle as O

Q4_0, Q8_0, Q4_K, Q6_K, TQ2_0, I2_S = 2, 8, 12, 14, 35, 36


def u16(v):
    return list(struct.pack("<H", v))


def test_q8_0_dequant_and_vec_dot_1056():
    # src/quant.rs:2593-2629
    raw = np.zeros(34, np.uint8)
    raw[0:2] = u16(0x4000)
    raw[2:] = np.arange(1, 33)
    out = O.dequantize_row_bytes(Q8_0, raw, 32)
    assert np.array_equal(out, 2.0 * np.arange(1, 33, dtype=np.float32))
    assert np.all(O.dequantize_row_bytes(Q8_0, np.zeros(34, np.uint8), 32) == 0.0)
    dot = O.vec_dot_f32(Q8_0, [1, 32], raw, np.ones(32, np.float32), 1)
    assert abs(dot[0] - 1056.0) < 1e-4


def test_q6_k_all_minus_30_dot_minus_7680():
    # src/quant.rs:2632-2663
    raw = np.zeros(210, np.uint8)
    raw[208:210] = u16(0x3C00)
    raw[192:208] = 1
    raw[0:128] = 0x22
    out = O.dequantize_row_bytes(Q6_K, raw, 256)
    assert np.all(out == -30.0)
    dot = O.vec_dot_f32(Q6_K, [1, 256], raw, np.ones(256, np.float32), 1)
    assert abs(dot[0] + 7680.0) < 1e-3


def test_q6_k_d2_half_input():
    # tests/kernel_phase2_tests.rs:275-305
    raw = np.zeros(210, np.uint8)
    raw[208:210] = u16(0x4000)
    raw[192:208] = 1
    raw[0:128] = 0x22
    assert np.all(O.dequantize_row_bytes(Q6_K, raw, 256) == -60.0)
    dot = O.vec_dot_f32(Q6_K, [1, 256], raw, np.full(256, 0.5, np.float32), 1)
    assert abs(dot[0] + 7680.0) < 1e-3


def test_q4_0_nibbles_and_gguf_orientation():
    # src/quant.rs:2727-2748: d = 0.5, low nibble 10 -> +1.0, high nibble 5 -> -1.5; shape [32, 1]
    raw = np.zeros(18, np.uint8)
    raw[0:2] = u16(0x3800)
    raw[2:] = (0x05 << 4) | 0x0A
    out = O.dequantize_row_bytes(Q4_0, raw, 32)
    assert np.all(out[:16] == 1.0) and np.all(out[16:] == -1.5)
    dot = O.vec_dot_f32(Q4_0, [32, 1], raw, np.full(32, 2.0, np.float32), 1)
    assert abs(dot[0] + 16.0) < 1e-4


def test_dequantize_token_row_q4_0_q8_0():
    # src/quant.rs:2782-2830
    q4 = np.zeros(3 * 18, np.uint8)
    q4[0:2] = u16(0x3800)
    q4[2:18] = (0x07 << 4) | 0x09
    q4[36:38] = u16(0x3C00)
    q4[38:54] = (0x06 << 4) | 0x0A
    r0 = O.dequantize_tensor_row(Q4_0, [32, 3], q4, 0, 32)
    r2 = O.dequantize_tensor_row(Q4_0, [32, 3], q4, 2, 32)
    assert np.all(r0[:16] == 0.5) and np.all(r0[16:] == -0.5)
    assert np.all(r2[:16] == 2.0) and np.all(r2[16:] == -2.0)
    q8 = np.zeros(2 * 34, np.uint8)
    q8[34:36] = u16(0x4000)
    q8[36:68] = np.arange(1, 33)
    r1 = O.dequantize_tensor_row(Q8_0, [32, 2], q8, 1, 32)
    assert r1[0] == 2.0 and r1[31] == 64.0
    assert O.status_of(O.dequantize_tensor_row, Q8_0, [32, 2], q8, 2, 32) == 1
    # 1D row 0 ok, row 1 and a 16-wide output fail closed (quant.rs:2890-2905)
    z = np.zeros(34, np.uint8)
    O.dequantize_tensor_row(Q8_0, [32], z, 0, 32)
    assert O.status_of(O.dequantize_tensor_row, Q8_0, [32], z, 1, 32) == 1
    assert O.status_of(O.dequantize_tensor_row, Q8_0, [32], z, 0, 16) == 1


def test_i2_s_interleaved_groups():
    # src/quant.rs:2905-2913: byte (1<<4)|(2<<2) -> {-1, 0, +1, -1} * 0.25 across the 4 groups
    blk = np.full(32, 0x55, np.uint8)
    blk[0] = (1 << 4) | (2 << 2)
    out = O.dequantize_i2_s_block(blk, 0.25)
    assert out[0] == -0.25 and out[32] == 0.0 and out[64] == 0.25 and out[96] == -0.25
    assert np.all(out[1:32] == 0.0)


def test_q8_0_scale_and_quant_bounds():
    # tests/empirical_challenge_m4.rs:382-419
    blk = np.zeros(34, np.uint8)
    blk[2:] = 127
    assert np.all(O.dequantize_row_bytes(Q8_0, blk, 32) == 0.0)
    blk[0:2] = u16(0x8000)
    assert np.all(O.dequantize_row_bytes(Q8_0, blk, 32) == 0.0)
    blk[0:2] = u16(0x3C00)
    blk[2], blk[3], blk[4] = 0x80, 0x7F, 0x00
    out = O.dequantize_row_bytes(Q8_0, blk, 32)
    assert out[0] == -128.0 and out[1] == 127.0 and out[2] == 0.0
    blk[0:2] = u16(0x7E00)
    out = O.dequantize_row_bytes(Q8_0, blk, 32)
    assert out[0] == 0.0 and out[1] == 0.0


def test_q8_0_two_row_matvec_plus_minus_64():
    # tests/kernel_phase2_tests.rs:232-272
    raw = np.zeros(68, np.uint8)
    raw[0:2] = u16(0x3C00)
    raw[2:34] = 1
    raw[34:36] = u16(0x3800)
    raw[36:68] = np.uint8(254)  # -2 as i8
    out = O.vec_dot_f32(Q8_0, [2, 32], raw, np.full(32, 2.0, np.float32), 2)
    assert abs(out[0] - 64.0) < 1e-4 and abs(out[1] + 64.0) < 1e-4


def test_q4_k_monotonic_rows():
    # src/lib.rs:1365-1396: d = 1, dmin = 0, scales[0..4] = 1; nibbles lo = blk + 1, hi = blk + 2
    raw = np.zeros(288, np.uint8)
    for blk in range(2):
        base = blk * 144
        raw[base:base + 2] = u16(0x3C00)
        raw[base + 4:base + 8] = 1
        raw[base + 16:base + 144] = ((blk + 2) << 4) | (blk + 1)
    out = O.vec_dot_f32(Q4_K, [256, 2], raw, np.ones(256, np.float32), 2)
    assert out[0] > 0.0 and out[1] > out[0]


def test_tq2_0_pattern_0x92_and_scale_edges():
    # tests/test_unpack_tq1_0_and_tq2_0.rs:19-81
    blk = np.zeros(66, np.uint8)
    blk[0:2] = u16(0x3E00)
    blk[2:] = 0x92
    s, t = O.unpack_tq2_0_block_i8(blk)
    assert abs(s - 1.5) < 1e-5
    assert np.all(t[0::4] == 1) and np.all(t[1::4] == -1) and np.all(t[2::4] == 0) and np.all(t[3::4] == 1)
    blk[0:2] = u16(0x0000)
    assert O.unpack_tq2_0_block_i8(blk)[0] == 0.0
    blk[0:2] = u16(0x7C00)
    assert O.unpack_tq2_0_block_i8(blk)[0] == 0.0


def test_tq2_0_exhaustive_2bit_unpack():
    # tests/empirical_challenge_m3_bitlinear.rs:143-186 (all 256 byte values at every position)
    blk = np.zeros(66, np.uint8)
    blk[0:2] = u16(0x4100)
    for val in range(256):
        exp = [((val >> (2 * j)) & 3) - 1 for j in range(4)]
        for pos in (0, 17, 63):
            blk[2:] = 0
            blk[2 + pos] = val
            s, t = O.unpack_tq2_0_block_i8(blk)
            assert s == 2.5
            assert list(t[4 * pos:4 * pos + 4]) == exp
            rest = np.delete(t, np.arange(4 * pos, 4 * pos + 4))
            assert np.all(rest == -1)


def test_bitlinear_tq2_0_all_plus_one_is_64():
    # tests/test_unpack_tq1_0_and_tq2_0.rs:212-263 (TQ2_0 half): 256 * (+1 * 2) * (1.0 * 0.125)
    rows, cols = 4, 256
    raw = np.zeros(rows * 66, np.uint8)
    for r in range(rows):
        raw[r * 66:r * 66 + 2] = u16(0x3C00)
        raw[r * 66 + 2:r * 66 + 66] = 0xAA
    out = O.bitlinear_i8(TQ2_0, [rows, cols], raw, np.full(cols, 2, np.int8), 0.125, rows)
    assert np.all(np.abs(out - 64.0) < 1e-4)


def test_subln_quantize_absmax_i8_kats():
    # tests/test_unpack_tq1_0_and_tq2_0.rs:269-318
    q, s = O.subln_quantize_absmax_i8(np.array([3, -3, 3, -3], np.float32), np.ones(4, np.float32), 1e-5)
    assert abs(s - 1.0 / 127.0) < 1e-5
    assert list(q) == [127, -127, 127, -127]
    q, s = O.subln_quantize_absmax_i8(np.zeros(128, np.float32), np.ones(128, np.float32), 1e-5)
    assert s > 0.0 and math.isfinite(s) and np.all(q == 0)
    q, s = O.subln_quantize_absmax_i8(np.full(64, 1e-15, np.float32), np.ones(64, np.float32), 1e-5)
    assert s > 0.0 and np.all(q == 0)
    assert O.status_of(O.subln_quantize_absmax_i8, np.zeros(0, np.float32), np.zeros(0, np.float32), 1e-5) == 1


def _test_f32_row(n, seed):
    # src/quant_q8.rs:3388-3395
    v = [((i * 37 + seed * 13) % 29) for i in range(n)]
    return (np.array(v, np.float32) - 14.0) * 0.125


def test_quantizer_sanitization_and_bounds():
    # src/quant_q8.rs:3414-3482
    assert O.status_of(O.quantize_row_q8_0, np.zeros(0, np.float32), 0) == 1
    assert O.status_of(O.quantize_row_q8_0, np.ones(31, np.float32), 1) == 1
    assert O.status_of(O.quantize_row_q8_k, np.ones(256, np.float32), 0) == 1
    x = _test_f32_row(96, 1)
    x[3] = np.nan
    x[11] = -np.nan
    x[32 + 7] = np.inf
    x[32 + 19] = -np.inf
    x[64:96] = np.nan
    x[64] = np.inf
    x[95] = 0.0
    q = O.quantize_row_q8_0(x)
    assert q[0]["d"] > 0 and q[0]["qs"][3] == 0 and q[0]["qs"][11] == 0 and np.any(q[0]["qs"] != 0)
    assert q[1]["d"] > 0 and q[1]["qs"][7] == 0 and q[1]["qs"][19] == 0 and np.any(q[1]["qs"] != 0)
    assert q[2]["d"] == 0 and np.all(q[2]["qs"] == 0)
    x = _test_f32_row(768, 2)
    x[3] = np.nan
    x[16 + 9] = -np.nan
    x[256 + 5] = -np.inf
    x[256 + 37] = np.inf
    x[512:768] = np.nan
    x[512] = -np.inf
    k = O.quantize_row_q8_k(x)
    assert k[0]["d"] > 0 and k[0]["qs"][3] == 0 and k[0]["qs"][25] == 0 and np.any(k[0]["qs"] != 0)
    assert k[1]["d"] > 0 and k[1]["qs"][5] == 0 and k[1]["qs"][37] == 0
    assert k[2]["d"] == 0 and np.all(k[2]["qs"] == 0) and np.all(k[2]["bsums"] == 0)
    for blk in k:
        assert np.array_equal(blk["bsums"], blk["qs"].astype(np.int32).reshape(16, 16).sum(1).astype(np.int16))


def test_block32_quantizer_sums():
    # src/repack.rs:5569-5586: 40 values of 0.5 with NaN/+Inf/-Inf at 3, 7, 9
    x = np.full(40, 0.5, np.float32)
    x[3], x[7], x[9] = np.nan, np.inf, -np.inf
    a = O.ActQ8(x, 1, 40)
    assert a.qs[0, 3] == 0 and a.qs[0, 7] == 0 and a.qs[0, 9] == 0
    assert abs(a.sums[0, 0] - 14.5) < 1e-5 and abs(a.sums[0, 1] - 4.0) < 1e-5
    assert np.all(a.qs[0, 40:] == 0)  # zero-padded tail


def _i2s_kat_tensor():
    """The I2_S weights of src/ime.rs:1243-1262 (3 rows x 256, trits from (r + gp) % 3 etc.)."""
    rows, bpr = 3, 2
    raw = np.zeros(rows * bpr * 32 + 32, np.uint8)
    for r in range(rows):
        for b in range(bpr):
            off = (r * bpr + b) * 32
            for gp in range(32):
                t0, t1, t2, t3 = (r + gp) % 3, (b + gp + 1) % 3, (r + b + gp) % 3, (gp + 2) % 3
                raw[off + gp] = (t0 << 6) | (t1 << 4) | (t2 << 2) | t3
    raw[rows * bpr * 32:rows * bpr * 32 + 4] = list(struct.pack("<f", 0.25))
    return raw


def test_convert_i2_s_blocks_to_tq2_0_kat():
    # src/ime.rs:1289-1303: the first two blocks of the test tensor with scale bits 0x3800 (0.5):
    # the TQ2_0 unpack gives scale 0.5 and the two I2_S unpacks, in order
    raw = _i2s_kat_tensor()
    tq2 = O.convert_i2_s_blocks_to_tq2_0(raw[0:32], raw[32:64], 0x3800)
    scale, t = O.unpack_tq2_0_block_i8(tq2)
    assert abs(scale - 0.5) < 1e-6
    assert np.array_equal(t[:128], O.unpack_i2_s_block_i8(raw[0:32]))
    assert np.array_equal(t[128:], O.unpack_i2_s_block_i8(raw[32:64]))
    assert list(tq2[:2]) == [0x00, 0x38]


def test_convert_i2_s_to_tq2_0_exhaustive_bytes_and_bitlinear_round_trip():
    # every byte value in every group position of both blocks: the unpacked trits agree with the
    # I2_S unpack (closed form: field f of byte g is element 32 f + g); an I2_S field value of 3
    # (not a trit, t = 2) must come out as TQ2_0 field 3 as well (the reference keeps & 0x03)
    for v in range(256):
        blk0 = np.full(32, v, np.uint8)
        blk1 = np.roll(np.arange(32, dtype=np.uint8) * 7 + v, v % 32).astype(np.uint8)
        out = O.convert_i2_s_blocks_to_tq2_0(blk0, blk1, 0x3C00)
        _, t = O.unpack_tq2_0_block_i8(out)
        ref = np.array([((int(b) >> (6 - 2 * f)) & 3) - 1 for blk in (blk0, blk1) for f in range(4) for b in blk],
                       np.int8)
        assert np.array_equal(t, ref), v
    # BitLinear over the converted rows equals BitLinear over the I2_S rows when the f16 scale is
    # the tensor scale exactly (0.25): same trits, same scale, same block order (two I2_S blocks
    # per TQ2_0 block, and the reference sums each block's integer dot before scaling)
    raw = _i2s_kat_tensor()
    rows, cols = 3, 256
    tq2 = np.concatenate([O.convert_i2_s_blocks_to_tq2_0(raw[64 * r:64 * r + 32], raw[64 * r + 32:64 * r + 64], 0x3400)
                          for r in range(rows)])
    act = np.array([(i % 15) - 7 for i in range(cols)], np.int8)
    y_i2s = O.bitlinear_i8(I2_S, [rows, cols], raw, act, 0.5, rows)
    y_tq2 = O.bitlinear_i8(TQ2_0, [rows, cols], tq2, act, 0.5, rows)
    ref = np.array([sum(float(w) * (float(a) * 0.5) for w, a in
                        zip(O.dequantize_tensor_row(I2_S, [rows, cols], raw, r, cols), act)) for r in range(rows)])
    assert np.allclose(y_i2s, ref, atol=1e-4) and np.allclose(y_tq2, ref, atol=1e-4)
