"""Known-answer tests of the oracle for Q5_0, Q5_K and TQ1_0, transcribed from the reference
crate's own tests (each names the test it transcribes, file:line).
"""
import struct

import numpy as np

import oracle as O

Q5_0, Q8_0, Q5_K, TQ1_0, TQ2_0 = 6, 8, 13, 34, 35


def u16(v):
    return list(struct.pack("<H", v))


class RefLcg:
    """tests/test_q5_k_dequant_and_matvec.rs:114-138"""

    def __init__(self, seed):
        self.s = seed

    def next_u32(self):
        self.s = (self.s * 6364136223846793005 + 1) & ((1 << 64) - 1)
        return self.s >> 32

    def next_u8(self):
        return self.next_u32() & 0xFF

    def next_f32(self, lo, hi):
        v = np.float32(self.next_u32() & 0x7FFFFF) / np.float32(1 << 23)
        return np.float32(lo) + v * (np.float32(hi) - np.float32(lo))


def golden_q5_k_block():
    # tests/test_q5_k_dequant_and_matvec.rs:169-203
    raw = np.zeros(176, np.uint8)
    raw[0:2] = u16(0x3C00)
    raw[2:4] = u16(0x3800)
    raw[4], raw[8], raw[5], raw[9] = 2, 1, 3, 2
    raw[6], raw[10], raw[7], raw[11] = 4, 3, 5, 4
    raw[16:48] = 0x09
    raw[48:80] = 0x53
    raw[80:112] = 0x24
    return raw


def test_q5_k_golden_vector_step_by_step():
    # tests/test_q5_k_dequant_and_matvec.rs:169-244
    out = O.dequantize_row_bytes(Q5_K, golden_q5_k_block(), 256)
    assert np.all(out[0:32] == 37.5) and np.all(out[32:64] == 14.0)
    assert np.all(out[64:96] == 14.5) and np.all(out[96:128] == 88.0)
    assert np.all(out[128:] == 0.0)
    assert abs(float(out.sum(dtype=np.float32)) - 4928.0) < 1e-3


def test_q5_k_upper_subblock_packing():
    # tests/test_q5_k_dequant_and_matvec.rs:248-289: sc = 25, m = 17 from the j >= 4 packing
    raw = np.zeros(176, np.uint8)
    raw[0:2] = u16(0x4000)
    raw[2:4] = u16(0x3C00)
    raw[4], raw[8], raw[12] = 0x40, 0x40, 0x19
    raw[16:48] = 0x10
    raw[112:144] = 0x07
    out = O.dequantize_row_bytes(Q5_K, raw, 256)
    assert np.all(out[128:160] == 1133.0)


def test_q5_k_all_32_levels():
    # tests/test_q5_k_dequant_and_matvec.rs:292-326
    raw = np.zeros(176, np.uint8)
    raw[0:2] = u16(0x3C00)
    raw[4] = 1
    for l in range(32):
        raw[48 + l] = l & 0x0F
        if l >= 16:
            raw[16 + l] = 0x01
    out = O.dequantize_row_bytes(Q5_K, raw, 256)
    assert np.array_equal(out[:32], np.arange(32, dtype=np.float32))


def test_q5_k_edge_blocks():
    # tests/test_q5_k_dequant_and_matvec.rs:329-417
    assert np.all(O.dequantize_row_bytes(Q5_K, np.zeros(176, np.uint8), 256) == 0.0)
    raw = np.zeros(176, np.uint8)
    raw[0:2] = u16(0x3C00)
    raw[4:8] = 1
    raw[12:16] = 0x11
    raw[16:176] = 0xFF
    assert np.all(O.dequantize_row_bytes(Q5_K, raw, 256) == 31.0)
    raw = np.zeros(176, np.uint8)
    raw[0:2] = u16(0x3400)
    raw[2:4] = u16(0x4000)
    raw[4], raw[8] = 1, 5
    raw[48:80] = 10
    assert np.all(O.dequantize_row_bytes(Q5_K, raw, 256)[:32] == -7.5)
    raw = np.zeros(176, np.uint8)
    raw[0:2] = u16(0x0001)  # subnormal d
    raw[2:4] = u16(0x7C00)  # +inf dmin decodes to 0.0
    out = O.dequantize_row_bytes(Q5_K, raw, 256)
    assert np.all(np.isfinite(out))


def test_matvec_q5_k_single_block_row():
    # tests/test_q5_k_dequant_and_matvec.rs:420-466
    raw = golden_q5_k_block()
    out = O.vec_dot_f32(Q5_K, [1, 256], raw, np.ones(256, np.float32), 1)
    assert abs(out[0] - 4928.0) < 1e-3
    alt = np.where(np.arange(256) % 2 == 0, 1.0, -1.0).astype(np.float32)
    assert abs(O.vec_dot_f32(Q5_K, [1, 256], raw, alt, 1)[0]) < 1e-4


def _ggml_q5_k_rows(raw, rows, cols):
    """The reference test's GGML restatement (tests/test_q5_k_dequant_and_matvec.rs:62-107),
    written here over numpy arrays: d * sc * q - dmin * m with get_scale_min_k4."""
    nb = cols // 256
    W = np.zeros((rows, cols), np.float32)
    for r in range(rows):
        for b in range(nb):
            blk = raw[(r * nb + b) * 176:(r * nb + b + 1) * 176]
            d = np.float32(np.frombuffer(blk[0:2].tobytes(), np.float16)[0])
            dmin = np.float32(np.frombuffer(blk[2:4].tobytes(), np.float16)[0])
            s = blk[4:16].astype(np.int64)
            for j in range(8):
                if j < 4:
                    sc, m = s[j] & 63, s[j + 4] & 63
                else:
                    sc = (s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4)
                    m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4)
                c, half = j // 2, j % 2
                nib = (blk[48 + 32 * c:80 + 32 * c] >> (4 * half)) & 0x0F
                hb = (blk[16:48] >> (2 * c + half)) & 1
                q = (nib.astype(np.int64) + 16 * hb).astype(np.float32)
                W[r, b * 256 + 32 * j:b * 256 + 32 * j + 32] = (d * np.float32(sc)) * q - dmin * np.float32(m)
    return W


def test_matvec_q5_k_multi_block_rows_and_cols():
    # tests/test_q5_k_dequant_and_matvec.rs:469-522
    rows, cols = 4, 512
    rng = RefLcg(0xCAFEBABE12345678)
    raw = np.array([rng.next_u8() for _ in range(rows * 2 * 176)], np.uint8)
    for blk in range(rows * 2):
        raw[blk * 176:blk * 176 + 2] = u16(0x3C00)
        raw[blk * 176 + 2:blk * 176 + 4] = u16(0x3800)
    x = np.array([rng.next_f32(-1.0, 1.0) for _ in range(cols)], np.float32)
    out = O.vec_dot_f32(Q5_K, [rows, cols], raw, x, rows)
    W = _ggml_q5_k_rows(raw, rows, cols)
    assert np.array_equal(W.reshape(-1), np.concatenate(
        [O.dequantize_tensor_row(Q5_K, [rows, cols], raw, r, cols) for r in range(rows)]))
    for r in range(rows):
        exp = np.float32(0.0)
        for b in range(2):
            s = np.float32(0.0)
            for e in range(256):
                s = np.float32(s + W[r, 256 * b + e] * x[256 * b + e])
            exp = np.float32(exp + s)
        assert abs(out[r] - exp) < 1e-2 and abs(out[r] - exp) / max(abs(exp), 1.0) < 1e-4
        assert out[r] == exp  # same order of f32 operations: bit-identical


def test_q5_k_property_sweep_against_ggml_restatement():
    # tests/test_q5_k_dequant_and_matvec.rs:601-628
    rng = RefLcg(0x1337BEEF5555AAAA)
    for trial in range(20):
        blk = np.array([rng.next_u8() for _ in range(176)], np.uint8)
        blk[0:2] = u16(0x3C00 + trial * 10)
        blk[2:4] = u16(0x3800 + trial * 5)
        got = O.dequantize_row_bytes(Q5_K, blk, 256)
        assert np.max(np.abs(got - _ggml_q5_k_rows(blk, 1, 256)[0])) < 1e-4


def test_matvec_q5_k_dimension_errors():
    # tests/test_q5_k_dequant_and_matvec.rs:562-598
    raw = np.zeros(176, np.uint8)
    one = np.ones(256, np.float32)
    v = O.View(12, [1, 256], raw)  # a Q4_K_M view handed to the Q5_K matvec
    out = np.zeros(1, np.float32)
    assert O.lib().or_vec_dot_q5_k(O._p(out), O._sz(1), O.C.byref(v.c), O._p(one), O._sz(256)) == 1
    assert O.status_of(O.vec_dot_f32, Q5_K, [1, 256], raw, one, 1) == 0
    assert O.status_of(O.vec_dot_f32, Q5_K, [1, 256], raw, one[:128], 1) == 1
    assert O.status_of(O.vec_dot_f32, Q5_K, [1, 256], raw, one, 2) == 1
    assert O.status_of(O.vec_dot_f32, Q5_K, [1, 250], raw, one[:250], 1) == 1
    assert O.status_of(O.vec_dot_f32, Q5_K, [1, 256], raw[:175], one, 1) == 1


def test_tq1_0_unpack_pattern_65():
    # tests/test_unpack_tq1_0_and_tq2_0.rs:46-73: byte 65 = digits 2,0,1,2,0 -> +1,-1,0,+1,-1
    blk = np.zeros(54, np.uint8)
    blk[0:2] = u16(0x4000)
    blk[2:53] = 65
    blk[53] = 2
    s, t = O.unpack_tq1_0_block_i8(blk)
    assert abs(s - 2.0) < 1e-5
    for j, v in enumerate((1, -1, 0, 1, -1)):
        assert np.all(t[j:255:5] == v)
    assert t[255] == 1


def test_bitlinear_tq1_0_equals_tq2_0_all_plus_one():
    # tests/test_unpack_tq1_0_and_tq2_0.rs:211-262: bit-identical outputs, 64.0
    rows, cols = 4, 256
    t2 = np.zeros(rows * 66, np.uint8)
    t1 = np.zeros(rows * 54, np.uint8)
    for r in range(rows):
        t2[r * 66:r * 66 + 2] = u16(0x3C00)
        t2[r * 66 + 2:r * 66 + 66] = 0xAA
        t1[r * 54:r * 54 + 2] = u16(0x3C00)
        t1[r * 54 + 2:r * 54 + 53] = 242
        t1[r * 54 + 53] = 2
    a = np.full(cols, 2, np.int8)
    o2 = O.bitlinear_i8(TQ2_0, [rows, cols], t2, a, 0.125, rows)
    o1 = O.bitlinear_i8(TQ1_0, [rows, cols], t1, a, 0.125, rows)
    assert np.array_equal(o1.view(np.uint32), o2.view(np.uint32))
    assert np.all(np.abs(o1 - 64.0) < 1e-4)


def test_bitlinear_tq1_0_multi_block():
    # Inputs of tests/test_unpack_tq1_0_and_tq2_0.rs:129-164 (TQ1_0 half: 0x55 payload, d = 1.0,
    # act (i % 17) - 8, scale 0.05); the expected value comes from a base-3 decode written here.
    rows, cols = 8, 512
    raw = np.full(rows * 2 * 54, 0x55, np.uint8)
    for blk in range(rows * 2):
        raw[blk * 54:blk * 54 + 2] = u16(0x3C00)
    a = ((np.arange(cols) % 17) - 8).astype(np.int8)
    out = O.bitlinear_i8(TQ1_0, [rows, cols], raw, a, 0.05, rows)
    digits = [(0x55 // 3 ** j) % 3 - 1 for j in range(5)]
    t = np.array(digits * 51 + [0x55 % 3 - 1], np.int64)
    assert list(t[:5]) == [0, 0, -1, -1, 0]
    exp = np.float32(0.0)
    for b in range(2):
        dot = int(np.dot(t, a[256 * b:256 * b + 256].astype(np.int64)))
        exp = np.float32(exp + np.float32(dot) * (np.float32(1.0) * np.float32(0.05)))
    assert np.all(out == exp)
