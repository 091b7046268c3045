"""Seeded input generators of the reference crate's integration tests, restated in numpy.

The reference synthesizes all test inputs in-test with an LCG
(s = s * 6364136223846793005 + 1442695040888963407, tests/wave4_quant_gemv_and_argmax.rs:31-36);
these functions produce inputs of the same construction for the parity tests here.
"""
from __future__ import annotations

import numpy as np

M64 = (1 << 64) - 1


class Lcg:
    def __init__(self, seed: int, inc: int = 1442695040888963407):
        self.s = seed & M64
        self.inc = inc

    def next(self) -> int:
        self.s = (self.s * 6364136223846793005 + self.inc) & M64
        return self.s

    def hi32(self) -> int:
        return self.next() >> 32


def gen_activation(n: int, seed: int) -> np.ndarray:
    """tests/wave4_quant_gemv_and_argmax.rs:38-48"""
    g = Lcg(seed)
    r = np.array([g.hi32() for _ in range(n)], dtype=np.float64).astype(np.float32) / np.float32(4294967296.0)
    i = np.arange(n, dtype=np.float32)
    return ((r - np.float32(0.35)) * np.float32(1.4) + np.sin(i * np.float32(0.013)) * np.float32(0.2)).astype(np.float32)


def _u16(v: int):
    return [v & 0xFF, v >> 8]


def fill_q4_0(rows: int, cols: int, seed: int) -> np.ndarray:
    """tests/wave4_quant_gemv_and_argmax.rs:77-96"""
    nb = cols // 32
    raw = np.zeros(rows * nb * 18, np.uint8)
    g = Lcg(seed)
    scales = [0x3000, 0x3200, 0x3400, 0x3600]
    for r in range(rows):
        for b in range(nb):
            off = (r * nb + b) * 18
            raw[off:off + 2] = _u16(scales[(r + b) % 4])
            for j in range(16):
                lo = (g.next() >> 32) % 16
                hi = (g.next() >> 40) % 16
                raw[off + 2 + j] = (hi << 4) | lo
    return raw


def fill_q8_0(rows: int, cols: int, seed: int) -> np.ndarray:
    """tests/wave4_quant_gemv_and_argmax.rs:116-133"""
    nb = cols // 32
    raw = np.zeros(rows * nb * 34, np.uint8)
    g = Lcg(seed)
    scales = [0x2800, 0x2C00, 0x3000, 0x3200]
    for r in range(rows):
        for b in range(nb):
            off = (r * nb + b) * 34
            raw[off:off + 2] = _u16(scales[(r + b) % 4])
            for j in range(32):
                q = (g.hi32() % 127) - 63
                raw[off + 2 + j] = q & 0xFF
    return raw


def fill_q4_k(rows: int, cols: int, seed: int) -> np.ndarray:
    """tests/wave4_quant_gemv_and_argmax.rs:135-153"""
    nb = cols // 256
    raw = np.zeros(rows * nb * 144, np.uint8)
    g = Lcg(seed)
    for blk in range(rows * nb):
        off = blk * 144
        raw[off:off + 2] = _u16(0x3000)
        raw[off + 2:off + 4] = _u16(0x2800)
        for idx in range(4, 16):
            raw[off + idx] = g.hi32() % 31 + 1
        for idx in range(16, 144):
            raw[off + idx] = g.hi32() & 0xFF
    return raw


def fill_q6_k(rows: int, cols: int, seed: int) -> np.ndarray:
    """tests/wave4_quant_gemv_and_argmax.rs:175-193"""
    nb = cols // 256
    raw = np.zeros(rows * nb * 210, np.uint8)
    g = Lcg(seed)
    for blk in range(rows * nb):
        off = blk * 210
        for idx in range(192):
            raw[off + idx] = g.hi32() & 0xFF
        for idx in range(192, 208):
            raw[off + idx] = ((g.hi32() % 15) - 7) & 0xFF
        raw[off + 208:off + 210] = _u16(0x3000)
    return raw


def fill_tq2_0(rows: int, cols: int, seed: int) -> np.ndarray:
    """tests/wave4_quant_gemv_and_argmax.rs:210-226"""
    nb = cols // 256
    raw = np.zeros(rows * nb * 66, np.uint8)
    g = Lcg(seed)
    for blk in range(rows * nb):
        off = blk * 66
        raw[off:off + 2] = _u16(0x3400)
        for idx in range(2, 66):
            raw[off + idx] = g.hi32() & 0xFF
    return raw


def fill_q5_0(rows: int, cols: int, seed: int) -> np.ndarray:
    """tests/wave4_quant_gemv_and_argmax.rs:97-115"""
    nb = cols // 32
    raw = np.zeros(rows * nb * 22, np.uint8)
    g = Lcg(seed)
    scales = [0x2C00, 0x3000, 0x3200, 0x3400]
    for r in range(rows):
        for b in range(nb):
            off = (r * nb + b) * 22
            raw[off:off + 2] = _u16(scales[(r + b) % 4])
            qh = g.hi32()
            raw[off + 2:off + 6] = [(qh >> (8 * i)) & 0xFF for i in range(4)]
            for j in range(16):
                raw[off + 6 + j] = g.hi32() & 0xFF
    return raw


def fill_q5_k(rows: int, cols: int, seed: int) -> np.ndarray:
    """tests/wave4_quant_gemv_and_argmax.rs:156-174"""
    nb = cols // 256
    raw = np.zeros(rows * nb * 176, np.uint8)
    g = Lcg(seed)
    for blk in range(rows * nb):
        off = blk * 176
        raw[off:off + 2] = _u16(0x3000)
        raw[off + 2:off + 4] = _u16(0x2800)
        for idx in range(4, 16):
            raw[off + idx] = g.hi32() % 31 + 1
        for idx in range(16, 176):
            raw[off + idx] = g.hi32() & 0xFF
    return raw


def fill_tq1_0(rows: int, cols: int, seed: int) -> np.ndarray:
    """tests/wave4_quant_gemv_and_argmax.rs:196-209"""
    nb = cols // 256
    raw = np.zeros(rows * nb * 54, np.uint8)
    g = Lcg(seed)
    for blk in range(rows * nb):
        off = blk * 54
        raw[off:off + 2] = _u16(0x3400)
        for idx in range(2, 54):
            raw[off + idx] = g.hi32() % 243
    return raw


# Q4_1, Q5_1, Q2_K, Q3_K, IQ4_NL block geometry
_SYN_BE = {3: 32, 7: 32, 20: 32, 10: 256, 11: 256}
_SYN_BB = {3: 20, 7: 24, 20: 18, 10: 84, 11: 110}


def _f16(v: float) -> int:
    return int(np.float16(v).view(np.uint16))


def _u16b(v: int):
    return [v & 0xFF, v >> 8]


def build_synthetic(quant: int, rows: int, cols: int, seed: int) -> np.ndarray:
    """build_synthetic_quant_tensor (tests/test_repack_gemv_gemm.rs:86-270) for these formats;
    f16 bits from its f32_to_f16_bits (31-45), exact for the values used."""
    nb = cols // _SYN_BE[quant]
    raw = np.zeros(rows * nb * _SYN_BB[quant], np.uint8)
    for r in range(rows):
        for b in range(nb):
            off = (r * nb + b) * _SYN_BB[quant]
            blk = raw[off:off + _SYN_BB[quant]]
            if quant == 3:
                blk[0:2] = _u16b(_f16(0.0625 * (1.0 + ((r + b) % 4) * 0.5)))
                blk[2:4] = _u16b(_f16(-0.25 + ((r * 3 + b) % 5) * 0.125))
                for i in range(16):
                    blk[4 + i] = ((r * 7 + b * 3 + i + seed) & 15) | (((r * 11 + b * 5 + i * 3 + seed) & 15) << 4)
            elif quant == 7:
                blk[0:2] = _u16b(_f16(0.0625 * (1.0 + ((r + b) % 3) * 0.25)))
                blk[2:4] = _u16b(_f16(-0.25 + ((r * 2 + b * 3) % 7) * 0.0625))
                qh = ((r * 0x517CC1B7) ^ (b * 0x27220A95) ^ seed) & 0xFFFFFFFF
                blk[4:8] = [(qh >> (8 * i)) & 0xFF for i in range(4)]
                for i in range(16):
                    blk[8 + i] = ((r * 9 + b * 7 + i + seed) & 15) | (((r * 3 + b * 11 + i * 7 + seed) & 15) << 4)
            elif quant == 10:
                for s in range(16):
                    blk[s] = (((r * 5 + b * 3 + s + 1) % 15 + 1) & 15) | ((((r * 3 + b * 7 + s + 2) % 13) & 15) << 4)
                for i in range(64):
                    blk[16 + i] = (r * 17 + b * 11 + i * 5 + seed) & 0xFF
                blk[80:82], blk[82:84] = _u16b(_f16(0.0625)), _u16b(_f16(0.03125))
            elif quant == 11:
                for i in range(96):
                    blk[i] = (r * 13 + b * 7 + i * 9 + seed) & 0xFF
                for s in range(12):
                    blk[96 + s] = (r * 19 + b * 23 + s * 11 + seed + 7) & 0xFF
                blk[108:110] = _u16b(_f16(0.0625))
            else:  # IQ4_NL
                blk[0:2] = _u16b(_f16(0.03125 * (1.0 + ((r + b) % 4) * 0.25)))
                for i in range(16):
                    blk[2 + i] = ((r * 5 + b * 3 + i + seed) & 15) | (((r * 7 + b * 9 + i * 3 + seed) & 15) << 4)
    return raw


def cosine(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


def rel_l2(got, ref) -> float:
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.linalg.norm(got - ref) / np.linalg.norm(ref))
