"""Seeded synthetic GGUF weights and activations for the quantized-matmul workloads.

Distributions (one GGUF block per row-block, little-endian):
  Q4_0   d = f16(|N(0,1)| * 0.02 / 8), 16 bytes of uniform nibbles
  Q5_0   d = f16(|N(0,1)| * 0.02 / 16), 4 random high-bit bytes, 16 bytes of uniform nibbles
  Q8_0   d = f16(|N(0,1)| * 0.02 / 127), 32 quants uniform in [-127, 127]
  Q4_K   d, dmin = f16(|N(0,1)| * 0.01), 12 random scale bytes, 128 random quant bytes
  Q5_K   d, dmin = f16(|N(0,1)| * 0.005), 12 random scale bytes, 160 random qh / quant bytes
  Q6_K   128 B ql + 64 B qh random, 16 i8 scales uniform in [-32, 31], d = f16(|N(0,1)| * 0.001)
  TQ1_0  trits uniform in {-1, 0, +1}, five base-3 digits per byte (element 5i+j = digit j of
         byte 2+i, element 255 = byte 53), d = f16(1.0)
  TQ2_0  trits uniform in {-1, 0, +1} packed 2 bits each (element 4i+j = bits 2j of qs[i]), d = f16(1.0)
  Q4_1, Q5_1  d = f16(|N(0,1)| * 0.02 / 16), m = f16(N(0,1) * 0.01), random quant (and high-bit) bytes
  IQ4_NL d = f16(|N(0,1)| * 0.02 / 127), 16 bytes of uniform nibble indices
  Q2_K   16 random scale / min bytes, 64 random quant bytes, d, dmin = f16(|N(0,1)| * 0.01)
  Q3_K   96 random hmask / quant bytes, 12 random packed scale bytes, d = f16(|N(0,1)| * 0.002)
  I2_S   trits uniform in {-1, 0, +1} (byte g: elements g, 32+g, 64+g, 96+g in bits 7:6..1:0),
         32-byte trailer holding the f32 tensor scale 1.0
Activations are f32 ~ N(0, 1).
"""
from __future__ import annotations

import numpy as np

from . import (BLOCK_BYTES, BLOCK_ELEMENTS, I2_S, IQ4_NL, Q2_K, Q3_K, Q4_0, Q4_1, Q4_K, Q5_0, Q5_1, Q5_K, Q6_K, Q8_0,
               TQ1_0, TQ2_0)


def _f16_bits(v: np.ndarray) -> np.ndarray:
    return np.asarray(v, dtype=np.float16).view(np.uint16)


def _put_u16(blocks: np.ndarray, off: int, bits: np.ndarray) -> None:
    b = bits.astype(np.uint16)
    blocks[..., off] = (b & 0xFF).astype(np.uint8)
    blocks[..., off + 1] = (b >> 8).astype(np.uint8)


def gguf_weights(quant: int, rows: int, cols: int, seed: int) -> np.ndarray:
    """Row-major GGUF payload (plus the I2_S trailer) of a [rows, cols] matrix."""
    rng = np.random.default_rng(seed)
    be, bb = BLOCK_ELEMENTS[quant], BLOCK_BYTES[quant]
    if cols % be:
        raise ValueError(f"cols {cols} not a multiple of {be}")
    nb = rows * (cols // be)
    blocks = np.empty((nb, bb), dtype=np.uint8)
    if quant == Q4_0:
        _put_u16(blocks, 0, _f16_bits(np.abs(rng.standard_normal(nb)) * 0.02 / 8))
        blocks[:, 2:] = rng.integers(0, 256, size=(nb, 16), dtype=np.uint8)
    elif quant == Q5_0:
        _put_u16(blocks, 0, _f16_bits(np.abs(rng.standard_normal(nb)) * 0.02 / 16))
        blocks[:, 2:] = rng.integers(0, 256, size=(nb, 20), dtype=np.uint8)
    elif quant == Q8_0:
        _put_u16(blocks, 0, _f16_bits(np.abs(rng.standard_normal(nb)) * 0.02 / 127))
        blocks[:, 2:] = rng.integers(-127, 128, size=(nb, 32), dtype=np.int8).view(np.uint8)
    elif quant == Q4_K:
        _put_u16(blocks, 0, _f16_bits(np.abs(rng.standard_normal(nb)) * 0.01))
        _put_u16(blocks, 2, _f16_bits(np.abs(rng.standard_normal(nb)) * 0.01))
        blocks[:, 4:] = rng.integers(0, 256, size=(nb, 140), dtype=np.uint8)
    elif quant == Q5_K:
        _put_u16(blocks, 0, _f16_bits(np.abs(rng.standard_normal(nb)) * 0.005))
        _put_u16(blocks, 2, _f16_bits(np.abs(rng.standard_normal(nb)) * 0.005))
        blocks[:, 4:] = rng.integers(0, 256, size=(nb, 172), dtype=np.uint8)
    elif quant == Q6_K:
        blocks[:, :192] = rng.integers(0, 256, size=(nb, 192), dtype=np.uint8)
        blocks[:, 192:208] = rng.integers(-32, 32, size=(nb, 16), dtype=np.int8).view(np.uint8)
        _put_u16(blocks, 208, _f16_bits(np.abs(rng.standard_normal(nb)) * 0.001))
    elif quant == TQ2_0:
        t = rng.integers(0, 3, size=(nb, 64, 4), dtype=np.uint8)  # 2-bit value = trit + 1
        blocks[:, 2:] = t[..., 0] | (t[..., 1] << 2) | (t[..., 2] << 4) | (t[..., 3] << 6)
        _put_u16(blocks, 0, np.full(nb, 0x3C00, dtype=np.uint16))
    elif quant in (Q4_1, Q5_1):
        _put_u16(blocks, 0, _f16_bits(np.abs(rng.standard_normal(nb)) * 0.02 / 16))
        _put_u16(blocks, 2, _f16_bits(rng.standard_normal(nb) * 0.01))
        blocks[:, 4:] = rng.integers(0, 256, size=(nb, bb - 4), dtype=np.uint8)
    elif quant == IQ4_NL:
        _put_u16(blocks, 0, _f16_bits(np.abs(rng.standard_normal(nb)) * 0.02 / 127))
        blocks[:, 2:] = rng.integers(0, 256, size=(nb, 16), dtype=np.uint8)
    elif quant == Q2_K:
        blocks[:, :80] = rng.integers(0, 256, size=(nb, 80), dtype=np.uint8)
        _put_u16(blocks, 80, _f16_bits(np.abs(rng.standard_normal(nb)) * 0.01))
        _put_u16(blocks, 82, _f16_bits(np.abs(rng.standard_normal(nb)) * 0.01))
    elif quant == Q3_K:
        blocks[:, :108] = rng.integers(0, 256, size=(nb, 108), dtype=np.uint8)
        _put_u16(blocks, 108, _f16_bits(np.abs(rng.standard_normal(nb)) * 0.002))
    elif quant == TQ1_0:
        t = rng.integers(0, 3, size=(nb, 256), dtype=np.int64)  # digit = trit + 1
        digits = t[:, :255].reshape(nb, 51, 5)
        blocks[:, 2:53] = (digits * np.array([1, 3, 9, 27, 81])).sum(axis=2).astype(np.uint8)
        blocks[:, 53] = t[:, 255].astype(np.uint8)
        _put_u16(blocks, 0, np.full(nb, 0x3C00, dtype=np.uint16))
    elif quant == I2_S:
        t = rng.integers(0, 3, size=(nb, 4, 32), dtype=np.uint8)  # [group][g] -> element 32*group + g
        blocks[:] = (t[:, 0] << 6) | (t[:, 1] << 4) | (t[:, 2] << 2) | t[:, 3]
    else:
        raise ValueError(f"unsupported quant {quant}")
    payload = blocks.reshape(-1)
    if quant == I2_S:
        trailer = np.zeros(32, dtype=np.uint8)
        trailer[:4] = np.frombuffer(np.float32(1.0).tobytes(), dtype=np.uint8)
        payload = np.concatenate([payload, trailer])
    return payload


def random_weights(quant: int, rows: int, cols: int, seed: int, specials: bool = False) -> np.ndarray:
    """Adversarial GGUF payload: uniformly random bytes in every field, and with
    ``specials`` a share of blocks whose scales are +-0, subnormal, Inf or NaN."""
    rng = np.random.default_rng(seed)
    be, bb = BLOCK_ELEMENTS[quant], BLOCK_BYTES[quant]
    nb = rows * (cols // be)
    blocks = rng.integers(0, 256, size=(nb, bb), dtype=np.uint8)
    # keep normal scales modest so sums stay finite; specials override some of them
    scale_offs = {Q4_0: [0], Q5_0: [0], Q8_0: [0], Q4_K: [0, 2], Q5_K: [0, 2], Q6_K: [208], TQ1_0: [0],
                  TQ2_0: [0], Q4_1: [0, 2], Q5_1: [0, 2], IQ4_NL: [0], Q2_K: [80, 82], Q3_K: [108]}.get(quant, [])
    for off in scale_offs:
        mag = rng.uniform(1e-4, 0.05, size=nb) * rng.choice([-1.0, 1.0], size=nb)
        _put_u16(blocks, off, _f16_bits(mag))
        if specials:
            pick = rng.random(nb) < 0.15
            sp = np.array([0x0000, 0x8000, 0x0001, 0x83FF, 0x7C00, 0xFC00, 0x7E00, 0x7C01], dtype=np.uint16)
            vals = blocks[pick]
            _put_u16(vals, off, rng.choice(sp, size=int(pick.sum())))
            blocks[pick] = vals
    payload = blocks.reshape(-1)
    if quant == I2_S:
        trailer = np.zeros(32, dtype=np.uint8)
        trailer[:4] = np.frombuffer(np.float32(rng.uniform(0.1, 2.0)).tobytes(), dtype=np.uint8)
        payload = np.concatenate([payload, trailer])
    return payload


def activations(shape, seed: int) -> np.ndarray:
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


# Workloads of the benchmark configurations (rows, cols per matrix).
LLAMA3_8B_LAYER = [  # (name, quant, rows, cols)
    ("attn_q", Q4_K, 4096, 4096),
    ("attn_k", Q4_K, 1024, 4096),
    ("attn_v", Q4_K, 1024, 4096),
    ("attn_output", Q4_K, 4096, 4096),
    ("ffn_gate", Q4_K, 14336, 4096),
    ("ffn_up", Q4_K, 14336, 4096),
    ("ffn_down", Q6_K, 4096, 14336),
]
