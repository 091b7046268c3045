"""ctypes binding of liboracle.so -- the CPU restatement of the reference's scalar path.

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() (which compares
the GPU result with it) and by bench.py's cpu_baseline leg. The product path never imports this module.
Status codes follow the product library: 0 ok, 1 TensorBoundsError, 2 CapabilityMismatch.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

BLOCK_Q8_0 = np.dtype([("d", "<f4"), ("qs", "i1", (32,))])
BLOCK_Q8K = np.dtype([("d", "<f4"), ("qs", "i1", (256,)), ("bsums", "<i2", (16,))])

_sz, _vp = C.c_size_t, C.c_void_p


class OracleError(RuntimeError):
    def __init__(self, status: int, what: str):
        super().__init__(f"{what}: oracle status {status}")
        self.status = status


class _View(C.Structure):
    _fields_ = [("quant", C.c_int), ("shape", C.POINTER(_sz)), ("ndim", _sz), ("bytes", _vp), ("byte_len", _sz)]


class _Act(C.Structure):
    _fields_ = [("m", _sz), ("k", _sz), ("k_padded", _sz), ("k_blocks32", _sz), ("k_chunks", _sz), ("sb256", _sz),
                ("qs", _vp), ("scales", _vp), ("sums", _vp), ("sums16", _vp), ("super256", _vp)]


_lib = None


def build() -> None:
    subprocess.run(["make", "-C", HERE, "-s"], check=True)


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        h = C.CDLL(LIB_PATH)
        h.or_f16_to_f32_ieee.restype = C.c_float
        h.or_f16_to_f32_ieee.argtypes = [C.c_uint16]
        h.or_f16_to_f32_finite.restype = C.c_float
        h.or_f16_to_f32_finite.argtypes = [C.c_uint16]
        h.or_unpack_tq2_0_block_i8.restype = C.c_float
        h.or_unpack_tq1_0_block_i8.restype = C.c_float
        h.or_unpack_q5_0_block_i8.restype = C.c_float
        h.or_unpack_iq4_nl_block_i8.restype = C.c_float
        h.or_read_i2_s_trailer_scale.restype = C.c_float
        h.or_act_q8_bytes.restype = _sz
        h.or_act_q8_bytes.argtypes = [_sz, _sz]
        _lib = h
    return _lib


def _p(a: np.ndarray) -> _vp:
    return _vp(a.ctypes.data)


class View:
    """Keeps the shape array and bytes of a TensorView alive for one call."""

    def __init__(self, quant: int, shape, data: np.ndarray):
        self.data = np.ascontiguousarray(data, dtype=np.uint8).reshape(-1)
        self.shape = (_sz * max(1, len(shape)))(*[int(s) for s in shape])
        self.c = _View(int(quant), C.cast(self.shape, C.POINTER(_sz)), len(shape), self.data.ctypes.data,
                       self.data.nbytes)


def _ok(st: int, what: str) -> None:
    if st != 0:
        raise OracleError(st, what)


def status_of(fn, *args) -> int:
    """Runs fn and returns its oracle status (0 when it succeeds)."""
    try:
        fn(*args)
        return 0
    except OracleError as e:
        return e.status


# ----------------------------------------------------------------- f16 / blocks
def f16_to_f32_ieee(bits: int) -> float:
    return lib().or_f16_to_f32_ieee(bits)


def f16_to_f32_finite(bits: int) -> float:
    return lib().or_f16_to_f32_finite(bits)


def dequantize_row_bytes(quant: int, row: np.ndarray, n_cols: int) -> np.ndarray:
    row = np.ascontiguousarray(row, dtype=np.uint8)
    out = np.zeros(n_cols, dtype=np.float32)
    _ok(lib().or_dequantize_row_bytes(quant, _p(row), _sz(row.size), _sz(n_cols), _p(out), _sz(out.size)),
        "dequantize_row_bytes")
    return out


def dequantize_tensor_row(quant: int, shape, data: np.ndarray, row: int, cols: int) -> np.ndarray:
    v = View(quant, shape, data)
    out = np.zeros(cols, dtype=np.float32)
    _ok(lib().or_dequantize_tensor_row(C.byref(v.c), _sz(row), _p(out), _sz(cols)), "dequantize_tensor_row")
    return out


def unpack_tq2_0_block_i8(block: np.ndarray):
    b = np.ascontiguousarray(block, dtype=np.uint8)
    out = np.zeros(256, dtype=np.int8)
    s = lib().or_unpack_tq2_0_block_i8(_p(b), _p(out))
    return s, out


def unpack_tq1_0_block_i8(block: np.ndarray):
    b = np.ascontiguousarray(block, dtype=np.uint8)
    out = np.zeros(256, dtype=np.int8)
    s = lib().or_unpack_tq1_0_block_i8(_p(b), _p(out))
    return s, out


def unpack_q5_0_block_i8(block: np.ndarray):
    b = np.ascontiguousarray(block, dtype=np.uint8)
    out = np.zeros(32, dtype=np.int8)
    s = lib().or_unpack_q5_0_block_i8(_p(b), _p(out))
    return s, out


def unpack_i2_s_block_i8(block: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(block, dtype=np.uint8)
    out = np.zeros(128, dtype=np.int8)
    lib().or_unpack_i2_s_block_i8(_p(b), _p(out))
    return out


def convert_i2_s_blocks_to_tq2_0(blk0: np.ndarray, blk1: np.ndarray, scale_f16_bits: int) -> np.ndarray:
    a = np.ascontiguousarray(blk0, dtype=np.uint8)
    b = np.ascontiguousarray(blk1, dtype=np.uint8)
    out = np.zeros(66, dtype=np.uint8)
    lib().or_convert_i2_s_blocks_to_tq2_0(_p(a), _p(b), C.c_uint16(scale_f16_bits), _p(out))
    return out


def dequantize_i2_s_block(block: np.ndarray, scale: float) -> np.ndarray:
    b = np.ascontiguousarray(block, dtype=np.uint8)
    out = np.zeros(128, dtype=np.float32)
    lib().or_dequantize_i2_s_block(_p(b), C.c_float(scale), _p(out))
    return out


# ----------------------------------------------------------------- quantizers
def quantize_row_q8_0(x: np.ndarray, out_len: int | None = None) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    n = x.size // 32 if out_len is None else out_len
    out = np.zeros(n, dtype=BLOCK_Q8_0)
    _ok(lib().or_quantize_row_q8_0(_p(x), _sz(x.size), _p(out), _sz(n)), "quantize_row_q8_0")
    return out


def quantize_row_q8_k(x: np.ndarray, out_len: int | None = None) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    n = x.size // 256 if out_len is None else out_len
    out = np.zeros(n, dtype=BLOCK_Q8K)
    _ok(lib().or_quantize_row_q8_k(_p(x), _sz(x.size), _p(out), _sz(n)), "quantize_row_q8_k")
    return out


class ActQ8:
    """Logical QuantizedActQ8 contents (numpy views into one storage buffer)."""

    def __init__(self, act: np.ndarray, m: int, k: int):
        act = np.ascontiguousarray(act, dtype=np.float32).reshape(-1)
        self.storage = np.zeros(lib().or_act_q8_bytes(m, k), dtype=np.uint8)
        self.c = _Act()
        _ok(lib().or_quantize_act_q8(_p(act), _sz(m), _sz(k), _p(self.storage), _sz(self.storage.size),
                                     C.byref(self.c)), "quantize_act_q8")
        c = self.c
        self.m, self.k, self.k_padded = c.m, c.k, c.k_padded
        self.k_blocks32, self.k_chunks, self.sb256 = c.k_blocks32, c.k_chunks, c.sb256
        base = self.storage.ctypes.data

        def arr(ptr, dtype, count):
            off = ptr - base
            return self.storage[off: off + count * np.dtype(dtype).itemsize].view(dtype)

        self.scales = arr(c.scales, np.float32, m * c.k_blocks32).reshape(m, -1)
        self.sums = arr(c.sums, np.float32, m * c.k_blocks32).reshape(m, -1)
        self.sums16 = arr(c.sums16, np.float32, m * c.k_chunks).reshape(m, -1)
        self.super256 = arr(c.super256, np.float32, m * c.sb256).reshape(m, -1)
        self.qs = arr(c.qs, np.int8, m * c.k_padded).reshape(m, -1)


def subln_quantize_absmax_i8(x: np.ndarray, w: np.ndarray, eps: float):
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    q = np.zeros(x.size, dtype=np.int8)
    s = C.c_float(0)
    _ok(lib().or_subln_quantize_absmax_i8(_p(q), _p(x), _p(w), _sz(x.size), C.c_float(eps), C.byref(s)), "subln")
    return q, s.value


def quantize_absmax_i8(x: np.ndarray):
    x = np.ascontiguousarray(x, dtype=np.float32)
    q = np.zeros(x.size, dtype=np.int8)
    s = C.c_float(0)
    _ok(lib().or_quantize_absmax_i8(_p(q), _p(x), _sz(x.size), C.byref(s)), "absmax")
    return q, s.value


# ----------------------------------------------------------------- quant_q8 path
_VEC_DOT_Q8 = {2: "or_vec_dot_q4_0_q8_0", 8: "or_vec_dot_q8_0_q8_0", 12: "or_vec_dot_q4_k_q8_k",
               14: "or_vec_dot_q6_k_q8_k", 35: "or_vec_dot_tq2_0_q8_k", 6: "or_vec_dot_q5_0_q8_0",
               13: "or_vec_dot_q5_k_q8_k", 34: "or_vec_dot_tq1_0_q8_k"}
_GEMV_Q8 = {2: "or_gemv_q4_0_q8_0", 8: "or_gemv_q8_0_q8_0", 12: "or_gemv_q4_k_q8_k", 14: "or_gemv_q6_k_q8_k",
            35: "or_gemv_tq2_0_q8_k", 6: "or_gemv_q5_0_q8_0", 13: "or_gemv_q5_k_q8_k", 34: "or_gemv_tq1_0_q8_k"}
# Formats whose GEMV takes BlockQ8_0 activations (the others take BlockQ8K).
Q8_0_ACT = (2, 6, 8)


def vec_dot_q8(quant: int, w_row: np.ndarray, x_blocks: np.ndarray) -> float:
    w = np.ascontiguousarray(w_row, dtype=np.uint8)
    x = np.ascontiguousarray(x_blocks)
    out = C.c_float(0)
    _ok(getattr(lib(), _VEC_DOT_Q8[quant])(_p(w), _sz(w.size), _p(x), _sz(x.size), C.byref(out)), "vec_dot_q8")
    return out.value


def gemv_q8(quant: int, shape, data: np.ndarray, x_blocks: np.ndarray, out_len: int) -> np.ndarray:
    v = View(quant, shape, data)
    x = np.ascontiguousarray(x_blocks)
    out = np.zeros(out_len, dtype=np.float32)
    _ok(getattr(lib(), _GEMV_Q8[quant])(_p(out), _sz(out_len), C.byref(v.c), _p(x), _sz(x.size)), "gemv_q8")
    return out


def gemv_rows(quant: int, data: np.ndarray, rows: int, cols: int, x_blocks: np.ndarray, r0: int, r1: int):
    """Rows [r0, r1) of the quant_q8 GEMV (row-partitioned CPU baseline)."""
    d = np.ascontiguousarray(data, dtype=np.uint8)
    x = np.ascontiguousarray(x_blocks)
    out = np.zeros(r1 - r0, dtype=np.float32)
    _ok(lib().or_gemv_rows(quant, _p(out), _p(d), _sz(rows), _sz(cols), _p(x), _sz(r0), _sz(r1)), "gemv_rows")
    return out


_VEC_DOT_F32 = {2: "or_vec_dot_q4_0", 8: "or_vec_dot_q8_0", 14: "or_vec_dot_q6_k", 12: "or_vec_dot_q4_k_m",
                36: "or_vec_dot_i2_s", 6: "or_vec_dot_q5_0", 13: "or_vec_dot_q5_k", 3: "or_vec_dot_q4_1",
                7: "or_vec_dot_q5_1", 10: "or_vec_dot_q2_k", 11: "or_vec_dot_q3_k", 20: "or_vec_dot_iq4_nl"}


def vec_dot_f32(quant: int, shape, data: np.ndarray, x: np.ndarray, out_len: int) -> np.ndarray:
    v = View(quant, shape, data)
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    out = np.zeros(out_len, dtype=np.float32)
    _ok(getattr(lib(), _VEC_DOT_F32[quant])(_p(out), _sz(out_len), C.byref(v.c), _p(x), _sz(x.size)),
        "vec_dot_f32")
    return out


# ----------------------------------------------------------------- repack GEMM
def repack_logical(quant: int, shape, data: np.ndarray, rows: int, cols: int):
    v = View(quant, shape, data)
    sg, hm, cps = _sz(0), C.c_int(0), C.c_int(0)
    _ok(lib().or_repack_logical(C.byref(v.c), _sz(rows), _sz(cols), None, None, None, C.byref(sg), C.byref(hm),
                                C.byref(cps)), "repack_logical")
    kp = (cols + 31) // 32 * 32
    q = np.zeros((rows, kp), dtype=np.int8)
    sc = np.zeros((rows, sg.value), dtype=np.float32)
    mn = np.zeros((rows, sg.value), dtype=np.float32) if hm.value else None
    _ok(lib().or_repack_logical(C.byref(v.c), _sz(rows), _sz(cols), _p(q), _p(sc),
                                _p(mn) if mn is not None else None, None, None, None), "repack_logical")
    return q, sc, mn, cps.value


def gemm_repacked(quant: int, shape, data: np.ndarray, rows: int, cols: int, act: ActQ8, r0: int, r1: int):
    v = View(quant, shape, data)
    out = np.zeros(act.m * (r1 - r0), dtype=np.float32)
    _ok(lib().or_gemm_repacked(_p(out), _sz(out.size), C.byref(v.c), _sz(rows), _sz(cols), C.byref(act.c), _sz(r0),
                               _sz(r1)), "gemm_repacked")
    return out.reshape(act.m, r1 - r0)


def gemm_logical_rows(q: np.ndarray, sc: np.ndarray, mn, cps: int, cols: int, act: ActQ8, m0: int, m1: int,
                      r0: int, r1: int) -> np.ndarray:
    """Tokens [m0, m1) x rows [r0, r1) of the repacked GEMM over weights already repacked by
    repack_logical (the reference repacks once at load time; the product is what a call costs)."""
    out = np.zeros((m1 - m0) * (r1 - r0), dtype=np.float32)
    _ok(lib().or_gemm_logical_rows(_p(out), _p(q), _p(sc), _p(mn) if mn is not None else None, _sz(cols),
                                   _sz(sc.shape[1]), C.c_int(cps), C.byref(act.c), _sz(m0), _sz(m1), _sz(r0),
                                   _sz(r1)), "gemm_logical_rows")
    return out.reshape(m1 - m0, r1 - r0)


def nibble_gemm_rows(quant: int, shape, data: np.ndarray, rows: int, cols: int, act: ActQ8, r0: int, r1: int):
    """PackedNibbleMatrix::gemm_rows restated (Q4_0, Q4_1, IQ4_NL, Q4_K)."""
    v = View(quant, shape, data)
    out = np.zeros(act.m * (r1 - r0), dtype=np.float32)
    _ok(lib().or_nibble_gemm_rows(_p(out), _sz(out.size), C.byref(v.c), _sz(rows), _sz(cols), C.byref(act.c),
                                  _sz(r0), _sz(r1)), "nibble_gemm_rows")
    return out.reshape(act.m, r1 - r0)


# ----------------------------------------------------------------- BitLinear
def bitlinear_i8(quant: int, shape, data: np.ndarray, act: np.ndarray, act_scale: float, out_len: int):
    v = View(quant, shape, data)
    a = np.ascontiguousarray(act, dtype=np.int8).reshape(-1)
    out = np.zeros(out_len, dtype=np.float32)
    _ok(lib().or_bitlinear_i8(_p(out), _sz(out_len), C.byref(v.c), _p(a), _sz(a.size), C.c_float(act_scale)),
        "bitlinear")
    return out


# ----------------------------------------------------------------- int8 primitives
def dot_i8(a: np.ndarray, b: np.ndarray) -> int:
    """dot_i8_scalar (ime.rs:490-496) over the zip of the two slices."""
    a = np.ascontiguousarray(a, dtype=np.int8).reshape(-1)
    b = np.ascontiguousarray(b, dtype=np.int8).reshape(-1)
    return int(lib().or_dot_i8(_p(a), _sz(a.size), _p(b), _sz(b.size)))


def gemm_i8_vector(a: np.ndarray, m: int, b: np.ndarray, n0: int, n1: int, k: int) -> np.ndarray:
    """gemm_i8_vector (ime.rs:563-583): [m][n1 - n0] i32."""
    a = np.ascontiguousarray(a, dtype=np.int8).reshape(-1)
    b = np.ascontiguousarray(b, dtype=np.int8).reshape(-1)
    assert a.size >= m * k and b.size >= n1 * k
    c = np.zeros(m * (n1 - n0), dtype=np.int32)
    lib().or_gemm_i8_vector(_p(c), _p(a), _sz(m), _p(b), _sz(n0), _sz(n1), _sz(k))
    return c.reshape(m, n1 - n0)


def pack_tiles(src: np.ndarray, rows: int, k: int) -> np.ndarray:
    """pack_tiles (ime.rs:81-94)."""
    s = np.ascontiguousarray(src, dtype=np.int8).reshape(-1)
    out = np.zeros((rows + 7) // 8 * (k // 16) * 128, dtype=np.int8)
    _ok(lib().or_pack_tiles(_p(out), _sz(out.size), _p(s), _sz(s.size), _sz(rows), _sz(k)), "pack_tiles")
    return out


def tile_dot_scalar_rows(a: np.ndarray, b: np.ndarray, k_chunks: int, active_m: int) -> np.ndarray:
    """tile_dot_scalar_rows (ime.rs:127-148): 64 i32."""
    a = np.ascontiguousarray(a, dtype=np.int8).reshape(-1)
    b = np.ascontiguousarray(b, dtype=np.int8).reshape(-1)
    assert a.size >= 128 * k_chunks and b.size >= 128 * k_chunks
    c = np.zeros(64, dtype=np.int32)
    lib().or_tile_dot_scalar_rows(_p(c), _p(a), _p(b), _sz(k_chunks), _sz(active_m))
    return c


def gemm_i8_ime(a_packed: np.ndarray, m_tiles: int, b_packed: np.ndarray, nt0: int, nt1: int, k_chunks: int):
    """gemm_i8_ime (ime.rs:449-486): [m_tiles][nt1 - nt0][64] i32."""
    a = np.ascontiguousarray(a_packed, dtype=np.int8).reshape(-1)
    b = np.ascontiguousarray(b_packed, dtype=np.int8).reshape(-1)
    assert a.size >= m_tiles * k_chunks * 128 and b.size >= nt1 * k_chunks * 128
    c = np.zeros(m_tiles * (nt1 - nt0) * 64, dtype=np.int32)
    lib().or_gemm_i8_ime(_p(c), _p(a), _sz(m_tiles), _p(b), _sz(nt0), _sz(nt1), _sz(k_chunks))
    return c.reshape(m_tiles, nt1 - nt0, 64)


# ----------------------------------------------------------------- gated activations, argmax
def swiglu_f32(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    g = np.ascontiguousarray(gate, dtype=np.float32).reshape(-1)
    u = np.ascontiguousarray(up, dtype=np.float32).reshape(-1)
    out = np.zeros(g.size, dtype=np.float32)
    _ok(lib().or_swiglu_f32(_p(out), _p(g), _p(u), _sz(g.size)), "swiglu")
    return out


def relu_squared_gate_f32(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    g = np.ascontiguousarray(gate, dtype=np.float32).reshape(-1)
    u = np.ascontiguousarray(up, dtype=np.float32).reshape(-1)
    out = np.zeros(g.size, dtype=np.float32)
    _ok(lib().or_relu_squared_gate_f32(_p(out), _p(g), _p(u), _sz(g.size)), "relu_squared")
    return out


def argmax_f32(x: np.ndarray) -> int:
    """Index of the maximum (lowest on ties), -1 for empty or all-NaN input."""
    a = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    f = lib().or_argmax_f32
    f.restype = C.c_long
    return int(f(_p(a) if a.size else None, _sz(a.size)))

