"""Python host mirror of the jero-kernels-rvv quantized-matmul API over libjk.so.

The functions keep the reference crate's names and argument meaning (quant_q8.rs,
quant.rs, repack.rs, ime.rs, lib.rs); errors raise the reference's two K3Error kinds.
All compute runs in libjk.so (hand-written HIP for gfx950); this module only marshals
arguments. A missing libjk.so is an ImportError-grade failure, never a fallback.

Two tiers, as in include/jk.h:
  * host tier   -- numpy in, numpy out, synchronous (``gemv_q4_k_q8_k(out, view, x)``);
  * device tier -- ``Weight`` handles plus device pointers (``int`` or any object with
                   ``data_ptr()``, e.g. a torch tensor) on a HIP stream.
"""
from __future__ import annotations

import ctypes as C
import os
import re

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
PACKAGE_DIR = os.path.dirname(_HERE)
LIB_PATH = os.path.join(PACKAGE_DIR, "libjk.so")
HEADER_PATH = os.path.join(os.path.dirname(PACKAGE_DIR), "include", "jk.h")

# ---------------------------------------------------------------- formats
Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K, TQ1_0, TQ2_0, I2_S = 2, 6, 8, 12, 13, 14, 34, 35, 36
Q4_1, Q5_1, Q2_K, Q3_K, IQ4_NL = 3, 7, 10, 11, 20
QUANT_NAMES = {Q4_0: "Q4_0", Q5_0: "Q5_0", Q8_0: "Q8_0", Q4_K: "Q4_K_M", Q5_K: "Q5_K", Q6_K: "Q6_K",
               TQ1_0: "TQ1_0", TQ2_0: "TQ2_0", I2_S: "I2_S", Q4_1: "Q4_1", Q5_1: "Q5_1", Q2_K: "Q2_K",
               Q3_K: "Q3_K", IQ4_NL: "IQ4_NL"}
BLOCK_ELEMENTS = {Q4_0: 32, Q5_0: 32, Q8_0: 32, Q4_K: 256, Q5_K: 256, Q6_K: 256, TQ1_0: 256, TQ2_0: 256, I2_S: 128,
                  Q4_1: 32, Q5_1: 32, IQ4_NL: 32, Q2_K: 256, Q3_K: 256}
BLOCK_BYTES = {Q4_0: 18, Q5_0: 22, Q8_0: 34, Q4_K: 144, Q5_K: 176, Q6_K: 210, TQ1_0: 54, TQ2_0: 66, I2_S: 32,
               Q4_1: 20, Q5_1: 24, IQ4_NL: 18, Q2_K: 84, Q3_K: 110}
# Formats with a quant_q8 GEMV, with an f32-activation vec_dot, with a BitLinear product.
GEMV_FORMATS = (Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K, TQ1_0, TQ2_0)
VEC_DOT_F32_FORMATS = (Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, IQ4_NL, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, I2_S)
BITLINEAR_FORMATS = (TQ1_0, TQ2_0, I2_S, Q8_0)
# Formats whose quant_q8 GEMV takes BlockQ8_0 activations (the others take BlockQ8K).
Q8_0_ACT = (Q4_0, Q5_0, Q8_0)
TRAILER_BYTES = {I2_S: 32}

# BlockQ8_0 (quant_q8.rs:37-44) and BlockQ8K (62-72), #[repr(C)] byte layouts.
BLOCK_Q8_0 = np.dtype([("d", "<f4"), ("qs", "i1", (32,))])
BLOCK_Q8K = np.dtype([("d", "<f4"), ("qs", "i1", (256,)), ("bsums", "<i2", (16,))])
assert BLOCK_Q8_0.itemsize == 36 and BLOCK_Q8K.itemsize == 292

OK, TENSOR_BOUNDS, CAPABILITY_MISMATCH, DEVICE_ERROR = 0, 1, 2, 3


class K3Error(RuntimeError):
    """Base of the errors the reference path returns. TensorBoundsError's payload (tensor_name,
    offset, byte_len, buffer_len, reason) comes from jk_last_error_info."""

    def __init__(self, reason: str, tensor_name: str = "", offset: int = 0, byte_len: int = 0,
                 buffer_len: int = 0):
        super().__init__(reason)
        self.reason = reason
        self.tensor_name = tensor_name
        self.offset = offset
        self.byte_len = byte_len
        self.buffer_len = buffer_len


class TensorBoundsError(K3Error):
    """K3Error::TensorBoundsError: shape, length, range or quant-type mismatch."""


class CapabilityMismatch(K3Error):
    """K3Error::CapabilityMismatch: format not supported by the entry point."""


class DeviceError(K3Error):
    """HIP runtime failure (no reference counterpart)."""


_ERRORS = {TENSOR_BOUNDS: TensorBoundsError, CAPABILITY_MISMATCH: CapabilityMismatch, DEVICE_ERROR: DeviceError}

# ---------------------------------------------------------------- ctypes
_sz = C.c_size_t
_vp = C.c_void_p


class TensorViewC(C.Structure):
    _fields_ = [("name", C.c_char_p), ("quant", C.c_int32), ("shape", C.POINTER(_sz)), ("ndim", _sz),
                ("bytes", _vp), ("byte_len", _sz), ("offset", _sz)]


class ErrorInfoC(C.Structure):
    _fields_ = [("status", C.c_int), ("tensor_name", C.c_char_p), ("offset", _sz), ("byte_len", _sz),
                ("buffer_len", _sz), ("reason", C.c_char_p)]


class HostStatsC(C.Structure):
    _fields_ = [("weight_uploads", C.c_uint64), ("cache_hits", C.c_uint64), ("cache_evictions", C.c_uint64),
                ("device_allocs", C.c_uint64), ("cached_weights", C.c_uint64), ("cached_bytes", C.c_uint64),
                ("cache_limit", C.c_uint64), ("stale_reuploads", C.c_uint64), ("verify", C.c_uint64)]


class ActQ8C(C.Structure):
    _fields_ = [("m", _sz), ("k", _sz), ("k_padded", _sz), ("k_blocks32", _sz), ("k_chunks", _sz), ("sb256", _sz),
                ("qs", _vp), ("scales", _vp), ("sums", _vp), ("sums16", _vp), ("super256", _vp)]


class GemvJobC(C.Structure):
    _fields_ = [("w", _vp), ("x_q8", _vp), ("x_f32", _vp), ("y", _vp), ("row_begin", _sz), ("row_end", _sz)]


class WeightInfoC(C.Structure):
    _fields_ = [("quant", C.c_int32), ("rows", _sz), ("cols", _sz), ("device_bytes", _sz), ("gguf_bytes", _sz)]


class WeightLayoutC(C.Structure):
    """BlockScaledTileLayout (repack.rs:1286-1449) plus the device layout's byte counts."""
    _fields_ = [("quant", C.c_int32), ("rows", _sz), ("cols", _sz), ("row_bytes", _sz), ("k_padded", _sz),
                ("n_tiles", _sz), ("k_chunks", _sz), ("chunks_per_scale", _sz), ("scale_groups", _sz),
                ("has_mins", C.c_int32), ("total_tiles", _sz), ("total_scales", _sz), ("total_mins", _sz),
                ("device_bytes", _sz), ("gguf_bytes", _sz), ("tensor_scale", C.c_float)]

    def scales_for_tiles(self, count: int) -> int:
        """BlockScaledTileLayout::scales_for_tiles (repack.rs:1446)."""
        return count * self.scale_groups * 8


_lib_handle = None


def lib() -> C.CDLL:
    """Loads libjk.so (built in-tree by ``make -C jero-kernels-rvv_amd``)."""
    global _lib_handle
    if _lib_handle is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"libjk.so not built: run `make -C {PACKAGE_DIR}` (expected {LIB_PATH})")
        h = C.CDLL(LIB_PATH)
        h.jk_last_error.restype = C.c_char_p
        h.jk_act_q8_bytes.restype = _sz
        h.jk_act_q8_bytes.argtypes = [_sz, _sz]
        _lib_handle = h
    return _lib_handle


def header_symbols() -> list[str]:
    """Every function name declared in include/jk.h."""
    text = open(HEADER_PATH).read()
    return sorted(set(re.findall(r"\b(jk_[a-z0-9_]+)\s*\(", text)))


def last_error_info() -> dict:
    """jk_last_error_info: the payload of the calling thread's most recent failure."""
    e = ErrorInfoC()
    lib().jk_last_error_info(C.byref(e))
    return {"status": e.status, "tensor_name": (e.tensor_name or b"").decode(errors="replace"), "offset": e.offset,
            "byte_len": e.byte_len, "buffer_len": e.buffer_len, "reason": (e.reason or b"").decode(errors="replace")}


def _check(status: int) -> None:
    if status != OK:
        info = last_error_info()
        raise _ERRORS.get(status, K3Error)(info["reason"], info["tensor_name"], info["offset"], info["byte_len"],
                                           info["buffer_len"])


def _ptr(x) -> int:
    """Device or host address of an int, numpy array or torch-like tensor."""
    if x is None:
        return 0
    if isinstance(x, int):
        return x
    if isinstance(x, np.ndarray):
        return x.ctypes.data
    return int(x.data_ptr())


class TensorView:
    """jero_core::TensorView fields the path reads: name, quant, shape, bytes, offset."""

    def __init__(self, name: str, quant: int, shape, data, offset: int = 0):
        self.name = name
        self.offset = int(offset)
        self.quant = int(quant)
        self.shape = tuple(int(s) for s in shape)
        self.data = np.ascontiguousarray(np.frombuffer(memoryview(data), dtype=np.uint8)
                                         if not isinstance(data, np.ndarray) else data.view(np.uint8).reshape(-1))
        self._name_b = name.encode()
        self._shape_c = (_sz * max(1, len(self.shape)))(*self.shape)

    def c(self) -> TensorViewC:
        return TensorViewC(self._name_b, self.quant, C.cast(self._shape_c, C.POINTER(_sz)), len(self.shape),
                           self.data.ctypes.data, self.data.nbytes, self.offset)


# ---------------------------------------------------------------- host-tier residency
def host_cache_set_limit(nbytes: int) -> None:
    _check(lib().jk_host_cache_set_limit(_sz(nbytes)))


def host_cache_invalidate(data) -> None:
    """Drops cached weights whose view overlaps the bytes of data (a numpy array or TensorView)."""
    a = data.data if isinstance(data, TensorView) else data
    _check(lib().jk_host_cache_invalidate(_vp(a.ctypes.data), _sz(a.nbytes)))


def host_cache_clear() -> None:
    _check(lib().jk_host_cache_clear())


def host_cache_set_verify(on: bool) -> None:
    """jk_host_cache_set_verify: every cache hit checks a hash of all of the view's bytes."""
    _check(lib().jk_host_cache_set_verify(C.c_int(int(on))))


def host_stats() -> dict:
    st = HostStatsC()
    _check(lib().jk_host_get_stats(C.byref(st)))
    return {name: getattr(st, name) for name, _ in HostStatsC._fields_}


def host_release_thread() -> None:
    _check(lib().jk_host_release_thread())


# ---------------------------------------------------------------- host tier
def _f32(x) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float32)


def quantize_row_q8_0(x) -> np.ndarray:
    """quantize_row_q8_0 (quant_q8.rs:395): f32[n] -> BlockQ8_0[n / 32]."""
    x = _f32(x).reshape(-1)
    out = np.zeros(x.size // 32 if x.size % 32 == 0 else 0, dtype=BLOCK_Q8_0)
    _check(lib().jk_host_quantize_row_q8_0(_vp(x.ctypes.data), _sz(x.size), _vp(out.ctypes.data), _sz(out.size)))
    return out


def quantize_row_q8_k(x) -> np.ndarray:
    """quantize_row_q8_k (quant_q8.rs:576): f32[n] -> BlockQ8K[n / 256]."""
    x = _f32(x).reshape(-1)
    out = np.zeros(x.size // 256 if x.size % 256 == 0 else 0, dtype=BLOCK_Q8K)
    _check(lib().jk_host_quantize_row_q8_k(_vp(x.ctypes.data), _sz(x.size), _vp(out.ctypes.data), _sz(out.size)))
    return out


def _vec_dot_row(fn: str, w_blocks, x_blocks) -> float:
    w = np.ascontiguousarray(w_blocks, dtype=np.uint8).reshape(-1)
    x = np.ascontiguousarray(x_blocks)
    out = C.c_float(0.0)
    _check(getattr(lib(), fn)(_vp(w.ctypes.data), _sz(w.size), _vp(x.ctypes.data), _sz(x.size), C.byref(out)))
    return out.value


def vec_dot_q4_0_q8_0(w_blocks, x_blocks) -> float:
    """quant_q8.rs:1463"""
    return _vec_dot_row("jk_host_vec_dot_q4_0_q8_0", w_blocks, x_blocks)


def vec_dot_q8_0_q8_0(w_blocks, x_blocks) -> float:
    """quant_q8.rs:1493"""
    return _vec_dot_row("jk_host_vec_dot_q8_0_q8_0", w_blocks, x_blocks)


def vec_dot_q4_k_q8_k(w_blocks, x_blocks) -> float:
    """quant_q8.rs:3019"""
    return _vec_dot_row("jk_host_vec_dot_q4_k_q8_k", w_blocks, x_blocks)


def vec_dot_q6_k_q8_k(w_blocks, x_blocks) -> float:
    """quant_q8.rs:3056"""
    return _vec_dot_row("jk_host_vec_dot_q6_k_q8_k", w_blocks, x_blocks)


def vec_dot_tq2_0_q8_k(w_blocks, x_blocks) -> float:
    """quant_q8.rs:3086"""
    return _vec_dot_row("jk_host_vec_dot_tq2_0_q8_k", w_blocks, x_blocks)


def vec_dot_q5_0_q8_0_blocks(w_blocks, x_blocks) -> float:
    """quant_q8.rs:1478"""
    return _vec_dot_row("jk_host_vec_dot_q5_0_q8_0", w_blocks, x_blocks)


def vec_dot_q5_k_q8_k(w_blocks, x_blocks) -> float:
    """quant_q8.rs:3041"""
    return _vec_dot_row("jk_host_vec_dot_q5_k_q8_k", w_blocks, x_blocks)


def vec_dot_tq1_0_q8_k(w_blocks, x_blocks) -> float:
    """quant_q8.rs:3071"""
    return _vec_dot_row("jk_host_vec_dot_tq1_0_q8_k", w_blocks, x_blocks)


def _gemv(fn: str, out: np.ndarray, weights: TensorView, x_blocks) -> None:
    x = np.ascontiguousarray(x_blocks)
    v = weights.c()
    _check(getattr(lib(), fn)(_vp(out.ctypes.data), _sz(out.size), C.byref(v), _vp(x.ctypes.data), _sz(x.size)))


def gemv_q4_0_q8_0(out, weights, x_blocks):
    """quant_q8.rs:1586 -- fills out[rows]."""
    _gemv("jk_host_gemv_q4_0_q8_0", out, weights, x_blocks)


def gemv_q8_0_q8_0(out, weights, x_blocks):
    """quant_q8.rs:1670"""
    _gemv("jk_host_gemv_q8_0_q8_0", out, weights, x_blocks)


def gemv_q4_k_q8_k(out, weights, x_blocks):
    """quant_q8.rs:3101"""
    _gemv("jk_host_gemv_q4_k_q8_k", out, weights, x_blocks)


def gemv_q6_k_q8_k(out, weights, x_blocks):
    """quant_q8.rs:3189"""
    _gemv("jk_host_gemv_q6_k_q8_k", out, weights, x_blocks)


def gemv_tq2_0_q8_k(out, weights, x_blocks):
    """quant_q8.rs:3250"""
    _gemv("jk_host_gemv_tq2_0_q8_k", out, weights, x_blocks)


def gemv_q5_0_q8_0(out, weights, x_blocks):
    """quant_q8.rs:1628"""
    _gemv("jk_host_gemv_q5_0_q8_0", out, weights, x_blocks)


def gemv_q5_k_q8_k(out, weights, x_blocks):
    """quant_q8.rs:3160"""
    _gemv("jk_host_gemv_q5_k_q8_k", out, weights, x_blocks)


def gemv_tq1_0_q8_k(out, weights, x_blocks):
    """quant_q8.rs:3219"""
    _gemv("jk_host_gemv_tq1_0_q8_k", out, weights, x_blocks)


def _vec_dot_f32(fn: str, out: np.ndarray, weights: TensorView, inp) -> None:
    x = _f32(inp).reshape(-1)
    v = weights.c()
    _check(getattr(lib(), fn)(_vp(out.ctypes.data), _sz(out.size), C.byref(v), _vp(x.ctypes.data), _sz(x.size)))


def vec_dot_q4_0(out, weights, inp):
    """quant.rs:1458"""
    _vec_dot_f32("jk_host_vec_dot_q4_0", out, weights, inp)


def vec_dot_q8_0(out, weights, inp):
    """quant.rs:1069"""
    _vec_dot_f32("jk_host_vec_dot_q8_0", out, weights, inp)


def vec_dot_q6_k(out, weights, inp):
    """quant.rs:1089"""
    _vec_dot_f32("jk_host_vec_dot_q6_k", out, weights, inp)


def vec_dot_q4_k_m(out, weights, inp):
    """VectorKernel::vec_dot_q4_k_m (lib.rs:157)"""
    _vec_dot_f32("jk_host_vec_dot_q4_k_m", out, weights, inp)


def vec_dot_i2_s(out, weights, inp):
    """quant.rs:2199"""
    _vec_dot_f32("jk_host_vec_dot_i2_s", out, weights, inp)


def vec_dot_q5_0(out, weights, inp):
    """quant.rs:2036"""
    _vec_dot_f32("jk_host_vec_dot_q5_0", out, weights, inp)


def vec_dot_q5_k(out, weights, inp):
    """quant.rs:1238"""
    _vec_dot_f32("jk_host_vec_dot_q5_k", out, weights, inp)


def vec_dot_q4_1(out, weights, inp):
    """quant.rs:2062"""
    _vec_dot_f32("jk_host_vec_dot_q4_1", out, weights, inp)


def vec_dot_q5_1(out, weights, inp):
    """quant.rs:2081"""
    _vec_dot_f32("jk_host_vec_dot_q5_1", out, weights, inp)


def vec_dot_q2_k(out, weights, inp):
    """quant.rs:2100"""
    _vec_dot_f32("jk_host_vec_dot_q2_k", out, weights, inp)


def vec_dot_q3_k(out, weights, inp):
    """quant.rs:2119"""
    _vec_dot_f32("jk_host_vec_dot_q3_k", out, weights, inp)


def vec_dot_iq4_nl(out, weights, inp):
    """quant.rs:2138"""
    _vec_dot_f32("jk_host_vec_dot_iq4_nl", out, weights, inp)


def dequantize_tensor_row(weights: TensorView, row: int, out: np.ndarray) -> None:
    """dequantize_tensor_row / dequantize_token_row (quant.rs:2492, 2580)."""
    v = weights.c()
    _check(lib().jk_host_dequantize_tensor_row(C.byref(v), _sz(row), _vp(out.ctypes.data), _sz(out.size)))


def bitlinear_i8(out: np.ndarray, weights: TensorView, act_i8, act_scale: float) -> None:
    """bitlinear_i8_rvv (ime.rs:882)."""
    a = np.ascontiguousarray(act_i8, dtype=np.int8).reshape(-1)
    v = weights.c()
    _check(lib().jk_host_bitlinear_i8(_vp(out.ctypes.data), _sz(out.size), C.byref(v), _vp(a.ctypes.data),
                                      _sz(a.size), C.c_float(act_scale)))


def convert_i2_s_blocks_to_tq2_0(blk0, blk1, scale_f16_bits: int) -> np.ndarray:
    """convert_i2_s_blocks_to_tq2_0 (ime.rs:767): two 32-byte I2_S blocks -> one 66-byte TQ2_0 block."""
    a = np.ascontiguousarray(blk0, dtype=np.uint8).reshape(-1)
    b = np.ascontiguousarray(blk1, dtype=np.uint8).reshape(-1)
    if a.size != 32 or b.size != 32:
        raise TensorBoundsError("convert_i2_s_blocks_to_tq2_0: I2_S blocks are 32 bytes")
    out = np.zeros(66, np.uint8)
    _check(lib().jk_host_convert_i2_s_blocks_to_tq2_0(_vp(a.ctypes.data), _vp(b.ctypes.data),
                                                      C.c_uint16(scale_f16_bits), _vp(out.ctypes.data)))
    return out


# ---------------------------------------------------------------- device tier
def init(device: int = 0) -> None:
    _check(lib().jk_init(C.c_int(device)))


def sync(stream=None) -> None:
    _check(lib().jk_stream_sync(_vp(stream or 0)))


def block_scaled_layout(view: TensorView, rows: int, cols: int) -> WeightLayoutC:
    """RepackedWeight::block_scaled_layout (repack.rs:2372)."""
    out = WeightLayoutC()
    v = view.c()
    _check(lib().jk_weight_layout_for(C.byref(v), _sz(rows), _sz(cols), C.byref(out)))
    return out


class Weight:
    """Device-resident weight (RepackedWeight::from_tensor, repack.rs:2288)."""

    def __init__(self, view: TensorView, rows: int = 0, cols: int = 0, stream=None):
        h = _vp()
        v = view.c()
        _check(lib().jk_weight_upload(_vp(stream or 0), C.byref(v), _sz(rows), _sz(cols), C.byref(h)))
        self._h = h
        self._info()

    def _info(self):
        info = WeightInfoC()
        _check(lib().jk_weight_get_info(self._h, C.byref(info)))
        self.quant, self.rows, self.cols = info.quant, info.rows, info.cols
        self.device_bytes, self.gguf_bytes = info.device_bytes, info.gguf_bytes

    @classmethod
    def create(cls, layout: WeightLayoutC, stream=None) -> "Weight":
        """An empty handle for layout, to be filled by tile ranges and sealed (the buffers of
        RepackedWeight::from_tile_buffers, repack.rs:2386, on the device)."""
        self = cls.__new__(cls)
        h = _vp()
        _check(lib().jk_weight_create(_vp(stream or 0), C.byref(layout), C.byref(h)))
        self._h = h
        self._info()
        return self

    def repack_into_tile_range(self, view: TensorView, tile_begin: int, tile_end: int, stream=None) -> None:
        """repack_into_tile_range (repack.rs:1579) into this handle."""
        v = view.c()
        _check(lib().jk_weight_upload_tile_range(_vp(stream or 0), self._h, C.byref(v), _sz(tile_begin),
                                                 _sz(tile_end)))

    def repack_tile_range(self, gguf_dev, gguf_len: int, tile_begin: int, tile_end: int, stream=None) -> None:
        """The same from GGUF bytes already in device memory (no allocation, asynchronous)."""
        _check(lib().jk_weight_repack_tile_range(_vp(stream or 0), self._h, _vp(_ptr(gguf_dev)), _sz(gguf_len),
                                                 _sz(tile_begin), _sz(tile_end)))

    @classmethod
    def _from_handle(cls, h) -> "Weight":
        self = cls.__new__(cls)
        self._h = h
        self._info()
        return self

    def seal(self) -> "Weight":
        """RepackedWeight::from_tile_buffers (repack.rs:2386): every tile written, then usable."""
        _check(lib().jk_weight_seal(self._h))
        return self

    @property
    def handle(self):
        return self._h

    def free(self) -> None:
        if getattr(self, "_h", None):
            lib().jk_weight_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class GgufFileInfoC(C.Structure):
    _fields_ = [("version", C.c_uint32), ("n_tensors", _sz), ("n_kv", _sz), ("alignment", _sz),
                ("data_offset", _sz), ("file_bytes", _sz)]


class GgufTensorC(C.Structure):
    _fields_ = [("name", C.c_char_p), ("ggml_type", C.c_uint32), ("n_dims", C.c_uint32), ("ne", C.c_uint64 * 4),
                ("offset", _sz), ("nbytes", _sz), ("data", _vp)]


class GGUF:
    """A GGUF v2 / v3 file opened by libjk (memory-mapped): tensor records and streaming
    loads of its weight matrices into device handles."""

    def __init__(self, path: str):
        h = _vp()
        _check(lib().jk_gguf_open(os.fsencode(path), C.byref(h)))
        self._h = h
        fi = GgufFileInfoC()
        _check(lib().jk_gguf_get_file_info(h, C.byref(fi)))
        self.version, self.alignment, self.data_offset = fi.version, fi.alignment, fi.data_offset
        self.n_kv, self.file_bytes = fi.n_kv, fi.file_bytes
        self.tensors = []
        for i in range(fi.n_tensors):
            t = GgufTensorC()
            _check(lib().jk_gguf_tensor_info(h, _sz(i), C.byref(t)))
            self.tensors.append({"name": t.name.decode(), "type": t.ggml_type, "shape": list(t.ne[:t.n_dims]),
                                 "offset": t.offset, "nbytes": t.nbytes, "data": t.data or 0})

    def index(self, name: str) -> int:
        i = _sz()
        _check(lib().jk_gguf_find(self._h, name.encode(), C.byref(i)))
        return int(i.value)

    def load(self, tensor, stream=None, chunk_bytes: int = 0) -> Weight:
        """The device weight of a 2D tensor (by name or index), streamed in tile-range chunks."""
        i = self.index(tensor) if isinstance(tensor, str) else int(tensor)
        h = _vp()
        _check(lib().jk_gguf_load_weight(_vp(stream or 0), self._h, _sz(i), _sz(chunk_bytes), C.byref(h)))
        return Weight._from_handle(h)

    def close(self) -> None:
        if getattr(self, "_h", None):
            lib().jk_gguf_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def act_q8_bytes(m: int, k: int) -> int:
    return int(lib().jk_act_q8_bytes(_sz(m), _sz(k)))


def act_q8_bind(storage, storage_len: int, m: int, k: int) -> ActQ8C:
    a = ActQ8C()
    _check(lib().jk_act_q8_bind(_vp(_ptr(storage)), _sz(storage_len), _sz(m), _sz(k), C.byref(a)))
    return a


def dev_quantize_row_q8_0(x, n, out, out_blocks, stream=None):
    _check(lib().jk_quantize_row_q8_0(_vp(stream or 0), _vp(_ptr(x)), _sz(n), _vp(_ptr(out)), _sz(out_blocks)))


def dev_quantize_row_q8_k(x, n, out, out_blocks, stream=None):
    _check(lib().jk_quantize_row_q8_k(_vp(stream or 0), _vp(_ptr(x)), _sz(n), _vp(_ptr(out)), _sz(out_blocks)))


def dev_quantize_act_q8(x, m, k, act: ActQ8C, stream=None):
    _check(lib().jk_quantize_act_q8(_vp(stream or 0), _vp(_ptr(x)), _sz(m), _sz(k), C.byref(act)))


def dev_subln_quantize_absmax_i8(x, norm_w, m, k, eps, q, scales, stream=None):
    _check(lib().jk_subln_quantize_absmax_i8(_vp(stream or 0), _vp(_ptr(x)), _vp(_ptr(norm_w)), _sz(m), _sz(k),
                                             C.c_float(eps), _vp(_ptr(q)), _vp(_ptr(scales))))


def dev_quantize_absmax_i8(x, m, k, q, scales, stream=None):
    _check(lib().jk_quantize_absmax_i8(_vp(stream or 0), _vp(_ptr(x)), _sz(m), _sz(k), _vp(_ptr(q)),
                                       _vp(_ptr(scales))))


_GEMV_FN = {Q4_0: "jk_gemv_q4_0_q8_0", Q8_0: "jk_gemv_q8_0_q8_0", Q4_K: "jk_gemv_q4_k_q8_k",
            Q6_K: "jk_gemv_q6_k_q8_k", TQ2_0: "jk_gemv_tq2_0_q8_k", Q5_0: "jk_gemv_q5_0_q8_0",
            Q5_K: "jk_gemv_q5_k_q8_k", TQ1_0: "jk_gemv_tq1_0_q8_k"}


def dev_gemv_q8(w: Weight, x, nx, y, y_len, stream=None, fn: str | None = None):
    name = fn or _GEMV_FN.get(w.quant, "jk_gemv_q4_0_q8_0")
    _check(getattr(lib(), name)(_vp(stream or 0), w.handle, _vp(_ptr(x)), _sz(nx), _vp(_ptr(y)), _sz(y_len)))


def dev_gemv_q8_rows(w: Weight, x, nx, y, r0, r1, stream=None):
    _check(lib().jk_gemv_q8_rows(_vp(stream or 0), w.handle, _vp(_ptr(x)), _sz(nx), _vp(_ptr(y)), _sz(r0), _sz(r1)))


def dev_gemv_q8_f32(w: Weight, x, n, y, y_len, stream=None):
    """quantize_row_q8_0/q8_k of f32 x and the matching gemv_* in one launch."""
    _check(lib().jk_gemv_q8_f32(_vp(stream or 0), w.handle, _vp(_ptr(x)), _sz(n), _vp(_ptr(y)), _sz(y_len)))


def gemv_jobs(jobs) -> C.Array:
    """ctypes array of jk_gemv_job from (weight, x_q8, x_f32, y, row_begin, row_end) tuples."""
    arr = (GemvJobC * max(1, len(jobs)))()
    for i, (w, xq, xf, y, r0, r1) in enumerate(jobs):
        arr[i] = GemvJobC(w.handle.value if isinstance(w, Weight) else w, _ptr(xq) or None, _ptr(xf) or None,
                          _ptr(y) or None, r0, r1)
    return arr


def dev_gemv_q8_batch(jobs, stream=None):
    """Grouped quant_q8 GEMV over (weight, x_q8, x_f32, y, row_begin, row_end) tuples."""
    arr = jobs if isinstance(jobs, C.Array) else gemv_jobs(jobs)
    n = len(jobs)
    _check(lib().jk_gemv_q8_batch(_vp(stream or 0), arr, _sz(n)))


def dev_vec_dot_f32(w: Weight, x, n, y, y_len, stream=None):
    _check(lib().jk_vec_dot_f32(_vp(stream or 0), w.handle, _vp(_ptr(x)), _sz(n), _vp(_ptr(y)), _sz(y_len)))


def dev_vec_dot_f32_tol(w: Weight, x, n, y, y_len, stream=None):
    """jk_vec_dot_f32_tol: the f32-activation matvec within 1e-5 of each output's row L2 norm."""
    _check(lib().jk_vec_dot_f32_tol(_vp(stream or 0), w.handle, _vp(_ptr(x)), _sz(n), _vp(_ptr(y)), _sz(y_len)))


def dev_gemm_repacked(w: Weight, act: ActQ8C, y, y_len, r0, r1, stream=None):
    _check(lib().jk_gemm_repacked(_vp(stream or 0), w.handle, C.byref(act), _vp(_ptr(y)), _sz(y_len), _sz(r0),
                                  _sz(r1)))


def dev_gemm_repacked_tol(w: Weight, act: ActQ8C, y, y_len, r0, r1, stream=None):
    """Tolerance-mode repacked GEMM (one fused multiply-add per scale group)."""
    _check(lib().jk_gemm_repacked_tol(_vp(stream or 0), w.handle, C.byref(act), _vp(_ptr(y)), _sz(y_len), _sz(r0),
                                      _sz(r1)))


def dev_gemv_repacked(w: Weight, act: ActQ8C, y, y_len, r0, r1, stream=None):
    _check(lib().jk_gemv_repacked(_vp(stream or 0), w.handle, C.byref(act), _vp(_ptr(y)), _sz(y_len), _sz(r0),
                                  _sz(r1)))


def dev_convert_i2_s_to_tq2_0(i2s, i2s_blocks, scale_f16_bits, tq2, tq2_blocks, stream=None):
    _check(lib().jk_convert_i2_s_to_tq2_0(_vp(stream or 0), _vp(_ptr(i2s)), _sz(i2s_blocks),
                                          C.c_uint16(scale_f16_bits), _vp(_ptr(tq2)), _sz(tq2_blocks)))


def dev_bitlinear_i8(w: Weight, act, act_scales, m, k, y, y_len, stream=None):
    _check(lib().jk_bitlinear_i8(_vp(stream or 0), w.handle, _vp(_ptr(act)), _vp(_ptr(act_scales)), _sz(m), _sz(k),
                                 _vp(_ptr(y)), _sz(y_len)))


def dev_bitlinear_i8_tol(w: Weight, act, act_scales, m, k, y, y_len, stream=None):
    """jk_bitlinear_i8_tol: BitLinear within 1e-5 of each token's output-row L2 norm (sums in any order)."""
    _check(lib().jk_bitlinear_i8_tol(_vp(stream or 0), w.handle, _vp(_ptr(act)), _vp(_ptr(act_scales)), _sz(m),
                                     _sz(k), _vp(_ptr(y)), _sz(y_len)))


def dev_dequantize_rows(w: Weight, r0, r1, out, out_len, stream=None):
    _check(lib().jk_weight_dequantize_rows(_vp(stream or 0), w.handle, _sz(r0), _sz(r1), _vp(_ptr(out)),
                                           _sz(out_len)))


def host_gemm_repacked_f32(out: np.ndarray, w: Weight, inp, m: int, r0: int, r1: int) -> None:
    """gemm_repacked_f32_rows (repack.rs:4143)."""
    x = _f32(inp).reshape(-1)
    _check(lib().jk_host_gemm_repacked_f32(_vp(out.ctypes.data), _sz(out.size), w.handle, _vp(x.ctypes.data), _sz(m),
                                           _sz(r0), _sz(r1)))


# ---------------------------------------------------------------- epilogues
ACT_SWIGLU, ACT_RELU2 = 1, 2


def swiglu_f32(out: np.ndarray, gate, up) -> None:
    """swiglu_f32 (swiglu.rs:62) on host slices."""
    g, u = _f32(gate).reshape(-1), _f32(up).reshape(-1)
    _check(lib().jk_host_swiglu_f32(_vp(out.ctypes.data), _sz(out.size), _vp(g.ctypes.data), _sz(g.size),
                                    _vp(u.ctypes.data), _sz(u.size)))


def relu_squared_gate_f32(out: np.ndarray, gate, up) -> None:
    """relu_squared_gate_f32 (lib.rs:1111) on host slices."""
    g, u = _f32(gate).reshape(-1), _f32(up).reshape(-1)
    _check(lib().jk_host_relu_squared_gate_f32(_vp(out.ctypes.data), _sz(out.size), _vp(g.ctypes.data), _sz(g.size),
                                               _vp(u.ctypes.data), _sz(u.size)))


def argmax_f32(logits):
    """argmax_f32 (lib.rs:662): the index, or None for empty / all-NaN input."""
    x = _f32(logits).reshape(-1)
    idx = C.c_int64(-1)
    _check(lib().jk_host_argmax_f32(_vp(x.ctypes.data if x.size else 0), _sz(x.size), C.byref(idx)))
    return None if idx.value < 0 else int(idx.value)


def dev_swiglu_f32(gate, up, n, out, stream=None):
    _check(lib().jk_swiglu_f32(_vp(stream or 0), _vp(_ptr(gate)), _vp(_ptr(up)), _sz(n), _vp(_ptr(out))))


def dev_relu_squared_gate_f32(gate, up, n, out, stream=None):
    _check(lib().jk_relu_squared_gate_f32(_vp(stream or 0), _vp(_ptr(gate)), _vp(_ptr(up)), _sz(n), _vp(_ptr(out))))


def dev_quantize_row_q8_k_gated(act: int, gate, up, n, out, out_blocks, stream=None):
    _check(lib().jk_quantize_row_q8_k_gated(_vp(stream or 0), C.c_int(act), _vp(_ptr(gate)), _vp(_ptr(up)), _sz(n),
                                            _vp(_ptr(out)), _sz(out_blocks)))


def dev_quantize_act_q8_gated(act: int, gate, up, m, k, act_q8: ActQ8C, stream=None):
    _check(lib().jk_quantize_act_q8_gated(_vp(stream or 0), C.c_int(act), _vp(_ptr(gate)), _vp(_ptr(up)), _sz(m),
                                          _sz(k), C.byref(act_q8)))


def argmax_workspace_bytes(n: int) -> int:
    """Device workspace bytes for an argmax over n values, or a fused GEMV argmax of n rows."""
    f = lib().jk_argmax_workspace_bytes
    f.restype = _sz
    return int(f(_sz(n)))


def _ws_bytes(ws, ws_bytes):
    return ws_bytes if ws_bytes is not None else (ws.numel() * ws.element_size() if ws is not None else 0)


def dev_argmax_f32(x, n, index, ws, stream=None, ws_bytes=None):
    _check(lib().jk_argmax_f32(_vp(stream or 0), _vp(_ptr(x)), _sz(n), _vp(_ptr(index)), _vp(_ptr(ws)),
                               _sz(_ws_bytes(ws, ws_bytes))))


def dev_gemv_q8_argmax(w: Weight, x_q8, x_f32, x_len, y, index, ws, stream=None, ws_bytes=None):
    _check(lib().jk_gemv_q8_argmax(_vp(stream or 0), w.handle, _vp(_ptr(x_q8)), _vp(_ptr(x_f32)), _sz(x_len),
                                   _vp(_ptr(y)), _vp(_ptr(index)), _vp(_ptr(ws)), _sz(_ws_bytes(ws, ws_bytes))))


def dev_gemv_q8_argmax_noalloc(w: Weight, x_q8, x_f32, x_len, y, index, stream=None):
    """jk_gemv_q8_argmax with the argmax slots in the library's static device scratch."""
    _check(lib().jk_gemv_q8_argmax_noalloc(_vp(stream or 0), w.handle, _vp(_ptr(x_q8)), _vp(_ptr(x_f32)),
                                           _sz(x_len), _vp(_ptr(y)), _vp(_ptr(index))))


def dev_gemm_i8(a, a_len, m, b, b_len, n0, n1, k, c, c_len, stream=None):
    """jk_gemm_i8: gemm_i8_vector (ime.rs:563-583), c[row][n - n0] in exact i32."""
    _check(lib().jk_gemm_i8(_vp(stream or 0), _vp(_ptr(a)), _sz(a_len), _sz(m), _vp(_ptr(b)), _sz(b_len), _sz(n0),
                            _sz(n1), _sz(k), _vp(_ptr(c)), _sz(c_len)))


def dev_gemm_i8_tiles(a_packed, a_len, m_tiles, b_packed, b_len, nt0, nt1, k_chunks, c, c_len, stream=None):
    """jk_gemm_i8_tiles: gemm_i8_ime (ime.rs:449-486) over pack_tiles layouts, 8 x 8 i32 tiles."""
    _check(lib().jk_gemm_i8_tiles(_vp(stream or 0), _vp(_ptr(a_packed)), _sz(a_len), _sz(m_tiles),
                                  _vp(_ptr(b_packed)), _sz(b_len), _sz(nt0), _sz(nt1), _sz(k_chunks), _vp(_ptr(c)),
                                  _sz(c_len)))


def dev_pack_tiles_i8(src, src_len, rows, k, dst, dst_len, stream=None):
    """jk_pack_tiles_i8: pack_tiles (ime.rs:81-94) on the device."""
    _check(lib().jk_pack_tiles_i8(_vp(stream or 0), _vp(_ptr(src)), _sz(src_len), _sz(rows), _sz(k), _vp(_ptr(dst)),
                                  _sz(dst_len)))


def dev_dot_i8(a, a_len, b, b_len, out, stream=None):
    """jk_dot_i8: dot_i8_vector (ime.rs:548-557) over the zip of the two slices, one i32."""
    _check(lib().jk_dot_i8(_vp(stream or 0), _vp(_ptr(a)), _sz(a_len), _vp(_ptr(b)), _sz(b_len), _vp(_ptr(out))))


def gemm_i8_vector(a: np.ndarray, m: int, b: np.ndarray, n0: int, n1: int, k: int) -> np.ndarray:
    """gemm_i8_vector (ime.rs:563-583) through jk_host_gemm_i8: [m][n1 - n0] i32 of host slices."""
    a = np.ascontiguousarray(a, dtype=np.int8).reshape(-1)
    b = np.ascontiguousarray(b, dtype=np.int8).reshape(-1)
    c = np.zeros(max(m * (n1 - n0), 0), dtype=np.int32)
    _check(lib().jk_host_gemm_i8(_vp(_ptr(a)), _sz(a.size), _sz(m), _vp(_ptr(b)), _sz(b.size), _sz(n0), _sz(n1),
                                 _sz(k), _vp(_ptr(c)), _sz(c.size)))
    return c.reshape(m, n1 - n0)


def dot_i8_vector(a: np.ndarray, b: np.ndarray) -> int:
    """dot_i8_vector (ime.rs:548-557) through jk_host_dot_i8, over the zip of the two slices."""
    a = np.ascontiguousarray(a, dtype=np.int8).reshape(-1)
    b = np.ascontiguousarray(b, dtype=np.int8).reshape(-1)
    out = C.c_int32(0)
    _check(lib().jk_host_dot_i8(_vp(_ptr(a)), _sz(a.size), _vp(_ptr(b)), _sz(b.size), C.byref(out)))
    return out.value


def op_counts() -> tuple[int, int]:
    """jk_op_counts: (ime_vmadot_count, vector_dot_count) of ime.rs:53-66 -- tile steps of
    jk_gemm_i8_tiles and dot products of jk_gemm_i8 and the BitLinear entry points."""
    t, v = C.c_uint64(0), C.c_uint64(0)
    lib().jk_op_counts(C.byref(t), C.byref(v))
    return t.value, v.value


def dev_measure_stream_read(buf, nbytes, sink, stream=None):
    """jk_measure_stream_read: a plain streaming read of nbytes of device memory (the roofline
    the GEMV launches are placed against)."""
    _check(lib().jk_measure_stream_read(_vp(stream or 0), _vp(_ptr(buf)), _sz(nbytes), _vp(_ptr(sink))))


def gemm_plan(w: Weight, act: ActQ8C, r0: int, r1: int, tolerance: bool) -> str | None:
    """jk_gemm_plan: the kernel jk_gemm_repacked(_tol) launches for this activation and row range."""
    k = C.c_char_p()
    _check(lib().jk_gemm_plan(w.handle, C.byref(act), _sz(r0), _sz(r1), C.c_int(int(tolerance)), C.byref(k)))
    return k.value.decode() if k.value else None


def bitlinear_plan(w: Weight, act, m: int, tolerance: bool = False) -> str:
    """jk_bitlinear_plan: the kernel jk_bitlinear_i8(_tol) launches for m tokens whose rows start at act."""
    k = C.c_char_p()
    _check(lib().jk_bitlinear_plan(w.handle, _vp(_ptr(act)), _sz(m), C.c_int(int(tolerance)), C.byref(k)))
    return k.value.decode()
