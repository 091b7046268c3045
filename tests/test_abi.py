"""C-ABI checks that need no GPU: libjk.so loads, exports every function include/jk.h
declares, its structs have the reference's byte layouts, and invalid arguments fail
closed with the reference's error kinds before any device work is attempted
(fail-closed tests: tests/test_repack_gemv_gemm.rs:883-917, src/quant_q8.rs:3414-3427)."""
import ctypes as C

import numpy as np
import pytest

import jk


def test_library_loads_and_exports_every_declared_symbol():
    lib = jk.lib()
    names = jk.header_symbols()
    assert len(names) > 40
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert lib.jk_abi_version() == 1


def test_block_struct_layouts():
    assert jk.BLOCK_Q8_0.itemsize == 36 and jk.BLOCK_Q8_0.fields["qs"][1] == 4
    assert jk.BLOCK_Q8K.itemsize == 292 and jk.BLOCK_Q8K.fields["bsums"][1] == 260


def test_act_q8_bytes_and_bind_layout():
    m, k = 7, 300
    need = jk.act_q8_bytes(m, k)
    buf = np.zeros(need + 64, np.uint8)
    base = (buf.ctypes.data + 15) & ~15
    a = jk.act_q8_bind(base, need, m, k)
    assert (a.k_padded, a.k_blocks32, a.k_chunks, a.sb256) == (320, 10, 20, 2)
    assert a.qs % 256 == 0 and a.qs + m * a.k_padded <= base + need
    with pytest.raises(jk.TensorBoundsError):
        jk.act_q8_bind(base, need - 1, m, k)
    with pytest.raises(jk.TensorBoundsError):
        jk.act_q8_bind(base, need, 0, k)


def test_quantize_validation_fails_closed():
    with pytest.raises(jk.TensorBoundsError):
        jk.quantize_row_q8_0(np.zeros(0, np.float32))
    with pytest.raises(jk.TensorBoundsError):
        jk.quantize_row_q8_0(np.ones(31, np.float32))
    with pytest.raises(jk.TensorBoundsError):
        jk.quantize_row_q8_k(np.ones(255, np.float32))


def test_gemv_validation_fails_closed():
    raw = np.zeros(4 * 18, np.uint8)
    x = np.zeros(1, jk.BLOCK_Q8_0)
    out = np.zeros(4, np.float32)
    # quant mismatch is a TensorBoundsError in the reference validators
    with pytest.raises(jk.TensorBoundsError, match="expected Q8_0"):
        jk.gemv_q8_0_q8_0(out, jk.TensorView("w", jk.Q4_0, [4, 32], raw), x)
    with pytest.raises(jk.TensorBoundsError):  # output length
        jk.gemv_q4_0_q8_0(np.zeros(3, np.float32), jk.TensorView("w", jk.Q4_0, [4, 32], raw), x)
    with pytest.raises(jk.TensorBoundsError):  # short buffer
        jk.gemv_q4_0_q8_0(out, jk.TensorView("w", jk.Q4_0, [4, 32], raw[:-1]), x)
    with pytest.raises(jk.TensorBoundsError):  # activation block count
        jk.gemv_q4_0_q8_0(out, jk.TensorView("w", jk.Q4_0, [4, 32], raw), np.zeros(2, jk.BLOCK_Q8_0))
    with pytest.raises(jk.TensorBoundsError):  # empty shape
        jk.gemv_q4_0_q8_0(out, jk.TensorView("w", jk.Q4_0, [], raw), x)
    with pytest.raises(jk.TensorBoundsError):  # single-row length mismatch
        jk.vec_dot_q4_0_q8_0(raw[:17], x)


def test_vec_dot_and_bitlinear_validation_fails_closed():
    raw = np.zeros(2 * 34, np.uint8)
    with pytest.raises(jk.TensorBoundsError):
        jk.vec_dot_q8_0(np.zeros(2, np.float32), jk.TensorView("w", jk.Q8_0, [2, 32], raw), np.zeros(16, np.float32))
    with pytest.raises(jk.TensorBoundsError):  # Q4_K view handed to the Q6_K entry
        jk.vec_dot_q6_k(np.zeros(1, np.float32), jk.TensorView("w", jk.Q4_K, [1, 256], np.zeros(144, np.uint8)),
                        np.zeros(256, np.float32))
    tq = np.zeros(66, np.uint8)
    with pytest.raises(jk.TensorBoundsError):  # unsupported format for BitLinear (ime.rs:666-683)
        jk.bitlinear_i8(np.zeros(1, np.float32), jk.TensorView("w", jk.Q4_K, [1, 256], np.zeros(144, np.uint8)),
                        np.zeros(256, np.int8), 1.0)
    with pytest.raises(jk.TensorBoundsError):  # I2_S without its 32-byte trailer
        jk.bitlinear_i8(np.zeros(1, np.float32), jk.TensorView("w", jk.I2_S, [1, 128], np.zeros(32, np.uint8)),
                        np.zeros(128, np.int8), 1.0)
    with pytest.raises(jk.TensorBoundsError):
        jk.bitlinear_i8(np.zeros(2, np.float32), jk.TensorView("w", jk.TQ2_0, [1, 256], tq), np.zeros(256, np.int8),
                        1.0)


def test_dequantize_row_validation_fails_closed():
    raw = np.zeros(2 * 34, np.uint8)
    v = jk.TensorView("t", jk.Q8_0, [32, 2], raw)
    with pytest.raises(jk.TensorBoundsError):
        jk.dequantize_tensor_row(v, 2, np.zeros(32, np.float32))
    with pytest.raises(jk.TensorBoundsError):
        jk.dequantize_tensor_row(v, 0, np.zeros(16, np.float32))
    with pytest.raises(jk.CapabilityMismatch):  # Q8_1 / MXFP4 and other formats
        jk.dequantize_tensor_row(jk.TensorView("t", 9, [32, 2], raw), 0, np.zeros(32, np.float32))


def test_weight_upload_validation_fails_closed():
    with pytest.raises(jk.CapabilityMismatch):  # F16 has no block-scaled layout here
        jk.Weight(jk.TensorView("w", 1, [2, 32], np.zeros(128, np.uint8)))
    with pytest.raises(jk.TensorBoundsError):  # cols not a multiple of the block size
        jk.Weight(jk.TensorView("w", jk.Q4_K, [2, 128], np.zeros(144, np.uint8)), rows=2, cols=128)
    with pytest.raises(jk.TensorBoundsError):  # buffer shorter than the matrix
        jk.Weight(jk.TensorView("w", jk.Q8_0, [4, 64], np.zeros(100, np.uint8)), rows=4, cols=64)
    with pytest.raises(jk.TensorBoundsError):  # 3D tensor
        jk.Weight(jk.TensorView("w", jk.Q8_0, [2, 2, 32], np.zeros(136, np.uint8)))
