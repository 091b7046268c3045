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
    assert lib.jk_abi_version() == 4


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


LAYOUT_FORMATS = [jk.Q4_0, jk.Q4_1, jk.Q5_0, jk.Q5_1, jk.Q8_0, jk.IQ4_NL, jk.Q2_K, jk.Q3_K, jk.Q4_K, jk.Q5_K,
                  jk.Q6_K, jk.TQ1_0, jk.TQ2_0, jk.I2_S]


@pytest.mark.parametrize("quant", LAYOUT_FORMATS)
@pytest.mark.parametrize("rows,cols", [(67, 512), (19, 256), (8, 768), (1, 256)])
def test_weight_layout_for(quant, rows, cols):
    """BlockScaledTileLayout::from_validated_dims (repack.rs:1339-1372) and its totals
    (1424-1449): tiles of 8 rows, 16-element K chunks over K padded to 32, one chunk per scale
    for the 16-element-scale formats, mins for the asymmetric ones; device bytes are the GGUF
    bytes except TQ1_0 (66 per 54-byte block) and Q3_K (112 per 110)."""
    nb = cols // jk.BLOCK_ELEMENTS[quant]
    raw = np.zeros(rows * nb * jk.BLOCK_BYTES[quant] + jk.TRAILER_BYTES.get(quant, 0), np.uint8)
    if quant == jk.I2_S:
        raw[-32:-28] = np.frombuffer(np.float32(0.75).tobytes(), np.uint8)
    L = jk.block_scaled_layout(jk.TensorView("w", quant, [cols, rows], raw), rows, cols)
    cps = 1 if quant in (jk.Q6_K, jk.Q3_K, jk.Q2_K) else 2
    k_padded = -(-cols // 32) * 32
    assert (L.quant, L.rows, L.cols, L.row_bytes) == (quant, rows, cols, nb * jk.BLOCK_BYTES[quant])
    assert (L.k_padded, L.n_tiles, L.k_chunks, L.chunks_per_scale) == (k_padded, -(-rows // 8), k_padded // 16, cps)
    assert L.scale_groups == k_padded // 16 // cps
    assert bool(L.has_mins) == (quant in (jk.Q4_K, jk.Q5_K, jk.Q4_1, jk.Q5_1, jk.Q2_K))
    assert L.total_tiles == L.n_tiles * L.k_chunks and L.total_scales == L.n_tiles * L.scale_groups * 8
    assert L.total_mins == (L.total_scales if L.has_mins else 0)
    assert L.scales_for_tiles(3) == 3 * L.scale_groups * 8
    dev_block = {jk.TQ1_0: 66, jk.Q3_K: 112}.get(quant, jk.BLOCK_BYTES[quant])
    assert L.device_bytes == rows * nb * dev_block and L.gguf_bytes == raw.size
    assert L.tensor_scale == (0.75 if quant == jk.I2_S else 0.0)


def test_weight_layout_validation_fails_closed():
    raw = np.zeros(67 * 2 * 144, np.uint8)
    with pytest.raises(jk.CapabilityMismatch):  # dense / unsupported (repack.rs:1325-1335)
        jk.block_scaled_layout(jk.TensorView("w", 1, [512, 67], raw), 67, 512)
    with pytest.raises(jk.TensorBoundsError):  # cols not a multiple of the block
        jk.block_scaled_layout(jk.TensorView("w", jk.Q4_K, [500, 67], raw), 67, 500)
    with pytest.raises(jk.TensorBoundsError):  # shape does not match
        jk.block_scaled_layout(jk.TensorView("w", jk.Q4_K, [512, 66], raw), 67, 512)
    with pytest.raises(jk.TensorBoundsError):  # short buffer
        jk.block_scaled_layout(jk.TensorView("w", jk.Q4_K, [512, 67], raw[:-1]), 67, 512)
    with pytest.raises(jk.TensorBoundsError):  # no inference from rows = cols = 0 (for_tensor)
        jk.block_scaled_layout(jk.TensorView("w", jk.Q4_K, [512, 67], raw), 0, 0)


def _err(fn, *args):
    with pytest.raises(jk.K3Error) as ei:
        fn(*args)
    return ei.value


def test_tensor_bounds_error_fields():
    """TensorBoundsError's payload (tensor_name, offset, byte_len, buffer_len, reason) as the
    reference's validators fill it: view checks report the view (validate_quant_matvec_dimensions,
    quant.rs:1816-1888: name, TensorView::offset, byte_len, buffer length); check_q8_block_len
    (quant_q8.rs:1562-1578) the block counts; validate_q8_block_row_bytes (quant_q8.rs:644-664)
    the row bytes; validate_activation_quant_slice (quant_q8.rs:111-149) the input bytes and the
    output block count. Every check runs before any device work, so no GPU is needed."""
    raw = np.zeros(4 * 18, np.uint8)
    x = np.zeros(1, jk.BLOCK_Q8_0)
    out = np.zeros(4, np.float32)
    e = _err(jk.gemv_q8_0_q8_0, out, jk.TensorView("blk.3.ffn_up.weight", jk.Q4_0, [4, 32], raw, offset=4096), x)
    assert isinstance(e, jk.TensorBoundsError)
    assert (e.tensor_name, e.offset, e.byte_len, e.buffer_len) == ("blk.3.ffn_up.weight", 4096, 72, 72)
    assert "expected Q8_0 quant type" in e.reason
    e = _err(jk.gemv_q4_0_q8_0, out, jk.TensorView("w", jk.Q4_0, [4, 32], raw[:-1], offset=7), x)
    assert (e.tensor_name, e.offset, e.byte_len, e.buffer_len) == ("w", 7, 71, 71)
    assert "buffer length 71 < required 72" in e.reason
    e = _err(jk.gemv_q4_0_q8_0, out, jk.TensorView("w", jk.Q4_0, [4, 32], raw), np.zeros(2, jk.BLOCK_Q8_0))
    assert isinstance(e, jk.TensorBoundsError) and e.tensor_name == "w"
    e = _err(jk.vec_dot_q4_0_q8_0, raw[:17], x)
    assert (e.tensor_name, e.offset, e.byte_len, e.buffer_len) == ("vec_dot_q4_0_q8_0", 0, 17, 18)
    e = _err(jk.quantize_row_q8_0, np.ones(31, np.float32))
    assert (e.tensor_name, e.offset, e.byte_len) == ("quantize_row_q8_0_f32", 0, 124)
    e = _err(jk.quantize_row_q8_k, np.ones(300, np.float32))
    assert (e.tensor_name, e.byte_len) == ("quantize_row_q8_k", 1200)
    e = _err(jk.bitlinear_i8, np.zeros(1, np.float32),
             jk.TensorView("bw", jk.I2_S, [1, 128], np.zeros(32, np.uint8), offset=64), np.zeros(128, np.int8), 1.0)
    assert (e.tensor_name, e.offset, e.byte_len, e.buffer_len) == ("bw", 64, 32, 32)
    info = jk.last_error_info()
    assert info["status"] == jk.TENSOR_BOUNDS and info["tensor_name"] == "bw" and info["reason"] == e.reason
    e = _err(jk.dequantize_tensor_row, jk.TensorView("emb", jk.Q8_0, [32, 2], np.zeros(68, np.uint8), offset=9), 2,
             np.zeros(32, np.float32))
    assert (e.tensor_name, e.offset, e.byte_len) == ("emb", 9, 68) and "out of bounds" in e.reason


def test_static_archive_exports_every_declared_symbol():
    """libjk.a (for a Rust build.rs) holds the same entry points as libjk.so."""
    import os
    import subprocess

    path = os.path.join(os.path.dirname(jk.LIB_PATH), "libjk.a")
    assert os.path.exists(path), "libjk.a not built"
    out = subprocess.run(["nm", "-g", "--defined-only", path], capture_output=True, text=True, check=True).stdout
    defined = {line.split()[-1] for line in out.splitlines() if line.strip() and not line.endswith(":")}
    missing = [n for n in jk.header_symbols() if n not in defined]
    assert not missing, missing
