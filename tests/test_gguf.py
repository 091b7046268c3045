"""The GGUF reader (jk_gguf_*) on files written by tests/gguf_writer.py, with no GPU: header,
metadata of every value type (nested arrays included), tensor records, the alignment rule,
the mapped bytes, and fail-closed errors for malformed files, including every truncation of
a file's header."""
import ctypes as C

import numpy as np
import pytest

import jk
from gguf_writer import ARR, BOOL, F32, F64, I8, I16, I32, I64, STR, U8, U16, U32, U64, write_gguf
from jk import synth

KV = [("general.architecture", STR, "llama"), ("llama.block_count", U32, 32), ("a.u8", U8, 7), ("a.i8", I8, -3),
      ("a.u16", U16, 65535), ("a.i16", I16, -2), ("a.i32", I32, -70000), ("a.f32", F32, 0.5), ("a.bool", BOOL, True),
      ("a.u64", U64, 1 << 40), ("a.i64", I64, -(1 << 40)), ("a.f64", F64, 2.25),
      ("tokenizer.ggml.tokens", ARR, (STR, ["<s>", "</s>", "hello"])), ("a.ints", ARR, (I32, [1, 2, 3])),
      ("a.nested", ARR, (ARR, [(U8, [1, 2]), (STR, ["x"])])), ("a.empty", ARR, (U64, []))]


def model_tensors():
    out = []
    for name, quant, rows, cols in [("blk.0.attn_q.weight", jk.Q4_K, 19, 512), ("blk.0.ffn_down.weight", jk.Q6_K, 8, 256),
                                    ("blk.0.attn_k.weight", jk.Q8_0, 5, 64), ("blk.0.ffn_up.weight", jk.TQ1_0, 3, 256),
                                    ("blk.0.ffn_gate.weight", jk.I2_S, 4, 128), ("blk.0.x.weight", jk.Q5_0, 9, 96)]:
        out.append((name, quant, [cols, rows], synth.gguf_weights(quant, rows, cols, seed=rows)))
    out.append(("token_embd_norm.weight", 0, [64], np.arange(256, dtype=np.uint8)))  # F32 [64]
    out.append(("output.weight", 1, [32, 2], np.arange(128, dtype=np.uint8)))  # F16 [2, 32]
    out.append(("blk.0.q8_vector", jk.Q8_0, [64], synth.gguf_weights(jk.Q8_0, 1, 64, seed=2)))
    return out


@pytest.mark.parametrize("alignment", [None, 64, 256])
def test_reader_records_and_bytes(tmp_path, alignment):
    path = tmp_path / "m.gguf"
    tensors = model_tensors()
    start, offsets = write_gguf(path, tensors, KV, alignment=alignment)
    g = jk.GGUF(str(path))
    assert (g.version, g.alignment, g.data_offset) == (3, alignment or 32, start)
    assert g.n_kv == len(KV) + (alignment is not None) and g.file_bytes == path.stat().st_size
    assert len(g.tensors) == len(tensors)
    for t, (name, quant, ne, data), off in zip(g.tensors, tensors, offsets):
        assert (t["name"], t["type"], t["shape"], t["offset"]) == (name, quant, ne, off)
        assert t["nbytes"] == len(data)
        assert C.string_at(t["data"], t["nbytes"]) == bytes(data)
        assert g.index(name) == g.tensors.index(t)
    with pytest.raises(jk.TensorBoundsError):
        g.index("missing.weight")
    with pytest.raises(jk.CapabilityMismatch):  # F16 is not a block format (repack.rs:1325-1335)
        g.load("output.weight")
    with pytest.raises(jk.CapabilityMismatch):
        g.load("token_embd_norm.weight")
    with pytest.raises(jk.TensorBoundsError):  # a 1-D tensor is not a weight matrix
        g.load("blk.0.q8_vector")
    with pytest.raises(jk.TensorBoundsError):
        g.load(len(tensors))
    g.close()


def test_version_2_reads_like_3(tmp_path):
    path = tmp_path / "v2.gguf"
    write_gguf(path, model_tensors()[:2], KV[:3], version=2)
    g = jk.GGUF(str(path))
    assert g.version == 2 and [t["name"] for t in g.tensors] == ["blk.0.attn_q.weight", "blk.0.ffn_down.weight"]


def _raises_closed(path):
    with pytest.raises((jk.TensorBoundsError, jk.CapabilityMismatch)):
        jk.GGUF(str(path))


def test_malformed_files_fail_closed(tmp_path):
    good = tmp_path / "good.gguf"
    start, _ = write_gguf(good, model_tensors()[:3], KV)
    blob = good.read_bytes()
    cases = {
        "magic": b"GGUX" + blob[4:],
        "version1": blob[:4] + (1).to_bytes(4, "little") + blob[8:],
        "version4": blob[:4] + (4).to_bytes(4, "little") + blob[8:],
        "no_data": blob[:start + 10],
        "huge_tensor_count": blob[:8] + (1 << 40).to_bytes(8, "little") + blob[16:],
        "huge_kv_count": blob[:16] + (1 << 40).to_bytes(8, "little") + blob[24:],
    }
    for name, data in cases.items():
        p = tmp_path / f"{name}.gguf"
        p.write_bytes(data)
        _raises_closed(p)
    # every truncation inside the header and tensor records is refused
    for cut in range(0, start, 7):
        p = tmp_path / "cut.gguf"
        p.write_bytes(blob[:cut])
        _raises_closed(p)
    with pytest.raises(jk.TensorBoundsError):
        jk.GGUF(str(tmp_path / "does_not_exist.gguf"))


def test_bad_alignment_and_offsets_fail_closed(tmp_path):
    t = model_tensors()[:2]
    p = tmp_path / "align3.gguf"
    write_gguf(p, t, [("general.alignment", U32, 3)])
    _raises_closed(p)
    p = tmp_path / "align_type.gguf"
    write_gguf(p, t, [("general.alignment", U64, 64)])
    _raises_closed(p)
    # a tensor record whose offset is not a multiple of the alignment
    p = tmp_path / "misaligned.gguf"
    write_gguf(p, t, [])
    blob = bytearray(p.read_bytes())
    name = t[1][0].encode()
    i = blob.index(name) + len(name) + 4 + 8 * 2 + 4  # n_dims, ne[2], type, then the offset
    off = int.from_bytes(blob[i:i + 8], "little")
    blob[i:i + 8] = (off + 4).to_bytes(8, "little")
    p.write_bytes(bytes(blob))
    _raises_closed(p)
    # a 5-dimensional tensor record
    p = tmp_path / "dims.gguf"
    write_gguf(p, [("t", jk.Q8_0, [32, 1, 1, 1, 1], np.zeros(34, np.uint8))], [])
    _raises_closed(p)


def test_wrapping_byte_count_fails_closed(tmp_path):
    # 32 x 542551296285575048 Q8_0 elements: the element count fits 64 bits, the byte count
    # (34 bytes per 32) wraps to 16 -- refused at open, not reported as a 16-byte tensor
    p = tmp_path / "wrap.gguf"
    write_gguf(p, [("w", jk.Q8_0, [32, 542551296285575048], np.zeros(34, np.uint8))], [])
    with pytest.raises(jk.TensorBoundsError, match="overflows"):
        jk.GGUF(str(p))
    # the same for a dense type: F32 with 2^62 elements
    p = tmp_path / "wrap_f32.gguf"
    write_gguf(p, [("f", 0, [1 << 31, 1 << 31], np.zeros(16, np.uint8))], [])
    with pytest.raises(jk.TensorBoundsError, match="overflows"):
        jk.GGUF(str(p))


def test_short_file_error_names_its_size(tmp_path):
    # a file shorter than the fixed header is refused with its own size in the message (the
    # message is formed before the handle is released)
    p = tmp_path / "short.gguf"
    p.write_bytes(b"GGUF" + bytes(17))
    with pytest.raises(jk.TensorBoundsError, match=r"\(21 bytes\)"):
        jk.GGUF(str(p))
