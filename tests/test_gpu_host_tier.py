"""Host tier (jk_host_*) as a drop-in for the reference's slice signatures: with residency on,
weights named by a TensorView stay resident after the first call, and warm calls perform no upload and no device
allocation (the reference's zero-allocation contract, tests/wave4_zero_alloc_gemv.rs:88-172),
with outputs bit-identical to the first call and to the oracle. Also the fail-closed cases of
tests/test_repack_gemv_gemm.rs:883-917 on the device tier, with TensorBoundsError's fields.
"""
import threading

import numpy as np
import pytest

import jk
import oracle as O
from jk import synth

pytestmark = pytest.mark.gpu

RESIDENT_LIMIT = 16 << 30


@pytest.fixture(autouse=True)
def resident_weights(gpu):
    """Weight residency is opt in (jk_host_cache_set_limit); these tests turn it on and leave the
    library's limit as they found it, verify off."""
    prev = jk.host_stats()["cache_limit"]
    jk.host_cache_set_limit(RESIDENT_LIMIT)
    yield
    jk.host_cache_set_verify(False)
    jk.host_cache_set_limit(prev)


def same_bits(a, b) -> bool:
    a, b = np.ascontiguousarray(a, np.float32), np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and bool(np.all(a.view(np.uint32) == b.view(np.uint32)))


ROWS, COLS = 13, 512  # the shapes of wave4_quant_q8_gemv_argmax_and_repack_m1_perform_zero_heap_allocations


def zero_alloc_calls():
    """One call of every host-tier path of the reference's zero-allocation test, returning outputs."""
    x = synth.activations(COLS, 3)
    q80, q8k = O.quantize_row_q8_0(x), O.quantize_row_q8_k(x)
    views = {q: jk.TensorView(f"w{q}", q, [COLS, ROWS], synth.gguf_weights(q, ROWS, COLS, seed=q))
             for q in (jk.Q4_0, jk.Q5_0, jk.Q8_0, jk.Q4_K, jk.Q5_K, jk.Q6_K, jk.TQ1_0, jk.TQ2_0)}
    logits = np.full(32000, 0.5, np.float32)
    logits[1234] = 2.0

    def run():
        outs = []
        outs.append(jk.quantize_row_q8_0(x)["qs"].astype(np.float32))
        outs.append(jk.quantize_row_q8_k(x)["qs"].astype(np.float32))
        for fn, q, xb in (("vec_dot_q4_0_q8_0", jk.Q4_0, q80), ("vec_dot_q5_0_q8_0_blocks", jk.Q5_0, q80),
                          ("vec_dot_q8_0_q8_0", jk.Q8_0, q80), ("vec_dot_q4_k_q8_k", jk.Q4_K, q8k),
                          ("vec_dot_q5_k_q8_k", jk.Q5_K, q8k), ("vec_dot_q6_k_q8_k", jk.Q6_K, q8k),
                          ("vec_dot_tq1_0_q8_k", jk.TQ1_0, q8k), ("vec_dot_tq2_0_q8_k", jk.TQ2_0, q8k)):
            row = views[q].data[:views[q].data.size // ROWS]
            outs.append(np.float32([getattr(jk, fn)(row, xb)]))
        for fn, q, xb in (("gemv_q4_0_q8_0", jk.Q4_0, q80), ("gemv_q5_0_q8_0", jk.Q5_0, q80),
                          ("gemv_q8_0_q8_0", jk.Q8_0, q80), ("gemv_q4_k_q8_k", jk.Q4_K, q8k),
                          ("gemv_q5_k_q8_k", jk.Q5_K, q8k), ("gemv_q6_k_q8_k", jk.Q6_K, q8k),
                          ("gemv_tq1_0_q8_k", jk.TQ1_0, q8k), ("gemv_tq2_0_q8_k", jk.TQ2_0, q8k)):
            out = np.zeros(ROWS, np.float32)
            getattr(jk, fn)(out, views[q], xb)
            outs.append(out)
        for fn, q in (("vec_dot_q4_0", jk.Q4_0), ("vec_dot_q5_0", jk.Q5_0), ("vec_dot_q8_0", jk.Q8_0),
                      ("vec_dot_q4_k_m", jk.Q4_K), ("vec_dot_q5_k", jk.Q5_K), ("vec_dot_q6_k", jk.Q6_K)):
            out = np.zeros(ROWS, np.float32)
            getattr(jk, fn)(out, views[q], x)
            outs.append(out)
        outs.append(np.float32([jk.argmax_f32(logits)]))
        return outs

    return run, views, x, q80, q8k


def test_warm_calls_upload_and_allocate_nothing(gpu):
    jk.host_cache_clear()
    run, views, x, q80, q8k = zero_alloc_calls()
    first = run()
    s0 = jk.host_stats()
    second = run()
    s1 = jk.host_stats()
    assert s1["weight_uploads"] == s0["weight_uploads"], (s0, s1)
    assert s1["device_allocs"] == s0["device_allocs"], (s0, s1)
    assert s1["cache_hits"] >= s0["cache_hits"] + 22
    assert all(same_bits(a, b) for a, b in zip(first, second))
    # and the outputs are the oracle's
    for k, (q, xb) in enumerate(((jk.Q4_0, q80), (jk.Q5_0, q80), (jk.Q8_0, q80), (jk.Q4_K, q8k), (jk.Q5_K, q8k),
                                 (jk.Q6_K, q8k), (jk.TQ1_0, q8k), (jk.TQ2_0, q8k))):
        assert same_bits(second[10 + k], O.gemv_q8(q, [ROWS, COLS], views[q].data, xb, ROWS))
    assert int(second[-1][0]) == 1234


def test_host_gemv_c3_gate_shape_resident(gpu):
    """gemv_q4_k_q8_k over the 14336 x 4096 gate matrix: the first call uploads 33 MB, later calls
    only the 4.7 KB of activation blocks."""
    rows, cols = 14336, 4096
    raw = synth.gguf_weights(jk.Q4_K, rows, cols, seed=5)
    v = jk.TensorView("blk.0.ffn_gate.weight", jk.Q4_K, [cols, rows], raw)
    ref_x = [O.quantize_row_q8_k(synth.activations(cols, s)) for s in (1, 2)]
    out = np.zeros(rows, np.float32)
    jk.gemv_q4_k_q8_k(out, v, ref_x[0])
    assert same_bits(out, O.gemv_q8(jk.Q4_K, [rows, cols], raw, ref_x[0], rows))
    s0 = jk.host_stats()
    jk.gemv_q4_k_q8_k(out, v, ref_x[1])
    s1 = jk.host_stats()
    assert (s1["weight_uploads"], s1["device_allocs"]) == (s0["weight_uploads"], s0["device_allocs"])
    assert same_bits(out, O.gemv_q8(jk.Q4_K, [rows, cols], raw, ref_x[1], rows))


def test_invalidate_limit_and_threads(gpu):
    rows, cols = 64, 1024
    raw = synth.gguf_weights(jk.Q6_K, rows, cols, seed=9)
    v = jk.TensorView("w", jk.Q6_K, [rows, cols], raw)
    xb = O.quantize_row_q8_k(synth.activations(cols, 4))
    out = np.zeros(rows, np.float32)
    jk.gemv_q6_k_q8_k(out, v, xb)
    # new bytes in the same buffer, announced: the next call sees them
    raw[:] = synth.gguf_weights(jk.Q6_K, rows, cols, seed=10)
    jk.host_cache_invalidate(v)
    jk.gemv_q6_k_q8_k(out, v, xb)
    assert same_bits(out, O.gemv_q8(jk.Q6_K, [rows, cols], raw, xb, rows))
    # cache off: every call uploads, results unchanged
    s0 = jk.host_stats()
    jk.host_cache_set_limit(0)
    try:
        assert jk.host_stats()["cached_weights"] == 0
        jk.gemv_q6_k_q8_k(out, v, xb)
        jk.gemv_q6_k_q8_k(out, v, xb)
        assert jk.host_stats()["weight_uploads"] == s0["weight_uploads"] + 2
        assert same_bits(out, O.gemv_q8(jk.Q6_K, [rows, cols], raw, xb, rows))
    finally:
        jk.host_cache_set_limit(s0["cache_limit"])
    # four threads on shared views, each with its own stream and scratch
    views = [jk.TensorView(f"t{i}", jk.Q4_K, [256, 2048], synth.gguf_weights(jk.Q4_K, 256, 2048, seed=20 + i))
             for i in range(3)]
    xs = [O.quantize_row_q8_k(synth.activations(2048, 30 + i)) for i in range(4)]
    errors = []

    def worker(t):
        try:
            for it in range(20):
                i = (t + it) % 3
                o = np.zeros(256, np.float32)
                jk.gemv_q4_k_q8_k(o, views[i], xs[t])
                if not same_bits(o, O.gemv_q8(jk.Q4_K, [256, 2048], views[i].data, xs[t], 256)):
                    errors.append((t, it))
            jk.host_release_thread()
        except Exception as e:  # noqa: BLE001 -- reported below
            errors.append(repr(e))

    ts = [threading.Thread(target=worker, args=(t,)) for t in range(4)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errors, errors


def test_repack_and_gemm_bounds_error_fields(gpu):
    """tests/test_repack_gemv_gemm.rs:883-917 with TensorBoundsError's fields as
    execute_gemm_repacked_rows / gemv_repacked_view_rows fill them (repack.rs:2725-2778, 4051-4060;
    buffer_len of the K check is the weight's stored bytes)."""
    torch = gpu
    raw = synth.gguf_weights(jk.Q8_0, 8, 64, seed=1)
    w = jk.Weight(jk.TensorView("w_err", jk.Q8_0, [64, 8], raw), 8, 64)

    def act(m, k):
        need = jk.act_q8_bytes(m, k)
        st = torch.empty(need, dtype=torch.uint8, device="cuda")
        a = jk.act_q8_bind(st, need, m, k)
        jk.dev_quantize_act_q8(torch.ones(m * k, dtype=torch.float32, device="cuda"), m, k, a)
        return st, a

    y = torch.zeros(16, dtype=torch.float32, device="cuda")
    _, bad = act(1, 32)
    with pytest.raises(jk.TensorBoundsError) as ei:  # K mismatch
        jk.dev_gemv_repacked(w, bad, y, 8, 0, 8)
    e = ei.value
    assert (e.tensor_name, e.offset, e.byte_len, e.buffer_len) == ("gemm_repacked", 0, 32, w.device_bytes)
    _, m2 = act(2, 64)
    with pytest.raises(jk.TensorBoundsError) as ei:  # M != 1 on gemv_repacked
        jk.dev_gemv_repacked(w, m2, y, 8, 0, 8)
    assert (ei.value.tensor_name, ei.value.offset, ei.value.byte_len) == ("gemv_repacked", 0, 32)
    _, ok = act(1, 64)
    with pytest.raises(jk.TensorBoundsError) as ei:  # out-of-range row slice 2..10
        jk.dev_gemm_repacked(w, ok, y, 8, 2, 10)
    assert (ei.value.tensor_name, ei.value.offset, ei.value.byte_len, ei.value.buffer_len) == ("gemm_repacked", 2, 8, 8)
    with pytest.raises(jk.TensorBoundsError) as ei:  # output slice length mismatch (7 of 8)
        jk.dev_gemm_repacked(w, ok, y, 7, 0, 8)
    assert (ei.value.tensor_name, ei.value.byte_len, ei.value.buffer_len) == ("gemm_repacked", 28, 32)
    torch.cuda.synchronize()
    w.free()


def test_unannounced_edit_of_unsampled_bytes(gpu):
    """An in-place edit of weight bytes that the cache key's fingerprint does not sample, made
    without jk_host_cache_invalidate: with residency off (the default) every call reads the bytes,
    as the reference does; with residency on, the stale device copy is used, as documented (the
    immutability contract), until invalidated; with verify on, the edit is caught by the full-content
    hash, the weight is uploaded again and the result is the oracle's for the new bytes."""
    rows, cols = 1024, 4096
    raw = synth.gguf_weights(jk.Q4_K, rows, cols, seed=11)
    v = jk.TensorView("w", jk.Q4_K, [cols, rows], raw)
    xb = O.quantize_row_q8_k(synth.activations(cols, 12))
    off = raw.nbytes // 256 + 2000  # between the fingerprint's first two sampled windows: a qs byte of row 4
    assert 1024 < off < raw.nbytes - 1024

    def gemv():
        out = np.zeros(rows, np.float32)
        jk.gemv_q4_k_q8_k(out, v, xb)
        return out

    def ref():
        return O.gemv_q8(jk.Q4_K, [rows, cols], raw, xb, rows)

    jk.host_cache_set_limit(0)  # the default: no residency
    a = gemv()
    assert same_bits(a, ref())
    raw[off] ^= 0x55
    b = gemv()
    assert same_bits(b, ref()) and not same_bits(a, b)
    jk.host_cache_set_limit(RESIDENT_LIMIT)  # residency: the caller promises immutable bytes
    c = gemv()
    raw[off] ^= 0x55
    assert same_bits(gemv(), c)  # the documented behaviour of a broken promise: the old bytes' result
    jk.host_cache_invalidate(v)
    assert same_bits(gemv(), ref())
    jk.host_cache_set_verify(True)  # verify: every hit hashes all bytes
    assert same_bits(gemv(), ref())
    s0 = jk.host_stats()
    assert s0["verify"] == 1
    raw[off] ^= 0x55
    assert same_bits(gemv(), ref())
    s1 = jk.host_stats()
    assert s1["stale_reuploads"] == s0["stale_reuploads"] + 1
    assert s1["weight_uploads"] == s0["weight_uploads"] + 1
    assert same_bits(gemv(), ref())  # and the new upload is then reused
    assert jk.host_stats()["weight_uploads"] == s1["weight_uploads"]
