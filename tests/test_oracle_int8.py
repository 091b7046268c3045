"""The oracle's int8 primitives (ime.rs:81-157, 449-496, 563-583) pinned without the GPU: the
reference's own unit tests for them (ime.rs:1157-1231), brute force in int64 numpy, and the
C ABI's argument checks (which return before any device work)."""
import ctypes as C

import numpy as np
import pytest

import oracle as O


def fill(n, seed):
    """The reference tests' input generator (ime.rs:1149-1153)."""
    return np.array([((i * 7 + seed * 13) % 17) - 8 for i in range(n)], dtype=np.int8)


def exact(a, m, b, n0, n1, k):
    return a.reshape(m, k).astype(np.int64) @ b.reshape(-1, k)[n0:n1].astype(np.int64).T


def test_pack_tiles_pads_and_orders_rows():
    # ime.rs:1203-1215
    src = np.arange(32, dtype=np.int8)
    p = O.pack_tiles(src, 2, 16)
    assert p.size == 128
    assert (p[:32] == src).all() and (p[32:] == 0).all()


def test_pack_tiles_layout_and_errors():
    rows, k = 13, 48
    src = np.random.default_rng(1).integers(-128, 128, rows * k, dtype=np.int8)
    p = O.pack_tiles(src, rows, k).reshape(2, 3, 8, 16)  # [tile][chunk][row][16]
    for r in range(16):
        for c in range(3):
            want = src[r * k + 16 * c: r * k + 16 * c + 16] if r < rows else np.zeros(16, np.int8)
            assert (p[r // 8, c, r % 8] == want).all()
    with pytest.raises(O.OracleError):
        O.pack_tiles(np.zeros(2 * 20, np.int8), 2, 20)  # k not a multiple of 16 (the reference asserts)


def test_gemm_i8_vector_and_ime_match_brute_force():
    # ime.rs:1157-1200 (ime_vector_and_scalar_paths_are_bit_identical), with the scalar dot
    # replaced by int64 numpy
    m, n, k = 6, 12, 64
    a, b = fill(m * k, 1), fill(n * k, 2)
    want = exact(a, m, b, 0, n, k)
    assert (O.gemm_i8_vector(a, m, b, 0, n, k) == want).all()
    t = O.gemm_i8_ime(O.pack_tiles(a, m, k), 1, O.pack_tiles(b, n, k), 0, 2, k // 16)
    full = t.reshape(1, 2, 8, 8).transpose(0, 2, 1, 3).reshape(8, 16)
    assert (full[:m, :n] == want).all()
    assert (full[m:] == 0).all() and (full[:, n:] == 0).all()


def test_tile_dot_rows_partial():
    # ime.rs:1217-1231 (tile_dot_rows_and_rvv_fallback_match_scalar)
    ap, bp = O.pack_tiles(fill(5 * 32, 3), 5, 32), O.pack_tiles(fill(8 * 32, 7), 8, 32)
    full = O.tile_dot_scalar_rows(ap, bp, 2, 8)
    part = O.tile_dot_scalar_rows(ap, bp, 2, 5)
    assert (part[:40] == full[:40]).all() and (part[40:] == 0).all()
    want = fill(5 * 32, 3).reshape(5, 32).astype(np.int64) @ fill(8 * 32, 7).reshape(8, 32).astype(np.int64).T
    assert (full.reshape(8, 8)[:5] == want).all()


@pytest.mark.parametrize("m,rows,n0,n1,k", [(1, 7, 0, 7, 1), (3, 40, 5, 33, 50), (17, 9, 2, 9, 256), (4, 4, 2, 2, 16)])
def test_gemm_i8_vector_ragged(m, rows, n0, n1, k):
    rng = np.random.default_rng(m * 1000 + k)
    a = rng.integers(-128, 128, m * k, dtype=np.int8)
    b = rng.integers(-128, 128, rows * k, dtype=np.int8)
    assert (O.gemm_i8_vector(a, m, b, n0, n1, k) == exact(a, m, b, n0, n1, k)).all()


def test_dot_i8_zip_and_extremes():
    a, b = fill(37, 4), fill(50, 5)
    assert O.dot_i8(a, b) == int((a.astype(np.int64) * b[:37]).sum())  # the zip stops at the shorter
    assert O.dot_i8(a[:0], b) == 0
    big = np.full(131071, -128, np.int8)
    assert O.dot_i8(big, big) == 131071 * 16384 == 2147467264  # the largest sum below 2^31
    mixed = np.full(131071, 127, np.int8)
    assert O.dot_i8(big, mixed) == -131071 * 128 * 127


def test_c_abi_int8_argument_checks():
    """Invalid arguments are rejected before any device work, so these run without a GPU."""
    import jk

    L = jk.lib()
    vp, sz = C.c_void_p, C.c_size_t
    one = vp(16)  # never dereferenced: every call below fails validation first
    assert L.jk_gemm_i8(vp(0), one, sz(2 * 131072), sz(2), one, sz(3 * 131072), sz(0), sz(3), sz(131072), one,
                        sz(6)) == jk.TENSOR_BOUNDS  # k above 131071
    assert L.jk_gemm_i8(vp(0), one, sz(8), sz(2), one, sz(12), sz(0), sz(4), sz(4), one, sz(8)) == jk.TENSOR_BOUNDS
    assert L.jk_gemm_i8(vp(0), one, sz(8), sz(2), one, sz(16), sz(3), sz(2), sz(4), one, sz(0)) == jk.TENSOR_BOUNDS
    assert L.jk_gemm_i8(vp(0), one, sz(8), sz(2), one, sz(16), sz(0), sz(4), sz(4), one, sz(7)) == jk.TENSOR_BOUNDS
    assert L.jk_gemm_i8(vp(0), vp(0), sz(0), sz(0), vp(0), sz(0), sz(0), sz(0), sz(4), vp(0), sz(0)) == jk.OK
    assert L.jk_gemm_i8_tiles(vp(0), one, sz(128), sz(1), one, sz(128), sz(0), sz(2), sz(1), one,
                              sz(128)) == jk.TENSOR_BOUNDS  # B holds one tile row, the range needs two
    assert L.jk_gemm_i8_tiles(vp(0), vp(17), sz(128), sz(1), vp(32), sz(128), sz(0), sz(1), sz(1), one,
                              sz(64)) == jk.TENSOR_BOUNDS  # unaligned packed tiles
    assert L.jk_pack_tiles_i8(vp(0), one, sz(40), sz(2), sz(20), one, sz(128)) == jk.TENSOR_BOUNDS
    assert L.jk_pack_tiles_i8(vp(0), one, sz(32), sz(2), sz(16), one, sz(64)) == jk.TENSOR_BOUNDS
    assert L.jk_dot_i8(vp(0), one, sz(131072), one, sz(131072), one) == jk.TENSOR_BOUNDS
    assert L.jk_dot_i8(vp(0), one, sz(4), one, sz(4), vp(0)) == jk.TENSOR_BOUNDS
