"""jk_gemm_i8 / jk_gemm_i8_tiles / jk_pack_tiles_i8 / jk_dot_i8 / jk_op_counts on the GPU against
the oracle's restatements of gemm_i8_vector, gemm_i8_ime, pack_tiles and dot_i8_scalar
(ime.rs:81-94, 449-496, 563-583) and int64 brute force; every result is compared bit for bit."""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


def fill(n, seed):
    """The reference tests' input generator (ime.rs:1149-1153)."""
    return np.array([((i * 7 + seed * 13) % 17) - 8 for i in range(n)], dtype=np.int8)


def dev(torch, x, offset=0):
    """x on the device, starting `offset` bytes into its allocation (offset 1: unaligned)."""
    buf = torch.zeros(x.size + offset + 16, dtype=torch.int8, device="cuda")
    buf[offset: offset + x.size] = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    return buf[offset: offset + x.size]


def run_gemm(torch, a, m, b, n0, n1, k, a_off=0, b_off=0):
    import jk

    da, db = dev(torch, a, a_off), dev(torch, b, b_off)
    c = torch.full((m * (n1 - n0),), 0x5A5A5A5A, dtype=torch.int32, device="cuda")
    jk.dev_gemm_i8(da, a.size, m, db, b.size, n0, n1, k, c, c.numel())
    torch.cuda.synchronize()
    return c.cpu().numpy().reshape(m, n1 - n0)


@pytest.mark.parametrize("m,rows,n0,n1,k,a_off,b_off", [
    (6, 12, 0, 12, 64, 0, 0),        # the reference's unit-test shape (ime.rs:1157-1200)
    (1, 100, 3, 97, 50, 0, 0),       # k not a multiple of 16: byte loads, zero-filled last piece
    (37, 45, 0, 45, 48, 1, 0),       # A unaligned
    (33, 70, 10, 70, 4096, 0, 3),    # B unaligned
    (128, 300, 17, 290, 4096, 0, 0),
    (65, 129, 0, 129, 272, 0, 0),    # ragged against the 64 x 64 tiles
    (512, 16384, 0, 16384, 256, 0, 0),  # the 128 x 128 tiles
    (520, 17000, 100, 16999, 160, 0, 0),  # 128 x 128 tiles, ragged
    (512, 16384, 0, 16384, 128, 0, 0),    # 128 x 128 tiles staged by global-to-LDS loads, one chunk
    (520, 17000, 100, 16999, 384, 0, 0),  # the same, ragged, an odd number of chunks
])
def test_gemm_i8_matches_oracle(gpu, m, rows, n0, n1, k, a_off, b_off):
    rng = np.random.default_rng(m + rows + k)
    if (m, rows, k) == (6, 12, 64):
        a, b = fill(m * k, 1), fill(rows * k, 2)
    else:
        a = rng.integers(-128, 128, m * k, dtype=np.int8)
        b = rng.integers(-128, 128, rows * k, dtype=np.int8)
    got = run_gemm(gpu, a, m, b, n0, n1, k, a_off, b_off)
    if m * (n1 - n0) * k <= 50_000_000:
        want = O.gemm_i8_vector(a, m, b, n0, n1, k)
    else:  # brute force in float64: every sum is an integer below 2^31, exact in a double
        want = (a.reshape(m, k).astype(np.float64) @ b.reshape(rows, k)[n0:n1].astype(np.float64).T).astype(np.int64)
    assert np.array_equal(got.astype(np.int64), want.astype(np.int64))


def test_gemm_i8_extreme_sums(gpu):
    k = 131071  # the largest k: |sum| reaches 131071 * 2^14 = 2147467264 < 2^31
    a = np.full(2 * k, -128, np.int8)
    b = np.concatenate([np.full(k, -128, np.int8), np.full(k, 127, np.int8), np.full(k, -127, np.int8)])
    got = run_gemm(gpu, a, 2, b, 0, 3, k)
    assert (got[:, 0] == 2147467264).all()
    assert (got[:, 1] == -128 * 127 * k).all() and (got[:, 2] == 128 * 127 * k).all()


def test_gemm_i8_tiles_and_pack(gpu):
    import jk

    for m, n, k, nt0, nt1 in [(6, 12, 64, 0, 2), (37, 300, 4096, 5, 33), (8, 16, 16, 1, 2), (20, 24, 0, 0, 3)]:
        rng = np.random.default_rng(m * n + k)
        a = rng.integers(-128, 128, m * k, dtype=np.int8)
        b = rng.integers(-128, 128, n * k, dtype=np.int8)
        kc = k // 16
        ap_want, bp_want = O.pack_tiles(a, m, k), O.pack_tiles(b, n, k)
        da, db = dev(gpu, a), dev(gpu, b)
        ap = gpu.full((ap_want.size,), 7, dtype=gpu.int8, device="cuda")
        bp = gpu.full((bp_want.size,), 7, dtype=gpu.int8, device="cuda")
        jk.dev_pack_tiles_i8(da, a.size, m, k, ap, ap.numel())
        jk.dev_pack_tiles_i8(db, b.size, n, k, bp, bp.numel())
        gpu.cuda.synchronize()
        assert np.array_equal(ap.cpu().numpy(), ap_want) and np.array_equal(bp.cpu().numpy(), bp_want)
        mt = (m + 7) // 8
        c = gpu.full((mt * (nt1 - nt0) * 64,), -1, dtype=gpu.int32, device="cuda")
        jk.dev_gemm_i8_tiles(ap, ap.numel(), mt, bp, bp.numel(), nt0, nt1, kc, c, c.numel())
        gpu.cuda.synchronize()
        want = O.gemm_i8_ime(ap_want, mt, bp_want, nt0, nt1, kc)
        assert np.array_equal(c.cpu().numpy().reshape(want.shape), want)
    # unaligned source rows are packed through the byte path
    a = fill(3 * 32, 9)
    da = dev(gpu, a, 1)
    ap = gpu.full((256,), 7, dtype=gpu.int8, device="cuda")
    jk.dev_pack_tiles_i8(da, a.size, 3, 32, ap, 256)
    gpu.cuda.synchronize()
    assert np.array_equal(ap.cpu().numpy(), O.pack_tiles(a, 3, 32))


@pytest.mark.parametrize("la,lb,off", [(0, 5, 0), (1, 1, 0), (15, 15, 1), (16, 16, 0), (17, 40, 0), (4096, 4096, 0),
                                       (4099, 4097, 3), (131071, 131071, 0)])
def test_dot_i8(gpu, la, lb, off):
    import jk

    rng = np.random.default_rng(la + lb)
    a = rng.integers(-128, 128, la, dtype=np.int8)
    b = rng.integers(-128, 128, lb, dtype=np.int8)
    out = gpu.full((1,), 12345, dtype=gpu.int32, device="cuda")
    jk.dev_dot_i8(dev(gpu, a, off), la, dev(gpu, b), lb, out)
    gpu.cuda.synchronize()
    assert int(out.item()) == O.dot_i8(a, b)


def test_dot_i8_extreme(gpu):
    import jk

    a = np.full(131071, -128, np.int8)
    out = gpu.zeros((1,), dtype=gpu.int32, device="cuda")
    jk.dev_dot_i8(dev(gpu, a), a.size, dev(gpu, a), a.size, out)
    gpu.cuda.synchronize()
    assert int(out.item()) == 2147467264


def test_op_counts(gpu):
    """ime_vmadot_count / vector_dot_count (ime.rs:53-66): tile steps of the tile GEMM, dot products
    of the vector GEMM and of BitLinear (one per weight block and token, ime.rs:919-936)."""
    import jk
    from jk import synth

    t0, v0 = jk.op_counts()
    run_gemm(gpu, fill(6 * 64, 1), 6, fill(12 * 64, 2), 2, 11, 64)
    t1, v1 = jk.op_counts()
    assert (t1, v1 - v0) == (t0, 6 * 9)
    ap = gpu.zeros((2 * 4 * 128,), dtype=gpu.int8, device="cuda")
    c = gpu.zeros((2 * 3 * 64,), dtype=gpu.int32, device="cuda")
    bp = gpu.zeros((5 * 4 * 128,), dtype=gpu.int8, device="cuda")
    jk.dev_gemm_i8_tiles(ap, ap.numel(), 2, bp, bp.numel(), 1, 4, 4, c, c.numel())
    t2, v2 = jk.op_counts()
    assert (t2 - t1, v2) == (2 * 3 * 4, v1)
    rows, cols, m = 64, 512, 3
    w = jk.Weight(jk.TensorView("w", jk.TQ2_0, (rows, cols), synth.gguf_weights(jk.TQ2_0, rows, cols, seed=3)), rows, cols)
    act = gpu.zeros((m * cols,), dtype=gpu.int8, device="cuda")
    sc = gpu.ones((m,), dtype=gpu.float32, device="cuda")
    y = gpu.zeros((m * rows,), dtype=gpu.float32, device="cuda")
    jk.dev_bitlinear_i8(w, act, sc, m, cols, y, m * rows)
    gpu.cuda.synchronize()
    w.free()
    t3, v3 = jk.op_counts()
    assert (t3, v3 - v2) == (t2, m * rows * (cols // 256))


def test_host_mirrors(gpu):
    """jk_host_gemm_i8 / jk_host_dot_i8: gemm_i8_vector and dot_i8_vector on host slices (the
    reference's signatures), equal to the oracle; short slices are TensorBoundsError."""
    import jk

    m, rows, k = 6, 12, 64
    a, b = fill(m * k, 1), fill(rows * k, 2)
    assert np.array_equal(jk.gemm_i8_vector(a, m, b, 3, 11, k), O.gemm_i8_vector(a, m, b, 3, 11, k))
    rng = np.random.default_rng(9)
    a2 = rng.integers(-128, 128, 33 * 1000, dtype=np.int8)
    b2 = rng.integers(-128, 128, 70 * 1000, dtype=np.int8)
    assert np.array_equal(jk.gemm_i8_vector(a2, 33, b2, 0, 70, 1000), O.gemm_i8_vector(a2, 33, b2, 0, 70, 1000))
    assert jk.dot_i8_vector(a2[:999], b2[:1003]) == O.dot_i8(a2[:999], b2[:1003])
    assert jk.dot_i8_vector(a2[:0], b2) == 0
    with pytest.raises(jk.TensorBoundsError):
        jk.gemm_i8_vector(a[:-1], m, b, 0, rows, k)  # A one byte short of m * k
    with pytest.raises(jk.TensorBoundsError):
        jk.gemm_i8_vector(a, m, b, 0, rows + 1, k)  # the range runs past B


def test_graph_replays_of_staged_and_tolerance_kernels(gpu):
    """The kernels staged by global-to-LDS loads (jk_gemm_i8 on 128 x 256 tiles, the Q8_0 tolerance
    and bit-exact 128 x 128 GEMM tiles) and the tolerance BitLinear / split-block vec_dot kernels,
    captured once in one HIP graph and replayed with new inputs, eager work and synchronizations in
    between: every replay equals the same calls made eagerly, bit for bit."""
    import jk
    from jk import synth

    torch = gpu
    M, N, K = 512, 14336, 256
    a = torch.empty(M * K, dtype=torch.int8, device="cuda")
    b = torch.from_numpy(np.random.default_rng(1).integers(-128, 128, N * K, dtype=np.int8)).cuda()
    c = torch.empty(M * N, dtype=torch.int32, device="cuda")
    wq = jk.Weight(jk.TensorView("wq", jk.Q8_0, (N, K), synth.gguf_weights(jk.Q8_0, N, K, seed=5)), N, K)
    x = torch.empty(M, K, device="cuda")
    need = jk.act_q8_bytes(M, K)
    st = torch.empty(need, dtype=torch.uint8, device="cuda")
    act = jk.act_q8_bind(st, need, M, K)
    assert jk.gemm_plan(wq, act, 0, N, True) == "gemm_q8_0_tol_dma_128"
    assert jk.gemm_plan(wq, act, 0, N, False) == "gemm_q8_0_exact_dma_128"
    yt = torch.empty(M * N, device="cuda")
    ye = torch.empty(M * N, device="cuda")
    rows, cols, m = 6912, 2560, 128
    wt = jk.Weight(jk.TensorView("wt", jk.TQ2_0, (rows, cols), synth.gguf_weights(jk.TQ2_0, rows, cols, seed=6)),
                   rows, cols)
    aq = torch.empty(m * cols, dtype=torch.int8, device="cuda")
    asc = torch.empty(m, device="cuda")
    yb = torch.empty(m * rows, device="cuda")
    wv = jk.Weight(jk.TensorView("wv", jk.Q4_K, (4096, 4096), synth.gguf_weights(jk.Q4_K, 4096, 4096, seed=7)),
                   4096, 4096)
    xv = torch.empty(4096, device="cuda")
    yv = torch.empty(4096, device="cuda")

    def step(s):
        jk.dev_gemm_i8(a, M * K, M, b, N * K, 0, N, K, c, M * N, s)
        jk.dev_quantize_act_q8(x, M, K, act, s)
        jk.dev_gemm_repacked_tol(wq, act, yt, M * N, 0, N, s)
        jk.dev_gemm_repacked(wq, act, ye, M * N, 0, N, s)
        jk.dev_bitlinear_i8_tol(wt, aq, asc, m, cols, yb, m * rows, s)
        jk.dev_vec_dot_f32_tol(wv, xv, 4096, yv, 4096, s)

    def fill(seed):
        g = torch.Generator().manual_seed(seed)
        a.copy_(torch.randint(-128, 128, (M * K,), dtype=torch.int8, generator=g))
        x.copy_(torch.randn(M, K, generator=g))
        aq.copy_(torch.randint(-127, 128, (m * cols,), dtype=torch.int8, generator=g))
        asc.copy_(torch.rand(m, generator=g) * 0.05)
        xv.copy_(torch.randn(4096, generator=g))

    outs = (c, yt, ye, yb, yv)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    fill(0)
    with torch.cuda.stream(side):
        step(side.cuda_stream)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step(torch.cuda.current_stream().cuda_stream)
    for seed in (1, 2, 3):
        fill(seed)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        replay = [o.clone() for o in outs]
        for o in outs:
            o.fill_(7)
        step(torch.cuda.current_stream().cuda_stream)  # the same calls, eagerly
        torch.cuda.synchronize()
        for name, r, e in zip(("gemm_i8", "gemm tol", "gemm exact", "bitlinear tol", "vec_dot tol"), replay, outs):
            assert torch.equal(r.view(torch.int32), e.view(torch.int32)), (seed, name)
    del g
    for w in (wq, wt, wv):
        w.free()
