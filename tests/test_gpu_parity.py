"""GPU parity: every libjk entry point against the oracle on identical seeded inputs.

The bar is bit-exactness for everything (quantizers, dequantization, and the f32 outputs
of GEMV / vec_dot / GEMM / BitLinear, whose per-block arithmetic and block-order
accumulation follow the reference exactly). `same_bits` compares float bit patterns,
so the sign of zero counts; two NaNs count as equal.
"""
import numpy as np
import pytest

import jk
import oracle as O
from jk import synth

pytestmark = pytest.mark.gpu

Q4_0, Q8_0, Q4_K, Q6_K, TQ2_0, I2_S = jk.Q4_0, jk.Q8_0, jk.Q4_K, jk.Q6_K, jk.TQ2_0, jk.I2_S
Q5_0, Q5_K, TQ1_0 = jk.Q5_0, jk.Q5_K, jk.TQ1_0
Q4_1, Q5_1, Q2_K, Q3_K, IQ4_NL = jk.Q4_1, jk.Q5_1, jk.Q2_K, jk.Q3_K, jk.IQ4_NL
GEMV_FORMATS = [Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K, TQ1_0, TQ2_0]
ALL_FORMATS = GEMV_FORMATS + [I2_S, Q4_1, Q5_1, Q2_K, Q3_K, IQ4_NL]
# device bytes per block where they differ from the GGUF bytes
DEVICE_BLOCK_BYTES = {TQ1_0: 66, Q3_K: 112}


def same_bits(a, b) -> bool:
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    if a.shape != b.shape:
        return False
    eq = a.view(np.uint32) == b.view(np.uint32)
    return bool(np.all(eq | (np.isnan(a) & np.isnan(b))))


def mismatch(a, b) -> str:
    a, b = np.asarray(a, np.float32).ravel(), np.asarray(b, np.float32).ravel()
    bad = np.nonzero(a.view(np.uint32) != b.view(np.uint32))[0]
    if bad.size == 0:
        return "ok"
    i = bad[0]
    return f"{bad.size} mismatches, first at {i}: gpu {a[i]!r} oracle {b[i]!r}"


def dev(torch, arr):
    a = np.ascontiguousarray(arr)
    return torch.from_numpy(a.view(np.uint8).reshape(-1).copy()).cuda()


def empty(torch, nbytes):
    return torch.empty(max(int(nbytes), 16), dtype=torch.uint8, device="cuda")


def host(t, dtype, count=None):
    a = t.cpu().numpy().view(dtype)
    return a if count is None else a[:count]


def x_blocks(quant, x):
    return O.quantize_row_q8_0(x) if quant in jk.Q8_0_ACT else O.quantize_row_q8_k(x)


def gpu_gemv(torch, w, xq, r0=0, r1=None):
    r1 = w.rows if r1 is None else r1
    dx = dev(torch, xq)
    dy = empty(torch, 4 * (r1 - r0))
    if r0 == 0 and r1 == w.rows:
        jk.dev_gemv_q8(w, dx, xq.size, dy, w.rows)
    else:
        jk.dev_gemv_q8_rows(w, dx, xq.size, dy, r0, r1)
    torch.cuda.synchronize()
    return host(dy, np.float32, r1 - r0)


# ------------------------------------------------------------------ quantizers
@pytest.mark.parametrize("n", [32, 4096, 14336, 32 * 1001])
def test_quantize_row_q8_0(gpu, n):
    torch = gpu
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) * rng.choice([1e-3, 1, 50], n)).astype(np.float32)
    x[rng.random(n) < 0.01] = np.nan
    x[rng.random(n) < 0.01] = np.inf
    x[:32] = 0.0
    ref = O.quantize_row_q8_0(x)
    dy = empty(torch, ref.nbytes)
    jk.dev_quantize_row_q8_0(dev(torch, x), n, dy, n // 32)
    torch.cuda.synchronize()
    got = host(dy, jk.BLOCK_Q8_0, ref.size)
    assert same_bits(got["d"], ref["d"]) and np.array_equal(got["qs"], ref["qs"])


@pytest.mark.parametrize("n", [256, 4096, 14336, 256 * 77])
@pytest.mark.parametrize("offset", [0, 1])
def test_quantize_row_q8_k(gpu, n, offset):
    """offset 1: the input one float past a 16-byte boundary (element-wise loads instead of one
    16-byte load per lane)."""
    torch = gpu
    rng = np.random.default_rng(n + 1)
    x = (rng.standard_normal(n) * rng.choice([1e-3, 1, 50], n)).astype(np.float32)
    x[rng.random(n) < 0.01] = -np.inf
    x[:256] = np.nan
    ref = O.quantize_row_q8_k(x)
    dy = empty(torch, ref.nbytes)
    dx = torch.zeros(n + 4, dtype=torch.float32, device="cuda")
    dx[offset:offset + n] = torch.from_numpy(x).cuda()
    jk.dev_quantize_row_q8_k(dx[offset:], n, dy, n // 256)
    torch.cuda.synchronize()
    got = host(dy, jk.BLOCK_Q8K, ref.size)
    assert same_bits(got["d"], ref["d"])
    assert np.array_equal(got["qs"], ref["qs"]) and np.array_equal(got["bsums"], ref["bsums"])


def gpu_act(torch, x, m, k):
    need = jk.act_q8_bytes(m, k)
    storage = empty(torch, need)
    act = jk.act_q8_bind(storage, need, m, k)
    jk.dev_quantize_act_q8(dev(torch, x), m, k, act)
    return storage, act


@pytest.mark.parametrize("m,k", [(1, 4096), (5, 300), (64, 4096), (3, 40), (2, 101), (7, 259)])
def test_quantize_act_q8(gpu, m, k):
    torch = gpu
    rng = np.random.default_rng(m * k)
    x = (rng.standard_normal((m, k)) * rng.choice([1e-3, 1, 50], (m, k))).astype(np.float32)
    x[rng.random((m, k)) < 0.01] = np.nan
    x[0, :32] = -0.0
    ref = O.ActQ8(x, m, k)
    storage, act = gpu_act(torch, x, m, k)
    torch.cuda.synchronize()
    base = storage.data_ptr()
    raw = storage.cpu().numpy()

    def arr(ptr, dtype, count):
        return raw[ptr - base: ptr - base + count * np.dtype(dtype).itemsize].view(dtype)

    assert np.array_equal(arr(act.qs, np.int8, m * act.k_padded).reshape(m, -1), ref.qs)
    for name, pa, refv in (("scales", act.scales, ref.scales), ("sums", act.sums, ref.sums),
                           ("sums16", act.sums16, ref.sums16), ("super256", act.super256, ref.super256)):
        got = arr(pa, np.float32, refv.size).reshape(refv.shape)
        assert same_bits(got, refv), (name, mismatch(got, refv))


@pytest.mark.parametrize("k", [2560, 6912, 100])
def test_absmax_quantizers(gpu, k):
    torch = gpu
    rng = np.random.default_rng(k)
    m = 4
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[1] = 0.0
    x[2] *= 1e-14
    w = rng.uniform(0.5, 1.5, k).astype(np.float32)
    dq, ds = empty(torch, m * k), empty(torch, 4 * m)
    jk.dev_subln_quantize_absmax_i8(dev(torch, x), dev(torch, w), m, k, 1e-5, dq, ds)
    dq2, ds2 = empty(torch, m * k), empty(torch, 4 * m)
    jk.dev_quantize_absmax_i8(dev(torch, x), m, k, dq2, ds2)
    torch.cuda.synchronize()
    for r in range(m):
        q, s = O.subln_quantize_absmax_i8(x[r], w, 1e-5)
        assert np.array_equal(host(dq, np.int8, m * k).reshape(m, k)[r], q)
        assert same_bits(host(ds, np.float32, m)[r:r + 1], np.float32([s]))
        q2, s2 = O.quantize_absmax_i8(x[r])
        assert np.array_equal(host(dq2, np.int8, m * k).reshape(m, k)[r], q2)
        assert same_bits(host(ds2, np.float32, m)[r:r + 1], np.float32([s2]))


# ------------------------------------------------------------------ weights
@pytest.mark.parametrize("quant", ALL_FORMATS)
def test_upload_and_dequantize_rows(gpu, quant):
    torch = gpu
    rows, cols = 19, 2048
    raw = synth.random_weights(quant, rows, cols, seed=quant, specials=True)
    w = jk.Weight(jk.TensorView("w", quant, [rows, cols], raw), rows, cols)
    nblk = rows * cols // jk.BLOCK_ELEMENTS[quant]
    assert w.quant == quant
    assert w.gguf_bytes == nblk * jk.BLOCK_BYTES[quant] + jk.TRAILER_BYTES.get(quant, 0)
    assert w.device_bytes == nblk * DEVICE_BLOCK_BYTES.get(quant, jk.BLOCK_BYTES[quant])
    dy = empty(torch, 4 * rows * cols)
    jk.dev_dequantize_rows(w, 0, rows, dy, rows * cols)
    torch.cuda.synchronize()
    got = host(dy, np.float32, rows * cols).reshape(rows, cols)
    for r in range(rows):
        ref = O.dequantize_tensor_row(quant, [rows, cols], raw, r, cols)
        assert same_bits(got[r], ref), (r, mismatch(got[r], ref))


def test_dequantize_every_f16_scale(gpu):
    """Device f16 scale decode on all 65,536 bit patterns: Q8_0 block i carries d = i (normal,
    subnormal, +-0, Inf and NaN patterns alike) and quants spanning -128..127, and its dequantized
    row is the oracle's bit for bit (f16_to_f32_finite, lib.rs:676-717: NaN/Inf -> 0)."""
    torch = gpu
    rows, cols = 2048, 1024  # 32 blocks per row: 65,536 blocks
    blk = np.zeros(65536, dtype=[("d", "<u2"), ("qs", "i1", 32)])
    blk["d"] = np.arange(65536, dtype=np.uint16)
    blk["qs"] = np.int8([1, -1, 127, -128, 0, 2, -2, 3, 5, -7, 11, -13, 64, -64, 100, -100,
                         17, -19, 23, -29, 31, -37, 41, -43, 47, -53, 59, -61, 67, -71, 73, -79])
    raw = blk.view(np.uint8).reshape(-1)
    w = jk.Weight(jk.TensorView("w", Q8_0, [rows, cols], raw), rows, cols)
    dy = empty(torch, 4 * rows * cols)
    jk.dev_dequantize_rows(w, 0, rows, dy, rows * cols)
    torch.cuda.synchronize()
    got = host(dy, np.float32, rows * cols).reshape(rows, cols)
    for r in range(rows):
        ref = O.dequantize_tensor_row(Q8_0, [rows, cols], raw, r, cols)
        assert same_bits(got[r], ref), (r, mismatch(got[r], ref))


# ------------------------------------------------------------------ quant_q8 GEMV
@pytest.mark.parametrize("quant", GEMV_FORMATS)
@pytest.mark.parametrize("rows,cols", [(1, 256), (3, 512), (5, 4352), (17, 1024), (33, 7168), (64, 2560)])
def test_gemv_q8_small_shapes(gpu, quant, rows, cols):
    torch = gpu
    if cols % jk.BLOCK_ELEMENTS[quant]:
        pytest.skip("shape not block aligned")
    raw = synth.random_weights(quant, rows, cols, seed=rows * 7 + quant, specials=True)
    rng = np.random.default_rng(cols)
    x = rng.standard_normal(cols).astype(np.float32)
    x[: jk.BLOCK_ELEMENTS[quant]] = 0.0  # one all-zero activation block
    xq = x_blocks(quant, x)
    ref = O.gemv_q8(quant, [rows, cols], raw, xq, rows)
    w = jk.Weight(jk.TensorView("w", quant, [rows, cols], raw), rows, cols)
    got = gpu_gemv(torch, w, xq)
    assert same_bits(got, ref), mismatch(got, ref)


@pytest.mark.parametrize("quant", GEMV_FORMATS)
def test_gemv_q8_row_slices_identical(gpu, quant):
    torch = gpu
    rows, cols = 61, 2048
    raw = synth.gguf_weights(quant, rows, cols, seed=quant)
    xq = x_blocks(quant, synth.activations(cols, 1))
    w = jk.Weight(jk.TensorView("w", quant, [cols, rows], raw), rows, cols)
    full = gpu_gemv(torch, w, xq)
    assert same_bits(full, O.gemv_q8(quant, [cols, rows], raw, xq, rows))
    for r0, r1 in ((0, 16), (7, 29), (57, 61), (60, 61)):
        assert same_bits(gpu_gemv(torch, w, xq, r0, r1), full[r0:r1])


CONFIG_MATRICES = [
    ("C1 Q4_0 4096x4096", Q4_0, 4096, 4096),
    ("C2 Q8_0 11008x4096", Q8_0, 11008, 4096),
] + [(f"C3 {n}", q, r, c) for n, q, r, c in synth.LLAMA3_8B_LAYER] + [
    ("C5 TQ2_0 6912x2560", TQ2_0, 6912, 2560),
    ("C5 TQ2_0 2560x6912", TQ2_0, 2560, 6912),
    ("Q5_0 4096x4096", Q5_0, 4096, 4096),
    ("Q5_K 14336x4096", Q5_K, 14336, 4096),
    ("Q5_K 4096x14336", Q5_K, 4096, 14336),
    ("TQ1_0 6912x2560", TQ1_0, 6912, 2560),
]


@pytest.mark.parametrize("name,quant,rows,cols", CONFIG_MATRICES, ids=[c[0] for c in CONFIG_MATRICES])
def test_gemv_q8_full_config_shapes(gpu, name, quant, rows, cols):
    torch = gpu
    raw = synth.gguf_weights(quant, rows, cols, seed=rows + cols + quant)
    xq = x_blocks(quant, synth.activations(cols, 5))
    ref = O.gemv_q8(quant, [cols, rows], raw, xq, rows)
    w = jk.Weight(jk.TensorView(name, quant, [cols, rows], raw), rows, cols)
    got = gpu_gemv(torch, w, xq)
    assert same_bits(got, ref), mismatch(got, ref)


# ------------------------------------------------- fused-quantize and grouped GEMV
def gpu_gemv_f32(torch, w, x):
    dx = torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()
    dy = empty(torch, 4 * w.rows)
    jk.dev_gemv_q8_f32(w, dx, x.size, dy, w.rows)
    torch.cuda.synchronize()
    return host(dy, np.float32, w.rows)


# K values cover one and several staging rounds, LPR 16 and 64 (K-quants with > 32
# blocks), and a K-quant row long enough for two 64-block iterations.
FUSED_SHAPES = [(1, 256), (5, 4352), (37, 4096), (33, 7168), (17, 8448), (9, 14336), (4, 17920), (3, 32000)]


@pytest.mark.parametrize("quant", GEMV_FORMATS)
@pytest.mark.parametrize("rows,cols", FUSED_SHAPES)
def test_gemv_q8_f32_fused_quantize(gpu, quant, rows, cols):
    """quantize_row_q8_* + gemv_* fused in one launch == oracle quantize + gemv, bit for bit."""
    torch = gpu
    if cols % jk.BLOCK_ELEMENTS[quant]:
        pytest.skip("shape not block aligned")
    raw = synth.random_weights(quant, rows, cols, seed=rows * 11 + quant, specials=True)
    rng = np.random.default_rng(cols + rows)
    x = (rng.standard_normal(cols) * rng.choice([1e-3, 1.0, 40.0], cols)).astype(np.float32)
    x[: jk.BLOCK_ELEMENTS[quant]] = 0.0
    x[rng.random(cols) < 0.005] = np.nan
    x[rng.random(cols) < 0.005] = -np.inf
    if cols >= 512:  # a block whose maximum is subnormal: 127 / amax overflows to inf
        x[256:512] = (rng.standard_normal(256) * 1e-40).astype(np.float32)
        x[256:512:7] = 0.0
    ref = O.gemv_q8(quant, [rows, cols], raw, x_blocks(quant, x), rows)
    w = jk.Weight(jk.TensorView("w", quant, [rows, cols], raw), rows, cols)
    got = gpu_gemv_f32(torch, w, x)
    assert same_bits(got, ref), mismatch(got, ref)


@pytest.mark.parametrize("quant,cols", [(Q4_K, 256 * 57), (Q6_K, 256 * 200), (Q8_0, 32 * 500), (Q4_0, 32 * 1500)])
def test_gemv_q8_long_rows_caller_blocks(gpu, quant, cols):
    """Caller blocks over several staging rounds, and past the LDS budget (global path)."""
    torch = gpu
    rows = 5
    raw = synth.random_weights(quant, rows, cols, seed=cols, specials=True)
    xq = x_blocks(quant, synth.activations(cols, 3))
    ref = O.gemv_q8(quant, [rows, cols], raw, xq, rows)
    w = jk.Weight(jk.TensorView("w", quant, [rows, cols], raw), rows, cols)
    got = gpu_gemv(torch, w, xq)
    assert same_bits(got, ref), mismatch(got, ref)


@pytest.mark.parametrize("quant", [Q6_K, TQ2_0])
@pytest.mark.parametrize("rows,cols", [(100, 256 * 40), (2000, 256 * 60), (2000, 256 * 56), (7, 256 * 33)])
def test_gemv_q8_caller_blocks_staging_rounds(gpu, quant, rows, cols):
    """The single-pass GEMV (one row a wave for rows of 33-64 blocks) with caller blocks of the formats
    whose dots read the recomputed per-16 sums: activations staged in two rounds (4-wave workgroups
    at 33 and 40 blocks, 8-wave ones at 60) and in one (8-wave workgroups at 56 blocks, the ffn_down
    shape), each == the oracle bit for bit."""
    torch = gpu
    raw = synth.random_weights(quant, rows, cols, seed=rows + cols, specials=True)
    xq = x_blocks(quant, synth.activations(cols, 4))
    ref = O.gemv_q8(quant, [rows, cols], raw, xq, rows)
    w = jk.Weight(jk.TensorView("w", quant, [rows, cols], raw), rows, cols)
    got = gpu_gemv(torch, w, xq)
    assert same_bits(got, ref), mismatch(got, ref)


def test_gemv_q8_caller_q8k_with_inconsistent_bsums(gpu):
    """Q6_K / TQ2_0 dots use the quants themselves, Q4_K uses bsums as given (quant_q8.rs:1834-2003)."""
    torch = gpu
    rows, cols = 7, 1024
    x = O.quantize_row_q8_k(synth.activations(cols, 9))
    x["bsums"] = np.random.default_rng(1).integers(-3000, 3000, x["bsums"].shape, dtype=np.int16)
    for quant in (Q4_K, Q5_K, Q6_K, TQ1_0, TQ2_0):
        raw = synth.gguf_weights(quant, rows, cols, seed=quant)
        ref = O.gemv_q8(quant, [rows, cols], raw, x, rows)
        w = jk.Weight(jk.TensorView("w", quant, [rows, cols], raw), rows, cols)
        got = gpu_gemv(torch, w, x)
        assert same_bits(got, ref), (quant, mismatch(got, ref))


def test_gemv_q8_batch_mixed_jobs(gpu):
    """One grouped call == the per-matrix calls: shared and distinct activations, f32 and
    caller blocks, row slices, an empty job and two weight formats (split launches)."""
    torch = gpu
    specs = [(Q4_K, 96, 4096), (Q4_K, 24, 4096), (Q4_K, 40, 4096), (Q6_K, 33, 14336), (Q4_0, 50, 4096),
             (Q4_K, 64, 4096)]
    xs = {c: synth.activations(c, c) for c in (4096, 14336)}
    dxf = {c: torch.from_numpy(xs[c]).cuda() for c in xs}
    dq = {}
    jobs, expect, outs = [], [], []
    for i, (quant, rows, cols) in enumerate(specs):
        raw = synth.gguf_weights(quant, rows, cols, seed=50 + i)
        w = jk.Weight(jk.TensorView(f"w{i}", quant, [rows, cols], raw), rows, cols)
        xq = x_blocks(quant, xs[cols])
        key = (quant in jk.Q8_0_ACT, cols)
        if key not in dq:
            dq[key] = dev(torch, xq)
        full = O.gemv_q8(quant, [rows, cols], raw, xq, rows)
        r0, r1 = (3, rows - 5) if i % 2 else (0, rows)
        if i == 5:
            r0 = r1 = 10  # empty job
        y = empty(torch, 4 * max(1, r1 - r0))
        use_f32 = i % 3 != 1
        jobs.append((w, None if use_f32 else dq[key], dxf[cols] if use_f32 else None, y, r0, r1))
        expect.append(full[r0:r1])
        outs.append((y, r1 - r0))
    jk.dev_gemv_q8_batch(jobs)
    torch.cuda.synchronize()
    for (y, n), ref in zip(outs, expect):
        if n:
            got = host(y, np.float32, n)
            assert same_bits(got, ref), mismatch(got, ref)


@pytest.mark.parametrize("use_f32", [True, False])
def test_gemv_q8_batch_uneven_jobs(gpu, use_f32):
    """Jobs of very different sizes in one call (the Q/K/V shape: 4096 + 1024 + 1024 rows, here
    with a sliced job and a row count that is no multiple of a workgroup's rows), which the
    launcher re-cuts into equal row ranges, == the oracle per matrix, bit for bit."""
    torch = gpu
    cols = 4096
    specs = [(4096, 5, 4000), (1024, 0, 1024), (1000, 0, 1000), (1024, 17, 1024)]
    x = synth.activations(cols, 77)
    xq = x_blocks(Q4_K, x)
    dxf, dxq = torch.from_numpy(x).cuda(), dev(torch, xq)
    jobs, expect, outs = [], [], []
    for i, (rows, r0, r1) in enumerate(specs):
        raw = synth.gguf_weights(Q4_K, rows, cols, seed=90 + i)
        w = jk.Weight(jk.TensorView(f"w{i}", Q4_K, [rows, cols], raw), rows, cols)
        y = empty(torch, 4 * (r1 - r0))
        jobs.append((w, None if use_f32 else dxq, dxf if use_f32 else None, y, r0, r1))
        expect.append(O.gemv_q8(Q4_K, [rows, cols], raw, xq, rows)[r0:r1])
        outs.append((y, r1 - r0))
    jk.dev_gemv_q8_batch(jobs)
    torch.cuda.synchronize()
    for i, ((y, n), ref) in enumerate(zip(outs, expect)):
        got = host(y, np.float32, n)
        assert same_bits(got, ref), (i, mismatch(got, ref))


def test_gemv_q8_batch_activation_beyond_lds_budget(gpu):
    """A caller-block job whose activation exceeds the LDS budget (Q4_K, K = 51200: 200 blocks of
    336 staged bytes > 60 KiB) runs on the global-activation kernel while small-K jobs of the same
    format in the same call, f32 included, stay on the staged kernels; an f32 job beyond the budget
    is refused before anything is launched (no output is written)."""
    torch = gpu
    specs = [(Q4_K, 40, 51200, False), (Q4_K, 96, 4096, True), (Q4_K, 24, 4096, False)]
    jobs, expect, outs = [], [], []
    for i, (quant, rows, cols, use_f32) in enumerate(specs):
        raw = synth.gguf_weights(quant, rows, cols, seed=70 + i)
        w = jk.Weight(jk.TensorView(f"w{i}", quant, [rows, cols], raw), rows, cols)
        x = synth.activations(cols, 80 + i)
        xq = x_blocks(quant, x)
        y = empty(torch, 4 * rows)
        jobs.append((w, None if use_f32 else dev(torch, xq), torch.from_numpy(x).cuda() if use_f32 else None, y, 0,
                     rows))
        expect.append(O.gemv_q8(quant, [rows, cols], raw, xq, rows))
        outs.append((y, rows))
    jk.dev_gemv_q8_batch(jobs)
    torch.cuda.synchronize()
    for (y, n), ref in zip(outs, expect):
        got = host(y, np.float32, n)
        assert same_bits(got, ref), mismatch(got, ref)
    # the same caller-block job first, then an f32 job with K beyond the budget: refused, and the
    # first job's output is left as it was
    big = jobs[0]
    xf_big = torch.from_numpy(synth.activations(51200, 90)).cuda()
    for y, _ in outs:
        y.fill_(7)
    with pytest.raises(jk.CapabilityMismatch, match="f32 activations need K"):
        jk.dev_gemv_q8_batch([big, (big[0], None, xf_big, outs[1][0], 0, 40)])
    torch.cuda.synchronize()
    assert bool((outs[0][0] == 7).all()) and bool((outs[1][0] == 7).all())


def test_gemv_q8_batch_validation(gpu):
    torch = gpu
    raw = synth.gguf_weights(Q4_K, 4, 256, seed=1)
    w = jk.Weight(jk.TensorView("w", Q4_K, [4, 256], raw), 4, 256)
    wi = jk.Weight(jk.TensorView("wi", I2_S, [4, 128], synth.gguf_weights(I2_S, 4, 128, seed=2)), 4, 128)
    x = torch.zeros(256, dtype=torch.float32, device="cuda")
    y = torch.zeros(4, dtype=torch.float32, device="cuda")
    with pytest.raises(jk.TensorBoundsError):  # neither activation
        jk.dev_gemv_q8_batch([(w, None, None, y, 0, 4)])
    with pytest.raises(jk.TensorBoundsError):  # both activations
        jk.dev_gemv_q8_batch([(w, x, x, y, 0, 4)])
    with pytest.raises(jk.TensorBoundsError):  # rows out of range
        jk.dev_gemv_q8_batch([(w, None, x, y, 0, 5)])
    with pytest.raises(jk.TensorBoundsError):  # misaligned f32 activation
        jk.dev_gemv_q8_batch([(w, None, x.data_ptr() + 4, y, 0, 4)])
    with pytest.raises(jk.CapabilityMismatch):  # I2_S has no quant_q8 GEMV
        jk.dev_gemv_q8_batch([(wi, None, x, y, 0, 4)])
    with pytest.raises(jk.TensorBoundsError):
        jk.dev_gemv_q8_f32(w, x, 255, y, 4)


# ------------------------------------------------------------------ f32 vec_dot
@pytest.mark.parametrize("quant", list(jk.VEC_DOT_F32_FORMATS))
@pytest.mark.parametrize("rows,cols", [(1, 256), (5, 4352), (33, 4096)])
def test_vec_dot_f32(gpu, quant, rows, cols):
    torch = gpu
    raw = synth.random_weights(quant, rows, cols, seed=rows + quant, specials=True)
    x = np.random.default_rng(rows).standard_normal(cols).astype(np.float32)
    ref = O.vec_dot_f32(quant, [rows, cols], raw, x, rows)
    w = jk.Weight(jk.TensorView("w", quant, [rows, cols], raw), rows, cols)
    dy = empty(torch, 4 * rows)
    jk.dev_vec_dot_f32(w, dev(torch, x), cols, dy, rows)
    torch.cuda.synchronize()
    got = host(dy, np.float32, rows)
    assert same_bits(got, ref), mismatch(got, ref)


@pytest.mark.parametrize("quant", list(jk.VEC_DOT_F32_FORMATS))
@pytest.mark.parametrize("rows,cols", [(1, 256), (37, 4096), (300, 4352), (11, 1024), (5, 8192), (9, 256 * 90)])
def test_vec_dot_f32_tol(gpu, quant, rows, cols):
    """Tolerance-mode f32 vec_dot (jk_vec_dot_f32_tol): rows of up to 32 blocks (each block's
    elements split over four waves; one and two blocks a lane, exactly 32 blocks), longer rows
    (64 lanes a row), activations too long for LDS (23040 columns), weights with special scales.
    Every output within 1e-5 of the output vector's L2 norm of the oracle and of the bit-exact GPU
    result."""
    torch = gpu
    raw = synth.random_weights(quant, rows, cols, seed=3 * rows + quant, specials=True)
    x = np.random.default_rng(rows + cols).standard_normal(cols).astype(np.float32)
    ref = O.vec_dot_f32(quant, [rows, cols], raw, x, rows)
    w = jk.Weight(jk.TensorView("w", quant, [rows, cols], raw), rows, cols)
    dy, dt = empty(torch, 4 * rows), empty(torch, 4 * rows)
    jk.dev_vec_dot_f32(w, dev(torch, x), cols, dy, rows)
    jk.dev_vec_dot_f32_tol(w, dev(torch, x), cols, dt, rows)
    torch.cuda.synchronize()
    exact, tol = host(dy, np.float32, rows), host(dt, np.float32, rows)
    assert same_bits(exact, ref)
    worst = assert_within_row_norm(tol[None, :], ref[None, :])
    print(f"vec_dot tol {quant} {rows}x{cols}: worst error / norm {worst:.2e}")
    w.free()


def test_vec_dot_i2_s_zero_scale_rows_are_zero(gpu):
    torch = gpu
    rows, cols = 6, 256
    raw = synth.gguf_weights(I2_S, rows, cols, seed=1)
    raw[-32:-28] = 0  # trailer scale 0.0
    w = jk.Weight(jk.TensorView("w", I2_S, [rows, cols], raw), rows, cols)
    dy = empty(torch, 4 * rows)
    jk.dev_vec_dot_f32(w, dev(torch, np.ones(cols, np.float32)), cols, dy, rows)
    torch.cuda.synchronize()
    assert same_bits(host(dy, np.float32, rows), np.zeros(rows, np.float32))
    dt = empty(torch, 4 * rows)
    jk.dev_vec_dot_f32_tol(w, dev(torch, np.ones(cols, np.float32)), cols, dt, rows)
    torch.cuda.synchronize()
    assert same_bits(host(dt, np.float32, rows), np.zeros(rows, np.float32))


# ------------------------------------------------------------------ repacked GEMM
def gpu_gemm(torch, w, x, m, r0=0, r1=None):
    r1 = w.rows if r1 is None else r1
    storage, act = gpu_act(torch, x, m, w.cols)
    dy = empty(torch, 4 * m * (r1 - r0))
    jk.dev_gemm_repacked(w, act, dy, m * (r1 - r0), r0, r1)
    torch.cuda.synchronize()
    return host(dy, np.float32, m * (r1 - r0)).reshape(m, r1 - r0)


@pytest.mark.parametrize("quant", ALL_FORMATS)
@pytest.mark.parametrize("m,rows,cols", [(1, 37, 512), (5, 64, 256), (70, 100, 1024), (64, 128, 4096)])
def test_gemm_repacked(gpu, quant, m, rows, cols):
    torch = gpu
    raw = synth.random_weights(quant, rows, cols, seed=m + quant, specials=True)
    x = np.random.default_rng(m + rows).standard_normal((m, cols)).astype(np.float32)
    w = jk.Weight(jk.TensorView("w", quant, [rows, cols], raw), rows, cols)
    got = gpu_gemm(torch, w, x, m)
    ref = O.gemm_repacked(quant, [rows, cols], raw, rows, cols, O.ActQ8(x, m, cols), 0, rows)
    assert same_bits(got, ref), mismatch(got, ref)
    got_slice = gpu_gemm(torch, w, x, m, 3, rows - 5)
    assert same_bits(got_slice, ref[:, 3:rows - 5])


@pytest.mark.parametrize("quant", ALL_FORMATS)
@pytest.mark.parametrize("m,rows,cols", [(1, 37, 512), (2, 100, 4096), (1, 33, 768), (2, 9, 160), (1, 4100, 1280),
                                         (2, 70, 14336), (2, 21, 33024), (1, 9, 32768), (2, 5, 16384)])
def test_gemv_repacked_one_or_two_tokens(gpu, quant, m, rows, cols):
    """m <= 2 runs a GEMV kernel (Q8_0 / Q4_0 / Q4_K / Q5_K / Q6_K: 16 lanes per row, block b on lane
    b % 16, terms chained across the lanes in K order; the other formats, and activations beyond
    the 32 KB staged in LDS (33024 columns at two tokens), the 32-row kernel whose waves split K):
    every repacked entry point == the oracle bit for bit -- one and several rounds of blocks, a
    partial last round and a partial last chunk (160 = 5 steps of 32), a partial last row tile, row
    slices (the two-token Q6_K launch offsets each token's output), both GEMM modes and
    jk_gemv_repacked. 32768 columns at one token and 16384 at two fill the LDS-staged activation
    exactly (every thread's eight 16-byte pieces distinct)."""
    torch = gpu
    if cols % jk.BLOCK_ELEMENTS[quant]:
        pytest.skip("shape not block aligned")
    raw = synth.random_weights(quant, rows, cols, seed=7 * m + quant + rows, specials=True)
    x = np.random.default_rng(m + cols).standard_normal((m, cols)).astype(np.float32)
    w = jk.Weight(jk.TensorView("w", quant, [rows, cols], raw), rows, cols)
    ref = O.gemm_repacked(quant, [rows, cols], raw, rows, cols, O.ActQ8(x, m, cols), 0, rows)
    got = gpu_gemm(torch, w, x, m)
    assert same_bits(got, ref), mismatch(got, ref)
    r0, r1 = min(3, rows - 1), rows - min(5, rows - 4)
    assert same_bits(gpu_gemm(torch, w, x, m, r0, r1), ref[:, r0:r1])
    assert same_bits(gpu_gemm_tol(torch, w, x, m), ref)
    if m == 1:
        storage, act = gpu_act(torch, x, m, cols)
        dy = empty(torch, 4 * rows)
        jk.dev_gemv_repacked(w, act, dy, rows, 0, rows)
        torch.cuda.synchronize()
        assert same_bits(host(dy, np.float32, rows).reshape(1, rows), ref)


@pytest.mark.parametrize("quant", ALL_FORMATS)
@pytest.mark.parametrize("m", [500, 250, 128, 30])
def test_gemm_tile_shapes(gpu, quant, m):
    """8200 rows: 500 tokens launch 128x64 tiles, 250 tokens 64x64, 128 tokens 32x32, 30
    tokens the single-wave 32x16 tiles (32x32 for Q6_K): the launcher takes the largest tile
    that gives 256 CUs two workgroups each. The last row tile and token tile are partial.
    Oracle on row windows."""
    torch = gpu
    rows, cols = 8200, 512
    raw = synth.random_weights(quant, rows, cols, seed=m + 3 * quant, specials=True)
    x = np.random.default_rng(m).standard_normal((m, cols)).astype(np.float32)
    w = jk.Weight(jk.TensorView("w", quant, [rows, cols], raw), rows, cols)
    got = gpu_gemm(torch, w, x, m)
    act = O.ActQ8(x, m, cols)
    for r0 in (0, 4091, rows - 45):
        ref = O.gemm_repacked(quant, [rows, cols], raw, rows, cols, act, r0, r0 + 45)
        assert same_bits(got[:, r0:r0 + 45], ref), (r0, mismatch(got[:, r0:r0 + 45], ref))


def gpu_gemm_tol(torch, w, x, m, r0=0, r1=None, expect=None):
    """Tolerance-mode GEMM; with `expect`, first checks (jk_gemm_plan) that the call launches
    that kernel, so a change of the launch rules cannot leave the test on another one."""
    r1 = w.rows if r1 is None else r1
    storage, act = gpu_act(torch, x, m, w.cols)
    if expect is not None:
        kernel = jk.gemm_plan(w, act, r0, r1, True)
        assert kernel == expect, f"{m} tokens x rows {r0}..{r1} launch {kernel}, not {expect}"
    dy = empty(torch, 4 * m * (r1 - r0))
    jk.dev_gemm_repacked_tol(w, act, dy, m * (r1 - r0), r0, r1)
    torch.cuda.synchronize()
    return host(dy, np.float32, m * (r1 - r0)).reshape(m, r1 - r0)


def assert_within_row_norm(got, ref, tol=1e-5):
    """The bar for f32 products: every output within tol of its token's output-row L2 norm."""
    ref64 = ref.astype(np.float64)
    norms = np.linalg.norm(ref64, axis=1)
    err = np.abs(got.astype(np.float64) - ref64).max(axis=1)
    bad = np.nonzero(err > tol * norms)[0]
    assert bad.size == 0, f"{bad.size} rows over the bar; first {bad[0]}: err {err[bad[0]]:.3e} norm {norms[bad[0]]:.3e}"
    return float((err / np.where(norms > 0, norms, 1.0)).max())


@pytest.mark.parametrize("m", [64, 128, 512, 2048])
def test_gemm_q8_0_prefill_shape_rows_sample(gpu, m):
    """C4 prefill shape 14336 x 4096 at its whole token sweep: the bit-exact GEMM is held to the
    oracle on row windows (full K, every token), and the tolerance-mode GEMM to the bit-exact
    output over the whole matrix at 1e-5 of each token's output-row L2 norm."""
    torch = gpu
    rows, cols = 14336, 4096
    raw = synth.gguf_weights(Q8_0, rows, cols, seed=4)
    x = synth.activations((m, cols), 6)
    w = jk.Weight(jk.TensorView("ffn", Q8_0, [cols, rows], raw), rows, cols)
    got = gpu_gemm(torch, w, x, m)
    act = O.ActQ8(x, m, cols)
    for r0 in (0, 7168, 14336 - 40):
        ref = O.gemm_repacked(Q8_0, [cols, rows], raw, rows, cols, act, r0, r0 + 40)
        assert same_bits(got[:, r0:r0 + 40], ref), (r0, mismatch(got[:, r0:r0 + 40], ref))
    tol = gpu_gemm_tol(torch, w, x, m)
    worst = assert_within_row_norm(tol, got)
    print(f"gemm tol Q8_0 14336x4096 M={m}: worst error / row norm {worst:.2e}")
    w.free()


def test_gemm_q8_0_prefill_full_matrix_vs_exact_product(gpu):
    """The C4 prefill GEMM at 512 tokens over all 14336 x 512 outputs against the exact product of
    its operands: the Q8_0 weights (d * q) times the QuantizedActQ8 activations (scale * q), both
    exact in float64, multiplied and summed in float64 -- a reference computed without the
    reference's recipe. Both modes within 1e-5 of each token's output-row L2 norm (the bit-exact
    mode's distance is the recipe's own f32 rounding)."""
    torch = gpu
    rows, cols, m = 14336, 4096, 512
    raw = synth.gguf_weights(Q8_0, rows, cols, seed=21)
    x = synth.activations((m, cols), 22)
    w = jk.Weight(jk.TensorView("ffn", Q8_0, [cols, rows], raw), rows, cols)
    blk = np.frombuffer(raw, dtype=np.dtype([("d", "<f2"), ("qs", "i1", (32,))])).reshape(rows, cols // 32)
    d = blk["d"].astype(np.float64)
    d = np.where(np.isfinite(d), d, 0.0)  # f16_to_f32_finite
    w64 = (d[..., None] * blk["qs"].astype(np.float64)).reshape(rows, cols)
    act = O.ActQ8(x, m, cols)
    x64 = (act.qs[:, :cols].astype(np.float64).reshape(m, cols // 32, 32)
           * act.scales[:, : cols // 32].astype(np.float64)[..., None]).reshape(m, cols)
    y64 = x64 @ w64.T
    del w64
    exact = gpu_gemm(torch, w, x, m)
    tol = gpu_gemm_tol(torch, w, x, m, expect="gemm_q8_0_tol_dma_128")
    we = assert_within_row_norm(exact, y64)
    wt = assert_within_row_norm(tol, y64)
    print(f"Q8_0 14336x4096 M=512 against the float64 product: bit-exact {we:.2e}, tolerance {wt:.2e} of the row norm")
    w.free()


@pytest.mark.parametrize("quant", ALL_FORMATS)
@pytest.mark.parametrize("m", [500, 250, 128, 30])
def test_gemm_tol_tile_shapes(gpu, quant, m):
    """Tolerance-mode GEMM on every format and tile shape (8200 rows: 128x64, 64x64 and 32x32
    tiles; partial last row and token tiles; weights with special scales): within 1e-5 of each
    token's output-row L2 norm of the oracle on row windows and of the bit-exact GPU output over
    the whole matrix, and row slices equal to the full call."""
    torch = gpu
    rows, cols = 8200, 512
    raw = synth.random_weights(quant, rows, cols, seed=m + 5 * quant, specials=True)
    x = np.random.default_rng(m + 1).standard_normal((m, cols)).astype(np.float32)
    w = jk.Weight(jk.TensorView("w", quant, [rows, cols], raw), rows, cols)
    exact = gpu_gemm(torch, w, x, m)
    tol = gpu_gemm_tol(torch, w, x, m)
    assert_within_row_norm(tol, exact)
    act = O.ActQ8(x, m, cols)
    ref = O.gemm_repacked(quant, [rows, cols], raw, rows, cols, act, 4091, 4091 + 45)
    assert same_bits(exact[:, 4091:4136], ref)
    norms = np.linalg.norm(exact.astype(np.float64), axis=1)
    assert np.all(np.abs(tol[:, 4091:4136] - ref).max(axis=1) <= 1e-5 * norms)
    sl = gpu_gemm_tol(torch, w, x, m, 3, rows - 5)
    assert_within_row_norm(sl, exact[:, 3:rows - 5])
    w.free()


@pytest.mark.parametrize("quant", [Q6_K, Q3_K])
def test_gemm_tol_q6_k_tiles(gpu, quant):
    """Q6_K / Q3_K in tolerance mode on 128 x 128 tiles (14300 rows, a partial last row tile; 500 tokens, a
    partial last token tile; weights with special scales): the two 16-element groups of a step
    combined in integers with their scales, then one fused multiply-add. Within 1e-5 of each
    token's output-row L2 norm of the bit-exact GPU output over the whole matrix and of the
    oracle on a row window; a row slice within the same bar."""
    torch = gpu
    rows, cols, m = 14300, 512, 500
    raw = synth.random_weights(quant, rows, cols, seed=61 + quant, specials=True)
    x = np.random.default_rng(62).standard_normal((m, cols)).astype(np.float32)
    w = jk.Weight(jk.TensorView("w", quant, [rows, cols], raw), rows, cols)
    exact = gpu_gemm(torch, w, x, m)
    tol = gpu_gemm_tol(torch, w, x, m)
    assert_within_row_norm(tol, exact)
    ref = O.gemm_repacked(quant, [rows, cols], raw, rows, cols, O.ActQ8(x, m, cols), 14250, 14300)
    assert same_bits(exact[:, 14250:], ref)
    norms = np.linalg.norm(exact.astype(np.float64), axis=1)
    assert np.all(np.abs(tol[:, 14250:] - ref).max(axis=1) <= 1e-5 * norms)
    assert_within_row_norm(gpu_gemm_tol(torch, w, x, m, 3, rows - 5), exact[:, 3:rows - 5])
    w.free()


def test_gemm_tol_q6_k_extreme_combination(gpu):
    """The Q6_K tolerance tiles add sc0 * c0 + sc1 * c1 in integers before converting: the largest
    magnitude a step can reach is 2 * 16 * 32 * 127 * 128 = 16,646,144, just under 2^24 (exact in
    f32). Every weight at q - 32 = -32 with scales -128 and d = 1.0, activations +1.0 (quants 127),
    12288 rows x 512 tokens: within the tolerance of the bit-exact output, which equals the
    oracle."""
    torch = gpu
    rows, cols, m = 12288, 256, 512
    blk = np.dtype([("ql", "u1", (128,)), ("qh", "u1", (64,)), ("scales", "i1", (16,)), ("d", "<f2")])
    wb = np.zeros((rows, cols // 256), dtype=blk)
    wb["scales"] = -128
    wb["d"] = 1.0
    raw = np.frombuffer(wb.tobytes(), dtype=np.uint8)
    x = np.ones((m, cols), np.float32)
    w = jk.Weight(jk.TensorView("w", Q6_K, [rows, cols], raw), rows, cols)
    exact = gpu_gemm(torch, w, x, m)
    tol = gpu_gemm_tol(torch, w, x, m)
    assert_within_row_norm(tol, exact)
    ref = O.gemm_repacked(Q6_K, [rows, cols], raw, rows, cols, O.ActQ8(x[:2], 2, cols), 100, 140)
    assert same_bits(exact[:2, 100:140], ref)
    assert exact[0, 0] == 2 * 8 * 16 * 32 * 127 * 128 / 127.0  # 16 groups of (-32 * -128) * 16 * 127, xs = 1/127
    w.free()


def test_gemm_tol_extreme_group_dots(gpu):
    """The 512-token tolerance tiles read each group's integer dot product out of a biased
    accumulator; its range must hold the largest |dot| a Q8_0 group can reach, 32 * 128 * 127 (-128
    weight quants against +-127 activation quants). Weights of +-128 / +127 quants with d = 1.0,
    activations of +-1.0 (quants +-127), 14336 rows x 512 tokens (448 128 x 128 tiles, which the
    launch plan confirms run gemm_q8_0_tol_dma_128): equal to the bit-exact output within the
    tolerance, and the bit-exact output equal to the oracle."""
    torch = gpu
    rows, cols, m = 14336, 256, 512
    blk = np.dtype([("d", "<f2"), ("qs", "i1", (32,))])
    w_blocks = np.zeros((rows, cols // 32), dtype=blk)
    w_blocks["d"] = 1.0
    w_blocks["qs"][0::2] = -128
    w_blocks["qs"][1::2] = 127
    raw = np.frombuffer(w_blocks.tobytes(), dtype=np.uint8)
    x = np.where((np.arange(m) % 3 == 0)[:, None], -1.0, 1.0).astype(np.float32) * np.ones((m, cols), np.float32)
    w = jk.Weight(jk.TensorView("w", Q8_0, [rows, cols], raw), rows, cols)
    exact = gpu_gemm(torch, w, x, m)
    tol = gpu_gemm_tol(torch, w, x, m, expect="gemm_q8_0_tol_dma_128")
    assert_within_row_norm(tol, exact)
    act = O.ActQ8(x, m, cols)
    ref = O.gemm_repacked(Q8_0, [rows, cols], raw, rows, cols, act, 4000, 4040)
    assert same_bits(exact[:, 4000:4040], ref)
    # every group dot is +-520192 or +-516128, i.e. -4096 / +4064 times 127; 8 groups per row
    assert np.allclose(exact[1, 0:2], [8 * -4096.0, 8 * 4064.0], rtol=1e-6)
    w.free()


def test_gemm_q8_0_exact_staged_tiles(gpu):
    """The bit-exact Q8_0 GEMM on the global-to-LDS staged 128 x 128 tiles (launched for 1.5 to 2 such
    tiles per CU): ragged rows (12328 = 96 x 128 + 40) and tokens (500 = 3 x 128 + 116), adversarial
    weights and activations, a row slice; equal to the oracle bit for bit on row windows at both ends
    and inside, every token. BitLinear's Q8_0 weights (one activation scale per token) keep the
    register-staged tiles."""
    torch = gpu
    rows, cols, m = 12328, 512, 500
    raw = synth.random_weights(Q8_0, rows, cols, seed=11, specials=True)
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((m, cols)) * rng.choice([1e-3, 1, 40], (m, cols))).astype(np.float32)
    x[rng.random((m, cols)) < 0.002] = np.nan
    w = jk.Weight(jk.TensorView("w", Q8_0, [rows, cols], raw), rows, cols)
    storage, act = gpu_act(torch, x, m, cols)
    assert jk.gemm_plan(w, act, 0, rows, False) == "gemm_q8_0_exact_dma_128"
    got = gpu_gemm(torch, w, x, m)
    oact = O.ActQ8(x, m, cols)
    for r0 in (0, 6000, rows - 40):
        ref = O.gemm_repacked(Q8_0, [rows, cols], raw, rows, cols, oact, r0, r0 + 40)
        assert same_bits(got[:, r0:r0 + 40], ref), (r0, mismatch(got[:, r0:r0 + 40], ref))
    sub = gpu_gemm(torch, w, x, m, 1000, rows - 17)  # a row slice (ragged at both ends of its tiles)
    assert same_bits(sub, got[:, 1000:rows - 17])
    w.free()


TOL128_FORMATS = [Q8_0, Q4_0, Q5_0, Q4_1, Q5_1, IQ4_NL, Q4_K, Q5_K, TQ2_0, I2_S]


@pytest.mark.parametrize("quant", TOL128_FORMATS)
def test_gemm_tol_128_tiles(gpu, quant):
    """Tolerance-mode 128 x 128 tiles of every 32-element-group format (gemm_tol_kernel; Q8_0 its
    DMA variant): 14300 rows x 500 tokens is 448 tiles, above the launch's 1.5 tiles per CU, with a
    partial last row tile and a partial last token tile; weights with special scales. Within 1e-5
    of each token's output-row L2 norm of the bit-exact GPU output over the whole matrix and of
    the oracle on two row windows (the first tile and the partial last one); a row slice within
    the same bar."""
    torch = gpu
    rows, cols, m = 14300, 512, 500
    raw = synth.random_weights(quant, rows, cols, seed=91 + quant, specials=True)
    x = np.random.default_rng(92 + quant).standard_normal((m, cols)).astype(np.float32)
    w = jk.Weight(jk.TensorView("w", quant, [rows, cols], raw), rows, cols)
    expect = "gemm_q8_0_tol_dma_128" if quant == Q8_0 else "gemm_tol_kernel"
    exact = gpu_gemm(torch, w, x, m)
    tol = gpu_gemm_tol(torch, w, x, m, expect=expect)
    worst = assert_within_row_norm(tol, exact)
    act = O.ActQ8(x, m, cols)
    norms = np.linalg.norm(exact.astype(np.float64), axis=1)
    for r0, r1 in ((0, 40), (14260, 14300)):
        ref = O.gemm_repacked(quant, [rows, cols], raw, rows, cols, act, r0, r1)
        assert same_bits(exact[:, r0:r1], ref), (r0, mismatch(exact[:, r0:r1], ref))
        assert np.all(np.abs(tol[:, r0:r1] - ref).max(axis=1) <= 1e-5 * norms)
    assert_within_row_norm(gpu_gemm_tol(torch, w, x, m, 3, rows - 5), exact[:, 3:rows - 5])
    print(f"gemm tol {quant} 14300x512 M=500 on {expect}: worst error / row norm {worst:.2e}")
    w.free()


@pytest.mark.parametrize("quant", [Q8_0, Q4_0, Q5_0, Q4_1, Q5_1, IQ4_NL])
@pytest.mark.parametrize("m,rows", [(64, 8200), (17, 16400)])
def test_gemm_tol_32x32_tiles_partial_chunk(gpu, quant, m, rows):
    """Tolerance-mode 32 x 32 tiles (gemm_repacked_kernel<32x32, tolerance>), the launch for K
    that is not a whole number of 128-element chunks (here 160: five 32-element groups) where the
    32 x 32 tiles give every CU two workgroups: 64 and 17 tokens (partial token tiles), a partial
    last row tile, weights with special scales. Within 1e-5 of each token's output-row L2 norm of
    the bit-exact GPU output and of the oracle on a row window."""
    torch = gpu
    cols = 160
    raw = synth.random_weights(quant, rows, cols, seed=m + rows + quant, specials=True)
    x = np.random.default_rng(m + quant).standard_normal((m, cols)).astype(np.float32)
    w = jk.Weight(jk.TensorView("w", quant, [rows, cols], raw), rows, cols)
    exact = gpu_gemm(torch, w, x, m)
    tol = gpu_gemm_tol(torch, w, x, m, expect="gemm_repacked_kernel<32x32, tolerance>")
    assert_within_row_norm(tol, exact)
    ref = O.gemm_repacked(quant, [rows, cols], raw, rows, cols, O.ActQ8(x, m, cols), rows - 50, rows)
    assert same_bits(exact[:, rows - 50:], ref)
    norms = np.linalg.norm(exact.astype(np.float64), axis=1)
    assert np.all(np.abs(tol[:, rows - 50:] - ref).max(axis=1) <= 1e-5 * norms)
    w.free()


SPLITK_FORMATS = [Q8_0, Q4_0, Q5_0, Q4_1, Q5_1, IQ4_NL, Q4_K, Q5_K, TQ2_0, I2_S, Q6_K, Q3_K]


@pytest.mark.parametrize("quant", SPLITK_FORMATS)
@pytest.mark.parametrize("m,chunks", [(3, 1), (17, 3), (32, 5), (33, 6), (64, 13), (100, 10), (200, 4)])
def test_gemm_tol_split_k(gpu, quant, m, chunks):
    """Tolerance-mode GEMM of a few tokens, where K is split over the waves of a workgroup: K of
    1 to 13 chunks of 128 (waves with no chunk, with one more chunk than the others), 32- and
    64-token tiles with a partial last one (Q6_K / Q3_K: 64-token tiles, the two 16-element groups of
    a step combined in integers), 200 rows (a partial last row tile) and a row slice.
    Held within 1e-5 of each token's output-row L2 norm of the bit-exact GPU output over the whole
    matrix and of the oracle on a row window."""
    torch = gpu
    block = 256 if quant in (Q4_K, Q5_K, TQ2_0, Q6_K, Q3_K) else 128  # K-quant super-blocks, I2_S blocks of 128
    cols = max(block, 128 * chunks // block * block)
    rows = 200
    raw = synth.random_weights(quant, rows, cols, seed=7 * m + chunks + quant, specials=True)
    x = np.random.default_rng(m + chunks).standard_normal((m, cols)).astype(np.float32)
    w = jk.Weight(jk.TensorView("w", quant, [rows, cols], raw), rows, cols)
    exact = gpu_gemm(torch, w, x, m)
    tol = gpu_gemm_tol(torch, w, x, m)
    assert_within_row_norm(tol, exact)
    act = O.ActQ8(x, m, cols)
    ref = O.gemm_repacked(quant, [rows, cols], raw, rows, cols, act, 150, 200)
    assert same_bits(exact[:, 150:200], ref)
    norms = np.linalg.norm(exact.astype(np.float64), axis=1)
    assert np.all(np.abs(tol[:, 150:200] - ref).max(axis=1) <= 1e-5 * norms)
    sl = gpu_gemm_tol(torch, w, x, m, 5, 171)
    assert_within_row_norm(sl, exact[:, 5:171])
    w.free()


# ------------------------------------------------------------------ BitLinear
@pytest.mark.parametrize("quant", [TQ1_0, TQ2_0, I2_S, Q8_0])
@pytest.mark.parametrize("m,rows,cols", [(1, 7, 256), (3, 64, 2560), (2, 2560, 6912),
                                         (1, 6912, 2560), (1, 2560, 6912),  # one token, the C5 shapes
                                         # token batches take the int8-MFMA path
                                         (16, 300, 2560), (37, 129, 768), (128, 2560, 6912), (128, 6912, 2560)])
def test_bitlinear(gpu, quant, m, rows, cols):
    torch = gpu
    raw = synth.gguf_weights(quant, rows, cols, seed=m + quant) if quant != Q8_0 else \
        synth.random_weights(quant, rows, cols, seed=m, specials=True)
    rng = np.random.default_rng(rows)
    a = rng.integers(-128, 128, (m, cols)).astype(np.int8)
    sc = rng.uniform(0.001, 0.1, m).astype(np.float32)
    w = jk.Weight(jk.TensorView("w", quant, [rows, cols], raw), rows, cols)
    dy = empty(torch, 4 * m * rows)
    jk.dev_bitlinear_i8(w, dev(torch, a), dev(torch, sc), m, cols, dy, m * rows)
    torch.cuda.synchronize()
    got = host(dy, np.float32, m * rows).reshape(m, rows)
    for i in range(m):
        ref = O.bitlinear_i8(quant, [rows, cols], raw, a[i], float(sc[i]), rows)
        assert same_bits(got[i], ref), (i, mismatch(got[i], ref))


@pytest.mark.parametrize("quant", [TQ1_0, TQ2_0, I2_S, Q8_0])
@pytest.mark.parametrize("m,rows,cols,offset", [(3, 64, 2560, 0), (16, 300, 2560, 0), (37, 129, 768, 0),
                                                (50, 40, 256, 0),  # fewer blocks than waves
                                                (20, 33, 512, 1),  # activation rows not 16-byte aligned
                                                (128, 2560, 6912, 0), (128, 6912, 2560, 0),
                                                (16, 40, 8448, 0)])  # K beyond the split kernel
def test_bitlinear_tol(gpu, quant, m, rows, cols, offset):
    """Tolerance-mode BitLinear (jk_bitlinear_i8_tol): every output within 1e-5 of its token's
    output-row L2 norm of the bit-exact GPU result over the whole matrix and of the oracle on
    the first and last tokens; the launch plan confirms that TQ2_0 / TQ1_0 / I2_S token batches
    with aligned rows and K up to 8192 run the K-split kernel (2 to 8 waves; longer K and the
    other cases the bit-exact launch), with weights with special scales and I2_S with a random
    tensor scale."""
    torch = gpu
    raw = synth.random_weights(quant, rows, cols, seed=m + rows + quant, specials=True)
    rng = np.random.default_rng(rows + cols)
    a = rng.integers(-128, 128, (m, cols)).astype(np.int8)
    sc = rng.uniform(0.001, 0.1, m).astype(np.float32)
    w = jk.Weight(jk.TensorView("w", quant, [rows, cols], raw), rows, cols)
    da = torch.zeros(m * cols + 16, dtype=torch.uint8, device="cuda")
    da[offset:offset + m * cols] = dev(torch, a)
    ds = dev(torch, sc)
    kernel = jk.bitlinear_plan(w, da[offset:], m, tolerance=True)
    split_k = cols // 256 <= 32 if quant != I2_S else cols // 128 <= 64  # K up to 8192
    if m >= 16 and quant != Q8_0 and offset == 0 and split_k:
        assert kernel.startswith("bitlinear_tol_kernel"), kernel
    dy, dt = empty(torch, 4 * m * rows), empty(torch, 4 * m * rows)
    jk.dev_bitlinear_i8(w, da[offset:], ds, m, cols, dy, m * rows)
    jk.dev_bitlinear_i8_tol(w, da[offset:], ds, m, cols, dt, m * rows)
    torch.cuda.synchronize()
    exact = host(dy, np.float32, m * rows).reshape(m, rows)
    tol = host(dt, np.float32, m * rows).reshape(m, rows)
    worst = assert_within_row_norm(tol, exact)
    for i in (0, m - 1):
        ref = O.bitlinear_i8(quant, [rows, cols], raw, a[i], float(sc[i]), rows)
        assert same_bits(exact[i], ref), (i, mismatch(exact[i], ref))
        assert np.abs(tol[i].astype(np.float64) - ref).max() <= 1e-5 * np.linalg.norm(ref.astype(np.float64))
    print(f"bitlinear tol {quant} {rows}x{cols} M={m} on {kernel}: worst error / row norm {worst:.2e}")
    w.free()


def test_bitlinear_tol_i2_s_extreme_sum(gpu):
    """The I2_S tolerance kernel sums a whole row in exact integers before one conversion: every
    weight +1 (2-bit field 2) and every activation +127 over K = 6912 gives 877,824 per output,
    exact in f32, so each output is f32(877824) * (scale * act_scale) -- one rounding."""
    torch = gpu
    rows, cols, m = 2560, 6912, 128
    payload = np.full(rows * cols // 4, 0b10101010, dtype=np.uint8)
    trailer = np.zeros(32, dtype=np.uint8)
    trailer[:4] = np.frombuffer(np.float32(0.75).tobytes(), dtype=np.uint8)
    raw = np.concatenate([payload, trailer])
    a = np.full((m, cols), 127, dtype=np.int8)
    sc = np.linspace(0.001, 0.1, m).astype(np.float32)
    w = jk.Weight(jk.TensorView("w", I2_S, [rows, cols], raw), rows, cols)
    dt = empty(torch, 4 * m * rows)
    jk.dev_bitlinear_i8_tol(w, dev(torch, a), dev(torch, sc), m, cols, dt, m * rows)
    torch.cuda.synchronize()
    tol = host(dt, np.float32, m * rows).reshape(m, rows)
    want = (np.float32(127 * cols) * (np.float32(0.75) * sc)).astype(np.float32)
    assert same_bits(tol, np.repeat(want[:, None], rows, axis=1))
    w.free()


@pytest.mark.parametrize("quant", [TQ1_0, TQ2_0, I2_S])
@pytest.mark.parametrize("m,rows,cols,offset", [(1, 9, 256 * 65, 0),   # more than 64 blocks a row
                                                (2, 13, 2560, 1),     # activation not 16-byte aligned
                                                (5, 11, 1024, 0)])
def test_bitlinear_few_tokens_paths(gpu, quant, m, rows, cols, offset):
    """The few-token BitLinear launches: the LDS-staged ternary kernel and the general kernel
    it leaves rows of more than 64 blocks and unaligned activation rows to."""
    torch = gpu
    raw = synth.gguf_weights(quant, rows, cols, seed=rows + quant)
    rng = np.random.default_rng(cols + offset)
    a = rng.integers(-128, 128, (m, cols)).astype(np.int8)
    sc = rng.uniform(0.001, 0.1, m).astype(np.float32)
    w = jk.Weight(jk.TensorView("w", quant, [rows, cols], raw), rows, cols)
    da = torch.zeros(m * cols + 16, dtype=torch.uint8, device="cuda")
    da[offset:offset + m * cols] = dev(torch, a)
    dy = empty(torch, 4 * m * rows)
    jk.dev_bitlinear_i8(w, da[offset:], dev(torch, sc), m, cols, dy, m * rows)
    torch.cuda.synchronize()
    got = host(dy, np.float32, m * rows).reshape(m, rows)
    for i in range(m):
        ref = O.bitlinear_i8(quant, [rows, cols], raw, a[i], float(sc[i]), rows)
        assert same_bits(got[i], ref), (i, mismatch(got[i], ref))


@pytest.mark.parametrize("quant", [TQ1_0, TQ2_0, I2_S])
@pytest.mark.parametrize("m,rows,cols", [(100, 6900, 2560), (16, 16400, 256)])
def test_bitlinear_wave_tiles_partial(gpu, quant, m, rows, cols):
    """The one-wave-per-tile BitLinear launch (enough 32 x 32 tiles for two waves per CU) with a
    partial last row tile (6900 = 215 x 32 + 20) and a partial last token tile (100 = 3 x 32 + 4),
    and with one half-empty token tile (16 tokens, 16400 rows: 513 tiles, one weight block a row):
    every token against the oracle, bit for bit."""
    torch = gpu
    raw = synth.gguf_weights(quant, rows, cols, seed=quant + 5)
    rng = np.random.default_rng(quant)
    a = rng.integers(-128, 128, (m, cols)).astype(np.int8)
    sc = rng.uniform(0.001, 0.1, m).astype(np.float32)
    w = jk.Weight(jk.TensorView("w", quant, [rows, cols], raw), rows, cols)
    dy = empty(torch, 4 * m * rows)
    jk.dev_bitlinear_i8(w, dev(torch, a), dev(torch, sc), m, cols, dy, m * rows)
    torch.cuda.synchronize()
    got = host(dy, np.float32, m * rows).reshape(m, rows)
    for i in range(m):
        ref = O.bitlinear_i8(quant, [rows, cols], raw, a[i], float(sc[i]), rows)
        assert same_bits(got[i], ref), (i, mismatch(got[i], ref))


@pytest.mark.parametrize("quant", [TQ1_0, TQ2_0, I2_S, Q8_0])
@pytest.mark.parametrize("m", [500, 250, 128, 30])
def test_bitlinear_tile_shapes(gpu, quant, m):
    """BitLinear token batches on each GEMM tile shape (as test_gemm_tile_shapes), with the
    block accumulation crossing chunk boundaries; oracle on every 23rd token and the last."""
    torch = gpu
    rows, cols = 8200, 512
    raw = synth.gguf_weights(quant, rows, cols, seed=m + quant) if quant != Q8_0 else \
        synth.random_weights(quant, rows, cols, seed=m, specials=True)
    rng = np.random.default_rng(m + 1)
    a = rng.integers(-128, 128, (m, cols)).astype(np.int8)
    sc = rng.uniform(0.001, 0.1, m).astype(np.float32)
    w = jk.Weight(jk.TensorView("w", quant, [rows, cols], raw), rows, cols)
    dy = empty(torch, 4 * m * rows)
    jk.dev_bitlinear_i8(w, dev(torch, a), dev(torch, sc), m, cols, dy, m * rows)
    torch.cuda.synchronize()
    got = host(dy, np.float32, m * rows).reshape(m, rows)
    for i in list(range(0, m, 23)) + [m - 1]:
        ref = O.bitlinear_i8(quant, [rows, cols], raw, a[i], float(sc[i]), rows)
        assert same_bits(got[i], ref), (i, mismatch(got[i], ref))


# ------------------------------------------------------------------ host tier
def test_host_tier_matches_oracle(gpu):
    rng = np.random.default_rng(0)
    x = rng.standard_normal(4096).astype(np.float32)
    assert np.array_equal(jk.quantize_row_q8_0(x).view(np.uint8), O.quantize_row_q8_0(x).view(np.uint8))
    assert np.array_equal(jk.quantize_row_q8_k(x).view(np.uint8), O.quantize_row_q8_k(x).view(np.uint8))
    raw = synth.gguf_weights(Q4_K, 9, 4096, seed=3)
    xq = O.quantize_row_q8_k(x)
    out = np.zeros(9, np.float32)
    jk.gemv_q4_k_q8_k(out, jk.TensorView("w", Q4_K, [4096, 9], raw), xq)
    assert same_bits(out, O.gemv_q8(Q4_K, [4096, 9], raw, xq, 9))
    v = jk.vec_dot_q4_k_q8_k(raw[:16 * 144], xq)
    assert same_bits(np.float32([v]), np.float32([O.vec_dot_q8(Q4_K, raw[:16 * 144], xq)]))
    f = np.zeros(9, np.float32)
    jk.vec_dot_q4_k_m(f, jk.TensorView("w", Q4_K, [4096, 9], raw), x)
    assert same_bits(f, O.vec_dot_f32(Q4_K, [4096, 9], raw, x, 9))
    row = np.zeros(4096, np.float32)
    jk.dequantize_tensor_row(jk.TensorView("w", Q4_K, [4096, 9], raw), 4, row)
    assert same_bits(row, O.dequantize_tensor_row(Q4_K, [4096, 9], raw, 4, 4096))
    tq = synth.gguf_weights(TQ2_0, 5, 512, seed=1)
    a = rng.integers(-128, 128, 512).astype(np.int8)
    bl = np.zeros(5, np.float32)
    jk.bitlinear_i8(bl, jk.TensorView("w", TQ2_0, [5, 512], tq), a, 0.02)
    assert same_bits(bl, O.bitlinear_i8(TQ2_0, [5, 512], tq, a, 0.02, 5))
    w8 = synth.gguf_weights(Q8_0, 40, 1024, seed=2)
    w = jk.Weight(jk.TensorView("w", Q8_0, [40, 1024], w8), 40, 1024)
    xs = rng.standard_normal((3, 1024)).astype(np.float32)
    g = np.zeros(3 * 30, np.float32)
    jk.host_gemm_repacked_f32(g, w, xs, 3, 5, 35)
    ref = O.gemm_repacked(Q8_0, [40, 1024], w8, 40, 1024, O.ActQ8(xs, 3, 1024), 5, 35)
    assert same_bits(g.reshape(3, 30), ref)


def test_tq1_0_and_tq2_0_jobs_share_a_batch(gpu):
    """TQ1_0 handles use the TQ2_0 device layout: a batch mixing the two formats runs as one
    launch and each job still matches its own format's oracle GEMV."""
    torch = gpu
    cols = 2560
    x = synth.activations(cols, 77)
    dxf = torch.from_numpy(x).cuda()
    jobs, expect, outs = [], [], []
    for i, (quant, rows) in enumerate(((TQ1_0, 300), (TQ2_0, 200), (TQ1_0, 77))):
        raw = synth.gguf_weights(quant, rows, cols, seed=90 + i)
        w = jk.Weight(jk.TensorView(f"t{i}", quant, [rows, cols], raw), rows, cols)
        y = empty(torch, 4 * rows)
        jobs.append((w, None, dxf, y, 0, rows))
        expect.append(O.gemv_q8(quant, [rows, cols], raw, O.quantize_row_q8_k(x), rows))
        outs.append((y, rows))
    jk.dev_gemv_q8_batch(jobs)
    torch.cuda.synchronize()
    for (y, n), ref in zip(outs, expect):
        got = host(y, np.float32, n)
        assert same_bits(got, ref), mismatch(got, ref)


def test_host_tier_new_formats(gpu):
    """Host-tier mirrors of the Q5_0 / Q5_K / TQ1_0 entries against the oracle."""
    rng = np.random.default_rng(4)
    x = rng.standard_normal(2048).astype(np.float32)
    x8, xk = O.quantize_row_q8_0(x), O.quantize_row_q8_k(x)
    for quant, gemv, xq in ((Q5_0, jk.gemv_q5_0_q8_0, x8), (Q5_K, jk.gemv_q5_k_q8_k, xk),
                            (TQ1_0, jk.gemv_tq1_0_q8_k, xk)):
        raw = synth.random_weights(quant, 6, 2048, seed=quant, specials=True)
        out = np.zeros(6, np.float32)
        gemv(out, jk.TensorView("w", quant, [2048, 6], raw), xq)
        assert same_bits(out, O.gemv_q8(quant, [2048, 6], raw, xq, 6)), quant
    raw = synth.random_weights(Q5_0, 3, 2048, seed=1, specials=True)
    v = jk.vec_dot_q5_0_q8_0_blocks(raw[:64 * 22], x8)
    assert same_bits(np.float32([v]), np.float32([O.vec_dot_q8(Q5_0, raw[:64 * 22], x8)]))
    raw = synth.random_weights(Q5_K, 3, 2048, seed=2, specials=True)
    v = jk.vec_dot_q5_k_q8_k(raw[:8 * 176], xk)
    assert same_bits(np.float32([v]), np.float32([O.vec_dot_q8(Q5_K, raw[:8 * 176], xk)]))
    raw = synth.gguf_weights(TQ1_0, 3, 2048, seed=3)
    v = jk.vec_dot_tq1_0_q8_k(raw[:8 * 54], xk)
    assert same_bits(np.float32([v]), np.float32([O.vec_dot_q8(TQ1_0, raw[:8 * 54], xk)]))
    for quant, fn in ((Q5_0, jk.vec_dot_q5_0), (Q5_K, jk.vec_dot_q5_k)):
        raw = synth.random_weights(quant, 5, 2048, seed=quant + 1, specials=True)
        f = np.zeros(5, np.float32)
        fn(f, jk.TensorView("w", quant, [2048, 5], raw), x)
        assert same_bits(f, O.vec_dot_f32(quant, [2048, 5], raw, x, 5)), quant
        row = np.zeros(2048, np.float32)
        jk.dequantize_tensor_row(jk.TensorView("w", quant, [2048, 5], raw), 3, row)
        assert same_bits(row, O.dequantize_tensor_row(quant, [2048, 5], raw, 3, 2048)), quant
    tq = synth.gguf_weights(TQ1_0, 5, 512, seed=1)
    a = rng.integers(-128, 128, 512).astype(np.int8)
    bl = np.zeros(5, np.float32)
    jk.bitlinear_i8(bl, jk.TensorView("w", TQ1_0, [5, 512], tq), a, 0.02)
    assert same_bits(bl, O.bitlinear_i8(TQ1_0, [5, 512], tq, a, 0.02, 5))


def test_new_format_validation(gpu):
    torch = gpu
    raw = synth.gguf_weights(TQ1_0, 4, 256, seed=1)
    w = jk.Weight(jk.TensorView("w", TQ1_0, [4, 256], raw), 4, 256)
    x = torch.zeros(256, dtype=torch.float32, device="cuda")
    y = torch.zeros(4, dtype=torch.float32, device="cuda")
    xq = dev(torch, O.quantize_row_q8_k(np.ones(256, np.float32)))
    with pytest.raises(jk.TensorBoundsError):  # a TQ1_0 handle is not a TQ2_0 weight
        jk.dev_gemv_q8(w, xq, 1, y, 4, fn="jk_gemv_tq2_0_q8_k")
    jk.dev_gemv_q8(w, xq, 1, y, 4)
    with pytest.raises(jk.CapabilityMismatch):  # no f32-activation matvec for TQ1_0
        jk.dev_vec_dot_f32(w, x, 256, y, 4)
    w5 = jk.Weight(jk.TensorView("w5", Q5_K, [4, 256], synth.gguf_weights(Q5_K, 4, 256, seed=2)), 4, 256)
    with pytest.raises(jk.TensorBoundsError):  # Q5_K is not a BitLinear format
        jk.dev_bitlinear_i8(w5, torch.zeros(256, dtype=torch.int8, device="cuda"), y[:1], 1, 256, y, 4)
    torch.cuda.synchronize()


@pytest.mark.parametrize("quant", [Q4_1, Q5_1, Q2_K, Q3_K, IQ4_NL, I2_S])
def test_formats_without_q8_gemv(gpu, quant):
    """Formats the reference offers no quant_q8 GEMV (nor BitLinear, except I2_S) for are refused
    with the reference's error kinds, before any device work."""
    torch = gpu
    rows, cols = 4, 256
    w = jk.Weight(jk.TensorView("w", quant, [rows, cols], synth.gguf_weights(quant, rows, cols, seed=1)), rows, cols)
    x = torch.zeros(cols, dtype=torch.float32, device="cuda")
    y = torch.zeros(rows, dtype=torch.float32, device="cuda")
    with pytest.raises(jk.CapabilityMismatch):
        jk.dev_gemv_q8_f32(w, x, cols, y, rows)
    with pytest.raises(jk.CapabilityMismatch):
        jk.dev_gemv_q8_rows(w, x, 1, y, 0, rows)
    if quant != I2_S:
        with pytest.raises(jk.TensorBoundsError):
            jk.dev_bitlinear_i8(w, torch.zeros(cols, dtype=torch.int8, device="cuda"), y[:1], 1, cols, y, rows)
    torch.cuda.synchronize()


def test_host_tier_vec_dot_more_formats(gpu):
    """Host-tier f32 matvec mirrors of the Q4_1 / Q5_1 / Q2_K / Q3_K / IQ4_NL entries."""
    x = np.random.default_rng(8).standard_normal(1024).astype(np.float32)
    for quant, fn in ((Q4_1, jk.vec_dot_q4_1), (Q5_1, jk.vec_dot_q5_1), (Q2_K, jk.vec_dot_q2_k),
                      (Q3_K, jk.vec_dot_q3_k), (IQ4_NL, jk.vec_dot_iq4_nl)):
        raw = synth.random_weights(quant, 7, 1024, seed=quant, specials=True)
        f = np.zeros(7, np.float32)
        fn(f, jk.TensorView("w", quant, [1024, 7], raw), x)
        assert same_bits(f, O.vec_dot_f32(quant, [1024, 7], raw, x, 7)), quant


# ------------------------------------------------------------ I2_S -> TQ2_0
def test_convert_i2_s_to_tq2_0(gpu):
    """convert_i2_s_blocks_to_tq2_0 (ime.rs:767-790) on the device over 5000 random block pairs
    (every byte value, I2_S field value 3 included) and through the host mirror, bit for bit
    against the oracle; then BitLinear over the converted weights equals the oracle's TQ2_0
    BitLinear of the same bytes."""
    torch = gpu
    rng = np.random.default_rng(11)
    n = 5000
    i2s = rng.integers(0, 256, size=(2 * n, 32), dtype=np.uint8)
    i2s[:256, 0] = np.arange(256)
    bits = 0x3555
    ref = np.concatenate([O.convert_i2_s_blocks_to_tq2_0(i2s[2 * k], i2s[2 * k + 1], bits) for k in range(n)])
    out = torch.full((n * 66,), 0xAB, dtype=torch.uint8, device="cuda")
    jk.dev_convert_i2_s_to_tq2_0(dev(torch, i2s), 2 * n, bits, out, n)
    torch.cuda.synchronize()
    got = host(out, np.uint8)
    assert np.array_equal(got, ref)
    for k in (0, 1, 4999):
        assert np.array_equal(jk.convert_i2_s_blocks_to_tq2_0(i2s[2 * k], i2s[2 * k + 1], bits), ref[66 * k:66 * k + 66])
    # the converted bytes as a TQ2_0 weight of 50 rows x 25600 (trits of field value 3 included)
    rows, cols = 50, 100 * 256
    w = jk.Weight(jk.TensorView("tq2", TQ2_0, [rows, cols], got), rows, cols)
    act = rng.integers(-128, 128, size=cols, dtype=np.int8)
    y = empty(torch, 4 * rows)
    sc = torch.tensor([0.375], dtype=torch.float32, device="cuda")
    jk.dev_bitlinear_i8(w, dev(torch, act), sc, 1, cols, y, rows)
    torch.cuda.synchronize()
    assert same_bits(host(y, np.float32, rows), O.bitlinear_i8(TQ2_0, [rows, cols], ref, act, 0.375, rows))
    with pytest.raises(jk.TensorBoundsError):
        jk.dev_convert_i2_s_to_tq2_0(dev(torch, i2s), 3, bits, out, 1)
