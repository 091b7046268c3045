"""GPU parity of the epilogue entry points: gated activations (alone and fused into the activation
quantizers) and argmax (alone and fused into the quant_q8 GEMV), through the C ABI.

SwiGLU uses the device's single-precision exp, so it is held to the reference's own tolerance for
its vector path, max(1e-6, 1e-5 |y|) (tests/wave1_rope_swiglu_fidelity.rs:295-297); everything
else is compared bit for bit.
"""
import numpy as np
import pytest

import jk
import oracle as O
from jk import synth

pytestmark = pytest.mark.gpu


def same_bits(a, b) -> bool:
    a, b = np.ascontiguousarray(a, np.float32), np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and bool(np.all((a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))))


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def gate_up(n, seed):
    rng = np.random.default_rng(seed)
    g = (rng.standard_normal(n) * 6).astype(np.float32)
    g[::97] = -100.0
    g[1::97] = 100.0
    g[2::97] = 0.0
    g[3::97] = -0.0
    g[4::97] = 20.0
    g[5::97] = -20.0
    u = rng.standard_normal(n).astype(np.float32)
    return g, u


@pytest.mark.parametrize("n", [1, 7, 1000, 14336, 14336 * 3 + 5])
def test_gated_activations(gpu, n):
    torch = gpu
    g, u = gate_up(n, n)
    dg, du = dev(torch, g), dev(torch, u)
    out = torch.empty(n, dtype=torch.float32, device="cuda")
    jk.dev_swiglu_f32(dg, du, n, out)
    torch.cuda.synchronize()
    got, ref = out.cpu().numpy(), O.swiglu_f32(g, u)
    assert np.all(np.abs(got - ref) <= np.maximum(1e-6, 1e-5 * np.abs(ref)))
    assert np.array_equal(got[(g > 20) | (g < -20)], ref[(g > 20) | (g < -20)])
    jk.dev_relu_squared_gate_f32(dg, du, n, out)
    torch.cuda.synchronize()
    assert same_bits(out.cpu().numpy(), O.relu_squared_gate_f32(g, u))


def test_gated_host_tier(gpu):
    g, u = gate_up(3000, 1)
    out = np.zeros(3000, np.float32)
    jk.relu_squared_gate_f32(out, g, u)
    assert same_bits(out, O.relu_squared_gate_f32(g, u))
    jk.swiglu_f32(out, g, u)
    ref = O.swiglu_f32(g, u)
    assert np.all(np.abs(out - ref) <= np.maximum(1e-6, 1e-5 * np.abs(ref)))
    with pytest.raises(jk.TensorBoundsError):
        jk.swiglu_f32(np.zeros(2, np.float32), g[:3], u[:3])


@pytest.mark.parametrize("n", [256, 14336, 256 * 57])
@pytest.mark.parametrize("offset", [0, 1])
def test_quantize_row_q8_k_gated(gpu, n, offset):
    """Fused activation + quantize_row_q8_k == the activation kernel followed by the quantizer
    (bit for bit), and for ReLU^2 == the oracle's quantize of the oracle's activation. offset 1:
    the fused call's gate and up rows one float past a 16-byte boundary (element-wise loads)."""
    torch = gpu
    g, u = gate_up(n, n + 1)
    dg, du = dev(torch, g), dev(torch, u)
    nb = n // 256
    ug, uu = torch.zeros(n + 4, dtype=torch.float32, device="cuda"), torch.zeros(n + 4, dtype=torch.float32, device="cuda")
    ug[offset:offset + n] = dg
    uu[offset:offset + n] = du
    fg, fu = ug[offset:], uu[offset:]
    for act in (jk.ACT_SWIGLU, jk.ACT_RELU2):
        h = torch.empty(n, dtype=torch.float32, device="cuda")
        (jk.dev_swiglu_f32 if act == jk.ACT_SWIGLU else jk.dev_relu_squared_gate_f32)(dg, du, n, h)
        q1 = torch.empty(nb * jk.BLOCK_Q8K.itemsize, dtype=torch.uint8, device="cuda")
        q2 = torch.empty_like(q1)
        jk.dev_quantize_row_q8_k(h, n, q1, nb)
        jk.dev_quantize_row_q8_k_gated(act, fg, fu, n, q2, nb)
        torch.cuda.synchronize()
        assert np.array_equal(q1.cpu().numpy(), q2.cpu().numpy()), act
        if act == jk.ACT_RELU2:
            ref = O.quantize_row_q8_k(O.relu_squared_gate_f32(g, u)).view(np.uint8).reshape(-1)
            assert np.array_equal(q2.cpu().numpy(), ref)


# Bound of a SwiGLU-fused quantizer against the oracle. The device SwiGLU is within
# max(1e-6, 1e-5 |h|) of the oracle's (glibc expf), so a block maximum -- and the scale
# d = amax / 127 -- moves by at most 1e-5 relative plus 1e-6 / 127, and h * 127 / amax by at
# most 127 * 2e-5 + 1e-6 * 127 / amax < 0.01 for the blocks here (amax > 0.5): a quant can
# only cross a rounding boundary, i.e. move by one level.
def assert_scale_close(got, ref):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    assert np.all(np.abs(got - ref) <= 1e-5 * np.abs(ref) + 1e-6 / 127), np.max(np.abs(got - ref) / np.abs(ref))


@pytest.mark.parametrize("n", [256, 14336, 256 * 57])
def test_quantize_row_q8_k_swiglu_vs_oracle(gpu, n):
    """SwiGLU fused into quantize_row_q8_k vs the oracle's quantize_row_q8_k of the oracle's SwiGLU:
    d within 1e-5 relative, every quant within one level, bsums the sums of the device's own quants
    (so within 16 of the oracle's)."""
    torch = gpu
    g, u = gate_up(n, n + 2)
    nb = n // 256
    q = torch.empty(nb * jk.BLOCK_Q8K.itemsize, dtype=torch.uint8, device="cuda")
    jk.dev_quantize_row_q8_k_gated(jk.ACT_SWIGLU, dev(torch, g), dev(torch, u), n, q, nb)
    torch.cuda.synchronize()
    got = q.cpu().numpy().view(jk.BLOCK_Q8K)
    ref = O.quantize_row_q8_k(O.swiglu_f32(g, u))
    assert np.all(np.abs(ref["d"]) * 127 > 0.5)  # the premise of the bound
    assert_scale_close(got["d"], ref["d"])
    dq = got["qs"].astype(np.int32) - ref["qs"].astype(np.int32)
    assert np.abs(dq).max() <= 1
    own = got["qs"].astype(np.int32).reshape(nb, 16, 16).sum(axis=2)
    assert np.array_equal(got["bsums"].astype(np.int32), own)
    assert np.abs(own - ref["bsums"].astype(np.int32)).max() <= 16
    assert np.mean(dq == 0) > 0.99  # a level moves only next to a rounding boundary


@pytest.mark.parametrize("m,k", [(1, 14336), (7, 4096)])
def test_quantize_act_q8_swiglu_vs_oracle(gpu, m, k):
    """SwiGLU fused into quantize_act_q8 vs the oracle's quantize of the oracle's SwiGLU: the 32-element
    scales within 1e-5 relative and quants within one level. (The derived sums of given quants and
    scales are pinned bit for bit by the non-fused quantizer's oracle test and the gated == two-call
    test below.)"""
    torch = gpu
    g, u = gate_up(m * k, m + k + 3)
    need = jk.act_q8_bytes(m, k)
    st = torch.zeros(need, dtype=torch.uint8, device="cuda")
    a = jk.act_q8_bind(st, need, m, k)
    jk.dev_quantize_act_q8_gated(jk.ACT_SWIGLU, dev(torch, g), dev(torch, u), m, k, a)
    torch.cuda.synchronize()
    raw, base = st.cpu().numpy(), st.data_ptr()
    ref = O.ActQ8(O.swiglu_f32(g, u), m, k)
    qs = raw[a.qs - base: a.qs - base + m * a.k_padded].view(np.int8).reshape(m, -1)
    sc = raw[a.scales - base: a.scales - base + 4 * ref.scales.size].view(np.float32).reshape(ref.scales.shape)
    live = ref.scales != 0
    assert np.array_equal(sc[~live], ref.scales[~live])
    assert np.all(np.abs(ref.scales[live]) * 127 > 0.5)
    assert_scale_close(sc[live], ref.scales[live])
    assert np.abs(qs.astype(np.int32) - ref.qs.astype(np.int32)).max() <= 1


@pytest.mark.parametrize("m,k", [(1, 14336), (7, 4096), (3, 300)])
def test_quantize_act_q8_gated(gpu, m, k):
    torch = gpu
    g, u = gate_up(m * k, m + k)
    dg, du = dev(torch, g), dev(torch, u)
    need = jk.act_q8_bytes(m, k)
    for act in (jk.ACT_SWIGLU, jk.ACT_RELU2):
        h = torch.empty(m * k, dtype=torch.float32, device="cuda")
        (jk.dev_swiglu_f32 if act == jk.ACT_SWIGLU else jk.dev_relu_squared_gate_f32)(dg, du, m * k, h)
        s1 = torch.zeros(need, dtype=torch.uint8, device="cuda")
        s2 = torch.zeros(need, dtype=torch.uint8, device="cuda")
        a1, a2 = jk.act_q8_bind(s1, need, m, k), jk.act_q8_bind(s2, need, m, k)
        jk.dev_quantize_act_q8(h, m, k, a1)
        jk.dev_quantize_act_q8_gated(act, dg, du, m, k, a2)
        torch.cuda.synchronize()
        assert np.array_equal(s1.cpu().numpy(), s2.cpu().numpy()), act


def argmax_cases():
    rng = np.random.default_rng(5)
    out = []
    for v in (32000, 128256, 262144):
        x = np.full(v, -12.5, np.float32)
        x[0] = x[v // 2] = np.nan
        x[v // 3 + 7] = x[v - 19] = 99.75
        out.append(x)
    out.append(np.zeros(0, np.float32))
    out.append(np.full(1000, np.nan, np.float32))
    out.append(np.float32([-0.0, 0.0, -1.0]))
    out.append(np.float32([np.nan, -np.inf, np.nan]))
    x = rng.standard_normal(100003).astype(np.float32)
    x[rng.random(100003) < 0.1] = np.nan
    out.append(x)
    # more values than one pass of the largest partial grid covers (1024 x 256 x 4)
    x = rng.standard_normal(3_000_001).astype(np.float32)
    x[2_999_999] = x[1_048_577] = 7.5
    out.append(x)
    return out


def test_argmax_f32(gpu):
    """Every case on one workspace, back to back, with no clearing between calls; the workspace
    starts out holding large keys so that a slot left unwritten would show."""
    torch = gpu
    cases = argmax_cases()
    ws = torch.full((jk.argmax_workspace_bytes(max(x.size for x in cases)),), 0xFF, dtype=torch.uint8,
                    device="cuda")
    idx = torch.empty(1, dtype=torch.int32, device="cuda")
    for x in cases:
        dx = dev(torch, x) if x.size else torch.empty(1, dtype=torch.float32, device="cuda")
        jk.dev_argmax_f32(dx, x.size, idx, ws)
        torch.cuda.synchronize()
        assert int(idx.cpu()[0]) == O.argmax_f32(x), x.size
        ref = O.argmax_f32(x)
        assert jk.argmax_f32(x) == (None if ref < 0 else ref)


@pytest.mark.parametrize("quant,rows,cols", [(jk.Q6_K, 32000, 4096), (jk.Q8_0, 8200, 4096), (jk.Q4_K, 300, 14336),
                                             (jk.Q4_K, 100, 256 * 70), (jk.Q8_0, 1000, 32 * 200),
                                             (jk.Q4_0, 77, 32 * 2000), (jk.Q4_K, 5, 256)])
def test_gemv_q8_argmax(gpu, quant, rows, cols):
    """GEMV + argmax in one launch: y equals the plain GEMV, the index equals the oracle's argmax of
    the oracle's GEMV; f32 and caller-block activations, with and without y, on the fast, looped
    and global-activation paths (Q4_0 with 2000 blocks a row exceeds the LDS budget)."""
    torch = gpu
    raw = synth.gguf_weights(quant, rows, cols, seed=rows)
    w = jk.Weight(jk.TensorView("lm_head", quant, [rows, cols], raw), rows, cols)
    x = synth.activations(cols, 3)
    xq = O.quantize_row_q8_0(x) if quant in jk.Q8_0_ACT else O.quantize_row_q8_k(x)
    ref_y = O.gemv_q8(quant, [rows, cols], raw, xq, rows)
    ref_i = O.argmax_f32(ref_y)
    ws = torch.full((jk.argmax_workspace_bytes(rows),), 0xFF, dtype=torch.uint8, device="cuda")
    idx = torch.empty(1, dtype=torch.int32, device="cuda")
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    dq = dev(torch, xq.view(np.uint8).reshape(-1))
    jk.dev_gemv_q8_argmax(w, dq, None, xq.size, y, idx, ws)
    torch.cuda.synchronize()
    assert same_bits(y.cpu().numpy(), ref_y) and int(idx.cpu()[0]) == ref_i
    staged = cols // jk.BLOCK_ELEMENTS[quant] * (48 if quant in jk.Q8_0_ACT else 336)
    if staged <= 60 * 1024:  # f32 activations are quantized into the staged LDS blocks
        jk.dev_gemv_q8_argmax(w, None, dev(torch, x), cols, None, idx, ws)
        torch.cuda.synchronize()
        assert int(idx.cpu()[0]) == ref_i


def test_epilogue_validation(gpu):
    torch = gpu
    x = torch.zeros(256, dtype=torch.float32, device="cuda")
    q = torch.zeros(292, dtype=torch.uint8, device="cuda")
    with pytest.raises(jk.TensorBoundsError):
        jk.dev_swiglu_f32(x, x, 0, x)
    with pytest.raises(jk.CapabilityMismatch):
        jk.dev_quantize_row_q8_k_gated(7, x, x, 256, q, 1)
    with pytest.raises(jk.TensorBoundsError):
        jk.dev_quantize_row_q8_k_gated(jk.ACT_SWIGLU, x, x, 255, q, 1)
    wi = jk.Weight(jk.TensorView("w", jk.I2_S, [4, 128], synth.gguf_weights(jk.I2_S, 4, 128, seed=1)), 4, 128)
    idx = torch.zeros(1, dtype=torch.int32, device="cuda")
    ws = torch.zeros(jk.argmax_workspace_bytes(4), dtype=torch.uint8, device="cuda")
    with pytest.raises(jk.CapabilityMismatch):
        jk.dev_gemv_q8_argmax(wi, None, x, 128, None, idx, ws)
    with pytest.raises(jk.TensorBoundsError):  # workspace too small for the values
        jk.dev_argmax_f32(x, 256, idx, ws)
    with pytest.raises(jk.TensorBoundsError):  # misaligned workspace
        jk.dev_argmax_f32(x, 4, idx, ws[1:])
    w = jk.Weight(jk.TensorView("w", jk.Q4_K, [4, 256], synth.gguf_weights(jk.Q4_K, 4, 256, seed=1)), 4, 256)
    with pytest.raises(jk.TensorBoundsError):  # both activations
        jk.dev_gemv_q8_argmax(w, x, x, 256, None, idx, ws)
    with pytest.raises(jk.TensorBoundsError):  # wrong length
        jk.dev_gemv_q8_argmax(w, None, x, 255, None, idx, ws)
    torch.cuda.synchronize()


def test_gemv_q8_argmax_graph_replays(gpu):
    """The fused GEMV + argmax and the standalone argmax captured once in a HIP graph (no memset
    nodes: the workspace needs no clearing) and replayed with new activations in between, eager
    work and synchronizations between the replays; every replay's index equals the oracle's."""
    torch = gpu
    rows, cols = 3000, 4096
    raw = synth.gguf_weights(jk.Q4_K, rows, cols, seed=11)
    w = jk.Weight(jk.TensorView("lm_head", jk.Q4_K, [cols, rows], raw), rows, cols)
    xq_dev = torch.empty(cols // 256 * jk.BLOCK_Q8K.itemsize, dtype=torch.uint8, device="cuda")
    ws = torch.full((jk.argmax_workspace_bytes(rows),), 0xFF, dtype=torch.uint8, device="cuda")
    ws2 = torch.full((jk.argmax_workspace_bytes(rows),), 0xFF, dtype=torch.uint8, device="cuda")
    idx = torch.empty(1, dtype=torch.int32, device="cuda")
    idx2 = torch.empty(1, dtype=torch.int32, device="cuda")
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up outside the capture
        jk.dev_gemv_q8_argmax(w, xq_dev, None, cols // 256, y, idx, ws, side.cuda_stream)
        jk.dev_argmax_f32(y, rows, idx2, ws2, side.cuda_stream)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        cs = torch.cuda.current_stream().cuda_stream
        jk.dev_gemv_q8_argmax(w, xq_dev, None, cols // 256, y, idx, ws, cs)
        jk.dev_argmax_f32(y, rows, idx2, ws2, cs)
    for seed in (1, 2, 3, 4):
        x = synth.activations(cols, 100 + seed)
        xq = O.quantize_row_q8_k(x)
        xq_dev.copy_(torch.from_numpy(xq.view(np.uint8).reshape(-1).copy()))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        ref = O.argmax_f32(O.gemv_q8(jk.Q4_K, [rows, cols], raw, xq, rows))
        assert int(idx.cpu()[0]) == ref and int(idx2.cpu()[0]) == ref, seed


def test_gated_quantizer_graph_replays(gpu):
    """SwiGLU fused into quantize_row_q8_k captured once and replayed with new gate / up values:
    every replay equals the eager activation + quantizer sequence bit for bit."""
    torch = gpu
    n, nb = 14336, 56
    dg = torch.empty(n, dtype=torch.float32, device="cuda")
    du = torch.empty_like(dg)
    q = torch.empty(nb * jk.BLOCK_Q8K.itemsize, dtype=torch.uint8, device="cuda")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        jk.dev_quantize_row_q8_k_gated(jk.ACT_SWIGLU, dg, du, n, q, nb, side.cuda_stream)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        jk.dev_quantize_row_q8_k_gated(jk.ACT_SWIGLU, dg, du, n, q, nb, torch.cuda.current_stream().cuda_stream)
    h = torch.empty_like(dg)
    ref = torch.empty_like(q)
    for seed in (1, 2, 3):
        gt, ut = gate_up(n, 500 + seed)
        dg.copy_(torch.from_numpy(gt))
        du.copy_(torch.from_numpy(ut))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        jk.dev_swiglu_f32(dg, du, n, h)
        jk.dev_quantize_row_q8_k(h, n, ref, nb)
        torch.cuda.synchronize()
        assert np.array_equal(q.cpu().numpy(), ref.cpu().numpy()), seed
