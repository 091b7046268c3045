"""Benchmark of the quantized-matmul hot path on one MI355X.

Headline (``value``): batch-1 decode GEMV throughput over Llama-3-8B layer shapes, in GB/s
of algorithmic bytes (GGUF weight bytes + Q8_K activation blocks + f32 outputs). One step
is one token's decode pass over ``--layers`` layers of distinct weights (32 = the whole
Llama-3-8B stack, 4.4 GB, far larger than the 256 MB Infinity Cache). Per layer the seven
GEMVs (Q/K/V/O 4096-wide and gate/up 14336x4096 in Q4_K, down 4096x14336 in Q6_K) run in
dependency order as grouped launches -- {Q,K,V}, {O}, {gate,up}, {down} -- each quantizing
its f32 activation to Q8_K on the device (bit-exact quantize_row_q8_k); the down projection's
input is SiLU(gate) * up of the layer's own gate / up outputs, fused into its quantizer. The
step is captured once in a HIP graph and replayed.

Also reported on the same JSON line:
  roofline      the dominant launch (grouped Q4_K gate+up GEMV, 2 x 14336x4096), timed per
                launch with HIP events on the launch stream, against 8 TB/s HBM;
  gemm_q8_0     Q8_0 prefill GEMM 14336x4096 at 512 tokens (QuantizedActQ8 quantization +
                int8-MFMA GEMM), in int8 TOPS against the 5.0 POPS dense int8 peak;
  cpu_baseline  the oracle (C restatement of the reference's scalar fallback) running the
                same layer GEMVs on one host core, for a bounded number of repetitions;
  cpu_baseline_all_cores  the same with every matrix's rows split over the host's cores.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "jero-kernels-rvv_amd"))

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
METRIC = "batch-1 Q4_K GEMV HBM GB/s (% peak) at 8B shapes; Q8_0 prefill GEMM int8 TOPS"
# HBM bytes per launch measured with rocprofv3 FETCH_SIZE / WRITE_SIZE (scaled by a copy
# kernel's reading); the file documents the runs and ends in "traffic <launch> <bytes>" lines.
TRAFFIC_FILE = os.path.join(REPO, "profiles", "hbm_traffic_decode_gemv_and_gemm_q8_0.md")


def read_traffic() -> dict:
    out = {}
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                parts = line.split()
                if len(parts) == 3 and parts[0] == "traffic":
                    out[parts[1]] = int(parts[2])
    except OSError:
        pass
    return out


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def graph_us(torch, launch, n, reps=5) -> float:
    """Per-launch time of n launches captured back to back in a HIP graph, replayed `reps`
    times with HIP events on the capturing stream (includes the graph's inter-launch gap)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(n):
            launch(i, side.cuda_stream)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        cs = torch.cuda.current_stream().cuda_stream
        for i in range(n):
            launch(i, cs)
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    del g
    return e0.elapsed_time(e1) * 1e3 / (reps * n)


def stream_read_us(torch, jk, buf, sink, nbytes) -> float:
    """jk_measure_stream_read of nbytes, graph-timed like the GEMV stages: back-to-back launches
    over distinct spans of buf (>= 600 MB in all where buf allows, beyond the 256 MB Infinity
    Cache), so every launch reads from HBM."""
    span = (nbytes + 65535) // 65536 * 65536
    n = max(1, min(buf.numel() // span, max(8, -(-600_000_000 // span))))
    base = buf.data_ptr()
    return graph_us(torch, lambda i, st: jk.dev_measure_stream_read(base + (i % n) * span, nbytes, sink, st), n)


def gemv_bytes(quant, rows, cols, jk) -> int:
    nb = cols // jk.BLOCK_ELEMENTS[quant]
    return rows * nb * jk.BLOCK_BYTES[quant] + (cols // 256) * jk.BLOCK_Q8K.itemsize + rows * 4


def gemv_bytes_q80(quant, rows, cols, jk) -> int:
    """Q4_0 / Q8_0 GEMV: weight bytes + BlockQ8_0 activation blocks + f32 outputs."""
    nb = cols // jk.BLOCK_ELEMENTS[quant]
    return rows * nb * jk.BLOCK_BYTES[quant] + (cols // 32) * jk.BLOCK_Q8_0.itemsize + rows * 4


class Layer:
    """Device weights and buffers of one decode layer."""

    def __init__(self, torch, jk, host_layer, layer_idx):
        self.mats = []
        for name, quant, rows, cols, data in host_layer:
            view = jk.TensorView(f"blk.{layer_idx}.{name}.weight", quant, (rows, cols), data)
            self.mats.append((name, quant, rows, cols, jk.Weight(view, rows, cols)))


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--variants", type=int, default=4, help="distinct synthetic layers (reused cyclically)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline budget (0 = skip)")
    ap.add_argument("--gemm-m", type=int, default=512, help="token count of the reported GEMM line (0 = skip)")
    ap.add_argument("--gemm-sweep", default="64,128,2048", help="further token counts timed for the GEMM sweep")
    ap.add_argument("--no-graph", action="store_true", help="launch the step eagerly instead of a HIP graph")
    ap.add_argument("--no-secondary", action="store_true",
                    help="skip the per-kernel lines of the other workloads (C1, C2, C5, vec_dot f32, quantizers)")
    ap.add_argument("--ffn", choices=("swiglu", "synthetic"), default="swiglu",
                    help="ffn_down input of the timed step: a fixed synthetic activation quantized to Q8_K, or "
                         "SwiGLU of the layer's gate / up outputs fused into its Q8_K quantizer (a Llama "
                         "feed-forward block; also reported as a secondary line)")
    ap.add_argument("--down", choices=("fused", "split"), default="split",
                    help="ffn_down activation: quantized inside the GEMV launch, or by its own launch")
    ap.add_argument("--profile-loop", choices=("bitlinear", "gemm", "vec_dot", "decode"),
                    help="instead of the benchmark: launch one workload's kernels eagerly (no graph) 20 times each "
                         "and exit -- the program a rocprofv3 counter pass runs (bitlinear: the 128-token C5 "
                         "BitLinear, both modes; gemm: the Q8_0 GEMM at 512, 64 and 128 tokens, both modes; vec_dot: the f32 "
                         "vec_dot lines, both modes; decode: the decode step's launches over eight layers, then "
                         "the streaming read of each launch's byte count)")
    args = ap.parse_args()

    if args.profile_loop:
        return profile_loop(args.profile_loop)
    if args.gpus != 1:
        print(f"bench.py: the library runs on one GPU; --gpus {args.gpus} is not supported "
              "(the row-sharded multi-GPU design is documented, not built)", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    import jk
    from jk import synth

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    jk.lib()
    jk.init(0)
    torch.cuda.init()
    dev = torch.device("cuda:0")

    # ------------------------------------------------------------ decode layers
    log(f"generating {args.variants} synthetic layer variants")
    host_layers = []
    for v in range(args.variants):
        hl = []
        for i, (name, quant, rows, cols) in enumerate(synth.LLAMA3_8B_LAYER):
            hl.append((name, quant, rows, cols, synth.gguf_weights(quant, rows, cols, seed=1000 * v + i)))
        host_layers.append(hl)
    log(f"uploading {args.layers} layers")
    layers = [Layer(torch, jk, host_layers[l % args.variants], l) for l in range(args.layers)]
    torch.cuda.synchronize()
    layer_bytes = sum(gemv_bytes(q, r, c, jk) for _, q, r, c in synth.LLAMA3_8B_LAYER)
    step_bytes = layer_bytes * args.layers
    weight_dev_bytes = sum(w.device_bytes for L in layers for *_, w in L.mats)
    log(f"layer algorithmic bytes {layer_bytes}, device weights {weight_dev_bytes / 1e9:.2f} GB")

    gen = torch.Generator(device="cpu").manual_seed(1234)
    acts = {"x": torch.randn(4096, generator=gen).to(dev), "attn": torch.randn(4096, generator=gen).to(dev),
            "ffn_in": torch.randn(4096, generator=gen).to(dev), "h": torch.randn(14336, generator=gen).to(dev)}
    h_q8 = torch.empty(56 * jk.BLOCK_Q8K.itemsize, dtype=torch.uint8, device=dev)
    outs = {name: torch.empty(rows, dtype=torch.float32, device=dev)
            for name, _, rows, _ in synth.LLAMA3_8B_LAYER}
    # The layer's GEMVs in dependency order: each stage is one grouped launch whose
    # activation is quantized to Q8_K inside the launch. ffn_down (K = 14336) takes its
    # activation pre-quantized by a quantize_row_q8_k launch with --down split.
    STAGES = [("qkv", ("attn_q", "attn_k", "attn_v"), "x"), ("attn_output", ("attn_output",), "attn"),
              ("ffn_gate_up", ("ffn_gate", "ffn_up"), "ffn_in"), ("ffn_down", ("ffn_down",), "h")]
    layer_jobs = []
    for L in layers:
        m = {name: (rows, w) for name, quant, rows, cols, w in L.mats}
        per = []
        for stage, names, act in STAGES:
            if stage == "ffn_down" and args.down == "split":
                jobs = [(m[n][1], h_q8, None, outs[n], 0, m[n][0]) for n in names]
            else:
                jobs = [(m[n][1], None, acts[act], outs[n], 0, m[n][0]) for n in names]
            per.append((stage, jk.gemv_jobs(jobs), len(jobs)))
        layer_jobs.append(per)
    lib = jk.lib()

    def launch_stage(stage, arr, n, stream, ffn):
        if stage == "ffn_down" and args.down == "split":
            if ffn == "swiglu":  # h = SiLU(gate) * up of this layer, quantized without writing h
                jk.dev_quantize_row_q8_k_gated(jk.ACT_SWIGLU, outs["ffn_gate"], outs["ffn_up"], 14336, h_q8, 56, stream)
            else:
                jk.dev_quantize_row_q8_k(acts["h"], 14336, h_q8, 56, stream)
        st = lib.jk_gemv_q8_batch(jk._vp(stream), arr, jk._sz(n))
        if st != 0:
            raise jk.K3Error(lib.jk_last_error().decode())

    def run_layers(stream, ffn=args.ffn):
        for per in layer_jobs:
            for stage, arr, n in per:
                launch_stage(stage, arr, n, stream, ffn)

    def capture(ffn):
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            run_layers(side.cuda_stream, ffn)  # warm-up outside capture
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            run_layers(torch.cuda.current_stream().cuda_stream, ffn)
        torch.cuda.synchronize()
        return g

    graph = None if args.no_graph else capture(args.ffn)

    def step():
        if graph is not None:
            graph.replay()
        else:
            run_layers(torch.cuda.current_stream().cuda_stream)

    log(f"warmup {args.warmup} steps")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(args.steps):
        step()
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = ev0.elapsed_time(ev1) / args.steps
    log(f"timed {args.steps} steps: {ms_per_step:.4f} ms/step (wall {wall * 1e3 / args.steps:.4f} ms/step)")
    value = step_bytes / (ms_per_step * 1e-3) / 1e9

    # Per-stage decomposition: each stage's launches for all layers captured back to back in
    # a HIP graph (distinct weights, so every launch streams from HBM), replayed with HIP
    # events on the capturing stream around the replays; per-launch time = elapsed /
    # (replays x layers). This includes the graph's inter-launch gap, which a kernel trace
    # does not.
    mat_bytes = {name: gemv_bytes(q, r, c, jk) for name, q, r, c in synth.LLAMA3_8B_LAYER}
    per_stage = {}
    reps = 5
    for si, (stage, names, _) in enumerate(STAGES):
        g = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for per in layer_jobs:
                launch_stage(stage, per[si][1], per[si][2], side.cuda_stream, args.ffn)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        with torch.cuda.graph(g):
            cs = torch.cuda.current_stream().cuda_stream
            for per in layer_jobs:
                launch_stage(stage, per[si][1], per[si][2], cs, args.ffn)
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        dur_us = e0.elapsed_time(e1) * 1e3 / (reps * len(layers))
        b = sum(mat_bytes[n] for n in names)
        per_stage[stage] = {"matrices": list(names), "bytes": b, "us": round(dur_us, 3),
                            "gbs": round(b / (dur_us * 1e-6) / 1e9, 1)}
        log(f"  {stage:12s} {b:>10d} B: {dur_us:.2f} us/launch, {per_stage[stage]['gbs']} GB/s")
        del g
    # Streaming-read ceiling of each stage: a plain read of the stage's algorithmic byte count
    # (jk_measure_stream_read), timed the same way, and the stage's time as a fraction of it;
    # plus one 1 GiB read for the asymptotic HBM read rate of this GPU.
    rd_buf = torch.empty(2_400_000_000, dtype=torch.uint8, device=dev)
    rd_sink = torch.zeros(4, dtype=torch.int32, device=dev)
    stream_ceiling = {}
    for stage, rec_ in per_stage.items():
        us = stream_read_us(torch, jk, rd_buf, rd_sink, rec_["bytes"])
        rec_["stream_read_us"] = round(us, 3)
        rec_["stream_read_gbs"] = round(rec_["bytes"] / (us * 1e-6) / 1e9, 1)
        rec_["frac_of_stream_read"] = round(us / rec_["us"], 4)
        stream_ceiling[stage] = {"bytes": rec_["bytes"], "us": round(us, 3), "gbs": rec_["stream_read_gbs"]}
        log(f"  stream read {rec_['bytes']:>10d} B: {us:.2f} us/launch, {rec_['stream_read_gbs']} GB/s "
            f"({stage} at {100 * us / rec_['us']:.1f}% of it)")
    big = 1 << 30
    us = stream_read_us(torch, jk, rd_buf, rd_sink, big)
    stream_ceiling["1 GiB"] = {"bytes": big, "us": round(us, 3), "gbs": round(big / (us * 1e-6) / 1e9, 1)}
    log(f"  stream read {big:>10d} B: {us:.2f} us/launch, {stream_ceiling['1 GiB']['gbs']} GB/s")
    stream_ceiling["kernel"] = ("jk_measure_stream_read: 256-thread workgroups of 32 KB, eight coalesced 16-byte "
                                "non-temporal loads per lane, nothing written")
    ceiling_cache = {}

    def ceiling_us(nbytes):
        """The streaming-read time of nbytes (rounded up to 16), measured once per size."""
        nb16 = (int(nbytes) + 15) // 16 * 16
        if nb16 not in ceiling_cache:
            ceiling_cache[nb16] = stream_read_us(torch, jk, rd_buf, rd_sink, nb16)
        return ceiling_cache[nb16]
    dom = per_stage["ffn_gate_up"]
    traffic = read_traffic()
    roofline = {"bound": "hbm", "achieved": dom["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(dom["gbs"] / HBM_PEAK_GBS, 4), "traffic": traffic.get("ffn_gate_up"),
                "kernel": "gemv_q8_fast_kernel<Q4_K> (ffn_gate + ffn_up, 2 x 14336x4096, f32 activation)",
                "avg_launch_us": dom["us"], "bytes_per_launch": dom["bytes"],
                "stream_read_us": dom["stream_read_us"], "frac_of_stream_read": dom["frac_of_stream_read"],
                "traffic_source": os.path.relpath(TRAFFIC_FILE, REPO)}

    # ------------------------------------------------------------ prefill GEMM (Q8_0)
    # Weights rotate over 10 device copies (620 MB, beyond the 256 MB Infinity Cache); the
    # kernel is timed with HIP events on its own stream around each launch, the activation
    # quantization (QuantizedActQ8::quantize_into) runs between the timed launches. Two modes:
    # tolerance (jk_gemm_repacked_tol: one fused multiply-add per scale group, within 1e-5 of
    # each token's output-row L2 norm -- the bar for f32 products; the reported
    # line) and bit-exact (jk_gemm_repacked: the reference's separately rounded epilogue).
    gemm, sweep, gemm_exact, sweep_exact = None, [], None, []
    gemm_host = None
    s = torch.cuda.current_stream().cuda_stream
    ms_list = [args.gemm_m] if args.gemm_m > 0 else []
    ms_list += [int(v) for v in args.gemm_sweep.split(",") if v.strip() and args.gemm_m > 0]
    if ms_list:
        N, K = 14336, 4096
        ncopies = 10
        gdata = synth.gguf_weights(jk.Q8_0, N, K, seed=77)
        gw = [jk.Weight(jk.TensorView(f"ffn_gate.{i}", jk.Q8_0, (N, K), gdata), N, K) for i in range(ncopies)]
        for M in ms_list:
            gx = torch.randn(M, K, generator=gen).to(dev)
            if M == args.gemm_m:
                gemm_host = (gdata, gx.cpu().numpy(), M, N, K)
            need = jk.act_q8_bytes(M, K)
            gstore = torch.empty(need, dtype=torch.uint8, device=dev)
            act = jk.act_q8_bind(gstore, need, M, K)
            gy = torch.empty(M * N, dtype=torch.float32, device=dev)
            for mode, fn in (("tolerance", jk.dev_gemm_repacked_tol), ("bit-exact", jk.dev_gemm_repacked)):
                for i in range(2):
                    jk.dev_quantize_act_q8(gx, M, K, act, s)
                    fn(gw[i], act, gy, M * N, 0, N, s)
                torch.cuda.synchronize()
                reps = 3 * ncopies
                g0, g1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                gev = []
                g0.record()
                for i in range(reps):
                    jk.dev_quantize_act_q8(gx, M, K, act, s)
                    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    e0.record()
                    fn(gw[i % ncopies], act, gy, M * N, 0, N, s)
                    e1.record()
                    gev.append((e0, e1))
                g1.record()
                torch.cuda.synchronize()
                ops = 2.0 * M * N * K
                step_ms = g0.elapsed_time(g1) / reps
                kern_us = float(np.mean([a.elapsed_time(b) * 1e3 for a, b in gev]))
                tops = ops / (kern_us * 1e-6) / 1e12
                row = {"m": M, "mode": mode, "kernel_us": round(kern_us, 2), "kernel_tops": round(tops, 1),
                       "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4),
                       "ms_per_call_incl_quantize": round(step_ms, 4)}
                log(f"gemm Q8_0 M={M} {mode}: kernel {kern_us:.1f} us = {tops:.1f} TOPS "
                    f"({step_ms:.3f} ms/call incl. quantize)")
                kname = jk.gemm_plan(gw[0], act, 0, N, mode == "tolerance")  # the kernel this call launches
                row["kernel"] = kname
                line = {"workload": f"Q8_0 {N}x{K} weights x {M} tokens (QuantizedActQ8 per-32 activations), "
                                    + ("outputs within 1e-5 of each token's output-row L2 norm of the reference "
                                       "recipe (one fused multiply-add per scale group)" if mode == "tolerance"
                                       else "outputs bit-identical to the reference recipe"),
                        "mode": mode, "ms_per_call": round(step_ms, 4), "tops": round(ops / (step_ms * 1e-3) / 1e12, 1),
                        "kernel_us": row["kernel_us"], "kernel_tops": row["kernel_tops"],
                        "roofline": {"bound": "mfma", "achieved": row["kernel_tops"], "peak": INT8_PEAK_TOPS,
                                     "unit": "TOPS", "frac": row["frac_int8_peak"],
                                     "traffic": traffic.get(f"gemm_q8_0_m{M}" + ("_tol" if mode == "tolerance"
                                                                                 else "")),
                                     "kernel": kname}}
                if M == args.gemm_m:
                    if mode == "tolerance" and gemm is None:
                        gemm = line
                    elif mode == "bit-exact" and gemm_exact is None:
                        gemm_exact = line
                else:
                    (sweep if mode == "tolerance" else sweep_exact).append(row)
            del gx, gstore, gy
        for w in gw:
            w.free()

    # ------------------------------------------------------------ other kernels of the path
    # Each line: one kernel at a configuration's shape, weights rotating over enough device
    # copies (>= 600 MB) that every launch streams from HBM, launches captured back to back in
    # a HIP graph and timed with HIP events on the capturing stream (per-launch time includes
    # the graph's inter-launch gap). Bytes are algorithmic (weight bytes + activation + output).
    secondary = {}
    cpu_jobs = []  # (kind, line, ...): the same tensors and inputs, timed on the host by the CPU leg

    def cpu_slices(name, make, unit, scale, what):
        """The CPU leg times make(O) -> [(callable, units)] (row or token slices of the line's work,
        built from the same host tensors) on one thread and on all cores."""
        cpu_jobs.append(("slices", name, make, unit, scale, what))

    def rows_of(data, quant, r0, r1, cols):
        rb = cols // jk.BLOCK_ELEMENTS[quant] * jk.BLOCK_BYTES[quant]
        return data[r0 * rb:r1 * rb]
    if not args.no_secondary and graph is not None:
        # The same step with ffn_down's input computed as in a Llama feed-forward block:
        # SwiGLU(gate, up) of the layer's own outputs, fused into the Q8_K quantizer.
        other = "swiglu" if args.ffn == "synthetic" else "synthetic"
        g2 = capture(other)
        for _ in range(args.warmup):
            g2.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.steps):
            g2.replay()
        e1.record()
        torch.cuda.synchronize()
        ms2 = e0.elapsed_time(e1) / args.steps
        del g2
        secondary[f"decode step, ffn_down input {other}"] = {
            "ms_per_step": round(ms2, 5), "gbs": round(step_bytes / (ms2 * 1e-3) / 1e9, 1),
            "workload": f"the headline step ({args.layers} layers) with ffn_down's Q8_K input "
                        + ("SwiGLU(gate, up) fused into its quantizer" if other == "swiglu" else "synthetic")}
        log(f"  decode step, ffn_down input {other}: {ms2:.4f} ms/step")
    if not args.no_secondary:
        def gus(launch, n, reps=5):
            return graph_us(torch, launch, n, reps)

        def copies(quant, rows, cols, seed):
            data = synth.gguf_weights(quant, rows, cols, seed=seed)
            copies.data = data
            n = max(4, int(600e6 // data.nbytes) + 1)
            return [jk.Weight(jk.TensorView(f"w{i}", quant, (rows, cols), data), rows, cols) for i in range(n)]

        def hbm_line(name, bytes_, us, note):
            gbs = bytes_ / (us * 1e-6) / 1e9
            cu = ceiling_us(bytes_)
            secondary[name] = {"us": round(us, 3), "bytes": int(bytes_), "gbs": round(gbs, 1),
                               "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4), "bound": "hbm",
                               "stream_read_us": round(cu, 3), "frac_of_stream_read": round(cu / us, 4),
                               "workload": note}
            log(f"  {name:28s} {us:8.2f} us  {gbs:7.1f} GB/s  ({100 * cu / us:.0f}% of a plain read's "
                f"{cu:.2f} us)  {note}")

        log("other kernels of the path:")
        # C1, C2: quant_q8 GEMV with caller Q8_0 blocks
        for name, quant, rows, cols in (("gemv_q4_0_q8_0 C1", jk.Q4_0, 4096, 4096),
                                        ("gemv_q8_0_q8_0 C2", jk.Q8_0, 11008, 4096)):
            ws = copies(quant, rows, cols, 500 + quant)
            xq = torch.empty(cols // 32 * jk.BLOCK_Q8_0.itemsize, dtype=torch.uint8, device=dev)
            jk.dev_quantize_row_q8_0(acts["x"], cols, xq, cols // 32)
            y = torch.empty(rows, dtype=torch.float32, device=dev)
            us = gus(lambda i, st: jk.dev_gemv_q8(ws[i % len(ws)], xq, cols // 32, y, rows, st), len(ws))
            b = gemv_bytes_q80(quant, rows, cols, jk)
            hbm_line(name, b, us, f"{rows}x{cols}, Q8_0 activation blocks")
            cpu_jobs.append(("gemv", name, quant, rows, cols, copies.data, acts["x"].cpu().numpy(), b))
            for w in ws:
                w.free()
        # Repacked GEMV (the m <= 2 route of the repacked GEMM, repack.rs:2892): one token's
        # QuantizedActQ8 against the block-scaled weights, at the C1 shape and the C3 gate and
        # down shapes
        for name, quant, rows, cols in (("gemv_repacked Q8_0 4096x4096 M=1", jk.Q8_0, 4096, 4096),
                                        ("gemv_repacked Q4_0 4096x4096 M=1", jk.Q4_0, 4096, 4096),
                                        ("gemv_repacked Q4_K 14336x4096 M=1", jk.Q4_K, 14336, 4096),
                                        ("gemv_repacked Q5_K 14336x4096 M=1", jk.Q5_K, 14336, 4096),
                                        ("gemv_repacked Q6_K 4096x14336 M=1", jk.Q6_K, 4096, 14336)):
            ws = copies(quant, rows, cols, 550 + quant)
            need = jk.act_q8_bytes(1, cols)
            store = torch.empty(need, dtype=torch.uint8, device=dev)
            act1 = jk.act_q8_bind(store, need, 1, cols)
            jk.dev_quantize_act_q8(acts["x" if cols == 4096 else "h"], 1, cols, act1)
            y = torch.empty(rows, dtype=torch.float32, device=dev)
            us = gus(lambda i, st: jk.dev_gemv_repacked(ws[i % len(ws)], act1, y, rows, 0, rows, st), len(ws))
            b = rows * (cols // jk.BLOCK_ELEMENTS[quant]) * jk.BLOCK_BYTES[quant] + need + 4 * rows
            hbm_line(name, b, us, f"{rows}x{cols}, one token's QuantizedActQ8")

            def mk(O, quant=quant, rows=rows, cols=cols, data=copies.data, b=b,
                   x1=acts["x" if cols == 4096 else "h"].cpu().numpy()[None, :]):
                q, sc, mn, cps = O.repack_logical(quant, (rows, cols), data, rows, cols)
                a1, R = O.ActQ8(x1, 1, cols), 512
                return [(lambda r0=r0: O.gemm_logical_rows(q, sc, mn, cps, cols, a1, 0, 1, r0, min(rows, r0 + R)),
                         b * (min(rows, r0 + R) - r0) / rows) for r0 in range(0, rows, R)]
            cpu_slices(name, mk, "GB/s", 1e9, "row slices of the repacked GEMV (the load-time repack not timed)")
            for w in ws:
                w.free()
        # Q5_0 / Q5_K / TQ1_0 quant_q8 GEMV with caller blocks (GGUF bytes; TQ1_0 streams its
        # 66-byte device blocks, 22% more than the 54 GGUF bytes counted here)
        for name, quant, rows, cols in (("gemv_q5_0_q8_0 4096x4096", jk.Q5_0, 4096, 4096),
                                        ("gemv_q5_k_q8_k 14336x4096", jk.Q5_K, 14336, 4096),
                                        ("gemv_q5_k_q8_k 4096x14336", jk.Q5_K, 4096, 14336),
                                        ("gemv_tq1_0_q8_k 6912x2560", jk.TQ1_0, 6912, 2560)):
            ws = copies(quant, rows, cols, 800 + quant)
            small = quant in jk.Q8_0_ACT
            be = 32 if small else 256
            bsz = (jk.BLOCK_Q8_0 if small else jk.BLOCK_Q8K).itemsize
            xq = torch.empty(cols // be * bsz, dtype=torch.uint8, device=dev)
            xin = torch.randn(cols, generator=gen).to(dev)
            if small:
                jk.dev_quantize_row_q8_0(xin, cols, xq, cols // 32)
            else:
                jk.dev_quantize_row_q8_k(xin, cols, xq, cols // 256)
            y = torch.empty(rows, dtype=torch.float32, device=dev)
            us = gus(lambda i, st: jk.dev_gemv_q8(ws[i % len(ws)], xq, cols // be, y, rows, st), len(ws))
            b = (gemv_bytes_q80 if small else gemv_bytes)(quant, rows, cols, jk)
            hbm_line(name, b, us, f"{rows}x{cols}, {'Q8_0' if small else 'Q8_K'} activation blocks")

            def mk(O, quant=quant, rows=rows, cols=cols, data=copies.data, b=b, small=small, xh=xin.cpu().numpy()):
                xb, R = (O.quantize_row_q8_0 if small else O.quantize_row_q8_k)(xh), 512
                return [(lambda r0=r0: O.gemv_rows(quant, data, rows, cols, xb, r0, min(rows, r0 + R)),
                         b * (min(rows, r0 + R) - r0) / rows) for r0 in range(0, rows, R)]
            cpu_slices(name, mk, "GB/s", 1e9, "row slices of the GEMV")
            for w in ws:
                w.free()
        # A8: f32-activation vec_dot (dequantize x f32 dot) at the Q4_K attn shape and Q6_K down
        for name, quant, rows, cols, xa in (("vec_dot_q4_k_m f32", jk.Q4_K, 4096, 4096, "x"),
                                            ("vec_dot_q6_k f32", jk.Q6_K, 4096, 14336, "h")):
            ws = copies(quant, rows, cols, 600 + quant)
            y = torch.empty(rows, dtype=torch.float32, device=dev)
            us = gus(lambda i, st: jk.dev_vec_dot_f32(ws[i % len(ws)], acts[xa], cols, y, rows, st), len(ws))
            b = rows * (cols // jk.BLOCK_ELEMENTS[quant]) * jk.BLOCK_BYTES[quant] + 4 * cols + 4 * rows
            hbm_line(name, b, us, f"{rows}x{cols}, f32 activation")

            def mk(O, quant=quant, rows=rows, cols=cols, data=copies.data, b=b, xh=acts[xa].cpu().numpy()):
                R = 256
                return [(lambda r0=r0: O.vec_dot_f32(quant, (min(rows, r0 + R) - r0, cols),
                                                     rows_of(data, quant, r0, min(rows, r0 + R), cols), xh,
                                                     min(rows, r0 + R) - r0),
                         b * (min(rows, r0 + R) - r0) / rows) for r0 in range(0, rows, R)]
            cpu_slices(name, mk, "GB/s", 1e9, "row slices of the f32 vec_dot")
            cpu_jobs.append(("same", name.replace(" f32", " f32 tolerance"), name))
            us = gus(lambda i, st: jk.dev_vec_dot_f32_tol(ws[i % len(ws)], acts[xa], cols, y, rows, st), len(ws))
            hbm_line(name.replace(" f32", " f32 tolerance"), b, us,
                     f"{rows}x{cols}, f32 activation, within 1e-5 of the output's L2 norm (four FMA accumulators "
                     "a block; rows of up to 32 blocks: each block over four waves)")
            for w in ws:
                w.free()
        # C5: ternary GEMV (Q8_K caller blocks) and BitLinear at batch 1 and 128
        for quant, qname in ((jk.TQ2_0, "tq2_0"), (jk.I2_S, "i2_s"), (jk.TQ1_0, "tq1_0")):
            for rows, cols in ((6912, 2560), (2560, 6912)):
                ws = copies(quant, rows, cols, 700 + rows)
                wbytes = rows * (cols // jk.BLOCK_ELEMENTS[quant]) * jk.BLOCK_BYTES[quant]
                if quant == jk.TQ2_0:
                    xq = torch.empty(cols // 256 * jk.BLOCK_Q8K.itemsize, dtype=torch.uint8, device=dev)
                    xin = torch.randn(cols, generator=gen).to(dev)
                    jk.dev_quantize_row_q8_k(xin, cols, xq, cols // 256)
                    y = torch.empty(rows, dtype=torch.float32, device=dev)
                    us = gus(lambda i, st: jk.dev_gemv_q8(ws[i % len(ws)], xq, cols // 256, y, rows, st), len(ws))
                    hbm_line(f"gemv_tq2_0_q8_k {rows}x{cols}", wbytes + cols // 256 * 292 + 4 * rows, us,
                             "C5, Q8_K activation blocks")

                    def mk(O, rows=rows, cols=cols, data=copies.data, b=wbytes + cols // 256 * 292 + 4 * rows,
                           xh=xin.cpu().numpy()):
                        xb, R = O.quantize_row_q8_k(xh), 512
                        return [(lambda r0=r0: O.gemv_rows(jk.TQ2_0, data, rows, cols, xb, r0, min(rows, r0 + R)),
                                 b * (min(rows, r0 + R) - r0) / rows) for r0 in range(0, rows, R)]
                    cpu_slices(f"gemv_tq2_0_q8_k {rows}x{cols}", mk, "GB/s", 1e9, "row slices of the GEMV")
                for m in (1, 128):
                    xin = torch.randn(m, cols, generator=gen).to(dev)
                    aq = torch.empty(m * cols, dtype=torch.int8, device=dev)
                    asc = torch.empty(m, dtype=torch.float32, device=dev)
                    jk.dev_quantize_absmax_i8(xin, m, cols, aq, asc)
                    y = torch.empty(m * rows, dtype=torch.float32, device=dev)
                    us = gus(lambda i, st: jk.dev_bitlinear_i8(ws[i % len(ws)], aq, asc, m, cols, y, m * rows, st),
                                  len(ws))
                    b = wbytes + m * (cols + 4) + 4 * m * rows
                    name = f"bitlinear_{qname} {rows}x{cols} M={m}"
                    cpu_jobs.append(("bitlinear", name, quant, rows, cols, copies.data, aq.cpu().numpy(),
                                     asc.cpu().numpy(), m, b))
                    if m == 1:
                        hbm_line(name, b, us, "C5, per-token absmax i8 activation")
                    else:
                        tops = 2.0 * m * rows * cols / (us * 1e-6) / 1e12
                        secondary[name] = {"us": round(us, 3), "tops": round(tops, 2),
                                           "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4),
                                           "gbs": round(b / (us * 1e-6) / 1e9, 1), "bound": "ridge",
                                           "kernel": jk.bitlinear_plan(ws[0], aq, m),
                                           "workload": "C5 at 128 tokens (AI 537-684 op/B, near the ridge)"}
                        log(f"  {name:28s} {us:8.2f} us  {tops:7.2f} TOPS")
                        # tolerance mode (jk_bitlinear_i8_tol: the per-block addends summed in any order)
                        us = gus(lambda i, st: jk.dev_bitlinear_i8_tol(ws[i % len(ws)], aq, asc, m, cols, y, m * rows,
                                                                       st), len(ws))
                        tops = 2.0 * m * rows * cols / (us * 1e-6) / 1e12
                        tname = name.replace("bitlinear_", "bitlinear_tol_")
                        secondary[tname] = {"us": round(us, 3), "tops": round(tops, 2),
                                            "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4),
                                            "gbs": round(b / (us * 1e-6) / 1e9, 1), "bound": "ridge",
                                            "kernel": jk.bitlinear_plan(ws[0], aq, m, tolerance=True),
                                            "workload": "C5 at 128 tokens, outputs within 1e-5 of each token's "
                                                        "output-row L2 norm of the reference's block-order sum"}
                        log(f"  {tname:28s} {us:8.2f} us  {tops:7.2f} TOPS")
                for w in ws:
                    w.free()
        # Repacked GEMM of every other weight format at the prefill shape (14336x4096, 512
        # tokens; the activation quantized once beforehand), kernel-only, graph-timed over weight
        # copies of >= 600 MB in all (beyond the 256 MB Infinity Cache: every launch streams its
        # weights from HBM)
        M, N, K = 512, 14336, 4096
        xin = torch.randn(M, K, generator=gen).to(dev)
        need = jk.act_q8_bytes(M, K)
        store = torch.empty(need, dtype=torch.uint8, device=dev)
        act = jk.act_q8_bind(store, need, M, K)
        jk.dev_quantize_act_q8(xin, M, K, act)
        y = torch.empty(M * N, dtype=torch.float32, device=dev)
        for quant in (jk.Q4_0, jk.Q4_1, jk.Q5_0, jk.Q5_1, jk.IQ4_NL, jk.Q4_K, jk.Q5_K, jk.Q6_K, jk.Q2_K, jk.Q3_K,
                      jk.TQ1_0):
            ws = copies(quant, N, K, 900 + quant)
            us = gus(lambda i, st: jk.dev_gemm_repacked(ws[i % len(ws)], act, y, M * N, 0, N, st), len(ws))
            tops = 2.0 * M * N * K / (us * 1e-6) / 1e12
            name = f"gemm_repacked {jk.QUANT_NAMES[quant]} M=512"
            secondary[name] = {"us": round(us, 3), "tops": round(tops, 2), "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4),
                               "bound": "mfma", "workload": f"{N}x{K} weights x {M} tokens, kernel only"}

            def mk(O, quant=quant, data=copies.data, xh=xin.cpu().numpy(), M=M, N=N, K=K):
                q, sc, mn, cps = O.repack_logical(quant, (N, K), data, N, K)
                ga, R = O.ActQ8(xh, M, K), 64
                return [(lambda r0=r0: O.gemm_logical_rows(q, sc, mn, cps, K, ga, 0, M, r0, min(N, r0 + R)),
                         2.0 * M * (min(N, r0 + R) - r0) * K) for r0 in range(0, N, R)]
            cpu_slices(name, mk, "TOPS", 1e12, f"slices of 64 weight rows x {M} tokens (the load-time repack not timed)")
            cpu_jobs.append(("same", f"gemm_repacked_tol {jk.QUANT_NAMES[quant]} M=512", name))
            log(f"  {name:28s} {us:8.2f} us  {tops:7.2f} TOPS")
            if quant in (jk.Q4_K, jk.Q6_K, jk.Q3_K):  # tolerance mode of the K-quant prefill formats
                us = gus(lambda i, st: jk.dev_gemm_repacked_tol(ws[i % len(ws)], act, y, M * N, 0, N, st), len(ws))
                tops = 2.0 * M * N * K / (us * 1e-6) / 1e12
                name = f"gemm_repacked_tol {jk.QUANT_NAMES[quant]} M=512"
                secondary[name] = {"us": round(us, 3), "tops": round(tops, 2),
                                   "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4), "bound": "mfma",
                                   "workload": f"{N}x{K} weights x {M} tokens, kernel only, outputs within 1e-5 of "
                                               "each token's output-row L2 norm of the bit-exact recipe"}
                log(f"  {name:28s} {us:8.2f} us  {tops:7.2f} TOPS")
            for w in ws:
                w.free()
        del xin, store, y
        # The plain int8 GEMM (gemm_i8_vector: C = A * B^T of row-major i8, exact i32) at the same
        # shape, B rotating over 11 device copies (646 MB)
        a_host = torch.randint(-128, 128, (M * K,), dtype=torch.int8, generator=gen)
        b_host = torch.randint(-128, 128, (N * K,), dtype=torch.int8, generator=gen)
        ai8 = a_host.to(dev)
        bi8 = [b_host.to(dev) for _ in range(11)]
        ci8 = torch.empty(M * N, dtype=torch.int32, device=dev)
        us = gus(lambda i, st: jk.dev_gemm_i8(ai8, M * K, M, bi8[i % len(bi8)], N * K, 0, N, K, ci8, M * N, st),
                 len(bi8))
        tops = 2.0 * M * N * K / (us * 1e-6) / 1e12
        name = f"gemm_i8 {M}x{N}x{K}"
        secondary[name] = {"us": round(us, 3), "tops": round(tops, 2), "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4),
                           "bound": "mfma", "workload": f"C = A * B^T, A {M}x{K} and B {N}x{K} row-major i8, exact i32 "
                                                        "outputs (gemm_i8_vector), kernel only"}
        log(f"  {name:28s} {us:8.2f} us  {tops:7.2f} TOPS")
        cpu_jobs.append(("gemm_i8", name, a_host.numpy(), b_host.numpy(), M, N, K))
        del ai8, bi8, ci8
        # f32-activation vec_dot of the other K-quants at the 4096x4096 attention shape
        for quant in (jk.Q5_K, jk.Q2_K, jk.Q3_K):
            rows, cols = 4096, 4096
            ws = copies(quant, rows, cols, 950 + quant)
            y = torch.empty(rows, dtype=torch.float32, device=dev)
            us = gus(lambda i, st: jk.dev_vec_dot_f32(ws[i % len(ws)], acts["x"], cols, y, rows, st), len(ws))
            b = rows * (cols // jk.BLOCK_ELEMENTS[quant]) * jk.BLOCK_BYTES[quant] + 4 * cols + 4 * rows
            hbm_line(f"vec_dot_{jk.QUANT_NAMES[quant].lower()} f32", b, us, f"{rows}x{cols}, f32 activation")

            def mk(O, quant=quant, rows=rows, cols=cols, data=copies.data, b=b, xh=acts["x"].cpu().numpy()):
                R = 256
                return [(lambda r0=r0: O.vec_dot_f32(quant, (min(rows, r0 + R) - r0, cols),
                                                     rows_of(data, quant, r0, min(rows, r0 + R), cols), xh,
                                                     min(rows, r0 + R) - r0),
                         b * (min(rows, r0 + R) - r0) / rows) for r0 in range(0, rows, R)]
            cpu_slices(f"vec_dot_{jk.QUANT_NAMES[quant].lower()} f32", mk, "GB/s", 1e9, "row slices of the f32 vec_dot")
            for w in ws:
                w.free()
        # Greedy lm_head: Q6_K 128256 x 4096 GEMV with argmax_f32 fused into the launch, against
        # the GEMV followed by a separate argmax launch (the logits written and read back)
        rows, cols = 128256, 4096
        ws_lm = copies(jk.Q6_K, rows, cols, 990)
        xq = torch.empty(cols // 256 * jk.BLOCK_Q8K.itemsize, dtype=torch.uint8, device=dev)
        jk.dev_quantize_row_q8_k(acts["x"], cols, xq, cols // 256)
        y = torch.empty(rows, dtype=torch.float32, device=dev)
        amw = torch.empty(jk.argmax_workspace_bytes(rows), dtype=torch.uint8, device=dev)
        idx = torch.empty(1, dtype=torch.int32, device=dev)
        b = gemv_bytes(jk.Q6_K, rows, cols, jk)
        us = gus(lambda i, st: jk.dev_gemv_q8_argmax(ws_lm[i % len(ws_lm)], xq, None, cols // 256, None, idx, amw, st),
                      len(ws_lm))
        hbm_line("lm_head Q6_K gemv+argmax", b - 4 * rows, us, f"{rows}x{cols}, fused argmax, no logits written")

        def mk(O, rows=rows, cols=cols, data=copies.data, b=b, xh=acts["x"].cpu().numpy()):
            xb, R = O.quantize_row_q8_k(xh), 2048
            return [(lambda r0=r0: O.gemv_rows(jk.Q6_K, data, rows, cols, xb, r0, min(rows, r0 + R)),
                     b * (min(rows, r0 + R) - r0) / rows) for r0 in range(0, rows, R)]
        cpu_slices("lm_head Q6_K gemv, argmax", mk, "GB/s", 1e9, "row slices of the lm_head GEMV (the argmax not timed)")
        cpu_jobs.append(("same", "lm_head Q6_K gemv+argmax", "lm_head Q6_K gemv, argmax"))

        def two(i, st):
            jk.dev_gemv_q8(ws_lm[i % len(ws_lm)], xq, cols // 256, y, rows, st)
            jk.dev_argmax_f32(y, rows, idx, amw, st)

        us = gus(two, len(ws_lm))
        hbm_line("lm_head Q6_K gemv, argmax", b + 4 * rows, us, f"{rows}x{cols}, logits written and re-read")
        for w in ws_lm:
            w.free()
        # Load time: one Llama-3-8B layer's seven matrices (138 MB of GGUF bytes) in a GGUF file
        # (page cache warm), streamed into device handles by jk_gguf_load_weight, against
        # jk_weight_upload from host memory and the oracle's CPU repack of the same tensors (the
        # reference repacks at load time on the host). GB/s of GGUF bytes.
        import tempfile
        sys.path.insert(0, os.path.join(REPO, "tests"))
        from gguf_writer import STR, write_gguf
        mats = [(f"blk.0.{n}.weight", q, [c, r], synth.gguf_weights(q, r, c, seed=700 + i))
                for i, (n, q, r, c) in enumerate(synth.LLAMA3_8B_LAYER)]
        total = sum(d.nbytes for *_, d in mats)
        with tempfile.TemporaryDirectory() as td:
            path = os.path.join(td, "layer.gguf")
            write_gguf(path, mats, [("general.architecture", STR, "llama")])
            g = jk.GGUF(path)
            best_file = best_up = float("inf")
            for _ in range(3):
                t0 = time.perf_counter()
                ws_ = [g.load(name) for name, *_ in mats]
                best_file = min(best_file, time.perf_counter() - t0)
                for w in ws_:
                    w.free()
                t0 = time.perf_counter()
                ws_ = [jk.Weight(jk.TensorView(n, q, ne, d), ne[1], ne[0]) for n, q, ne, d in mats]
                torch.cuda.synchronize()
                best_up = min(best_up, time.perf_counter() - t0)
                for w in ws_:
                    w.free()
            g.close()
        load = {"gguf_bytes": total, "gguf_load_s": round(best_file, 4),
                "gguf_load_gbs": round(total / best_file / 1e9, 2), "upload_from_host_s": round(best_up, 4),
                "upload_from_host_gbs": round(total / best_up / 1e9, 2),
                "workload": "Llama-3-8B layer: Q/K/V/O/gate/up Q4_K, down Q6_K; GGUF file in the page cache"}
        secondary["load_layer_gguf"] = load
        load_mats = mats  # the CPU baseline below times the host repack of the same tensors
        log(f"  load layer from GGUF {best_file * 1e3:.1f} ms ({total / best_file / 1e9:.2f} GB/s), "
            f"upload from host {best_up * 1e3:.1f} ms")
        # Host tier, the reference's slice signature gemv_q4_k_q8_k(out, &TensorView, &[BlockQ8K])
        # over the 14336 x 4096 gate matrix in host memory: the first call uploads the weight (33
        # MB over PCIe), later calls reuse the resident copy and move only the 4.7 KB of activation
        # blocks and the 57 KB of outputs; wall clock per call, synchronous.
        rows, cols = 14336, 4096
        hraw = synth.gguf_weights(jk.Q4_K, rows, cols, seed=1200)
        hv = jk.TensorView("blk.0.ffn_gate.weight", jk.Q4_K, [cols, rows], hraw)
        hxq = jk.quantize_row_q8_k(synth.activations(cols, seed=1201))
        hout = np.zeros(rows, np.float32)
        jk.host_cache_set_limit(16 << 30)  # weight residency (opt in)
        s0 = jk.host_stats()
        t0 = time.perf_counter()
        jk.gemv_q4_k_q8_k(hout, hv, hxq)
        first_ms = (time.perf_counter() - t0) * 1e3
        s1 = jk.host_stats()
        warm = []
        for _ in range(200):
            t0 = time.perf_counter()
            jk.gemv_q4_k_q8_k(hout, hv, hxq)
            warm.append(time.perf_counter() - t0)
        s2 = jk.host_stats()
        warm_us = float(np.median(warm)) * 1e6
        secondary["host_tier gemv_q4_k_q8_k 14336x4096"] = {
            "first_call_ms": round(first_ms, 3), "us_per_call_warm": round(warm_us, 2),
            "uploads_first": s1["weight_uploads"] - s0["weight_uploads"],
            "uploads_warm": s2["weight_uploads"] - s1["weight_uploads"],
            "device_allocs_warm": s2["device_allocs"] - s1["device_allocs"],
            "workload": "host-memory TensorView + BlockQ8K slice, synchronous (copy in, GEMV, copy out), weight "
                        "residency on; median of 200 warm calls, wall clock, PCIe-inclusive"}
        log(f"  host tier gemv_q4_k_q8_k 14336x4096: first call {first_ms:.2f} ms, warm {warm_us:.1f} us/call "
            f"({s2['weight_uploads'] - s1['weight_uploads']} uploads, "
            f"{s2['device_allocs'] - s1['device_allocs']} device allocations over 200 warm calls)")
        jk.host_cache_invalidate(hv)
        jk.host_cache_set_limit(0)
        cpu_jobs.append(("percall", "host_tier gemv_q4_k_q8_k 14336x4096",
                         lambda O, d=hraw, rows=rows, cols=cols: (
                             lambda xb=O.quantize_row_q8_k(synth.activations(cols, seed=1201)):
                             (lambda: O.gemv_q8(jk.Q4_K, (rows, cols), d, xb, rows)))(),
                         "gemv_q4_k_q8_k over the same host slices"))
        del hv
        # A3-A5: quantizers (one activation row of the decode step; the prefill activation)
        yq = torch.empty(56 * jk.BLOCK_Q8K.itemsize, dtype=torch.uint8, device=dev)
        us = gus(lambda i, st: jk.dev_quantize_row_q8_k(acts["h"], 14336, yq, 56, st), 64)
        secondary["quantize_row_q8_k 14336"] = {"us": round(us, 3), "bound": "latency",
                                                "workload": "ffn_down input, 56 blocks"}
        cpu_jobs.append(("percall", "quantize_row_q8_k 14336",
                         lambda O, xh=acts["h"].cpu().numpy(): (lambda: O.quantize_row_q8_k(xh)),
                         "quantize_row_q8_k of the same 14336 values"))
        log(f"  {'quantize_row_q8_k 14336':28s} {us:8.2f} us")
        M, K = 512, 4096
        xin = torch.randn(M, K, generator=gen).to(dev)
        need = jk.act_q8_bytes(M, K)
        store = torch.empty(need, dtype=torch.uint8, device=dev)
        act = jk.act_q8_bind(store, need, M, K)
        us = gus(lambda i, st: jk.dev_quantize_act_q8(xin, M, K, act, st), 32)
        b = M * K * 4 + M * K + M * (K // 32) * 8
        hbm_line("quantize_act_q8 512x4096", b, us, "QuantizedActQ8::quantize_into for the prefill GEMM")

        def mk(O, xh=xin.cpu().numpy(), M=M, K=K, b=b):
            R = 32
            return [(lambda t0=t0: O.ActQ8(xh[t0:t0 + R], R, K), b * R / M) for t0 in range(0, M, R)]
        cpu_slices("quantize_act_q8 512x4096", mk, "GB/s", 1e9, "32-token slices of the same quantization")
        del xin, store

    del rd_buf
    # ------------------------------------------------------------ CPU baseline (oracle)
    cpu = cpu_all = None
    if args.cpu_seconds > 0:
        sys.path.insert(0, os.path.join(REPO, "oracle"))
        import oracle as O

        if "load_layer_gguf" in secondary:  # load time on the host: the reference's CPU repack
            t0 = time.perf_counter()
            for n, q, ne, d in load_mats:
                O.repack_logical(q, ne, d, ne[1], ne[0])
            el = time.perf_counter() - t0
            secondary["load_layer_gguf"].update({
                "cpu_repack_s": round(el, 3),
                "cpu_repack_gbs": round(secondary["load_layer_gguf"]["gguf_bytes"] / el / 1e9, 3),
                "cpu_repack_kind": "port: the oracle's C restatement of the reference's repack, 1 thread"})
            log(f"cpu repack of the layer: {el * 1e3:.0f} ms")

        hl = host_layers[0]
        x = synth.activations(4096, seed=5)
        h = synth.activations(14336, seed=6)
        xq, hq = O.quantize_row_q8_k(x), O.quantize_row_q8_k(h)
        reps = 0
        t0 = time.perf_counter()
        while True:
            for name, quant, rows, cols, data in hl:
                O.gemv_q8(quant, (rows, cols), data, hq if cols == 14336 else xq, rows)
            reps += 1
            el = time.perf_counter() - t0
            if el >= args.cpu_seconds:
                break
        cpu_gbs = layer_bytes * reps / el / 1e9
        cpu = {"value": round(cpu_gbs, 3), "unit": "GB/s", "cores": 1, "kind": "port",
               "sample": f"{reps} passes over one Llama-3-8B layer's 7 GEMVs ({layer_bytes} B) in {el:.1f} s, "
                         "oracle C restatement of the scalar fallback, -O3 -march=x86-64, 1 thread",
               "cpu_model": _cpu_model(), "host_cpus": os.cpu_count()}
        log(f"cpu baseline: {cpu_gbs:.3f} GB/s ({reps} layer passes)")

        # Second labelled run: every matrix's rows partitioned over the host's cores (the
        # reference's row_range APIs), one thread per slice over the same C restatement
        # (ctypes releases the GIL during each call).
        from concurrent.futures import ThreadPoolExecutor
        ncores = max(1, min(16, os.cpu_count() or 1))
        slices = []
        for name, quant, rows, cols, data in hl:
            xb = hq if cols == 14336 else xq
            step = (rows + ncores - 1) // ncores
            slices += [(quant, data, rows, cols, xb, r0, min(rows, r0 + step)) for r0 in range(0, rows, step)]
        with ThreadPoolExecutor(ncores) as ex:
            reps = 0
            t0 = time.perf_counter()
            while True:
                list(ex.map(lambda j: O.gemv_rows(*j), slices))
                reps += 1
                el = time.perf_counter() - t0
                if el >= max(2.0, args.cpu_seconds / 2):
                    break
        cpu_all_gbs = layer_bytes * reps / el / 1e9
        cpu_all = {"value": round(cpu_all_gbs, 3), "unit": "GB/s", "cores": ncores, "kind": "port",
                   "sample": f"{reps} passes over the same layer in {el:.1f} s, rows of each matrix split over "
                             f"{ncores} threads (row_range partitioning)"}
        log(f"cpu baseline, {ncores} threads: {cpu_all_gbs:.3f} GB/s ({reps} layer passes)")

        # The same scalar restatement beside every other GPU figure: the prefill GEMM (TOPS over the
        # 64-row x all-token slices done; the load-time repack is not timed, as in the reference,
        # which repacks once), the C1 / C2 GEMVs and the C5 BitLinear lines. One thread, then the
        # rows (GEMV, GEMM, one-token BitLinear) or tokens (128-token BitLinear) split over the cores.
        def attach(target, unit, scale, one, alln, what):
            (u1, el1, c1), (un, eln, cn) = one, alln
            target["cpu_baseline"] = {"value": round(u1 / el1 / scale, 4), "unit": unit, "cores": 1, "kind": "port",
                                      "sample": f"{c1} {what} in {el1:.1f} s, oracle C restatement of the scalar "
                                                "fallback, -O3 -march=x86-64, 1 thread"}
            target["cpu_baseline_all_cores"] = {"value": round(un / eln / scale, 4), "unit": unit, "cores": ncores,
                                                "kind": "port", "sample": f"{cn} {what} in {eln:.1f} s on {ncores} threads"}
            log(f"cpu baseline {unit}: {u1 / el1 / scale:.4g} (1 thread), {un / eln / scale:.4g} ({ncores} threads)")

        if gemm_host is not None and (gemm is not None or gemm_exact is not None):
            gd, gxh, M, N, K = gemm_host
            q, sc, mn, cps = O.repack_logical(jk.Q8_0, (N, K), gd, N, K)
            gact = O.ActQ8(gxh, M, K)
            R = 64
            sl = [(lambda r0=r0: O.gemm_logical_rows(q, sc, mn, cps, K, gact, 0, M, r0, min(N, r0 + R)),
                   2.0 * M * (min(N, r0 + R) - r0) * K) for r0 in range(0, N, R)]
            gsec = max(2.0, args.cpu_seconds)
            res = (cpu_rate(sl, gsec, 1), cpu_rate(sl, max(1.0, gsec / 3), ncores))
            for line in (gemm, gemm_exact):
                if line is not None:
                    attach(line, "TOPS", 1e12, *res, f"slices of {R} weight rows x {M} tokens of the same GEMM")
            del q, sc, mn, gact
        for job in cpu_jobs:
            sec = secondary.get(job[1])
            if sec is None or job[0] == "same":
                continue
            if job[0] == "slices":
                _, name, make, unit, scale, what = job
                attach(sec, unit, scale, *(lambda sl: (cpu_rate(sl, 1.5, 1), cpu_rate(sl, 0.75, ncores)))(make(O)), what)
                continue
            if job[0] == "percall":
                _, name, make, what = job
                fn = make(O)
                calls, t0 = 0, time.perf_counter()
                while time.perf_counter() - t0 < 1.0:
                    fn()
                    calls += 1
                el = time.perf_counter() - t0
                sec["cpu_baseline"] = {"value": round(el / calls * 1e6, 2), "unit": "us per call", "cores": 1,
                                       "kind": "port", "sample": f"{calls} calls of {what} in {el:.1f} s, oracle C "
                                                                 "restatement of the scalar fallback, 1 thread"}
                log(f"cpu baseline {name}: {el / calls * 1e6:.1f} us per call")
                continue
            if job[0] == "gemm_i8":
                _, name, ah, bh, M, N, K = job
                R = 64
                sl = [(lambda r0=r0: O.gemm_i8_vector(ah, M, bh, r0, min(N, r0 + R), K), 2.0 * M * (min(N, r0 + R) - r0) * K)
                      for r0 in range(0, N, R)]
                attach(sec, "TOPS", 1e12, cpu_rate(sl, 2.0, 1), cpu_rate(sl, 1.0, ncores),
                       f"slices of {R} rows of B x {M} rows of A of the same product")
            elif job[0] == "gemv":
                _, name, quant, rows, cols, data, xh, b = job
                xb = O.quantize_row_q8_0(xh)
                one = [(lambda: O.gemv_q8(quant, (rows, cols), data, xb, rows), b)]
                step = -(-rows // ncores)
                par = [(lambda r0=r0: O.gemv_rows(quant, data, rows, cols, xb, r0, min(rows, r0 + step)),
                        b * (min(rows, r0 + step) - r0) / rows) for r0 in range(0, rows, step)]
                attach(sec, "GB/s", 1e9, cpu_rate(one, 2.0, 1), cpu_rate(par, 1.0, ncores),
                       f"GEMVs (or row slices) of the {rows}x{cols} matrix")
            else:
                _, name, quant, rows, cols, data, aqh, asch, m, b = job
                ops = 2.0 * rows * cols
                if m == 1:  # rows split over the cores: row-range views of the same tensor
                    one = [(lambda: O.bitlinear_i8(quant, (rows, cols), data, aqh, float(asch[0]), rows), b)]
                    rb = cols // jk.BLOCK_ELEMENTS[quant] * jk.BLOCK_BYTES[quant]
                    tail = data[rows * rb:]  # the I2_S tensor trailer (empty for TQ2_0)
                    step = -(-rows // ncores)
                    par = []
                    for r0 in range(0, rows, step):
                        r1 = min(rows, r0 + step)
                        part = np.concatenate([data[r0 * rb:r1 * rb], tail])
                        par.append((lambda part=part, n=r1 - r0: O.bitlinear_i8(quant, (n, cols), part, aqh,
                                                                                float(asch[0]), n), b * (r1 - r0) / rows))
                    attach(sec, "GB/s", 1e9, cpu_rate(one, 2.0, 1), cpu_rate(par, 1.0, ncores),
                           f"one-token BitLinear products (or row slices) of the {rows}x{cols} matrix")
                else:  # one token per call
                    aq2 = aqh.reshape(m, cols)
                    sl = [(lambda t=t: O.bitlinear_i8(quant, (rows, cols), data, aq2[t], float(asch[t]), rows), ops)
                          for t in range(m)]
                    attach(sec, "TOPS", 1e12, cpu_rate(sl, 2.0, 1), cpu_rate(sl, 1.0, ncores),
                           f"tokens of the {m}-token BitLinear over the {rows}x{cols} matrix")
                    tsec = secondary.get(name.replace("bitlinear_", "bitlinear_tol_"))
                    if tsec is not None:  # the same reference computation beside the tolerance-mode line
                        tsec["cpu_baseline"] = sec["cpu_baseline"]
                        tsec["cpu_baseline_all_cores"] = sec["cpu_baseline_all_cores"]
        # lines whose reference computation is another line's (tolerance modes, the fused argmax, the
        # synthetic-input decode step) carry that line's CPU figures
        for job in cpu_jobs:
            if job[0] == "same" and job[1] in secondary and "cpu_baseline" in secondary.get(job[2], {}):
                for key in ("cpu_baseline", "cpu_baseline_all_cores"):
                    if key in secondary[job[2]]:
                        secondary[job[1]][key] = secondary[job[2]][key]
        for k, v in secondary.items():
            if k.startswith("decode step") and isinstance(v, dict):
                v["cpu_baseline"], v["cpu_baseline_all_cores"] = cpu, cpu_all

    rec = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "i8", "data": "synthetic",
        "config": {"workload": f"Llama-3-8B decode GEMVs, batch 1, {args.layers} layers: Q/K/V/O/gate/up Q4_K, "
                               "down Q6_K, activations Q8_K (quantized on device each layer)",
                   "layers": args.layers, "hidden": 4096, "ffn": 14336, "kv_rows": 1024,
                   "bytes_per_step": step_bytes, "launch": "eager" if graph is None else "hip_graph",
                   "launches_per_layer": 4 + (args.down == "split"), "down_activation": args.down,
                   "ffn_down_input": "SwiGLU(gate, up) fused into its Q8_K quantizer" if args.ffn == "swiglu"
                   else "synthetic",
                   "parallelism": "single_gpu"},
        "frac_of_hbm_peak": round(value / HBM_PEAK_GBS, 4),
        "decode_tok_s_equiv": round(1e3 / ms_per_step * args.layers / 32, 1),
        "roofline": roofline, "per_stage": per_stage, "stream_read_ceiling": stream_ceiling,
        "gemm_q8_0": gemm, "gemm_q8_0_sweep": sweep,
        "gemm_q8_0_bit_exact": gemm_exact, "gemm_q8_0_bit_exact_sweep": sweep_exact,
        "secondary": secondary,
        "cpu_baseline": cpu,
        "cpu_baseline_all_cores": cpu_all,
    }
    print(json.dumps(rec), flush=True)
    return 0


def profile_loop(which: str) -> int:
    """Eager launches of one workload's kernels (20 per configuration and mode), for counter passes."""
    import torch

    import jk
    from jk import synth

    jk.lib()
    jk.init(0)
    gen = torch.Generator(device="cpu").manual_seed(99)
    n = 20
    if which == "bitlinear":
        for quant in (jk.TQ2_0, jk.I2_S):
            for rows, cols in ((6912, 2560), (2560, 6912)):
                m = 128
                w = jk.Weight(jk.TensorView("w", quant, (rows, cols), synth.gguf_weights(quant, rows, cols, seed=7)),
                              rows, cols)
                xin = torch.randn(m, cols, generator=gen).cuda()
                aq = torch.empty(m * cols, dtype=torch.int8, device="cuda")
                asc = torch.empty(m, dtype=torch.float32, device="cuda")
                jk.dev_quantize_absmax_i8(xin, m, cols, aq, asc)
                y = torch.empty(m * rows, dtype=torch.float32, device="cuda")
                for fn in (jk.dev_bitlinear_i8, jk.dev_bitlinear_i8_tol):
                    for _ in range(n):
                        fn(w, aq, asc, m, cols, y, m * rows)
                torch.cuda.synchronize()
                w.free()
    elif which == "gemm":
        N, K = 14336, 4096
        w = jk.Weight(jk.TensorView("w", jk.Q8_0, (N, K), synth.gguf_weights(jk.Q8_0, N, K, seed=77)), N, K)
        for M in (512, 64, 128):
            x = torch.randn(M, K, generator=gen).cuda()
            need = jk.act_q8_bytes(M, K)
            st = torch.empty(need, dtype=torch.uint8, device="cuda")
            act = jk.act_q8_bind(st, need, M, K)
            jk.dev_quantize_act_q8(x, M, K, act)
            y = torch.empty(M * N, dtype=torch.float32, device="cuda")
            for fn in (jk.dev_gemm_repacked_tol, jk.dev_gemm_repacked):
                for _ in range(n):
                    fn(w, act, y, M * N, 0, N)
            torch.cuda.synchronize()
        w.free()
    elif which == "decode":
        # the decode step's launches on eight distinct layers (so the weights stream from HBM), in
        # the step's order, then the streaming read of each launch's byte count
        L = 8
        mats = {name: (q, r, c) for name, q, r, c in synth.LLAMA3_8B_LAYER}
        raw = {name: synth.gguf_weights(q, r, c, seed=3 + i) for i, (name, (q, r, c)) in enumerate(mats.items())}
        ws = [{name: jk.Weight(jk.TensorView(name, q, (r, c), raw[name]), r, c) for name, (q, r, c) in mats.items()}
              for _ in range(L)]
        x = torch.randn(4096, generator=gen).cuda()
        outs = {name: torch.empty(r, dtype=torch.float32, device="cuda") for name, (q, r, c) in mats.items()}
        h_q8 = torch.empty(56 * jk.BLOCK_Q8K.itemsize, dtype=torch.uint8, device="cuda")
        groups = (("attn_q", "attn_k", "attn_v"), ("attn_output",), ("ffn_gate", "ffn_up"))
        for i in range(n):
            lw = ws[i % L]
            for names in groups:
                jk.dev_gemv_q8_batch([(lw[nm], None, x, outs[nm], 0, mats[nm][1]) for nm in names])
            jk.dev_quantize_row_q8_k_gated(jk.ACT_SWIGLU, outs["ffn_gate"], outs["ffn_up"], 14336, h_q8, 56)
            jk.dev_gemv_q8_batch([(lw["ffn_down"], h_q8, None, outs["ffn_down"], 0, 4096)])
        torch.cuda.synchronize()
        buf = torch.empty(800_000_000, dtype=torch.uint8, device="cuda")
        sink = torch.zeros(4, dtype=torch.int32, device="cuda")
        for names in groups + (("ffn_down",),):
            nb = sum(gemv_bytes(*mats[nm], jk) for nm in names)
            span = (nb + 65535) // 65536 * 65536
            for i in range(n):
                jk.dev_measure_stream_read(buf.data_ptr() + (i % (buf.numel() // span)) * span, nb, sink)
        torch.cuda.synchronize()
        for lw in ws:
            for w in lw.values():
                w.free()
    else:
        for quant, rows, cols in ((jk.Q4_K, 4096, 4096), (jk.Q6_K, 4096, 14336)):
            w = jk.Weight(jk.TensorView("w", quant, (rows, cols), synth.gguf_weights(quant, rows, cols, seed=8)),
                          rows, cols)
            x = torch.randn(cols, generator=gen).cuda()
            y = torch.empty(rows, dtype=torch.float32, device="cuda")
            for fn in (jk.dev_vec_dot_f32, jk.dev_vec_dot_f32_tol):
                for _ in range(n):
                    fn(w, x, cols, y, rows)
            torch.cuda.synchronize()
            w.free()
    print(json.dumps({"profile_loop": which, "launches_per_configuration_and_mode": n}), flush=True)
    return 0


def cpu_rate(slices, seconds, threads=1):
    """Runs the (callable, work units) slices in order, cyclically, until `seconds` have
    passed: one at a time on one thread, or `threads` at a time on a thread pool (ctypes
    releases the GIL during each oracle call). Returns (units done, elapsed s, calls)."""
    from concurrent.futures import ThreadPoolExecutor

    done, calls, i = 0.0, 0, 0
    t0 = time.perf_counter()
    if threads == 1:
        while True:
            fn, u = slices[i % len(slices)]
            fn()
            done, calls, i = done + u, calls + 1, i + 1
            el = time.perf_counter() - t0
            if el >= seconds:
                return done, el, calls
    with ThreadPoolExecutor(threads) as ex:
        while True:
            batch = [slices[(i + j) % len(slices)] for j in range(threads)]
            list(ex.map(lambda sl: sl[0](), batch))
            done, calls, i = done + sum(u for _, u in batch), calls + threads, i + threads
            el = time.perf_counter() - t0
            if el >= seconds:
                return done, el, calls


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


if __name__ == "__main__":
    sys.exit(main())
