"""bench.py's contract on the CPU: one GPU only, and the HBM traffic figures it reports as
roofline.traffic parse from the committed counter summary and agree with the algorithmic bytes."""
import importlib.util
import os
import subprocess
import sys

import jk
from jk import synth

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def load_bench():
    spec = importlib.util.spec_from_file_location("bench_module", os.path.join(REPO, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)  # defines functions only: main() runs under __name__ == "__main__"
    return mod


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_traffic_lines_match_the_algorithmic_bytes():
    """Every traffic line bench.py reads is present and positive. The decode GEMVs read their weights
    once (HBM bytes within 0-5% above the algorithmic bytes: GGUF weight bytes + Q8_K activation
    blocks + f32 outputs); the Q8_0 GEMM at 512 tokens re-reads weight tiles (1-2x)."""
    bench = load_bench()
    traffic = bench.read_traffic()
    for key in ("ffn_gate_up", "ffn_down", "qkv", "attn_output", "gemm_q8_0_m512_tol", "gemm_q8_0_m512",
                "gemm_q8_0_m2048_tol", "gemm_q8_0_m2048"):
        assert traffic.get(key, 0) > 0, key
    mats = {name: (quant, rows, cols) for name, quant, rows, cols in synth.LLAMA3_8B_LAYER}
    stages = {"ffn_gate_up": ("ffn_gate", "ffn_up"), "ffn_down": ("ffn_down",),
              "qkv": ("attn_q", "attn_k", "attn_v"), "attn_output": ("attn_output",)}
    for stage, names in stages.items():
        algo = sum(bench.gemv_bytes(*mats[n], jk) for n in names)
        assert 1.0 <= traffic[stage] / algo <= 1.05, (stage, traffic[stage], algo)
    m, n, k = 512, 14336, 4096
    unique = n * (k // 32) * 34 + m * k + m * (k // 32) * 4 + m * n * 4  # Q8_0 weights, int8 acts + scales, f32 out
    for key in ("gemm_q8_0_m512_tol", "gemm_q8_0_m512"):
        assert 1.0 <= traffic[key] / unique <= 2.0, (key, traffic[key], unique)
