"""Writes the golden fixtures of this directory: small seeded cases of every entry point.

Inputs follow the reference's own test construction (the LCG generators of
tests/wave4_quant_gemv_and_argmax.rs:31-226, restated in tests/refgen.py); I2_S weights,
which that file does not build, come from the seeded synthetic generator. Expected outputs
are computed by the CPU oracle, whose functions are pinned by the reference's known-answer
tests (tests/test_oracle_kat.py) and by closed-form / float64 properties
(tests/test_oracle_properties.py). The fixtures freeze those outputs so that the GPU tests
check the HIP library against fixed data, and a later change of the oracle shows up as a
fixture mismatch.

Run from the repository root:  python tests/golden/make_golden.py [--all]
(without --all only the missing fixtures are written). Each case is one .npz (no pickled
objects) holding its inputs and expected outputs.
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(REPO, "oracle"))
sys.path.insert(0, os.path.join(REPO, "tests"))
sys.path.insert(0, os.path.join(REPO, "jero-kernels-rvv_amd"))

import oracle as O  # noqa: E402
import refgen as R  # noqa: E402

Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K, TQ1_0, TQ2_0, I2_S = 2, 6, 8, 12, 13, 14, 34, 35, 36
Q4_1, Q5_1, Q2_K, Q3_K, IQ4_NL = 3, 7, 10, 11, 20

# quant -> (LCG weight filler of the reference's tests, weight seed, activation seed)
CASES = {
    Q4_0: (R.fill_q4_0, 0x51, 0x61),
    Q8_0: (R.fill_q8_0, 0x52, 0x62),
    Q4_K: (R.fill_q4_k, 0x53, 0x63),
    Q6_K: (R.fill_q6_k, 0x54, 0x64),
    TQ2_0: (R.fill_tq2_0, 0x55, 0x65),
    Q5_0: (R.fill_q5_0, 0x57, 0x67),
    Q5_K: (R.fill_q5_k, 0x58, 0x68),
    TQ1_0: (R.fill_tq1_0, 0x59, 0x69),
    # formats without a quant_q8 GEMV: the construction of tests/test_repack_gemv_gemm.rs:86-270
    Q4_1: (lambda r, c, s: R.build_synthetic(Q4_1, r, c, s), 0x5A, 0x6A),
    Q5_1: (lambda r, c, s: R.build_synthetic(Q5_1, r, c, s), 0x5B, 0x6B),
    Q2_K: (lambda r, c, s: R.build_synthetic(Q2_K, r, c, s), 0x5C, 0x6C),
    Q3_K: (lambda r, c, s: R.build_synthetic(Q3_K, r, c, s), 0x5D, 0x6D),
    IQ4_NL: (lambda r, c, s: R.build_synthetic(IQ4_NL, r, c, s), 0x5E, 0x6E),
}
NAMES = {Q4_0: "q4_0", Q8_0: "q8_0", Q4_K: "q4_k", Q6_K: "q6_k", TQ2_0: "tq2_0", I2_S: "i2_s", Q5_0: "q5_0",
         Q5_K: "q5_k", TQ1_0: "tq1_0", Q4_1: "q4_1", Q5_1: "q5_1", Q2_K: "q2_k", Q3_K: "q3_k", IQ4_NL: "iq4_nl"}
F32_PATH = {Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K, I2_S, Q4_1, Q5_1, Q2_K, Q3_K, IQ4_NL}  # f32-activation vec_dot
GEMV_PATH = {Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K, TQ1_0, TQ2_0}  # quant_q8 GEMV
Q8_0_ACT = (Q4_0, Q5_0, Q8_0)  # formats whose GEMV takes BlockQ8_0 activations
ROWS, COLS, TOKENS = 8, 512, 3


def weights(quant: int, seed: int) -> np.ndarray:
    if quant == I2_S:
        from jk import synth

        return synth.gguf_weights(I2_S, ROWS, COLS, seed)
    return CASES[quant][0](ROWS, COLS, seed)


def activations(seed: int, n: int) -> np.ndarray:
    return R.gen_activation(n, seed)


def case(quant: int, wseed: int, xseed: int) -> dict:
    w = weights(quant, wseed)
    shape = [ROWS, COLS]
    x = activations(xseed, COLS)
    X = activations(xseed + 1, TOKENS * COLS).reshape(TOKENS, COLS)
    out = {"quant": np.int32(quant), "rows": np.int32(ROWS), "cols": np.int32(COLS), "wseed": np.int64(wseed),
           "xseed": np.int64(xseed), "w": w, "x": x, "X": X}
    out["deq"] = np.stack([O.dequantize_tensor_row(quant, shape, w, r, COLS) for r in range(ROWS)])
    if quant in GEMV_PATH:
        xq = O.quantize_row_q8_0(x) if quant in Q8_0_ACT else O.quantize_row_q8_k(x)
        out["xq"] = xq.view(np.uint8).reshape(-1)
        out["y_gemv"] = O.gemv_q8(quant, shape, w, xq, ROWS)
    if quant != I2_S:
        act = O.ActQ8(X, TOKENS, COLS)
        out["y_gemm"] = O.gemm_repacked(quant, shape, w, ROWS, COLS, act, 0, ROWS)
        out["y_gemm_rows"] = O.gemm_repacked(quant, shape, w, ROWS, COLS, act, 2, 7)
    if quant in F32_PATH:
        out["y_vec_f32"] = O.vec_dot_f32(quant, shape, w, x, ROWS)
    if quant in (TQ1_0, TQ2_0, I2_S):
        a, s = O.quantize_absmax_i8(x)
        out["act_i8"], out["act_scale"] = a, np.float32(s)
        out["y_bitlinear"] = O.bitlinear_i8(quant, shape, w, a, s, ROWS)
    return out


def quantizer_case() -> dict:
    """Quantizers on a row with the sanitized specials: NaN, +-Inf, a subnormal-only block,
    exact ties and a large-magnitude block."""
    x = activations(0x71, 1024).astype(np.float32)
    x[3], x[40], x[77] = np.nan, np.inf, -np.inf
    x[256:288] = np.float32(1e-40)                 # one all-subnormal Q8_0 block
    x[512:520] = np.float32([0.5, -0.5, 1.5, -2.5, 127.0, -127.0, 63.5, -63.5])
    x[768:1024] *= np.float32(3.0e4)
    norm_w = activations(0x72, 1024)
    q, s = O.subln_quantize_absmax_i8(x, norm_w, 1e-5)
    qa, sa = O.quantize_absmax_i8(np.nan_to_num(x, nan=0.0, posinf=0.0, neginf=0.0))
    return {"x": x, "norm_w": norm_w,
            "q8_0": O.quantize_row_q8_0(x).view(np.uint8).reshape(-1),
            "q8_k": O.quantize_row_q8_k(x).view(np.uint8).reshape(-1),
            "subln_q": q, "subln_scale": np.float32(s), "absmax_q": qa, "absmax_scale": np.float32(sa)}


def main() -> None:
    O.build()
    everything = "--all" in sys.argv[1:]
    todo = {f"{NAMES[q]}.npz": (lambda q=q, ws=ws, xs=xs: case(q, ws, xs)) for q, (_, ws, xs) in CASES.items()}
    todo["i2_s.npz"] = lambda: case(I2_S, 0x56, 0x66)
    todo["quantizers.npz"] = quantizer_case
    written = []
    for name, make in todo.items():
        path = os.path.join(HERE, name)
        if everything or not os.path.exists(path):
            np.savez(path, **make())
            written.append(name)
    print("wrote", sorted(written))


if __name__ == "__main__":
    main()
