"""Writes the committed golden fixtures of tests/golden/ from the oracle.

The reference (Mojo) cannot run here and ships no vectors, so these fixtures
freeze the oracle's outputs after the oracle itself was pinned by the
independent checks in tests/test_oracle_*.py; they guard the oracle (and the
GPU path, which is compared with them) against regressions.

    python tests/golden/make_golden.py
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402


def main():
    oracle.build()
    words = {str(s): [f"{int(w):016x}" for w in oracle.rng_words(s, 16)] for s in (0, 1, 2, 3, 4, 5)}
    with open(os.path.join(HERE, "rng_words.json"), "w") as f:
        json.dump({"source": "oracle.rng_words (creation.mojo:57-131)", "words": words}, f, indent=1)

    # small fixtures: fp32 16x16x16 matmul, Linear 8->12 with bias and ReLU,
    # int8 rows with constructed ties, a 64x256 W8A16 GEMV
    A = oracle.randn_f32((16, 16), seed=1)
    B = oracle.randn_f32((16, 16), seed=2)
    x = oracle.randn_f32((5, 8), seed=3)
    W = oracle.randn_f32((12, 8), seed=4)
    b = oracle.randu_f32((12,), -1 / 16, 1 / 16, seed=5)
    s = np.float32(2.0 ** -6)
    ties = np.concatenate([(np.arange(-64, 64, dtype=np.float32) + 0.5) * s,
                           np.array([127 * s, -127 * s], np.float32),
                           np.zeros(126, np.float32)]).reshape(1, 256)
    Wq_src = np.concatenate([ties, oracle.randn_f32((7, 256), std=0.02, seed=6),
                             np.zeros((1, 256), np.float32)])
    Qr, sr = oracle.quantize_rowwise_rhe(Wq_src)
    Ql, sl = oracle.quantize_rowwise_legacy(Wq_src)
    xv = oracle.f32_to_bf16(oracle.randn_f32((1, 256), seed=7))
    Wg = oracle.randn_f32((64, 256), std=0.02, seed=8)
    Qg, sg = oracle.quantize_rowwise_rhe(Wg)
    bg = oracle.randu_f32((64,), -1 / 16, 1 / 16, seed=9)
    yb, yf = oracle.linear_w8a16(xv, Qg, sg, bg)
    np.savez_compressed(
        os.path.join(HERE, "small_cases.npz"),
        mm_A=A, mm_B=B, mm_C=oracle.matmul_f32(A, B),
        lin_x=x, lin_W=W, lin_b=b, lin_relu_y=oracle.linear_act_f32(x, W, b, oracle.EPI_RELU),
        q_W=Wq_src, q_rhe=Qr, q_rhe_s=sr, q_legacy=Ql, q_legacy_s=sl,
        gemv_x=xv, gemv_Q=Qg, gemv_s=sg, gemv_b=bg, gemv_y_bf16=yb, gemv_y_f32=yf,
    )
    print("wrote", os.listdir(HERE))


if __name__ == "__main__":
    main()
