"""Writes the small Q8_0 golden vectors in tests/golden/q8_cases.npz.

Inputs come from numpy's PCG64 (seeded); expected outputs from the CPU
oracle (weights: quantize_row_q8_0_ref rule, activations: x86 rule).  The
file holds, per case: W and x floats (small cases), the GGUF Q8_0 bytes of
both, the int32 per-block sums and the fp64 / sequential-fp32 outputs.
Run from the repository root:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import oracle  # noqa: E402

CASES = [(1, 32, 1), (7, 64, 3), (5, 96, 2), (64, 1024, 1), (8, 2048, 1), (3, 6144, 2)]


def main():
    out = {}
    for i, (N, K, M) in enumerate(CASES):
        rng = np.random.default_rng(1000 + i)
        w = rng.normal(0, 0.02, (N, K)).astype(np.float32)
        x = rng.normal(0, 1, (M, K)).astype(np.float32)
        wq = oracle.quantize_rows(w, oracle.QUANT_REF)
        xq = oracle.quantize_rows(x, oracle.QUANT_X86)
        tag = f"c{i}"
        out[f"{tag}_shape"] = np.array([N, K, M], np.int64)
        if N * K <= 8192:
            out[f"{tag}_w"] = w
        out[f"{tag}_x"] = x
        out[f"{tag}_wq"] = wq
        out[f"{tag}_xq"] = xq
        out[f"{tag}_sums"] = oracle.block_dots(wq, xq, N, K, M)
        out[f"{tag}_y64"] = oracle.mul_mat_f64(wq, xq, N, K, M)
        out[f"{tag}_y32"] = oracle.mul_mat(wq, xq, N, K, M)
    np.savez_compressed(os.path.join(ROOT, "tests", "golden", "q8_cases.npz"), **out)


if __name__ == "__main__":
    main()
