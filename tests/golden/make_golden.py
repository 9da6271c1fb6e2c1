"""Writes the committed golden fixtures of tests/ from library routines.

sgemm_small.npz: seeded fp32 operands for the four NN/NT/TN/TT variants and
their products computed by numpy in float64 (library matmul, independent of
the oracle).  conv_small.npz: a seeded conv layer (3->8, 3x3, stride 1, pad 1,
leaky 0.1) with its output from torch.nn.functional.conv2d in float64.

Run: python tests/golden/make_golden.py
"""
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def main():
    rng = np.random.default_rng(20240601)
    out = {}
    M, N, K = 19, 27, 45
    for v in ("nn", "nt", "tn", "tt"):
        ta, tb = v[0] == "t", v[1] == "t"
        A = rng.uniform(-1, 1, (K, M) if ta else (M, K)).astype(np.float32)
        B = rng.uniform(-1, 1, (N, K) if tb else (K, N)).astype(np.float32)
        C = (A.T if ta else A).astype(np.float64) @ (B.T if tb else B).astype(np.float64)
        out[f"{v}_A"], out[f"{v}_B"], out[f"{v}_C64"] = A, B, C
    np.savez_compressed(os.path.join(HERE, "sgemm_small.npz"), **out)

    import torch
    import torch.nn.functional as F

    x = rng.uniform(0, 1, (1, 3, 16, 16)).astype(np.float32)
    W = rng.normal(0, 0.05, (8, 3, 3, 3)).astype(np.float32)
    b = rng.normal(0, 0.1, 8).astype(np.float32)
    y = F.conv2d(torch.from_numpy(x).double(), torch.from_numpy(W).double(), torch.from_numpy(b).double(),
                 padding=1)
    y = torch.where(y < 0, 0.1 * y, y).numpy()
    np.savez_compressed(os.path.join(HERE, "conv_small.npz"), x=x, W=W.reshape(8, 27), b=b, y64=y)


if __name__ == "__main__":
    main()
