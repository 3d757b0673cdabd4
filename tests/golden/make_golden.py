"""Generate tests/golden/vnni_vectors.npz from the (pinned) CPU oracle.

Inputs follow the reference's TestMatMulPackedVNNIExact recipe
(internal/tensor/vnni_test.go:83-98): a ~ U[-2,2), bT ~ U[-1,1), and one rail
row 127.4, -127.4, 1e-4 when k > 2, drawn here with numpy PCG64 seeds
(Go's math/rand stream is not reproducible outside Go). Outputs: quantized
weights, colSum, scales, quantized activations, row scales, int32
accumulators and the dequantized result — all exact.

Run: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as O  # noqa: E402

SHAPES = [(1, 1, 16), (1, 3, 16), (2, 4, 16), (3, 5, 32), (4, 8, 16), (5, 7, 48),
          (13, 129, 64), (64, 100, 128)]
SEED = 0x5EED0003


def main():
    rng = np.random.Generator(np.random.PCG64(SEED))
    out = {"seed": np.array([SEED], np.int64)}
    for (m, k, n) in SHAPES:
        a = (rng.random((m, k), dtype=np.float32) * 4 - 2).astype(np.float32)
        bT = (rng.random((n, k), dtype=np.float32) * 2 - 1).astype(np.float32)
        if k > 2:
            a[0, :3] = [127.4, -127.4, 0.0001]
        st, q, sc, cs = O.pack_b8_vnni(bT, k, n)
        assert st == 0
        dst, qa, rs, acc = O.matmul_vnni(a, q, cs, sc)
        tag = f"{m}x{k}x{n}"
        for name, arr in (("a", a), ("bT", bT), ("q", q), ("scales", sc), ("colsum", cs),
                          ("qa", qa), ("rs", rs), ("acc", acc), ("dst", dst)):
            out[f"{tag}/{name}"] = arr
    np.savez_compressed(os.path.join(HERE, "vnni_vectors.npz"), **out)
    print("wrote", os.path.join(HERE, "vnni_vectors.npz"))


if __name__ == "__main__":
    main()
