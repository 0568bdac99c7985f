"""Writes the golden fixtures of this directory (run from the repository root: python tests/golden/make_golden.py).

The reference ships no data files for this path: its test/model_data/ is produced by a PyTorch script and is not
committed.  Its known-answer tests are generators — check_qmatmul's LCG cases (reference test/model_test.c:384-446)
— so the fixtures here are those cases, written down with expected outputs computed by a restatement that is
independent of both the oracle and the GPU path: int64 dot products of the same int8 values and the reference's
fp32 steps done one numpy float32 operation at a time (reference include/kernix_model.h:112-178).

  qmatmul_lcg.npz   check_qmatmul cases: (k, n, rows) ∈ CASES, accumulate 0 and 1
  i8gemm_cases.npz  int8 GEMM with per-row / per-column scales, bias, ReLU: ragged shapes, K % 128 == 64
  mlp_int8.knx      KNX2 int8 MLP 20-16-12-5 (ReLU hidden), weights from the reference LCG
  mlp_int8.npz      its input (1 and 2 rows: the int8 path of the reference dispatch) and expected outputs
"""
import os
import struct
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
CASES = [(55, 31, 1), (64, 256, 1), (128, 512, 3), (114, 512, 32), (16, 16, 1), (1, 1, 1)]
F = np.float32


class LCG:
    """reference test/model_test.c:384-385"""

    def __init__(self, seed=12345):
        self.x = seed

    def __call__(self):
        self.x = (self.x * 1664525 + 1013904223) & 0xFFFFFFFF
        return self.x >> 8


def qcase(rng, k, n, rows):
    """reference test/model_test.c:396-398"""
    q = np.array([(rng() % 255) - 127 for _ in range(k * n)], np.int8).reshape(k, n)
    scale = np.zeros(n, F)
    bias = np.zeros(n, F)
    for i in range(n):
        scale[i] = F(0.001) + F(rng() % 1000) * F(1e-5)
        bias[i] = F(rng() % 200) * F(0.01) - F(1.0)
    x = np.array([F(rng() % 2001) * F(0.003) - F(3.0) for _ in range(rows * k)], F).reshape(rows, k)
    return q, scale, bias, x


def quantize_row(xr):
    """x → (int8 values as int64, sx): reference include/kernix_model.h:121-142"""
    if not np.all(np.isfinite(xr)):
        return None, F(np.nan)
    m = F(np.max(np.abs(xr))) if xr.size else F(0)
    sx = F(m / F(127.0)) if m > 0 else F(1.0)
    inv = F(F(1.0) / sx)
    v = np.rint((xr * inv).astype(F))
    return np.clip(v, -127, 127).astype(np.int64), sx


def qmatmul_expected(x, q, scale, bias, y_old=None):
    out = np.zeros((x.shape[0], q.shape[1]), F)
    for r in range(x.shape[0]):
        v, sx = quantize_row(x[r])
        if v is None:
            out[r] = np.nan
            continue
        acc = v @ q.astype(np.int64)
        y = (acc.astype(F) * sx).astype(F)
        y = (y * scale).astype(F)
        y = (y + bias).astype(F)
        out[r] = y if y_old is None else (y_old[r] + y).astype(F)
    return out


def i8gemm_expected(A, W, sa, sw, bias):
    acc = A.astype(np.int64) @ W.astype(np.int64).T
    assert np.abs(acc).max() < 2**31
    y = (acc.astype(F) * sa[:, None]).astype(F)
    y = (y * sw[None, :]).astype(F)
    y = (y + bias[None, :]).astype(F)
    y = np.where(y >= 0, y, F(0)).astype(F)
    return acc.astype(np.int32), y


def write_knx2_int8_mlp(path, layers):
    """KNX2 (reference docs/int8-quantization-design.md:67-87): LINEAR with an I8_COL weight block, ACT relu between.
    Written here byte by byte from the format description, independently of the package writer (kernix_amd/knxfile.py)."""
    recs = []
    for i, (q, scale, bias) in enumerate(layers):
        k, n = q.shape
        # kind LINEAR, in, out, has_bias, then the weight block (dtype I8_COL, scale[out], int8 in×out), bias[out]
        recs.append(struct.pack("<5I", 0, k, n, 1, 1) + scale.astype("<f4").tobytes() + q.astype(np.int8).tobytes()
                    + bias.astype("<f4").tobytes())
        if i + 1 < len(layers):
            recs.append(struct.pack("<2I", 1, 0))
    with open(path, "wb") as f:
        f.write(b"KNX2" + struct.pack("<I", len(recs)) + b"".join(recs))


def main():
    rng = LCG()
    d = {}
    for i, (k, n, rows) in enumerate(CASES):
        q, scale, bias, x = qcase(rng, k, n, rows)
        y_old = (np.arange(rows * n) % 7 * 0.5).astype(F).reshape(rows, n)
        d.update({f"q{i}": q, f"scale{i}": scale, f"bias{i}": bias, f"x{i}": x, f"yold{i}": y_old,
                  f"y{i}": qmatmul_expected(x, q, scale, bias), f"yacc{i}": qmatmul_expected(x, q, scale, bias, y_old)})
    np.savez_compressed(os.path.join(HERE, "qmatmul_lcg.npz"), cases=np.array(CASES, np.int32), **d)

    g = {}
    shapes = [(37, 70, 192), (96, 80, 320), (5, 100, 64), (1, 48, 128)]
    for i, (M, N, K) in enumerate(shapes):
        A = np.array([(rng() % 255) - 127 for _ in range(M * K)], np.int8).reshape(M, K)
        W = np.array([(rng() % 255) - 127 for _ in range(N * K)], np.int8).reshape(N, K)
        sa = np.array([F(0.001) + F(rng() % 1000) * F(9e-6) for _ in range(M)], F)
        sw = np.array([F(0.001) + F(rng() % 1000) * F(9e-6) for _ in range(N)], F)
        bias = np.array([F(rng() % 200) * F(0.001) - F(0.1) for _ in range(N)], F)
        acc, y = i8gemm_expected(A, W, sa, sw, bias)
        g.update({f"A{i}": A, f"W{i}": W, f"sa{i}": sa, f"sw{i}": sw, f"bias{i}": bias, f"acc{i}": acc, f"y{i}": y})
    np.savez_compressed(os.path.join(HERE, "i8gemm_cases.npz"), shapes=np.array(shapes, np.int32), **g)

    dims = [20, 16, 12, 5]
    layers = []
    for k, n in zip(dims[:-1], dims[1:]):
        q, scale, bias, _ = qcase(rng, k, n, 1)
        layers.append((q, scale, bias))
    write_knx2_int8_mlp(os.path.join(HERE, "mlp_int8.knx"), layers)
    x = np.array([F(rng() % 2001) * F(0.003) - F(3.0) for _ in range(2 * dims[0])], F).reshape(2, dims[0])
    outs = {}
    for rows in (1, 2):
        h = x[:rows]
        for i, (q, scale, bias) in enumerate(layers):
            h = qmatmul_expected(h, q, scale, bias)
            if i + 1 < len(layers):
                h = np.where(h >= 0, h, F(0)).astype(F)
        outs[f"y{rows}"] = h
    np.savez_compressed(os.path.join(HERE, "mlp_int8.npz"), x=x, **outs)
    print("wrote fixtures to", HERE, file=sys.stderr)


if __name__ == "__main__":
    main()
