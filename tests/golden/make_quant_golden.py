"""Fixture that pins the weight quantizer and the weight-block bytes to the reference's own exporter.

Run in the build container (it needs the reference repository, which the GPU machines do not have):

    python tests/golden/make_quant_golden.py /root/reference

It imports the reference's tools/knx_quant.py and writes tests/golden/quant_blocks.npz: for each weight matrix w
below (float64), the reference's quantize(w, "col") and quantize(w, "row") results and the bytes of weight_block(w, m)
for m in f32 / i8_col / i8_row (KNX2) and of the KNX1 float32 block.  The matrices hold the cases where a plausible
restatement goes wrong:
  * all-zero columns and rows (scale 1, q 0);
  * exact ties (a column whose maximum is 127, so the scale is exactly 1, with values ±0.5, 1.5, 2.5, 63.5, …):
    numpy's rint rounds half to even;
  * values next to a half-way point of w / scale where the quotient computed in float32 (or as w · (1/scale))
    rounds to the other integer than the reference's float64 quotient;
  * float64 weights (not float32 values) whose column maximum / 127 rounds to another float32 when the maximum is
    first rounded to float32.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def boundary_values(rng, scale, count):
    """float32 values w near (j + ½)·scale whose float32 quotient w / scale (or w · (1/scale)) rounds to another
    integer than the float64 quotient"""
    out = []
    s32 = np.float32(scale)
    inv32 = np.float32(1.0) / s32
    tries = 0
    while len(out) < count and tries < 200000:
        tries += 1
        j = int(rng.integers(-126, 126))
        w = np.float32((j + 0.5) * float(s32))
        for cand in (w, np.nextafter(w, np.float32(np.inf)), np.nextafter(w, np.float32(-np.inf))):
            q64 = np.rint(np.float64(cand) / np.float64(s32))
            q32 = np.rint(np.float32(cand) / s32)
            qm = np.rint(np.float32(cand) * inv32)
            if abs(q64) <= 126 and (q64 != q32 or q64 != qm):
                out.append(np.float32(cand))
                break
    return np.array(out, np.float32)


def float32_weights(rng):
    k, n = 64, 12
    w = rng.normal(0, 0.05, (k, n)).astype(np.float32).astype(np.float64)
    w[:, 0] = 0.0                                                     # all-zero column
    ties = np.array([127.0, 63.5, -0.5, 0.5, 1.5, -1.5, 2.5, -2.5, 3.5, 126.5, -126.5, 4.5])
    w[:, 1] = 0.0
    w[: len(ties), 1] = ties                                          # scale exactly 1: round half to even
    w[5, :] = 0.0                                                     # an all-zero row (I8_ROW: scale 1)
    for c in range(2, n):
        peak = float(np.float32(rng.uniform(0.05, 3.0)))
        w[0, c] = peak if c % 2 else -peak                            # the column maximum fixes the scale
        scale = np.float32(peak / 127.0)
        vals = boundary_values(rng, scale, 20)
        w[6 : 6 + len(vals), c] = vals
    return w


def float64_weights(rng):
    k, n = 16, 10
    w = rng.normal(0, 1.0, (k, n))
    for c in range(n):  # a column maximum whose float32 rounding changes float32(max / 127)
        for _ in range(100000):
            m = rng.uniform(0.5, 4.0)
            if np.float32(m / 127.0) != np.float32(np.float32(m) / np.float32(127.0)):
                break
        w[0, c] = m
        w[1:, c] = np.clip(w[1:, c], -m * 0.999, m * 0.999)
    return w


def main(reference):
    sys.path.insert(0, os.path.join(reference, "tools"))
    import knx_quant  # the reference's quantizer and weight-block writer

    rng = np.random.default_rng(20240611)
    cases = {"w32": float32_weights(rng), "w64": float64_weights(rng)}
    out = {}
    for name, w in cases.items():
        out[f"{name}_w"] = w
        for axis in ("col", "row"):
            scale, q = knx_quant.quantize(w, axis)
            out[f"{name}_scale_{axis}"] = scale
            out[f"{name}_q_{axis}"] = q
        for mode in ("f32", "i8_col", "i8_row"):
            out[f"{name}_block_{mode}"] = np.frombuffer(knx_quant.weight_block(w, mode), np.uint8)
        out[f"{name}_block_v1"] = np.frombuffer(knx_quant.weight_block(w, "f32", v2=False), np.uint8)
    np.savez_compressed(os.path.join(HERE, "quant_blocks.npz"), **out)
    print("wrote", os.path.join(HERE, "quant_blocks.npz"), sorted(out))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
