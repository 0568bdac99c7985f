"""Check a .knx model against known outputs and time it (the role of the reference's tools/verify.py:57-80).

    python -m kernix_amd.knx_verify model.knx --input x.npy --expect y.npy [--tol 1e-4] [--mode ref|i8]
    python -m kernix_amd.knx_verify model.knx --batch 64          # random N(0, 1) input: timing only

From Python, `verify(path, x, expect)` takes the expected outputs as an array or as a callable (for example a torch
module wrapped as `lambda x: module(torch.from_numpy(x)).detach().numpy()`), runs the model on the GPU and returns a
`Report`: the maximum error relative to the largest expected magnitude (absolute when every expected value is 0), the
share of samples whose arg-max class agrees (for outputs with two or more classes), and the median forward time at
batch 1 and at the full batch.  Exit status 1 when the error is above the tolerance.
"""
import argparse
import statistics
import sys
import time
from dataclasses import dataclass
from typing import Optional

import numpy as np

from .kernix import INT8_I8, Model


@dataclass
class Report:
    max_rel_err: float
    argmax_agree: Optional[float]   # None when the output has fewer than two classes
    ms_batch1: float
    ms_batch: float
    batch: int
    ok: bool


def compare(want, got):
    """(max |want − got| / max |want|, or the absolute error when want is all zero; arg-max agreement or None)"""
    want = np.asarray(want, np.float64)
    got = np.asarray(got, np.float64).reshape(want.shape)
    peak = float(np.max(np.abs(want))) if want.size else 0.0
    diff = float(np.max(np.abs(want - got))) if want.size else 0.0
    err = diff / peak if peak > 0.0 else diff
    if np.isnan(got).any() != np.isnan(want).any():
        err = float("inf")
    agree = None
    if want.ndim >= 2 and want.shape[-1] >= 2:
        agree = float(np.mean(np.argmax(want, axis=-1) == np.argmax(got, axis=-1)))
    return err, agree


def median_ms(fn, x, runs=20, warmup=3):
    """median wall time of fn(x) in ms over `runs` back-to-back calls after `warmup` calls (no pauses in between:
    an idle GPU lowers its clock and a small model would read slow)"""
    for _ in range(warmup):
        fn(x)
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn(x)
        times.append((time.perf_counter() - t0) * 1e3)
    return statistics.median(times)


def verify(path, x, expect, tol=1e-4, mode="ref", workspace_mb=None, runs=20):
    """Run the .knx model at `path` on x and compare it with `expect` (array, or callable of x)."""
    model = Model(path, workspace_mb=workspace_mb)
    try:
        if mode == "i8":
            model.set_int8_mode(INT8_I8)
        x = np.ascontiguousarray(x, np.float32)
        got = model(x)
        want = expect(x) if callable(expect) else expect
        err, agree = compare(want, got)
        t1 = median_ms(model, x[:1], runs)
        tb = median_ms(model, x, runs)
    finally:
        model.close()
    return Report(err, agree, t1, tb, len(x), bool(err <= tol))


def main(argv=None):
    ap = argparse.ArgumentParser(description="compare a .knx model's GPU forward with expected outputs and time it")
    ap.add_argument("knx")
    ap.add_argument("--input", help=".npy input, first axis the batch (default: N(0, 1) of --batch samples)")
    ap.add_argument("--expect", help=".npy expected output for --input (without it only the timing is reported)")
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--tol", type=float, default=1e-4, help="largest accepted relative error (default 1e-4)")
    ap.add_argument("--mode", choices=("ref", "i8"), default="ref", help="int8 dispatch: the reference's, or int8 at every M")
    ap.add_argument("--workspace-mb", type=float, default=None)
    a = ap.parse_args(argv)
    if a.batch < 1:
        ap.error("--batch must be at least 1")
    probe = Model(a.knx)
    in_shape = probe.in_shape
    probe.close()
    if a.input:
        x = np.load(a.input, allow_pickle=False)
        if x.ndim < 2 or tuple(x.shape[1:]) != in_shape:
            ap.error(f"--input shape {x.shape}: expected (batch, {', '.join(map(str, in_shape))})")
    else:
        x = np.random.default_rng(0).standard_normal((a.batch,) + in_shape).astype(np.float32)
    expect = np.load(a.expect, allow_pickle=False) if a.expect else None
    if expect is None:
        model = Model(a.knx, workspace_mb=a.workspace_mb)
        if a.mode == "i8":
            model.set_int8_mode(INT8_I8)
        print(f"batch 1: {median_ms(model, x[:1]):.3f} ms   batch {len(x)}: {median_ms(model, x):.3f} ms")
        model.close()
        return 0
    r = verify(a.knx, x, expect, a.tol, a.mode, a.workspace_mb)
    agree = "-" if r.argmax_agree is None else f"{100 * r.argmax_agree:.1f}%"
    print(f"max relative error {r.max_rel_err:.2e} (tolerance {a.tol:g}), arg-max agreement {agree}")
    print(f"batch 1: {r.ms_batch1:.3f} ms   batch {r.batch}: {r.ms_batch:.3f} ms")
    print("PASS" if r.ok else "FAIL")
    return 0 if r.ok else 1


if __name__ == "__main__":
    sys.exit(main())
