"""Runs tests/c/knx_model_test.c (the reference's test/model_test.c checks, in C against libkernix.so).

Fixtures: the reference generates small/wide/inplace_first models and their expected outputs with PyTorch
(reference test/mlp_bench.py:36-62).  Here the same architectures are written with random weights by the numpy .knx
writer and the expected outputs come from the CPU oracle; the checks and tolerances are the reference's.
"""
import os
import struct
import subprocess

import numpy as np
import pytest

from kernix_amd import knx_write
from oracle import knx_ref

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIBDIR = os.path.join(ROOT, "kernix_amd")


def _lin(rng, i, o):
    k = 1.0 / np.sqrt(i)
    return rng.uniform(-k, k, (i, o)), rng.uniform(-k, k, o)


def _save(path, a):
    a = np.ascontiguousarray(a, np.float32)
    with open(path, "wb") as f:
        f.write(struct.pack("<2I", *a.shape) + a.tobytes())


@pytest.fixture(scope="module")
def fixtures(tmp_path_factory):
    d = tmp_path_factory.mktemp("cfix")
    rng = np.random.default_rng(0)
    s = knx_write.Sequential()
    w, b = _lin(rng, 64, 128); s.linear(w, b).act("gelu")
    s.layernorm(128, 1e-5, rng.normal(1.0, 0.5, 128), rng.normal(0.0, 0.5, 128))
    w, _ = _lin(rng, 128, 96); s.linear(w).act("silu")
    w, b = _lin(rng, 96, 96); s.linear(w, b).act("tanh")
    w, b = _lin(rng, 96, 80); s.linear(w, b).act("sigmoid")
    w, b = _lin(rng, 80, 32); s.linear(w, b).act("relu")
    s.layernorm(32, 1e-5)
    w, b = _lin(rng, 32, 10); s.linear(w, b).softmax()
    wide = knx_write.Sequential()
    w, b = _lin(rng, 4, 9000); wide.linear(w, b).act("silu").act("gelu")
    w, b = _lin(rng, 9000, 3); wide.linear(w, b)
    inpl = knx_write.Sequential().act("tanh")
    w, b = _lin(rng, 8, 4); inpl.linear(w, b)
    for name, model, in_dim, batches in (("small", s, 64, (1, 37, 4096)), ("wide", wide, 4, (5,)),
                                         ("inplace_first", inpl, 8, (3,))):
        p = str(d / f"{name}.knx")
        model.write(p)
        ref = knx_ref.parse(p)
        for bsz in batches:
            x = rng.standard_normal((bsz, in_dim)).astype(np.float32)
            y, _ = knx_ref.forward(ref, x)
            _save(str(d / f"{name}_x_{bsz}.bin"), x)
            _save(str(d / f"{name}_y_{bsz}.bin"), y)
    return str(d)


@pytest.fixture(scope="module")
def binary(tmp_path_factory):
    if not os.path.exists(os.path.join(LIBDIR, "libkernix.so")):
        pytest.fail("kernix_amd/libkernix.so is not built (run __graft_entry__.build())")
    out = str(tmp_path_factory.mktemp("cbin") / "knx_model_test")
    cmd = ["gcc", "-O1", "-std=c11", "-D_GNU_SOURCE", "-Wall", "-I", os.path.join(ROOT, "include"),
           os.path.join(ROOT, "tests", "c", "knx_model_test.c"), "-o", out, "-L", LIBDIR, "-lkernix",
           f"-Wl,-rpath,{LIBDIR}", "-lm"]
    subprocess.run(cmd, check=True)
    return out


def _run(binary, mode, d):
    r = subprocess.run([binary, mode, d], capture_output=True, text=True, timeout=600)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr[-3000:]


def test_loader_checks_cpu(binary, fixtures):
    """loader rejection/acceptance, KNX2 dtype rules, int8 pack/unpack, ws_fixed (no GPU involved)"""
    _run(binary, "cpu", fixtures)


@pytest.mark.gpu
def test_runtime_checks_gpu(binary, fixtures):
    """forward accuracy, buffer reuse, LSTM, chunking/trim, int8 kernel, KNX2 forward on the MI355X"""
    _run(binary, "gpu", fixtures)
