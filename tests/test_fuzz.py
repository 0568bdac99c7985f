"""Loader fuzzing (the reference's test/knx_fuzz_test.py:47-90 procedure): every graph family of
tests/graph_models.py is written as a valid .knx, then damaged — truncated at a random length, one u32 set to a
boundary value (0, 1, 2, 3, 7, 255, 65535, 65536, 2³¹−1, 2³¹, 2³²−1), 1–3 random bytes in the first 1600 replaced,
or 1–8 garbage bytes appended.  The harness (tests/c/knx_fuzz.c) is built with AddressSanitizer and UBSan over the
host runtime sources (loader, planner, C ABI), linked to the library for the device entry points, and must load
every valid file and either reject each damaged one or accept it without a memory error.  Loading only: a forward
of an accepted damaged model would run on the GPU, which this CPU test does not use.
"""
import os
import struct
import subprocess

import numpy as np
import pytest

from tests.graph_models import FAMILIES, make

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIBDIR = os.path.join(ROOT, "kernix_amd")
HOST = os.path.join(ROOT, "kernix_amd", "csrc", "host")
BOUNDARY = [0, 1, 2, 3, 7, 255, 65535, 65536, 2**31 - 1, 2**31, 2**32 - 1]


def mutations(rng, data, n):
    words = len(data) // 4
    for i in range(n):
        b = bytearray(data)
        kind = i % 4
        if kind == 0:
            yield bytes(b[: int(rng.integers(0, len(b)))])
        elif kind == 1:
            w = int(rng.integers(0, min(words, 400)))
            b[4 * w:4 * w + 4] = struct.pack("<I", int(rng.choice(BOUNDARY)))
            yield bytes(b)
        elif kind == 2:
            for _ in range(int(rng.integers(1, 4))):
                b[int(rng.integers(0, min(len(b), 1600)))] = int(rng.integers(0, 256))
            yield bytes(b)
        else:
            yield bytes(b) + bytes(rng.integers(0, 256, int(rng.integers(1, 9))).astype(np.uint8))


@pytest.fixture(scope="module")
def harness(tmp_path_factory):
    if not os.path.exists(os.path.join(LIBDIR, "libkernix.so")):
        pytest.fail("kernix_amd/libkernix.so is not built (run __graft_entry__.build())")
    out = str(tmp_path_factory.mktemp("fuzzbin") / "knx_fuzz")
    srcs = [os.path.join(HOST, f) for f in ("knx_decode.c", "knx_graph.c", "knx_forward.c", "knx_capi.c")]
    cmd = ["gcc", "-O1", "-g", "-std=c11", "-D_GNU_SOURCE", "-fsanitize=address,undefined", "-fno-omit-frame-pointer",
           "-I", os.path.join(ROOT, "include"), "-I", HOST, os.path.join(ROOT, "tests", "c", "knx_fuzz.c"), *srcs,
           "-o", out, "-L", LIBDIR, "-lkernix", f"-Wl,-rpath,{LIBDIR}", "-lm"]
    subprocess.run(cmd, check=True)
    return out


def _run(harness, files):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    r = subprocess.run([harness] + files, capture_output=True, text=True, env=env, timeout=600)
    assert r.returncode == 0, r.stderr[-4000:]
    return int(r.stdout.split()[1])


@pytest.mark.parametrize("family", sorted(FAMILIES))
@pytest.mark.parametrize("quantize", [None, "int8"])
def test_loader_fuzz(harness, tmp_path, family, quantize):
    p, _ = make(tmp_path, family, quantize)
    assert _run(harness, [p]) == 1
    data = open(p, "rb").read()
    rng = np.random.default_rng(sum(map(ord, family)) + (7 if quantize else 0))
    files = []
    for i, m in enumerate(mutations(rng, data, 400)):
        q = str(tmp_path / f"m{i}.knx")
        with open(q, "wb") as f:
            f.write(m)
        files.append(q)
    accepted = _run(harness, files)
    assert accepted < len(files)  # truncations at least are rejected
