"""Loader fuzzing.  Each graph family of tests/graph_models.py (float32 and int8 weights) is written as a valid .knx
and then damaged in the ways the reference's fuzz test damages files (reference test/knx_fuzz_test.py:47-90): cut short
at a random length, one u32 word replaced by a boundary value (0, 1, 2, 3, 7, 255, 65535, 65536, 2³¹−1, 2³¹, 2³²−1),
one to three random bytes overwritten in the first 1600, one to eight random bytes appended.  On top of those random
cases, every one of the first 48 words is set to every boundary value in turn.  The harness (tests/c/knx_fuzz.c)
is built with AddressSanitizer and UBSan over the host runtime sources and must accept the valid file, survive every
damaged one without a memory error, and leave every model it accepts consistent.  Loading only: no GPU is used.
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
BOUNDARY = (0, 1, 2, 3, 7, 255, 65535, 65536, 2**31 - 1, 2**31, 2**32 - 1)


def cut(rng, data):
    return data[: int(rng.integers(0, len(data)))]


def poke_word(rng, data):
    b = bytearray(data)
    w = int(rng.integers(0, min(len(b) // 4, 400)))
    b[4 * w: 4 * w + 4] = struct.pack("<I", int(rng.choice(BOUNDARY)))
    return bytes(b)


def scramble(rng, data):
    b = bytearray(data)
    for _ in range(int(rng.integers(1, 4))):
        b[int(rng.integers(0, min(len(b), 1600)))] = int(rng.integers(0, 256))
    return bytes(b)


def append(rng, data):
    return data + rng.integers(0, 256, int(rng.integers(1, 9)), dtype=np.uint8).tobytes()


MUTATORS = (cut, poke_word, scramble, append)


def damaged(rng, data, n_random):
    for i in range(n_random):
        yield MUTATORS[i % len(MUTATORS)](rng, data)
    for w in range(min(48, len(data) // 4)):  # the header and first records, word by word
        for v in BOUNDARY:
            b = bytearray(data)
            b[4 * w: 4 * w + 4] = struct.pack("<I", v)
            if bytes(b) != data:
                yield bytes(b)


@pytest.fixture(scope="module")
def harness(tmp_path_factory):
    if not os.path.exists(os.path.join(LIBDIR, "libkernix.so")):
        pytest.fail("kernix_amd/libkernix.so is not built (run __graft_entry__.build())")
    out = str(tmp_path_factory.mktemp("fuzzbin") / "knx_fuzz")
    srcs = [os.path.join(HOST, f) for f in ("knx_decode.c", "knx_graph.c", "knx_forward.c", "knx_capi.c")]
    cmd = ["gcc", "-O1", "-g", "-std=c11", "-D_GNU_SOURCE", "-fsanitize=address,undefined", "-fno-omit-frame-pointer",
           "-I", os.path.join(ROOT, "include"), "-I", HOST, os.path.join(ROOT, "tests", "c", "knx_fuzz.c"), *srcs,
           "-o", out, "-L", LIBDIR, "-lkernix", f"-Wl,-rpath,{LIBDIR}", "-lm", "-lpthread"]
    subprocess.run(cmd, check=True)
    return out


def _accepted(harness, files):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    r = subprocess.run([harness] + files, capture_output=True, text=True, env=env, timeout=600)
    assert r.returncode == 0, r.stderr[-4000:]
    return int(r.stdout.split()[1])


@pytest.mark.parametrize("family", sorted(FAMILIES))
@pytest.mark.parametrize("quantize", [None, "int8"])
def test_loader_fuzz(harness, tmp_path, family, quantize):
    p, _ = make(tmp_path, family, quantize)
    assert _accepted(harness, [p]) == 1
    data = open(p, "rb").read()
    rng = np.random.default_rng(sum(map(ord, family)) + (7 if quantize else 0))
    files = []
    for i, blob in enumerate(damaged(rng, data, 400)):
        q = str(tmp_path / f"d{i}.knx")
        with open(q, "wb") as f:
            f.write(blob)
        files.append(q)
    accepted = _accepted(harness, files)
    assert accepted < len(files)  # cut-short files at least are rejected
