"""The C API (include/kernix_model.h) exercised from C: tests/c/capi_driver.c runs a manifest of checks that this
module writes, with every model, malformed file and expected output prepared here.

What is checked is the reference's C-level contract (reference test/model_test.c): the files its loader accepts and
rejects (cases of :51-98, :246-293 and :471-537, kept as data — the byte layouts, sizes and bounds), the fields its tests
read (n_steps after activation folding, in/out dims, seq_len, ws_fixed, which int8 weights stay int8), exact int8
pack/unpack and dequantization at load, and on the GPU: forward accuracy against the CPU oracle, output-buffer reuse,
empty and malformed inputs, chunked execution under a workspace limit with trim, the dequantized-copy rule (an fp32
copy of int8 weights only above 2 rows), KNX1 ≡ KNX2-F32 bit for bit, and kernix_qmatmul on the reference's LCG
known-answer cases (tests/golden/qmatmul_lcg.npz, bit-exact) including NaN and zero rows and the int32 bound.
Tolerances: 1e-4 absolute for fp32 models against the oracle, 1e-5 for the recurrent ones (reference
test/model_test.c:127-142, :268-272), 1e-2 between the int8 and dequantized paths of one model (:651).
"""
import os
import struct
import subprocess

import numpy as np
import pytest

from kernix_amd import configs
from kernix_amd.knxfile import ModelBuilder
from oracle import knx_ref
from tests.golden.make_golden import LCG, qcase
from tests.graph_models import FAMILIES, make

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIBDIR = os.path.join(ROOT, "kernix_amd")
MAX_K = 131072


def _u32(*v):
    return struct.pack(f"<{len(v)}I", *v)


def _f32(a):
    return np.asarray(a, "<f4").tobytes()


def _tensor(path, a, dtype="<f4"):
    a = np.ascontiguousarray(a, dtype)
    a2 = a.reshape(a.shape[0], -1) if a.ndim != 2 else a
    with open(path, "wb") as f:
        f.write(_u32(*a2.shape) + a2.tobytes())
    return path


class Fixtures:
    """files in one directory and the manifest lines that use them"""

    def __init__(self, d):
        self.d = str(d)
        self.cpu, self.gpu = [], []

    def path(self, name):
        return os.path.join(self.d, name)

    def raw(self, name, data):
        with open(self.path(name), "wb") as f:
            f.write(data)
        return self.path(name)

    def reject(self, name, data):
        self.cpu.append(f"reject {self.raw(name, data)}")


def _lin(rng, i, o):
    k = 1.0 / np.sqrt(i)
    return rng.uniform(-k, k, (i, o)), rng.uniform(-k, k, o)


def _oracle(path, x, mode="ref"):
    y, _ = knx_ref.forward(knx_ref.parse(path), np.ascontiguousarray(x, np.float32), mode=mode)
    return y


def _sequential_models(fx, rng):
    """the reference test models' architectures (reference test/mlp_bench.py:36-62), random weights"""
    b = ModelBuilder((64,))
    w, bias = _lin(rng, 64, 128)
    h = b.linear(b.input, w, bias, activation="gelu")
    h = b.layer_norm(h, rng.normal(1.0, 0.5, 128), rng.normal(0.0, 0.5, 128))
    for (i, o, act, has_b) in ((128, 96, "silu", False), (96, 96, "tanh", True), (96, 80, "sigmoid", True),
                               (80, 32, "relu", True)):
        w, bias = _lin(rng, i, o)
        h = b.linear(h, w, bias if has_b else None, activation=act)
    h = b.layer_norm(h)
    w, bias = _lin(rng, 32, 10)
    b.linear(h, w, bias, activation="softmax")
    small = b.save(fx.path("small.knx"))
    assert open(small, "rb").read(4) == b"KNX1"

    b = ModelBuilder((4,))
    w, bias = _lin(rng, 4, 9000)
    h = b.activation(b.linear(b.input, w, bias, activation="silu"), "gelu")
    w, bias = _lin(rng, 9000, 3)
    b.linear(h, w, bias)
    wide = b.save(fx.path("wide.knx"))

    b = ModelBuilder((8,))
    w, bias = _lin(rng, 8, 4)
    b.linear(b.activation(b.input, "tanh"), w, bias)
    inplace = b.save(fx.path("inplace_first.knx"))

    b = ModelBuilder((4,))
    b.linear(b.input, np.eye(4), None)
    ident = b.save(fx.path("id.knx"))

    fx.cpu += [f"load {small} 9 64 10 1", f"load {wide} 3 4 3 1", f"load {inplace} 2 8 4 1", f"load {ident} 1 4 4 1"]
    for name, path, in_dim, batches in (("small", small, 64, (1, 37, 4096)), ("wide", wide, 4, (5,)),
                                        ("inplace", inplace, 8, (3,))):
        for n in batches:
            x = rng.standard_normal((n, in_dim)).astype(np.float32)
            xp = _tensor(fx.path(f"{name}_x{n}.bin"), x)
            fx.gpu.append(f"forward {path} {xp} {_tensor(fx.path(f'{name}_y{n}.bin'), _oracle(path, x))} 1e-4")
    x37 = fx.path("small_x37.bin")
    x = (np.arange(8, dtype=np.float32) - 3.0).reshape(2, 4)
    fx.gpu += [f"reuse {small} {x37}", f"edges {small}", f"own {ident} {_tensor(fx.path('id_x.bin'), x)}",
               f"forward {ident} {fx.path('id_x.bin')} {_tensor(fx.path('id_y.bin'), x)} 0",
               f"chunks {small} {x37} 1e-5"]
    xc = np.array([((i * 29) % 17 - 8) * 0.2 for i in range(80)], np.float32).reshape(10, 8)
    fx.gpu.append(f"chunks {inplace} {_tensor(fx.path('inplace_xc.bin'), xc)} 1e-5")
    return small


def _recurrent_models(fx, rng):
    """LSTM(7→5, tanh, sequences, T=4) → LSTM(5→6, ReLU, last) → Linear(6→3): float32 (KNX1 and the same weights as
    KNX2 F32 blocks) and with int8 recurrent / Linear weights (KNX2 I8_COL)"""
    w1, u1, b1 = rng.uniform(-0.5, 0.5, (7, 20)), rng.uniform(-0.5, 0.5, (5, 20)), rng.uniform(-0.5, 0.5, 20)
    w2, u2, b2 = rng.uniform(-0.5, 0.5, (5, 24)), rng.uniform(-0.5, 0.5, (6, 24)), rng.uniform(-0.5, 0.5, 24)
    wd, bd = rng.uniform(-0.5, 0.5, (6, 3)), rng.uniform(-0.5, 0.5, 3)

    def build(int8):
        b = ModelBuilder((4, 7))
        h = b.recurrent(b.input, "LSTM", 5, [(w1, u1, b1)], activation="tanh", return_sequences=True,
                        fmt_input="f32", fmt_recurrent="i8_col" if int8 else "f32")
        h = b.recurrent(h, "LSTM", 6, [(w2, u2, b2)], activation="relu", fmt_input="f32",
                        fmt_recurrent="i8_col" if int8 else "f32")
        b.linear(h, wd, bd if int8 else None, fmt="i8_col" if int8 else "f32")
        return b

    lstm = build(False).save(fx.path("lstm.knx"))
    lstm2 = build(False).save(fx.path("lstm_v2f.knx"), version=2)
    qlstm = build(True).save(fx.path("qlstm.knx"))
    assert open(lstm, "rb").read(4) == b"KNX1" and open(qlstm, "rb").read(4) == b"KNX2"
    x = np.array([((i * 37) % 23 - 11) * 0.1 for i in range(40 * 4 * 7)], np.float32).reshape(40 * 4, 7)
    xp = _tensor(fx.path("lstm_x40.bin"), x)
    x3p = _tensor(fx.path("lstm_x3.bin"), x[:12])
    x10p = _tensor(fx.path("lstm_x10.bin"), x[:40])
    fx.cpu += [f"load {lstm} 3 7 3 4", f"load {qlstm} 3 7 3 4", f"fixed {qlstm} {5 * 20 + 6 * 24 + 6 * 3}",
               f"int8 {qlstm} 0 1 1 0", f"int8 {qlstm} 2 1 0 0", f"int8 {lstm} 0 0 1 1", f"ane {qlstm}"]
    fx.gpu += [f"forward {lstm} {x3p} {_tensor(fx.path('lstm_y3.bin'), _oracle(lstm, x[:12]))} 1e-5",
               f"same {lstm} {lstm2} {xp}", f"badrows {lstm} 7", f"chunks {lstm} {x10p} 1e-5"]
    # int8 recurrences: int8 arithmetic at <= 2 samples (the recurrence's rows), the fp32 copy above
    per_sample = []
    for n in (1, 2, 3, 40):
        want = _oracle(qlstm, x[: 4 * n])
        xn = _tensor(fx.path(f"qlstm_x{n}.bin"), x[: 4 * n])
        fx.gpu += [f"forward {qlstm} {xn} {_tensor(fx.path(f'qlstm_y{n}.bin'), want)} 1e-5",
                   f"deq {qlstm} {xp} {n} {int(n > 2)}"]
        if n == 40:
            per_sample = np.concatenate([_oracle(qlstm, x[4 * s: 4 * s + 4]) for s in range(40)])
            assert np.max(np.abs(per_sample - want)) <= 1e-2  # int8 path vs dequantized path of one model
    fx.gpu += [f"chunks {qlstm} {xp} 1e-2", f"limit_deq {qlstm} {xp} 10"]
    return lstm


def _malformed(fx, small):
    """loader rejections: the reference's cases (test/model_test.c:51-98, :246-293, :471-537) as byte layouts"""
    data = open(small, "rb").read()
    fx.reject("truncated.knx", data[: len(data) // 2])
    fx.reject("trailing.knx", data + b"\0\0\0\0")
    fx.reject("v1_as_v2.knx", b"KNX2" + data[4:])
    K1 = b"KNX1"
    fx.reject("zero_ops.knx", K1 + _u32(0))
    fx.reject("many_ops.knx", K1 + _u32(1025))
    fx.reject("huge.knx", K1 + _u32(1, 0, 0xFFFFFFFF, 0xFFFFFFFF, 1))
    fx.reject("big_no_data.knx", K1 + _u32(1, 0, 30000, 30000, 0))
    fx.reject("zero_dim.knx", K1 + _u32(1, 0, 0, 4, 0))
    lin48 = _u32(0, 4, 8, 0) + _f32(np.zeros(32))
    fx.reject("chain.knx", K1 + _u32(2) + lin48 + _u32(0, 9, 2, 0) + _f32(np.zeros(18)))
    fx.reject("ln_size.knx", K1 + _u32(2) + lin48 + _u32(2, 7, 0) + _f32([1e-5]))
    fx.reject("kind9.knx", K1 + _u32(1, 9))
    fx.reject("act9.knx", K1 + _u32(1, 1, 9))
    fx.reject("act_only.knx", K1 + _u32(1, 1, 0))
    ok = fx.raw("chain_ok.knx", K1 + _u32(2) + lin48 + _u32(0, 8, 2, 0) + _f32(np.zeros(16)))
    fx.cpu.append(f"load {ok} 2 4 2 1")

    def lstm_rec(i, u, act, ret, seq):
        return _u32(4, i, u, act, ret, seq) + _f32(np.full(i * 4 * u + u * 4 * u + 4 * u, 0.1))

    fx.reject("lstm_seq0.knx", K1 + _u32(1) + lstm_rec(7, 5, 4, 0, 0))
    fx.reject("lstm_gelu.knx", K1 + _u32(1) + lstm_rec(7, 5, 1, 0, 4))
    fx.reject("lstm_ret2.knx", K1 + _u32(1) + lstm_rec(7, 5, 4, 2, 4))
    fx.reject("lstm_after_end.knx", K1 + _u32(2) + lstm_rec(7, 5, 4, 0, 4) + lstm_rec(5, 6, 0, 0, 4))
    fx.reject("lstm_units.knx", K1 + _u32(1, 4, 7, 100000, 0, 0, 4))
    fx.reject("lstm_short.knx", (K1 + _u32(1) + lstm_rec(7, 5, 4, 0, 4))[:-4])

    K2 = b"KNX2"
    head = _u32(1, 0, 4, 2, 0)
    lcg = LCG(777)
    q = np.array([(lcg() % 255) - 127 for _ in range(8)], np.int8)
    sc = np.array([0.01 + (lcg() % 100) * 1e-4 for _ in range(2)], np.float32)
    col = head + _u32(1) + _f32(sc) + q.tobytes()
    fx.reject("v3_magic.knx", b"KNX3" + head + _u32(0) + _f32(np.zeros(8)))
    fx.reject("dtype3.knx", K2 + head + _u32(3) + _f32(np.full(8, 0.1)))
    fx.reject("short_scales.knx", K2 + head + _u32(1) + _f32([0.1]))
    fx.reject("short_int8.knx", (K2 + col)[:-1])
    for i, bad in enumerate((0.0, -1.0, np.nan, np.inf)):
        blob = bytearray(K2 + col)
        blob[4 + 4 + 16 + 4: 4 + 4 + 16 + 8] = _f32([bad])
        fx.reject(f"scale{i}.knx", bytes(blob))
    fx.reject("k_over.knx", K2 + _u32(1, 0, MAX_K + 1, 1, 0, 1) + _f32([0.01]) + b"\x01" * (MAX_K + 1))
    kb = fx.raw("k_bound.knx", K2 + _u32(1, 0, MAX_K, 1, 0, 1) + _f32([0.01]) + b"\x01" * MAX_K)
    fx.cpu.append(f"int8 {kb} 0 1 0 0")
    # I8_ROW Linear: dequantized at load, w[k][n] = q·scale[k] exactly
    q15 = np.array([(lcg() % 255) - 127 for _ in range(15)], np.int8).reshape(3, 5)
    s3 = np.array([0.01 + (lcg() % 100) * 1e-4 for _ in range(3)], np.float32)
    row = fx.raw("i8_row.knx", K2 + _u32(1, 0, 3, 5, 0, 2) + _f32(s3) + q15.tobytes())
    fx.cpu += [f"int8 {row} 0 0 1 0",
               f"weight {row} 0 w {_tensor(fx.path('i8_row_w.bin'), q15.astype(np.float32) * s3[:, None])}"]
    # KNX2 LSTM: I8_COL input weight dequantized (q·scale[n]), float recurrent weight kept
    q24 = np.array([(lcg() % 255) - 127 for _ in range(24)], np.int8).reshape(3, 8)
    s8 = np.array([0.01 + (lcg() % 100) * 1e-4 for _ in range(8)], np.float32)
    u = np.linspace(-0.5, 0.5, 16, dtype=np.float32)
    lst = fx.raw("v2_lstm.knx", K2 + _u32(1, 4, 3, 2, 4, 0, 2) + _u32(1) + _f32(s8) + q24.tobytes() + _u32(0) + _f32(u) +
                 _f32(np.zeros(8)))
    fx.cpu += [f"int8 {lst} 0 0 1 1",
               f"weight {lst} 0 w {_tensor(fx.path('v2_lstm_w.bin'), q24.astype(np.float32) * s8[None, :])}",
               f"weight {lst} 0 rec {_tensor(fx.path('v2_lstm_u.bin'), u.reshape(2, 8))}"]


def _int8_kernel(fx):
    g = np.load(os.path.join(ROOT, "tests", "golden", "qmatmul_lcg.npz"), allow_pickle=False)
    for i in range(len(g["cases"])):
        p = fx.path(f"qm{i}")
        _tensor(p + "_q.bin", g[f"q{i}"], np.int8)
        for name in ("scale", "bias"):
            _tensor(p + f"_{name}.bin", g[f"{name}{i}"][None, :])
        for name in ("x", "yold", "y", "yacc"):
            _tensor(p + f"_{name}.bin", g[f"{name}{i}"])
        fx.gpu.append(f"qmatmul {p}")
        if g["cases"][i][2] >= 3:
            fx.gpu.append(f"qspecial {p}")
    fx.gpu.append("qbound")
    lcg = LCG()
    q, scale, _, _ = qcase(lcg, 55, 31, 1)
    fx.cpu.append(f"qpack {_tensor(fx.path('pack_q.bin'), q, np.int8)} {_tensor(fx.path('pack_s.bin'), scale[None, :])}")


@pytest.fixture(scope="module")
def manifest(tmp_path_factory):
    d = tmp_path_factory.mktemp("capi")
    fx = Fixtures(d)
    rng = np.random.default_rng(0)
    small = _sequential_models(fx, rng)
    _recurrent_models(fx, rng)
    _malformed(fx, small)
    _int8_kernel(fx)
    # storage-plan invariants on every graph family and on the benchmark architectures at reduced size
    for fam in sorted(FAMILIES):
        for qz in (None, "int8"):
            p, _ = make(d, fam, qz)
            fx.cpu.append(f"plan {p}")
    for name, kw in (("cnn", dict(batch=1, hw=8, widths=(8, 8, 16, 16))),
                     ("transformer", dict(batch=1, seq=8, d=16, heads=2, ffn=32, layers=2)),
                     ("int8_mlp", dict(batch=1)), ("fp32_mlp", dict(batch=1, dims=(32, 32, 32, 10)))):
        p = str(d / f"{name}.knx")
        getattr(configs, name)(p, **kw)
        fx.cpu.append(f"plan {p}")
    fx.cpu += [f"plan {small}", f"plan {fx.path('qlstm.knx')}"]
    files = {}
    for mode, lines in (("cpu", fx.cpu), ("gpu", fx.gpu)):
        files[mode] = str(d / f"{mode}.manifest")
        with open(files[mode], "w") as f:
            f.write("\n".join(lines) + "\n")
    return files


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    if not os.path.exists(os.path.join(LIBDIR, "libkernix.so")):
        pytest.fail("kernix_amd/libkernix.so is not built (run __graft_entry__.build())")
    out = str(tmp_path_factory.mktemp("capibin") / "capi_driver")
    subprocess.run(["gcc", "-O1", "-std=c11", "-D_GNU_SOURCE", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"),
                    os.path.join(ROOT, "tests", "c", "capi_driver.c"), "-o", out, "-L", LIBDIR, "-lkernix",
                    f"-Wl,-rpath,{LIBDIR}", "-lm"], check=True)
    return out


def _run(driver, manifest):
    r = subprocess.run([driver, manifest], capture_output=True, text=True, timeout=600)
    print(r.stdout)
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-2000:]
    return r.stdout


def test_capi_host_checks(driver, manifest):
    """loader acceptance/rejection, fields, int8 dispositions, pack/unpack, storage plan (no GPU involved)"""
    out = _run(driver, manifest["cpu"])
    assert " 0 failed" in out


@pytest.mark.gpu
def test_capi_device_checks(driver, manifest):
    """forward accuracy and buffer contracts, chunking and trim, dequantized copies, kernix_qmatmul known answers"""
    out = _run(driver, manifest["gpu"])
    assert " 0 failed" in out
