"""The committed golden fixtures (tests/golden/, written by tests/golden/make_golden.py from the reference's
known-answer generators with an independent int64 / float32 restatement) against the oracle (CPU) and against the
GPU path through the C ABI.  Integer work and the int8 epilogue are compared bit for bit."""
import ctypes
import os

import numpy as np
import pytest

from kernix_amd import hipabi
from oracle import knx_ref

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def same(a, b):
    return np.array_equal(a, b, equal_nan=True)


# ---------------------------------------------------------------- oracle (CPU)

def test_oracle_qmatmul_golden():
    d = load("qmatmul_lcg.npz")
    for i in range(len(d["cases"])):
        x, q, scale, bias, y_old = d[f"x{i}"], d[f"q{i}"], d[f"scale{i}"], d[f"bias{i}"], d[f"yold{i}"]
        assert same(knx_ref.qmatmul(x, q, scale, bias), d[f"y{i}"])
        assert same(knx_ref.qmatmul(x, q, scale, bias, y_old=y_old), d[f"yacc{i}"])


def test_oracle_i8gemm_golden():
    d = load("i8gemm_cases.npz")
    for i in range(len(d["shapes"])):
        y, acc = knx_ref.i8gemm(d[f"A{i}"], d[f"W{i}"], d[f"sa{i}"], d[f"sw{i}"], d[f"bias{i}"], act_id=0)
        assert np.array_equal(acc, d[f"acc{i}"])
        assert np.array_equal(y, d[f"y{i}"])


def test_oracle_forward_golden():
    d = load("mlp_int8.npz")
    model = knx_ref.parse(os.path.join(GOLDEN, "mlp_int8.knx"))
    for rows in (1, 2):
        y, _ = knx_ref.forward(model, d["x"][:rows])
        assert np.array_equal(y, d[f"y{rows}"])


def test_library_loads_golden_model():
    """the loader accepts the fixture model (written from the format description, not by this repository's writer)"""
    from kernix_amd.kernix import Model

    m = Model(os.path.join(GOLDEN, "mlp_int8.knx"))
    assert (m.in_dim, m.out_dim, m.seq_len) == (20, 5, 1)
    m.close()


def test_quantizer_matches_reference_exporter():
    """tests/golden/quant_blocks.npz, written by the reference's own tools/knx_quant.py (make_quant_golden.py): the
    package writer's quantize and weight blocks and the oracle's ko_quantize_cols reproduce its scales, int8 values
    and bytes exactly, on matrices holding all-zero columns and rows, exact ties, quotients next to a half-way point
    and float64 weights whose column maximum rounds differently through float32; the fixture also tells apart the
    plausible restatement mistakes (float32 quotient, reciprocal multiply, ties away from zero, scale from a float32
    maximum)"""
    from kernix_amd import knxfile

    d = load("quant_blocks.npz")
    for name in ("w32", "w64"):
        w = d[f"{name}_w"]
        for axis, per in (("col", "column"), ("row", "row")):
            scale, q = knxfile.quantize(w, per)
            assert np.array_equal(scale, d[f"{name}_scale_{axis}"]) and scale.dtype == np.float32, (name, axis)
            assert np.array_equal(q, d[f"{name}_q_{axis}"]), (name, axis)
        scale, q = knx_ref.quantize_cols(w)
        assert np.array_equal(scale, d[f"{name}_scale_col"]) and np.array_equal(q, d[f"{name}_q_col"]), name
        for mode in ("f32", "i8_col", "i8_row"):
            assert knxfile._weight(w, mode, 2) == d[f"{name}_block_{mode}"].tobytes(), (name, mode)
        assert knxfile._weight(w, "f32", 1) == d[f"{name}_block_v1"].tobytes(), name
    # the mistakes the fixture must catch, planted here on the CPU
    w, s, q = d["w32_w"], d["w32_scale_col"], d["w32_q_col"]
    assert (np.clip(np.rint(w.astype(np.float32) / s), -127, 127).astype(np.int8) != q).any()
    assert (np.clip(np.rint(w.astype(np.float32) * (np.float32(1) / s)), -127, 127).astype(np.int8) != q).any()
    away = np.clip(np.trunc(w / s.astype(np.float64) + 0.5 * np.sign(w)), -127, 127).astype(np.int8)
    assert (away != q).any()
    w64, s64 = d["w64_w"], d["w64_scale_col"]
    m32 = np.abs(w64.astype(np.float32)).max(axis=0)
    assert (np.where(m32 > 0, m32 / np.float32(127), np.float32(1)).astype(np.float32) != s64).any()


# ---------------------------------------------------------------- GPU path

@pytest.fixture(scope="module")
def L():
    lib = hipabi.lib()
    hipabi.check(lib.knx_hip_init())
    lib.kernix_qweight_pack.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int]
    lib.kernix_qweight_pack.restype = ctypes.c_void_p
    lib.kernix_qweight_free.argtypes = [ctypes.c_void_p]
    lib.kernix_qweight_free.restype = None
    lib.kernix_qmatmul.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                   ctypes.c_void_p]
    lib.kernix_qmatmul.restype = ctypes.c_int
    return lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


@pytest.mark.gpu
def test_gpu_qmatmul_golden(L):
    """kernix_qmatmul (host pointers, computed on the GPU) on the reference's check_qmatmul cases"""
    d = load("qmatmul_lcg.npz")
    for i, (k, n, rows) in enumerate(d["cases"]):
        q = np.ascontiguousarray(d[f"q{i}"])
        scale, bias = np.ascontiguousarray(d[f"scale{i}"]), np.ascontiguousarray(d[f"bias{i}"])
        x = np.ascontiguousarray(d[f"x{i}"])
        w = L.kernix_qweight_pack(_p(q), _p(scale), int(k), int(n))
        assert w
        try:
            y = np.zeros((rows, n), np.float32)
            assert L.kernix_qmatmul(_p(x), int(rows), w, _p(bias), 0, _p(y)) == 0
            assert same(y, d[f"y{i}"]), (k, n, rows)
            y = np.ascontiguousarray(d[f"yold{i}"]).copy()
            assert L.kernix_qmatmul(_p(x), int(rows), w, _p(bias), 1, _p(y)) == 0
            assert same(y, d[f"yacc{i}"]), (k, n, rows)
        finally:
            L.kernix_qweight_free(w)


class _QWeight(ctypes.Structure):
    _fields_ = [("k", ctypes.c_int), ("n", ctypes.c_int), ("kp", ctypes.c_int), ("np", ctypes.c_int),
                ("q", ctypes.POINTER(ctypes.c_int8)), ("scale", ctypes.POINTER(ctypes.c_float))]


@pytest.mark.gpu
def test_gpu_qmatmul_reads_the_weight_every_call(L):
    """a weight whose values change in place between calls gives the new values' results (the reference reads w->q
    and w->scale on every call, include/kernix_model.h:143-175); the struct has the reference's six fields"""
    d = load("qmatmul_lcg.npz")
    k, n, rows = (int(v) for v in d["cases"][1])
    q = np.ascontiguousarray(d["q1"])
    scale, bias, x = (np.ascontiguousarray(d[f"{v}1"]) for v in ("scale", "bias", "x"))
    w = L.kernix_qweight_pack(_p(q), _p(scale), k, n)
    assert w
    try:
        y = np.zeros((rows, n), np.float32)
        assert L.kernix_qmatmul(_p(x), rows, w, _p(bias), 0, _p(y)) == 0
        assert same(y, d["y1"])
        s = _QWeight.from_address(w)
        assert (s.k, s.n) == (k, n)
        qv = np.ctypeslib.as_array(s.q, shape=(s.np * s.kp,))
        sv = np.ctypeslib.as_array(s.scale, shape=(s.np,))
        qv[:] = -qv                         # every weight negated in place, every scale halved (exact)
        sv[:n] = sv[:n] * np.float32(0.5)
        y2 = np.zeros((rows, n), np.float32)
        assert L.kernix_qmatmul(_p(x), rows, w, _p(bias), 0, _p(y2)) == 0
        want = knx_ref.qmatmul(x, -q, scale * np.float32(0.5), bias)
        assert same(y2, want)
        assert not same(y2, y)
    finally:
        L.kernix_qweight_free(w)


@pytest.mark.gpu
def test_gpu_i8gemm_golden(L):
    import torch

    d = load("i8gemm_cases.npz")
    for i, (M, N, K) in enumerate(d["shapes"]):
        M, N, K = int(M), int(N), int(K)
        dA, dW = (torch.from_numpy(np.ascontiguousarray(d[f"{n}{i}"])).cuda() for n in ("A", "W"))
        dsa, dsw, db = (torch.from_numpy(np.ascontiguousarray(d[f"{n}{i}"])).cuda() for n in ("sa", "sw", "bias"))
        Y = torch.empty((M, N), dtype=torch.float32, device="cuda")
        acc = torch.empty((M, N), dtype=torch.int32, device="cuda")
        P = hipabi.ptr
        hipabi.check(L.knx_hip_i8gemm(M, N, K, P(dA), K, P(dsa), P(dW), K, P(dsw), P(db), 0, 0.0, 0,
                                      P(Y), N, P(acc), N, hipabi.stream()))
        torch.cuda.synchronize()
        assert np.array_equal(acc.cpu().numpy(), d[f"acc{i}"]), (M, N, K)
        assert np.array_equal(Y.cpu().numpy(), d[f"y{i}"]), (M, N, K)


@pytest.mark.gpu
def test_gpu_forward_golden():
    """the KNX2 int8 fixture model at 1 and 2 rows (the reference's int8 dispatch), bit for bit"""
    from kernix_amd.kernix import Model

    d = load("mlp_int8.npz")
    m = Model(os.path.join(GOLDEN, "mlp_int8.knx"))
    try:
        for rows in (1, 2):
            assert np.array_equal(m(d["x"][:rows]), d[f"y{rows}"])
    finally:
        m.close()
