"""Pins the CPU oracle (oracle/knx_oracle.c, oracle/knx_ref.py) before it is trusted as the parity checker.

Each oracle function is checked against (a) the reference's own known-answer tests for this path
(reference test/model_test.c: check_qmatmul :387-446, check_v2_load :471-537, ref_lstm :219-239), reproduced with the
reference's LCG (x = x·1664525 + 1013904223, >> 8, seed 12345), and (b) closed forms / brute force computed
independently in float64 or int64, chosen so that a plausible mistake (wrong rounding, dropped bias, transposed
weight order, wrong axis, wrong constant) fails one of them.
"""
import math

import numpy as np
import pytest

import struct

from kernix_amd import knxfile
from oracle import knx_ref


class LCG:
    """reference test/model_test.c:384-385"""

    def __init__(self, seed=12345):
        self.x = seed

    def __call__(self):
        self.x = (self.x * 1664525 + 1013904223) & 0xFFFFFFFF
        return self.x >> 8


def qcase(rng, k, n, rows):
    """One check_qmatmul case (reference test/model_test.c:396-398)."""
    q = np.array([(rng() % 255) - 127 for _ in range(k * n)], np.int8).reshape(k, n)
    scale = np.zeros(n, np.float32)
    bias = np.zeros(n, np.float32)
    for i in range(n):
        scale[i] = np.float32(0.001) + np.float32(rng() % 1000) * np.float32(1e-5)
        bias[i] = np.float32(rng() % 200) * np.float32(0.01) - np.float32(1.0)
    x = np.array([np.float32(rng() % 2001) * np.float32(0.003) - np.float32(3.0) for _ in range(rows * k)],
                 np.float32).reshape(rows, k)
    return q, scale, bias, x


def int_reference(x, q, scale, bias, y_old=None):
    """Independent restatement of the reference's ref_qmatmul (int64 accumulation of the same int8 values)."""
    rows, k = x.shape
    out = np.zeros((rows, q.shape[1]), np.float32)
    for r in range(rows):
        m = np.float32(np.max(np.abs(x[r]))) if k else np.float32(0)
        sx = np.float32(m / np.float32(127.0)) if m > 0 else np.float32(1.0)
        inv = np.float32(np.float32(1.0) / sx)
        v = np.rint((x[r] * inv).astype(np.float32))
        v = np.clip(v, -127, 127).astype(np.int64)
        acc = v @ q.astype(np.int64)
        y = (acc.astype(np.float32) * sx).astype(np.float32) * scale
        y = (y.astype(np.float32) + (bias if bias is not None else 0)).astype(np.float32)
        out[r] = y if y_old is None else (y_old[r] + y).astype(np.float32)
    return out


CASES = [(55, 31, 1), (64, 256, 1), (128, 512, 3), (114, 512, 32), (16, 16, 1), (1, 1, 1)]


def test_qmatmul_reference_cases():
    """reference test/model_test.c:387-412: kernel vs ref_qmatmul ≤ 1e-5 rel, accumulate 0/1"""
    rng = LCG()
    for k, n, rows in CASES:
        q, scale, bias, x = qcase(rng, k, n, rows)
        for acc in (0, 1):
            y_old = (np.arange(rows * n) % 7 * 0.5).astype(np.float32).reshape(rows, n)
            got = knx_ref.qmatmul(x, q, scale, bias, y_old=y_old if acc else None)
            want = int_reference(x, q, scale, bias, y_old if acc else None)
            mx = max(1e-30, float(np.max(np.abs(want))))
            assert float(np.max(np.abs(got - want))) / mx <= 1e-5
            assert np.array_equal(got, want)  # same arithmetic, no FMA: bit-exact


def test_qmatmul_nan_and_zero_rows():
    """reference test/model_test.c:413-426: a NaN makes its row all NaN; an all-zero row gives exactly bias"""
    rng = LCG()
    for k, n, rows in CASES:
        q, scale, bias, x = qcase(rng, k, n, rows)
        if rows < 3:
            continue
        x[1, 0] = np.nan
        x[2, :] = 0.0
        y = knx_ref.qmatmul(x, q, scale, bias)
        assert np.all(np.isnan(y[1]))
        assert np.array_equal(y[2], bias)
        want0 = int_reference(x[:1], q, scale, bias)
        assert np.allclose(y[0], want0[0], rtol=1e-5, atol=1e-5)
        x[0, 3] = np.inf
        assert np.all(np.isnan(knx_ref.qmatmul(x[:1], q, scale, bias)))


def test_qmatmul_int32_boundary():
    """reference test/model_test.c:428-441: K = 131072, q = −128, x = 1 → exact, no int32 overflow"""
    K = 131072
    q = np.full((K, 1), -128, np.int8)
    x = np.ones((1, K), np.float32)
    y, acc = knx_ref.qmatmul(x, q, np.ones(1, np.float32), None, return_acc=True)
    assert acc[0, 0] == -128 * 127 * K
    assert y[0, 0] == np.float32(np.float32(-128.0 * 127.0 * K) * (np.float32(1.0) / np.float32(127.0)))


def test_quantize_rows_rounding_and_scale():
    """per-row scale m/127 makes the largest |x| exactly ±127; ties round to even (NEON vcvtn / rintf)"""
    x = np.array([[127.0, 0.5, 1.5, 2.5, -0.5, -1.5, 126.5, -127.0],
                  [0.0] * 8,
                  [3.0, -1.0, 0.25, 1e-9, 0, 0, 0, 0]], np.float32)
    xq, sx, bad = knx_ref.quantize_rows(x)
    assert list(xq[0]) == [127, 0, 2, 2, 0, -2, 126, -127]
    assert sx[0] == 1.0 and sx[1] == 1.0 and not xq[1].any()
    assert xq[2, 0] == 127 and sx[2] == np.float32(3.0) / np.float32(127.0)
    rng = np.random.default_rng(0)
    x = rng.normal(0, 3, (50, 300)).astype(np.float32)
    xq, sx, _ = knx_ref.quantize_rows(x)
    assert np.all(np.abs(xq).max(axis=1) == 127)
    inv = (np.float32(1) / sx).astype(np.float32)
    assert np.all(np.abs(x * inv[:, None] - xq) <= 0.5 + 1e-3)


def test_i8gemm_accumulators_vs_int64_matmul():
    rng = np.random.default_rng(1)
    A = rng.integers(-127, 128, (33, 200), dtype=np.int8)
    W = rng.integers(-128, 128, (45, 200), dtype=np.int8)
    sa = rng.uniform(0.001, 0.01, 33).astype(np.float32)
    sw = rng.uniform(0.001, 0.01, 45).astype(np.float32)
    b = rng.normal(0, 0.1, 45).astype(np.float32)
    Y, acc = knx_ref.i8gemm(A, W, sa, sw, b, act_id=0)
    want = A.astype(np.int64) @ W.astype(np.int64).T
    assert np.array_equal(acc, want)
    v = (want.astype(np.float64) * sa[:, None] * sw[None, :] + b[None, :])
    assert np.allclose(Y, np.maximum(v, 0), rtol=1e-6, atol=1e-7)
    assert np.all(Y >= 0)


def test_qweight_unpack_exact():
    """reference test/model_test.c:403-404: unpack == (float)q·scale exactly (here: the dequantized file weight)"""
    rng = LCG()
    q, scale, _, _ = qcase(rng, 37, 19, 1)
    w = q.astype(np.float32) * scale[None, :]
    blob = struct.pack("<I", 1) + scale.astype("<f4").tobytes() + q.tobytes()
    r = knx_ref._R(blob)
    kind, w2 = knx_ref._weight(r, 2, 37, 19, False)
    assert kind == "f32" and np.array_equal(w2, w)


def test_quantize_cols_invariants():
    """quantizer of tools/knx_quant.py:18-25: per column max|q| = 127, all-zero column → scale 1, q 0, |w/s − q| ≤ ½,
    half-way values rounded to even; the C oracle and the package writer agree bit for bit"""
    rng = np.random.default_rng(2)
    w = rng.normal(0, 1, (70, 9))
    w[:, 3] = 0.0
    w[:, 5] = np.array([127.0, 63.5, -0.5, 1.5] + [0.0] * 66)  # scale exactly 1 → ties
    scale, q = knx_ref.quantize_cols(w)
    s2, q2 = knxfile.quantize(w, "column")
    assert np.array_equal(scale, s2) and np.array_equal(q, q2)
    assert scale[3] == 1.0 and not q[:, 3].any()
    assert list(q[:4, 5]) == [127, 64, 0, 2]
    for c in range(9):
        if c == 3:
            continue
        assert np.abs(q[:, c]).max() == 127
        assert np.all(np.abs(w[:, c] / np.float64(scale[c]) - q[:, c]) <= 0.5)
    # per-row axis
    sr, qr = knxfile.quantize(w.T, "row")
    assert np.array_equal(sr, scale) and np.array_equal(qr, q.T)


# ---------------------------------------------------------------- activations: closed forms in float64
def _gelu_exact(x):
    return 0.5 * x * (1.0 + np.array([math.erf(v / math.sqrt(2.0)) for v in x]))


def test_activations_closed_forms():
    x = np.linspace(-8, 8, 4001).astype(np.float32)
    xd = x.astype(np.float64)
    sig = 1.0 / (1.0 + np.exp(-xd))
    sp = np.log1p(np.exp(xd))
    r6 = np.clip(xd, 0, 6)
    forms = {
        0: np.maximum(xd, 0), 1: _gelu_exact(xd), 2: xd * sig, 3: sig, 4: np.tanh(xd), 5: np.where(xd < 0, 0.1 * xd, xd),
        6: np.where(xd < 0, 0.1 * np.expm1(xd), xd), 7: 1.0507009873554805 * np.where(xd < 0, 1.6732632423543772 * np.expm1(xd), xd),
        8: np.where(xd > 20, xd, sp), 9: r6, 10: np.clip(xd + 3, 0, 6) / 6, 11: xd * np.clip(xd + 3, 0, 6) / 6,
        12: 0.5 * xd * (1 + np.tanh(math.sqrt(2 / math.pi) * (xd + 0.044715 * xd ** 3))), 13: np.exp(xd),
        14: xd * np.tanh(sp), 15: xd / (1 + np.abs(xd)),
    }
    for a, want in forms.items():
        got = knx_ref.act(x, a, 0.1).astype(np.float64)
        tol = 4e-7 if a == 1 else 2e-7  # A&S 7.1.26: |erf error| ≤ 1.5e-7
        err = np.abs(got - want) / np.maximum(1.0, np.abs(want))
        assert err.max() <= tol, (a, float(err.max()))
    assert knx_ref.act(np.array([np.nan], np.float32), 0)[0] == 0.0  # threshold semantics


# ---------------------------------------------------------------- fp32 ops
def test_dense_layernorm_softmax_closed_forms():
    rng = np.random.default_rng(3)
    A = rng.normal(0, 1, (40, 300)).astype(np.float32)
    W = rng.normal(0, 0.1, (300, 70)).astype(np.float32)
    b = rng.normal(0, 0.1, 70).astype(np.float32)
    C = np.zeros((40, 70), np.float32)
    knx_ref.lib().ko_dense(40, 70, 300, knx_ref._p(A), knx_ref._p(W), knx_ref._p(b), -1, 0.0, knx_ref._p(C))
    want = A.astype(np.float64) @ W.astype(np.float64) + b
    assert np.max(np.abs(C - want)) <= 1e-5 * max(1, np.abs(want).max())
    assert not np.allclose(C, A.astype(np.float64) @ W.astype(np.float64))  # bias present
    x = rng.normal(2, 3, (20, 100)).astype(np.float32)
    g = rng.normal(1, 0.3, 100).astype(np.float32)
    bt = rng.normal(0, 0.3, 100).astype(np.float32)
    xd = x.astype(np.float64)
    mu, var = xd.mean(1, keepdims=True), xd.var(1, keepdims=True)
    want = (xd - mu) / np.sqrt(var + 1e-5) * g + bt
    assert np.max(np.abs(knx_ref.layernorm(x, g, bt, 1e-5) - want)) <= 1e-5
    plain = knx_ref.layernorm(x, None, None, 0.0).astype(np.float64)
    assert np.allclose(plain.mean(1), 0, atol=1e-6) and np.allclose(plain.var(1), 1, atol=1e-5)
    e = np.exp(xd - xd.max(1, keepdims=True))
    sm = knx_ref.softmax(x)
    assert np.max(np.abs(sm - e / e.sum(1, keepdims=True))) <= 1e-6 and np.allclose(sm.sum(1), 1, atol=1e-6)


def test_conv_vs_brute_force():
    """(ky, kx, ci)-ordered weight rows, stride, dilation, padding and groups against a direct 7-loop convolution"""
    rng = np.random.default_rng(4)
    for (B, H, W, C, Co, kh, kw, sh, sw, dh, dw, pt, pl, g) in [(2, 6, 5, 4, 6, 3, 2, 1, 2, 1, 1, 1, 0, 2),
                                                               (1, 7, 7, 3, 5, 3, 3, 2, 2, 2, 1, 2, 1, 1)]:
        cg, cog = C // g, Co // g
        Ho = (H + 2 * pt - dh * (kh - 1) - 1) // sh + 1
        Wo = (W + 2 * pl - dw * (kw - 1) - 1) // sw + 1
        x = rng.normal(0, 1, (B, H, W, C)).astype(np.float32)
        w = rng.normal(0, 1, (kh * kw * cg, Co)).astype(np.float32)
        b = rng.normal(0, 1, Co).astype(np.float32)
        want = np.zeros((B, Ho, Wo, Co))
        for bb in range(B):
            for oy in range(Ho):
                for ox in range(Wo):
                    for co in range(Co):
                        gi = co // cog
                        s = float(b[co])
                        for ky in range(kh):
                            for kx in range(kw):
                                iy, ix = oy * sh - pt + ky * dh, ox * sw - pl + kx * dw
                                if 0 <= iy < H and 0 <= ix < W:
                                    for ci in range(cg):
                                        s += float(x[bb, iy, ix, gi * cg + ci]) * float(w[(ky * kw + kx) * cg + ci, co])
                        want[bb, oy, ox, co] = s
        y = np.zeros((B * Ho * Wo, Co), np.float32)
        knx_ref.lib().ko_conv(B, H, W, C, Ho, Wo, Co, kh, kw, sh, sw, dh, dw, pt, pl, g, knx_ref._p(x), knx_ref._p(w),
                              knx_ref._p(b), -1, 0.0, knx_ref._p(y))
        assert np.max(np.abs(y - want.reshape(-1, Co))) <= 1e-5
        op = dict(cin=C, cout=Co, k=(kh, kw), s=(sh, sw), d=(dh, dw), p=(pt, pt, pl, pl), g=g, w=w, b=b)
        y2, _ = knx_ref._conv(x.reshape(-1, C), B, H, W, op)
        assert np.max(np.abs(y2 - want.reshape(-1, Co))) <= 1e-5


def test_attention_core_closed_form():
    rng = np.random.default_rng(5)
    B, H, Rq, S, dk, dv = 2, 3, 6, 6, 4, 5
    Q = rng.normal(0, 1, (B * Rq, H * dk)).astype(np.float32)
    K = rng.normal(0, 1, (B * S, H * dk)).astype(np.float32)
    V = rng.normal(0, 1, (B * S, H * dv)).astype(np.float32)
    for causal in (0, 1):
        got = np.zeros((B * Rq, H * dv), np.float32)
        knx_ref.lib().ko_attention_core(knx_ref._p(Q), knx_ref._p(K), knx_ref._p(V), knx_ref._p(got), B, H, Rq, S, dk, dv,
                                        float(1 / np.sqrt(dk)), causal)
        q = Q.reshape(B, Rq, H, dk).transpose(0, 2, 1, 3).astype(np.float64)
        k = K.reshape(B, S, H, dk).transpose(0, 2, 1, 3).astype(np.float64)
        v = V.reshape(B, S, H, dv).transpose(0, 2, 1, 3).astype(np.float64)
        s = q @ k.transpose(0, 1, 3, 2) / np.sqrt(dk)
        if causal:
            s = np.where(np.triu(np.ones((Rq, S), bool), 1), -np.inf, s)
        p = np.exp(s - s.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        want = (p @ v).transpose(0, 2, 1, 3).reshape(B * Rq, H * dv)
        assert np.max(np.abs(got - want)) <= 1e-5
        if causal:
            assert np.allclose(got.reshape(B, Rq, H, dv)[:, 0], V.reshape(B, S, H, dv)[:, 0], atol=1e-6)


def test_binary_and_global_pool_vs_numpy():
    rng = np.random.default_rng(6)
    B, R, C = 2, 5, 4
    a = rng.normal(0, 1, (B, R, C)).astype(np.float32)
    b = rng.normal(0, 1, (B, 1, C)).astype(np.float32) + 3
    for op, fn in enumerate([np.add, np.subtract, np.multiply, np.divide, np.maximum, np.minimum]):
        y = np.zeros((B * R, C), np.float32)
        knx_ref.lib().ko_binary(op, knx_ref._p(a), R, C, knx_ref._p(b), 1, C, knx_ref._p(y), B, R, C)
        assert np.array_equal(y, fn(a, b).reshape(-1, C).astype(np.float32))
    x = rng.normal(0, 1, (B, R, C)).astype(np.float32)
    for t in (0, 1):
        y = np.zeros((B, C), np.float32)
        knx_ref.lib().ko_global_pool(t, knx_ref._p(x), B, R, C, knx_ref._p(y))
        want = x.max(1) if t == 0 else x.astype(np.float64).mean(1)
        assert np.allclose(y, want, atol=1e-6)


# ---------------------------------------------------------------- model-level known answers
def test_v2_zero_column_gives_bias(tmp_path):
    """reference test/model_test.c:492-509: all-zero int8 column (scale 1) → exactly its bias"""
    zq = np.array([10, 0, 20, 0, 30, 0, 40, 0], np.int8).reshape(4, 2)
    zs = np.array([0.02, 1.0], np.float32)
    zb = np.array([0.25, -0.75], np.float32)
    blob = b"KNX2" + struct.pack("<6I", 1, 0, 4, 2, 1, 1) + zs.astype("<f4").tobytes() + zq.tobytes() + zb.astype("<f4").tobytes()
    p = tmp_path / "v2.knx"
    p.write_bytes(blob)
    m = knx_ref.parse(str(p))
    x = np.array([[1.0, -2.0, 0.5, 3.0]], np.float32)
    y, _ = knx_ref.forward(m, x)
    assert y[0, 1] == np.float32(-0.75)
    assert abs(y[0, 0] - int_reference(x, zq, zs, zb)[0, 0]) <= 1e-6


def test_lstm_vs_double_reference():
    """reference test/model_test.c:219-239 (ref_lstm, double accumulation, Keras gate order i f g o)"""
    rng = np.random.default_rng(7)
    T, cin, u, B = 4, 7, 5, 3
    W = rng.uniform(-0.5, 0.5, (cin, 4 * u)).astype(np.float32)
    U = rng.uniform(-0.5, 0.5, (u, 4 * u)).astype(np.float32)
    bias = rng.uniform(-0.5, 0.5, 4 * u).astype(np.float32)
    x = rng.normal(0, 1, (B * T, cin)).astype(np.float32)
    op = dict(kind=4, u=u, act=4, ret=1, dirs=[(W, ("f32", U), bias)], merge=0)
    y, _ = knx_ref._rnn(op, x, (T, cin), B, "ref")
    sig = lambda v: 1 / (1 + np.exp(-v))  # noqa: E731
    want = np.zeros((B, T, u))
    for b in range(B):
        h = np.zeros(u)
        c = np.zeros(u)
        for t in range(T):
            z = bias + x[b * T + t].astype(np.float64) @ W + h @ U
            c = sig(z[u:2 * u]) * c + sig(z[:u]) * np.tanh(z[2 * u:3 * u])
            h = sig(z[3 * u:]) * np.tanh(c)
            want[b, t] = h
    assert np.max(np.abs(y.reshape(B, T, u) - want)) <= 1e-5
