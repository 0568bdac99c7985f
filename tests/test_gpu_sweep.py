"""Randomized parity sweep through the C ABI over shapes drawn log-uniformly within each entry point's contract: the
int8 GEMM (with accumulate, residual and raw accumulators), the row quantizer (zero, NaN, ±inf and integral rows),
the quantize + int8 GEMM call (both of its paths), the fp32 NT GEMM, the convolutions (groups, depthwise, stride,
dilation, asymmetric padding, both weight layouts, residual), the row and elementwise ops and the attention core.
The dispatch rules pick a different kernel by shape, so a sweep reaches tile/edge combinations that fixed cases miss.

References: int8 — exact int32 sums (float64 products of int8 values are exact integers below 2^53) and the
epilogue's fp32 steps in order, bit-exact (reference include/kernix_model.h:112-178); fp32 GEMM and convolution —
float64, max|a−b| / max(1, max|ref|) ≤ 1e-4 (reference include/kernix.h:951-977, include/kernix_model.h:711-771);
row ops, activations, binary ops and attention — the oracle's restatements, at the tolerances of their kernel tests.
"""
import ctypes

import numpy as np
import pytest

from kernix_amd import hipabi
from kernix_amd.hipabi import ptr

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
F32 = np.float32


@pytest.fixture(scope="module")
def L():
    lib = hipabi.lib()
    hipabi.check(lib.knx_hip_init())
    return lib


class Device:
    """Device copies that stay alive until the case is checked (a freed tensor's memory can be handed out again)."""

    def __init__(self):
        self.held = []

    def __call__(self, a):
        if a is None:
            return None
        t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
        self.held.append(t)
        return t


def opt(t):
    return ptr(t) if t is not None else None


def logu(rng, lo, hi):
    return int(np.exp(rng.uniform(np.log(lo), np.log(hi + 1))))


def epilogue(acc, sa, sw, bias, act, yold=None, R=None):
    """((float)acc · sa[m]) · sw[n] (+ bias[n]) (+ Y) → act (none / ReLU) (+ R), each step rounded to fp32"""
    v = acc.astype(F32) * sa[:, None]
    v = (v * sw[None, :]).astype(F32)
    if bias is not None:
        v = (v + bias[None, :]).astype(F32)
    if yold is not None:
        v = (yold + v).astype(F32)
    if act == 0:
        v = np.where(v >= 0, v, F32(0)).astype(F32)
    if R is not None:
        v = (v + R).astype(F32)
    return v


def quantize(x, k, kp):
    """per row: s = max|x|/127 (1 for a zero row, NaN for a row with NaN or ±inf, its bytes 0), q = clamp(rint(x/s))"""
    q = np.zeros((x.shape[0], kp), np.int8)
    s = np.zeros(x.shape[0], F32)
    for r in range(x.shape[0]):
        a = np.abs(x[r, :k])
        if not np.all(np.isfinite(a)):
            s[r] = np.nan
            continue
        m = a.max()
        sx = F32(m) / F32(127) if m > 0 else F32(1)
        inv = F32(1) / F32(sx)
        q[r, :k] = np.clip(np.rint((x[r, :k] * inv).astype(F32)), -127, 127).astype(np.int8)
        s[r] = sx
    return q, s


def int_dot(a, w):
    return (a.astype(np.float64) @ w.astype(np.float64).T).astype(np.int64).astype(np.int32)


def rel_err(got, want):
    return float(np.max(np.abs(got - want)) / max(1.0, float(np.max(np.abs(want))))) if want.size else 0.0


@pytest.mark.parametrize("seed", [1, 2])
def test_i8gemm_sweep(L, seed):
    rng = np.random.default_rng(seed)
    st = hipabi.stream()
    for case in range(60):
        M, N, K = logu(rng, 1, 3000), logu(rng, 1, 3000), 64 * logu(rng, 1, 64)
        lda, ldw = K + 16 * int(rng.integers(0, 2)), K + 16 * int(rng.integers(0, 2))
        act, hasb = int(rng.choice([-1, 0])), bool(rng.random() < 0.7)
        accu = int(rng.random() < 0.2)
        res = not accu and rng.random() < 0.3
        raw = not res and rng.random() < 0.3
        ldy = N + int(rng.integers(0, 5))
        name = f"case {case}: M {M} N {N} K {K} lda {lda} ldw {ldw} act {act} bias {hasb} accumulate {accu} res {res}"
        print(name, flush=True)
        A = rng.integers(-127, 128, (M, lda), dtype=np.int8)
        W = rng.integers(-127, 128, (N, ldw), dtype=np.int8)
        A[:, K:] = 0
        W[:, K:] = 0
        sa, sw = rng.uniform(0.001, 0.02, M).astype(F32), rng.uniform(0.001, 0.02, N).astype(F32)
        b = rng.normal(0, 1, N).astype(F32) if hasb else None
        Y0 = rng.normal(0, 1, (M, ldy)).astype(F32)
        R = rng.normal(0, 1, (M, ldy)).astype(F32) if res else None
        d = Device()
        dY = d(Y0)
        dacc = torch.zeros((M, N), dtype=torch.int32, device="cuda") if raw else None
        if res:
            hipabi.check(L.knx_hip_i8gemm_res(M, N, K, ptr(d(A)), lda, ptr(d(sa)), ptr(d(W)), ldw, ptr(d(sw)), opt(d(b)),
                                              act, 0.0, ptr(d(R)), ldy, ptr(dY), ldy, st))
        else:
            hipabi.check(L.knx_hip_i8gemm(M, N, K, ptr(d(A)), lda, ptr(d(sa)), ptr(d(W)), ldw, ptr(d(sw)), opt(d(b)), act,
                                          0.0, accu, ptr(dY), ldy, opt(dacc), N, st))
        torch.cuda.synchronize()
        acc = int_dot(A[:, :K], W[:, :K])
        want = epilogue(acc, sa, sw, b, act, Y0[:, :N] if accu else None, R[:, :N] if res else None)
        got = dY.cpu().numpy()
        assert np.array_equal(got[:, :N], want), name
        assert np.array_equal(got[:, N:], Y0[:, N:]), name  # the row padding is not written
        if raw:
            assert np.array_equal(dacc.cpu().numpy(), acc), name


@pytest.mark.parametrize("seed", [1, 2])
def test_quantize_rows_sweep(L, seed):
    rng = np.random.default_rng(seed)
    st = hipabi.stream()
    for case in range(60):
        rows, k = logu(rng, 1, 5000), logu(rng, 1, 4096)
        kp = (k + 63) // 64 * 64 + 64 * int(rng.integers(0, 2))
        ldq, ldx = kp + 16 * int(rng.integers(0, 3)), k + int(rng.integers(0, 9))
        name = f"case {case}: rows {rows} k {k} kp {kp} ldq {ldq} ldx {ldx}"
        print(name, flush=True)
        x = rng.normal(0, 1, (rows, ldx)).astype(F32) * rng.uniform(0.01, 100, (rows, 1)).astype(F32)
        for r in rng.choice(rows, min(rows, 3), replace=False):
            kind = int(rng.integers(0, 4))
            if kind == 0:
                x[r, :k] = 0
            elif kind == 1:
                x[r, int(rng.integers(0, k))] = np.inf
            elif kind == 2:
                x[r, int(rng.integers(0, k))] = np.nan
            else:
                x[r, :k] = np.round(x[r, :k])  # integral values: exact ties after scaling are likelier
        d = Device()
        dq = torch.full((rows, ldq), 99, dtype=torch.int8, device="cuda")
        ds = torch.zeros(rows, device="cuda")
        hipabi.check(L.knx_hip_quantize_rows(ptr(d(x)), ldx, rows, k, kp, ptr(dq), ldq, ptr(ds), st))
        torch.cuda.synchronize()
        q, s = quantize(x, k, kp)
        gq, gs = dq.cpu().numpy(), ds.cpu().numpy()
        assert np.array_equal(gq[:, :kp], q), name
        assert np.all(gq[:, kp:] == 99), name  # past kp nothing is written
        assert np.array_equal(np.isnan(gs), np.isnan(s)) and np.array_equal(gs[~np.isnan(s)], s[~np.isnan(s)]), name


@pytest.mark.parametrize("seed", [1, 2])
def test_qlinear_sweep(L, seed):
    """both paths of knx_hip_qlinear (the quantizer inside the GEMM at <= 16 rows, else the quantizer then the GEMM)"""
    rng = np.random.default_rng(seed)
    st = hipabi.stream()
    for case in range(50):
        rows, k, n = logu(rng, 1, 300), logu(rng, 1, 3000), logu(rng, 1, 3000)
        kp = (k + 63) // 64 * 64
        ldw, ldx = kp + 16 * int(rng.integers(0, 2)), k + int(rng.integers(0, 5))
        act, hasb, res = int(rng.choice([-1, 0])), bool(rng.random() < 0.7), bool(rng.random() < 0.3)
        name = f"case {case}: rows {rows} k {k} n {n} kp {kp} ldw {ldw} ldx {ldx} act {act} bias {hasb} res {res}"
        print(name, flush=True)
        x = rng.normal(0, 1, (rows, ldx)).astype(F32)
        W = rng.integers(-127, 128, (n, ldw), dtype=np.int8)
        W[:, k:] = 0
        sw = rng.uniform(0.001, 0.02, n).astype(F32)
        b = rng.normal(0, 1, n).astype(F32) if hasb else None
        R = rng.normal(0, 1, (rows, n)).astype(F32) if res else None
        d = Device()
        dxq = torch.zeros((rows, kp), dtype=torch.int8, device="cuda")
        dsx = torch.zeros(rows, device="cuda")
        dY = torch.full((rows, n), 5.0, device="cuda")
        hipabi.check(L.knx_hip_qlinear(ptr(d(x)), ldx, rows, k, kp, ptr(dxq), ptr(dsx), ptr(d(W)), ldw, n, ptr(d(sw)),
                                       opt(d(b)), act, 0.0, 0, opt(d(R)), n, ptr(dY), n, st))
        torch.cuda.synchronize()
        q, s = quantize(x, k, kp)
        assert np.array_equal(dY.cpu().numpy(), epilogue(int_dot(q[:, :k], W[:, :k]), s, sw, b, act, None, R)), name


@pytest.mark.parametrize("seed", [1, 2])
def test_sgemm_nt_sweep(L, seed):
    rng = np.random.default_rng(seed)
    st = hipabi.stream()
    for case in range(50):
        M, N, K = logu(rng, 1, 3000), logu(rng, 1, 3000), logu(rng, 1, 2048)
        lda, ldb, ldc = K + int(rng.integers(0, 9)), K + int(rng.integers(0, 9)), N + int(rng.integers(0, 5))
        act, hasb = int(rng.choice([-1, 0, 1])), bool(rng.random() < 0.7)
        name = f"case {case}: M {M} N {N} K {K} lda {lda} ldb {ldb} ldc {ldc} act {act} bias {hasb}"
        print(name, flush=True)
        A = rng.normal(0, 1, (M, lda)).astype(F32)
        B = rng.normal(0, 1, (N, ldb)).astype(F32)
        b = rng.normal(0, 1, N).astype(F32) if hasb else None
        d = Device()
        dC = d(np.full((M, ldc), 3.0, F32))
        hipabi.check(L.knx_hip_sgemm_nt_ep(M, N, K, ptr(d(A)), lda, ptr(d(B)), ldb, opt(d(b)), act, 0.0, ptr(dC), ldc, st))
        torch.cuda.synchronize()
        ref = A[:, :K].astype(np.float64) @ B[:, :K].astype(np.float64).T
        if hasb:
            ref = ref + b[None, :]
        if act == 0:
            ref = np.maximum(ref, 0)
        elif act == 1:
            ref = torch.nn.functional.gelu(torch.from_numpy(ref)).numpy()
        got = dC.cpu().numpy()
        assert rel_err(got[:, :N], ref) <= 1e-4, name
        assert np.all(got[:, N:] == 3.0), name


@pytest.mark.parametrize("seed", [1, 2])
def test_conv_sweep(L, seed):
    import torch.nn.functional as Fn

    rng = np.random.default_rng(seed)
    st = hipabi.stream()
    for case in range(60):
        g = int(rng.choice([1, 1, 1, 2, 4]))
        C = g * int(rng.choice([1, 2, 3, 4, 8, 16, 32, 64] if g == 1 else [1, 2, 8, 16, 32]))
        Co = g * int(rng.choice([1, 3, 8, 16, 32, 64, 96, 128] if g == 1 else [1, 4, 16, 32]))
        if g == 1 and rng.random() < 0.15:
            g = C = Co = int(rng.choice([8, 32, 64]))  # depthwise
        kh, kw = int(rng.integers(1, 6)), int(rng.integers(1, 6))
        sh, sw = int(rng.integers(1, 4)), int(rng.integers(1, 4))
        dh, dw = int(rng.integers(1, 3)), int(rng.integers(1, 3))
        B, H, W = logu(rng, 1, 16), logu(rng, 1, 40), logu(rng, 1, 40)
        pt, pb = int(rng.integers(0, kh)), int(rng.integers(0, kh))
        pl, pr = int(rng.integers(0, kw)), int(rng.integers(0, kw))
        Ho = (H + pt + pb - dh * (kh - 1) - 1) // sh + 1
        Wo = (W + pl + pr - dw * (kw - 1) - 1) // sw + 1
        if Ho < 1 or Wo < 1:
            continue
        act, hasb, res = int(rng.choice([-1, 0])), bool(rng.random() < 0.7), bool(rng.random() < 0.3)
        transposed = res or rng.random() < 0.6
        name = (f"case {case}: B {B} H {H} W {W} C {C} Co {Co} k {kh}x{kw} s {sh}x{sw} d {dh}x{dw} pad {pt},{pb},{pl},{pr}"
                f" groups {g} act {act} bias {hasb} res {res} transposed {transposed}")
        print(name, flush=True)
        x = rng.normal(0, 1, (B, H, W, C)).astype(F32)
        wt = rng.normal(0, 0.2, (Co, kh, kw, C // g)).astype(F32)  # Co × (ky, kx, ci)
        b = rng.normal(0, 1, Co).astype(F32) if hasb else None
        R = rng.normal(0, 1, (B, Ho, Wo, Co)).astype(F32) if res else None
        geom = hipabi.ConvGeom(B, H, W, C, Ho, Wo, Co, kh, kw, sh, sw, dh, dw, pt, pl, g)
        d = Device()
        dy = torch.full((B, Ho, Wo, Co), 7.0, device="cuda")
        if res:
            hipabi.check(L.knx_hip_conv_t_res(ctypes.byref(geom), ptr(d(x)), ptr(d(wt.reshape(Co, -1))), opt(d(b)), act, 0.0,
                                              ptr(d(R)), ptr(dy), st))
        elif transposed:
            hipabi.check(L.knx_hip_conv_t(ctypes.byref(geom), ptr(d(x)), ptr(d(wt.reshape(Co, -1))), opt(d(b)), act, 0.0,
                                          ptr(dy), st))
        else:  # (ky, kx, ci) rows × Co columns
            hipabi.check(L.knx_hip_conv(ctypes.byref(geom), ptr(d(x)), ptr(d(wt.reshape(Co, -1).T)), opt(d(b)), act, 0.0,
                                        ptr(dy), st))
        torch.cuda.synchronize()
        xt = Fn.pad(torch.from_numpy(x).double().permute(0, 3, 1, 2), (pl, pr, pt, pb))
        ref = Fn.conv2d(xt, torch.from_numpy(wt).double().permute(0, 3, 1, 2),
                        torch.from_numpy(b).double() if hasb else None, stride=(sh, sw), dilation=(dh, dw), groups=g)
        if act == 0:
            ref = torch.relu(ref)
        ref = ref.permute(0, 2, 3, 1).numpy()
        if res:
            ref = ref + R
        assert rel_err(dy.cpu().numpy(), ref) <= 1e-4, name


@pytest.mark.parametrize("seed", [1, 2])
def test_row_ops_sweep(L, seed):
    """layer_norm (in place or not), layer_norm + quantize (the bits of layer_norm then the quantizer), softmax with
    masked (−inf) entries, bias + each activation, elementwise binary ops with broadcast rows or channels: against the
    oracle's restatements (layer_norm 1e-5, activations 2e-6 as their kernel test, binary ops and the quantized rows
    bit-exact) and softmax against float64 (1e-5)"""
    from oracle import knx_ref

    rng = np.random.default_rng(seed)
    st = hipabi.stream()
    for case in range(40):
        rows, cols = logu(rng, 1, 20000), logu(rng, 1, 4096)
        while rows * cols > 2e7:
            rows //= 2
        inplace, eps = bool(rng.random() < 0.5), float(rng.choice([1e-5, 1e-6, 1e-3]))
        act = int(rng.integers(-1, 16))
        name = f"case {case}: rows {rows} cols {cols} in place {inplace} eps {eps} act {act}"
        print(name, flush=True)
        x = (rng.standard_normal((rows, cols)) * 3).astype(F32)
        g = (1 + rng.normal(0, 0.5, cols)).astype(F32)
        bt = rng.normal(0, 0.5, cols).astype(F32)
        d = Device()
        dx = d(x)
        y = dx if inplace else torch.empty_like(dx)
        hipabi.check(L.knx_hip_layernorm(ptr(dx), ptr(y), rows, cols, ptr(d(g)), ptr(d(bt)), eps, st))
        torch.cuda.synchronize()
        ln = y.cpu().numpy()
        assert rel_err(ln, knx_ref.layernorm(x, g, bt, eps)) <= 1e-5, name
        if cols % 4 == 0 and cols <= 2048:
            kp = cols + 4 * int(rng.integers(0, 17))
            dxq = torch.full((rows, kp), 99, dtype=torch.int8, device="cuda")
            dsx = torch.zeros(rows, device="cuda")
            dx2 = d(x)
            hipabi.check(L.knx_hip_layernorm_quantize(ptr(dx2), rows, cols, ptr(d(g)), ptr(d(bt)), eps, kp, ptr(dxq),
                                                      ptr(dsx), st))
            torch.cuda.synchronize()
            q, s = quantize(ln, cols, kp)  # the GPU layer_norm's own bits, quantized
            assert np.array_equal(dxq.cpu().numpy(), q) and np.array_equal(dsx.cpu().numpy(), s), name
        xm = x.copy()
        if cols >= 2:
            for r in rng.choice(rows, min(rows, 5), replace=False):
                xm[r, int(rng.integers(1, cols)):] = -np.inf  # a causal row's masked tail (never the whole row)
        dm = d(xm)
        hipabi.check(L.knx_hip_softmax(ptr(dm), ptr(dm), rows, cols, st))
        torch.cuda.synchronize()
        xd = xm.astype(np.float64)
        e = np.exp(xd - xd.max(axis=1, keepdims=True))
        # against float64: the oracle's sequential float32 row sum (the reference's order) itself drifts by up to
        # 1.5e-5 at 4096 columns
        assert rel_err(dm.cpu().numpy(), e / e.sum(axis=1, keepdims=True)) <= 1e-5, name
        xa = (x * 4 / 3).astype(F32)
        ba = rng.normal(0, 1, cols).astype(F32)
        da = d(xa)
        hipabi.check(L.knx_hip_bias_act(ptr(da), ptr(da), rows, cols, ptr(d(ba)), act, 0.2, st))
        torch.cuda.synchronize()
        xb = (xa + ba).astype(F32)
        want = xb if act == -1 else knx_ref.act(xb, act, 0.2)
        assert np.allclose(da.cpu().numpy(), want, rtol=2e-6, atol=2e-6, equal_nan=True), name
    for case in range(60):
        op = int(rng.integers(0, 6))
        B, R, C = logu(rng, 1, 16), logu(rng, 1, 300), logu(rng, 1, 600)
        ra, ca = (R if rng.random() < 0.7 else 1), (C if rng.random() < 0.7 else 1)
        rb, cb = (R if rng.random() < 0.7 else 1), (C if rng.random() < 0.7 else 1)
        alias = ra == R and ca == C and rng.random() < 0.3
        name = f"binary {case}: op {op} B {B} R {R} C {C} a {ra}x{ca} b {rb}x{cb} y is a {alias}"
        print(name, flush=True)
        a = rng.normal(0, 1, (B * ra, ca)).astype(F32)
        b = (rng.normal(0, 1, (B * rb, cb)) + 2.5).astype(F32)
        want = np.zeros((B * R, C), F32)
        knx_ref.lib().ko_binary(op, knx_ref._p(a), ra, ca, knx_ref._p(b), rb, cb, knx_ref._p(want), B, R, C)
        d = Device()
        da = d(a)
        y = da if alias else torch.empty((B * R, C), dtype=torch.float32, device="cuda")
        hipabi.check(L.knx_hip_binary(op, ptr(da), ra, ca, ptr(d(b)), rb, cb, ptr(y), B, R, C, st))
        torch.cuda.synchronize()
        assert np.array_equal(y.cpu().numpy(), want), name


@pytest.mark.parametrize("seed", [1, 2])
def test_attention_sweep(L, seed):
    """the attention core (fused where the shape allows, else the scores GEMM, softmax and P·V) over random batch,
    heads, query and key counts, head widths, causal masks, and the strided form with and without the Vᵀ scratch,
    against the oracle's loop (reference include/kernix_model.h:1021-1046), 1e-4"""
    from oracle import knx_ref

    rng = np.random.default_rng(seed)
    st = hipabi.stream()
    for case in range(40):
        B, H, Rq, S = logu(rng, 1, 16), logu(rng, 1, 8), logu(rng, 1, 300), logu(rng, 1, 300)
        while B * H * Rq * S > 4e6:
            B = max(1, B // 2)
            if B == 1:
                Rq = max(1, Rq // 2)
        dk = int(rng.choice([4, 8, 16, 32, 64, 128])) if rng.random() < 0.7 else logu(rng, 1, 128)
        dv = dk if rng.random() < 0.6 else logu(rng, 1, 128)
        causal, strided = int(rng.random() < 0.5), bool(rng.random() < 0.4)
        use_vt = strided and rng.random() < 0.5
        name = f"case {case}: B {B} H {H} Rq {Rq} S {S} dk {dk} dv {dv} causal {causal} strided {strided} vt {use_vt}"
        print(name, flush=True)
        Q = rng.standard_normal((B * Rq, H * dk)).astype(F32)
        K = rng.standard_normal((B * S, H * dk)).astype(F32)
        V = rng.standard_normal((B * S, H * dv)).astype(F32)
        scale = F32(1.0) / np.sqrt(F32(dk))
        want = np.zeros((B * Rq, H * dv), F32)
        knx_ref.lib().ko_attention_core(knx_ref._p(Q), knx_ref._p(K), knx_ref._p(V), knx_ref._p(want), B, H, Rq, S, dk,
                                        dv, float(scale), causal)
        d = Device()
        ctx = torch.empty((B * Rq, H * dv), dtype=torch.float32, device="cuda")
        sc = torch.empty((B * H * Rq, S), dtype=torch.float32, device="cuda")
        if strided:
            pq, pk, pv = (4 * int(rng.integers(0, 3)) for _ in range(3))  # row padding (16-byte steps)
            Qp = np.zeros((B * Rq, H * dk + pq), F32)
            Kp = np.zeros((B * S, H * dk + pk), F32)
            Vp = np.zeros((B * S, H * dv + pv), F32)
            Qp[:, :H * dk], Kp[:, :H * dk], Vp[:, :H * dv] = Q, K, V
            dvt = torch.empty((H * dv, B * S), dtype=torch.float32, device="cuda") if use_vt else None
            hipabi.check(L.knx_hip_attention_core_ex(ptr(d(Qp)), H * dk + pq, ptr(d(Kp)), H * dk + pk, ptr(d(Vp)),
                                                     H * dv + pv, opt(dvt), ptr(ctx), ptr(sc), B, H, Rq, S, dk, dv,
                                                     float(scale), causal, st))
        else:
            hipabi.check(L.knx_hip_attention_core(ptr(d(Q)), ptr(d(K)), ptr(d(V)), ptr(ctx), ptr(sc), B, H, Rq, S, dk,
                                                  dv, float(scale), causal, st))
        torch.cuda.synchronize()
        got = ctx.cpu().numpy()
        ok = np.isfinite(want)  # a causal query row with no key at or before it has an empty softmax
        assert np.array_equal(np.isfinite(got), ok), name
        assert rel_err(got[ok], want[ok]) <= 1e-4, name
