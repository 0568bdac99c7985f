"""CPU oracle for whole-model forward of .knx files.  TEST INFRASTRUCTURE ONLY.

An independent restatement of the reference's runtime semantics (reference include/kernix_model.h), used by tests/
and bench.py's cpu_baseline leg to check the GPU library.  It parses .knx bytes itself (sharing no code with the
product's C loader) and computes every op on the CPU:
  - GEMMs (Linear, convolution, attention projections and products) in float64, rounded to float32 per op —
    the closed form the reference's Accelerate/AMX path approximates (pinned in the reference only by tolerance);
  - int8 Linear / recurrence in the reference's int8 arithmetic (per-row int8 input, int32 accumulation,
    ((float)acc·sx)·scale + bias) through the C oracle (knx_oracle.c), bit-exact by construction;
  - activations, layer_norm, softmax through the C oracle (float32, the reference formulas).
int8 dispatch: mode "ref" uses the int8 arithmetic at ≤ 2 rows and the dequantized float copy above (reference
include/kernix_model.h:1853-1860); mode "i8" uses the int8 arithmetic at every row count.
"""
import ctypes
import os
import struct

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libknx_oracle.so")
INT8_MAX_ROWS = 2

_lib = None


def lib():
    """The C oracle (built by oracle/Makefile)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            import subprocess
            subprocess.run(["make", "-s", "-C", HERE], check=True)
        L = ctypes.CDLL(LIB_PATH)
        P, I, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
        sig = {
            "ko_set_threads": ([I], None), "ko_get_threads": ([], I),
            "ko_quantize_cols": ([P, I, I, P, P], None),
            "ko_quantize_rows": ([P, I, I, P, P, P], None),
            "ko_qmatmul": ([P, I, I, I, P, P, P, I, P, P], None),
            "ko_i8gemm": ([I, I, I, P, P, P, P, P, I, F, P, P], None),
            "ko_act": ([P, ctypes.c_size_t, I, F], None),
            "ko_dense": ([I, I, I, P, P, P, I, F, P], None),
            "ko_dense_f64": ([I, I, I, P, P, P, I, F, P], None),
            "ko_layernorm": ([P, P, I, I, P, P, F], None),
            "ko_softmax": ([P, P, I, I], None),
            "ko_conv": ([I] * 16 + [P, P, P, I, F, P], None),
            "ko_attention_core": ([P, P, P, P, I, I, I, I, I, I, F, I], None),
            "ko_binary": ([I, P, I, I, P, I, I, P, I, I, I], None),
            "ko_global_pool": ([I, P, I, I, I, P], None),
        }
        for name, (args, res) in sig.items():
            f = getattr(L, name)
            f.argtypes, f.restype = args, res
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


def f32c(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---------------------------------------------------------------- C oracle wrappers
def act(x, a, alpha=0.0):
    y = f32c(x).copy()
    if a is not None and a >= 0:
        lib().ko_act(_p(y), y.size, int(a), float(alpha))
    return y


def qmatmul(x, q_kn, scale, bias=None, y_old=None, return_acc=False):
    """Reference int8 product: x rows×k fp32, q k×n int8 (file layout), scale n."""
    x = f32c(x)
    rows, k = x.shape
    n = q_kn.shape[1]
    q = np.ascontiguousarray(q_kn, dtype=np.int8)
    y = f32c(y_old).copy() if y_old is not None else np.zeros((rows, n), np.float32)
    acc = np.zeros((rows, n), np.int32)
    lib().ko_qmatmul(_p(x), rows, k, n, _p(q), _p(f32c(scale)), _p(None if bias is None else f32c(bias)),
                     int(y_old is not None), _p(y), _p(acc))
    return (y, acc) if return_acc else y


def quantize_rows(x):
    x = f32c(x)
    rows, k = x.shape
    xq = np.zeros((rows, k), np.int8)
    sx = np.zeros(rows, np.float32)
    bad = np.zeros(rows, np.int32)
    lib().ko_quantize_rows(_p(x), rows, k, _p(xq), _p(sx), _p(bad))
    return xq, sx, bad


def i8gemm(A, W, sa, sw, bias, act_id=0, alpha=0.0, want_y=True, threads=None):
    A = np.ascontiguousarray(A, np.int8)
    W = np.ascontiguousarray(W, np.int8)
    M, K = A.shape
    N = W.shape[0]
    Y = np.zeros((M, N), np.float32) if want_y else None
    acc = np.zeros((M, N), np.int32)
    L = lib()
    old = L.ko_get_threads()
    if threads:
        L.ko_set_threads(int(threads))
    try:
        L.ko_i8gemm(M, N, K, _p(A), _p(f32c(sa)), _p(W), _p(f32c(sw)), _p(None if bias is None else f32c(bias)),
                    int(act_id), float(alpha), _p(Y), _p(acc))
    finally:
        L.ko_set_threads(old)
    return Y, acc


def quantize_cols(w):
    w = np.ascontiguousarray(w, np.float64)
    k, n = w.shape
    scale = np.zeros(n, np.float32)
    q = np.zeros((k, n), np.int8)
    lib().ko_quantize_cols(_p(w), k, n, _p(scale), _p(q))
    return scale, q


def layernorm(x, gamma, beta, eps):
    x = f32c(x)
    y = np.empty_like(x)
    lib().ko_layernorm(_p(x), _p(y), x.shape[0], x.shape[1], _p(None if gamma is None else f32c(gamma)),
                       _p(None if beta is None else f32c(beta)), float(eps))
    return y


def softmax(x):
    x = f32c(x)
    y = np.empty_like(x)
    lib().ko_softmax(_p(x), _p(y), x.shape[0], x.shape[1])
    return y


def dense64(x, w, b=None):
    y = np.asarray(x, np.float64) @ np.asarray(w, np.float64)
    if b is not None:
        y = y + np.asarray(b, np.float64)
    return y.astype(np.float32)


# ---------------------------------------------------------------- .knx parsing
class _R:
    def __init__(self, data):
        self.d, self.o = data, 0

    def u32(self, n=1):
        v = struct.unpack_from(f"<{n}I", self.d, self.o)
        self.o += 4 * n
        return v if n > 1 else v[0]

    def f32(self, n):
        v = np.frombuffer(self.d, "<f4", n, self.o).astype(np.float32)
        self.o += 4 * n
        return v

    def i8(self, n):
        v = np.frombuffer(self.d, np.int8, n, self.o).copy()
        self.o += n
        return v


def _weight(r, ver, k, n, keep_int8):
    """→ ("f32", W k×n) or ("i8", q k×n, scale n)"""
    dt = r.u32() if ver >= 2 else 0
    if dt == 0:
        return ("f32", r.f32(k * n).reshape(k, n))
    ns = n if dt == 1 else k
    sc = r.f32(ns)
    q = r.i8(k * n).reshape(k, n)
    if keep_int8 and dt == 1:
        return ("i8", q, sc)
    w = q.astype(np.float32) * (sc[None, :] if dt == 1 else sc[:, None])
    return ("f32", w.astype(np.float32))


def parse(path):
    data = open(path, "rb").read()
    r = _R(data)
    magic = data[:4]
    r.o = 4
    ver = {b"KNX1": 1, b"KNX2": 2, b"KNX3": 3}[magic]
    n_ops = r.u32()
    layout, in_shape = 0, None
    if ver == 3:
        layout, nd = r.u32(2)
        in_shape = tuple(int(v) for v in (r.u32(nd) if nd > 1 else (r.u32(),)))
    ops = []
    for i in range(n_ops):
        kind = r.u32()
        if ver == 3:
            n_in = r.u32()
            inp = list(r.u32(n_in)) if n_in > 1 else [r.u32()]
        else:
            inp = [i]
        op = dict(kind=kind, inp=inp)
        if kind == 0:  # LINEAR
            k, n, hb = r.u32(3)
            op.update(k=k, n=n, w=_weight(r, ver, k, n, True), b=r.f32(n) if hb else None)
        elif kind == 1:  # ACT
            op["act"] = r.u32()
            op["alpha"] = float(r.f32(1)[0]) if ver >= 3 else 0.0
        elif kind == 2:  # LAYERNORM
            c, aff = r.u32(2)
            op["cols"] = c
            op["eps"] = float(r.f32(1)[0])
            op["g"], op["b"] = (r.f32(c), r.f32(c)) if aff else (None, None)
        elif kind == 3:
            pass
        elif kind in (4, 5, 6):  # LSTM / GRU / RNN
            G = {4: 4, 5: 3, 6: 1}[kind]
            seq = None
            if ver < 3:
                cin, u, a, ret, seq = r.u32(5)
                dirs, merge = 1, 0
            else:
                cin, u, a, ret, dirs, merge = r.u32(6)
            op.update(cin=cin, seq=seq)
            gu = G * u
            nb = 2 * gu if kind == 5 else gu
            ds = []
            for _ in range(dirs):
                W = _weight(r, ver, cin, gu, False)[1]
                U = _weight(r, ver, u, gu, True)
                ds.append((W, U, r.f32(nb)))
            op.update(u=u, act=a, ret=ret, dirs=ds, merge=merge)
        elif kind == 7:  # CONV
            a = r.u32(14)
            cin, cout, kh, kw_, sh, sw, dh, dw, pt, pb, pl, pr, g, hb = a
            op.update(cin=cin, cout=cout, k=(kh, kw_), s=(sh, sw), d=(dh, dw), p=(pt, pb, pl, pr), g=g,
                      w=_weight(r, ver, kh * kw_ * (cin // g), cout, False)[1], b=r.f32(cout) if hb else None)
        elif kind == 8:  # POOL
            a = r.u32(10)
            op.update(type=a[0], k=(a[1], a[2]), s=(a[3], a[4]), p=(a[5], a[6], a[7], a[8]), cp=a[9])
        elif kind == 9:
            op["type"] = r.u32()
        elif kind in (10, 11):
            nd = r.u32()
            op["v"] = tuple(r.u32(nd)) if nd > 1 else (r.u32(),)
        elif kind == 12:
            op["op"] = r.u32()
        elif kind == 13:
            op["axis"] = r.u32()
        elif kind == 14:
            V, D = r.u32(2)
            op.update(V=V, D=D, w=_weight(r, ver, V, D, False)[1])
        elif kind == 15:
            c = r.u32()
            op.update(scale=r.f32(c), shift=r.f32(c))
        elif kind == 16:
            c = r.u32()
            op["c"] = r.f32(c)
        elif kind == 17:  # ATTENTION
            H, dk, dv, causal, cq, cv, ck, cout, hb = r.u32(9)
            ws = []
            for (k_, n_) in ((cq, H * dk), (ck, H * dk), (cv, H * dv), (H * dv, cout)):
                ws.append((_weight(r, ver, k_, n_, False)[1], r.f32(n_) if hb else None))
            op.update(H=H, dk=dk, dv=dv, causal=causal, ws=ws)
        elif kind == 18:
            op.update(zip(("axis", "start", "len", "squeeze"), r.u32(4)))
        elif kind == 19:
            op["p"] = r.u32(4)
        elif kind == 20:
            op["s"] = r.u32(2)
        ops.append(op)
    assert r.o == len(data), "trailing bytes"
    if ver < 3:  # the first sized op gives the input width; the first LSTM gives the sequence length
        first = next(o for o in ops if o["kind"] in (0, 2, 4))
        in_dim = first["k"] if first["kind"] == 0 else first["cols"] if first["kind"] == 2 else first["cin"]
        seq = next((o["seq"] for o in ops if o["kind"] == 4), None)
        in_shape = (seq, in_dim) if seq else (in_dim,)
    return dict(ver=ver, layout=layout, in_shape=in_shape, ops=ops)


# ---------------------------------------------------------------- forward
def _shape_rows(shape):
    return int(np.prod(shape[:-1])) if len(shape) > 1 else 1


def _conv(x, B, H, W, op, act_id=-1, alpha=0.0):
    kh, kw_ = op["k"]
    sh, sw = op["s"]
    dh, dw = op["d"]
    pt, pb, pl, pr = op["p"]
    g = op["g"]
    C = op["cin"]
    cg, Co = C // g, op["cout"]
    cog = Co // g
    Ho = (H + pt + pb - dh * (kh - 1) - 1) // sh + 1
    Wo = (W + pl + pr - dw * (kw_ - 1) - 1) // sw + 1
    xi = np.zeros((B, H + pt + pb, W + pl + pr, C), np.float64)
    xi[:, pt:pt + H, pl:pl + W, :] = x.reshape(B, H, W, C)
    out = np.zeros((B, Ho, Wo, Co), np.float64)
    wt = op["w"].astype(np.float64).reshape(kh, kw_, cg, Co)
    for gi in range(g):
        acc = np.zeros((B, Ho, Wo, cog))
        for ky in range(kh):
            for kx in range(kw_):
                patch = xi[:, ky * dh: ky * dh + sh * (Ho - 1) + 1: sh, kx * dw: kx * dw + sw * (Wo - 1) + 1: sw,
                           gi * cg:(gi + 1) * cg]
                acc += patch @ wt[ky, kx, :, gi * cog:(gi + 1) * cog]
        out[..., gi * cog:(gi + 1) * cog] = acc
    if op["b"] is not None:
        out += op["b"].astype(np.float64)
    y = out.astype(np.float32).reshape(B * Ho * Wo, Co)
    return act(y, act_id, alpha), (Ho, Wo)


def forward(model, x, mode="ref"):
    """x: (batch·seq_len) × in_dim float32 (channels-last). Returns (outputs batch × out_dim, shapes)."""
    ops = model["ops"]
    in_shape = model["in_shape"]
    x = f32c(x)
    R0 = _shape_rows(in_shape)
    B = x.shape[0] // R0
    vals = [x]
    shapes = [tuple(in_shape)]
    for op in ops:
        k = op["kind"]
        a, sa = vals[op["inp"][0]], shapes[op["inp"][0]]
        if k == 0:
            w = op["w"]
            if w[0] == "i8":
                q, sc = w[1], w[2]
                if mode == "i8" or a.shape[0] <= INT8_MAX_ROWS:
                    y = qmatmul(a, q, sc, op["b"])
                else:
                    y = dense64(a, q.astype(np.float32) * sc[None, :], op["b"])
            else:
                y = dense64(a, w[1], op["b"])
            s = sa[:-1] + (op["n"],)
        elif k == 1:
            y, s = act(a, op["act"], op["alpha"]), sa
        elif k == 2:
            y, s = layernorm(a, op["g"], op["b"], op["eps"]), sa
        elif k == 3:
            y, s = softmax(a), sa
        elif k in (4, 5, 6):
            y, s = _rnn(op, a, sa, B, mode)
        elif k == 7:
            H, W = sa[0], (sa[1] if len(sa) == 3 else 1)
            y, (Ho, Wo) = _conv(a, B, H, W, op)
            s = ((Ho, Wo, op["cout"]) if len(sa) == 3 else (Ho, op["cout"]))
        elif k == 8:
            y, s = _pool(op, a, sa, B)
        elif k == 9:
            R, C = _shape_rows(sa), sa[-1]
            t = a.reshape(B, R, C)
            y = (t.max(axis=1) if op["type"] == 0 else _seq_sum(t) * np.float32(1.0 / R)).astype(np.float32)
            s = (C,)
        elif k == 10:
            y, s = a, tuple(op["v"])
            y = y.reshape(B * _shape_rows(s), s[-1])
        elif k == 11:
            perm = op["v"]
            t = a.reshape((B,) + sa).transpose((0,) + tuple(p + 1 for p in perm))
            s = tuple(sa[p] for p in perm)
            y = np.ascontiguousarray(t).reshape(B * _shape_rows(s), s[-1])
        elif k == 12:
            b, sb = vals[op["inp"][1]], shapes[op["inp"][1]]
            ra, rb = _shape_rows(sa), _shape_rows(sb)
            R, C = max(ra, rb), max(sa[-1], sb[-1])
            ta = a.reshape(B, ra, sa[-1])
            tb = b.reshape(B, rb, sb[-1])
            fn = [np.add, np.subtract, np.multiply, np.divide, np.maximum, np.minimum][op["op"]]
            with np.errstate(divide="ignore", invalid="ignore"):
                y = fn(ta, tb).astype(np.float32).reshape(B * R, C)
            big = sa if ra * sa[-1] >= rb * sb[-1] else sb
            s = big[:-1] + (C,)
        elif k == 13:
            parts = [vals[i].reshape((B,) + shapes[i]) for i in op["inp"]]
            ax = 1 if op["axis"] == 0 else len(sa)
            t = np.concatenate(parts, axis=ax)
            s = t.shape[1:]
            y = t.reshape(B * _shape_rows(s), s[-1])
        elif k == 14:
            ids = a.reshape(-1)
            V, D = op["V"], op["D"]
            y = np.full((ids.size, D), np.nan, np.float32)
            ok = (ids >= 0) & (ids < V) & (ids == np.floor(ids))
            y[ok] = op["w"][ids[ok].astype(np.int64)]
            s = sa + (D,)
            y = y.reshape(B * _shape_rows(s), D)
        elif k == 15:
            y, s = (a * op["scale"] + op["shift"]).astype(np.float32), sa
        elif k == 16:
            y = (a.reshape(B, -1) + op["c"][None, :]).astype(np.float32).reshape(a.shape)
            s = sa
        elif k == 17:
            y, s = _attention(op, vals, shapes, B)
        elif k == 18:
            t = a.reshape((B,) + sa)
            ax = 1 if op["axis"] == 0 else len(sa)
            t = np.take(t, range(op["start"], op["start"] + op["len"]), axis=ax)
            s = list(sa)
            s[ax - 1] = op["len"]
            if op["squeeze"] and op["len"] == 1 and len(s) > 1:
                del s[ax - 1]
            s = tuple(s)
            y = np.ascontiguousarray(t).reshape(B * _shape_rows(s), s[-1])
        elif k == 19:
            pt, pb, pl, pr = op["p"]
            H, W = sa[0], (sa[1] if len(sa) == 3 else 1)
            t = np.zeros((B, H + pt + pb, W + pl + pr, sa[-1]), np.float32)
            t[:, pt:pt + H, pl:pl + W] = a.reshape(B, H, W, sa[-1])
            s = ((H + pt + pb, W + pl + pr, sa[-1]) if len(sa) == 3 else (H + pt + pb, sa[-1]))
            y = t.reshape(-1, sa[-1])
        elif k == 20:
            sh, sw = op["s"]
            H, W = sa[0], (sa[1] if len(sa) == 3 else 1)
            t = a.reshape(B, H, W, sa[-1]).repeat(sh, axis=1).repeat(sw, axis=2)
            s = ((H * sh, W * sw, sa[-1]) if len(sa) == 3 else (H * sh, sa[-1]))
            y = t.reshape(-1, sa[-1])
        else:
            raise ValueError(f"op kind {k}")
        vals.append(f32c(y))
        shapes.append(tuple(s))
    out = vals[-1]
    return out.reshape(B, -1), shapes[-1]


def _seq_sum(t):
    o = t[:, 0, :].astype(np.float32).copy()
    for i in range(1, t.shape[1]):
        o = (o + t[:, i, :]).astype(np.float32)
    return o


def _pool(op, a, sa, B):
    kh, kw_ = op["k"]
    sh, sw = op["s"]
    pt, pb, pl, pr = op["p"]
    H, W, C = sa[0], (sa[1] if len(sa) == 3 else 1), sa[-1]
    Ho = (H + pt + pb - kh) // sh + 1
    Wo = (W + pl + pr - kw_) // sw + 1
    t = a.reshape(B, H, W, C)
    y = np.zeros((B, Ho, Wo, C), np.float32)
    for oy in range(Ho):
        for ox in range(Wo):
            y0, x0 = oy * sh - pt, ox * sw - pl
            ys, xs = max(y0, 0), max(x0, 0)
            ye, xe = min(y0 + kh, H), min(x0 + kw_, W)
            win = t[:, ys:ye, xs:xe, :].reshape(B, -1, C)
            if op["type"] == 0:
                y[:, oy, ox] = win.max(axis=1)
            else:
                cnt = kh * kw_ if op["cp"] else win.shape[1]
                y[:, oy, ox] = (win.astype(np.float64).sum(axis=1) / cnt).astype(np.float32)
    s = (Ho, Wo, C) if len(sa) == 3 else (Ho, C)
    return y.reshape(-1, C), s


def _attention(op, vals, shapes, B):
    inp = op["inp"]
    q = vals[inp[0]]
    vi = inp[1] if len(inp) > 1 else inp[0]
    ki = inp[2] if len(inp) > 2 else vi
    v, k_ = vals[vi], vals[ki]
    Rq, S = _shape_rows(shapes[inp[0]]), _shape_rows(shapes[vi])
    H, dk, dv = op["H"], op["dk"], op["dv"]
    (wq, bq), (wk, bk), (wv, bv), (wo, bo) = op["ws"]
    Q = dense64(q, wq, bq).astype(np.float64).reshape(B, Rq, H, dk).transpose(0, 2, 1, 3)
    K = dense64(k_, wk, bk).astype(np.float64).reshape(B, S, H, dk).transpose(0, 2, 1, 3)
    V = dense64(v, wv, bv).astype(np.float64).reshape(B, S, H, dv).transpose(0, 2, 1, 3)
    scale = np.float32(1.0) / np.sqrt(np.float32(dk))
    sc = (float(scale) * (Q @ K.transpose(0, 1, 3, 2))).astype(np.float32)
    if op["causal"]:
        sc = np.where(np.triu(np.ones((Rq, S), bool), 1)[None, None], -np.inf, sc).astype(np.float32)
    P = softmax(sc.reshape(-1, S)).reshape(B, H, Rq, S)
    ctx = (P.astype(np.float64) @ V).astype(np.float32).transpose(0, 2, 1, 3).reshape(B * Rq, H * dv)
    s = shapes[inp[0]][:-1] + (wo.shape[1],)
    return dense64(ctx, wo, bo), s


def _rnn(op, a, sa, B, mode, dense=None):
    """dense: the product x·W + b used for the input projection and the fp32 recurrence (default: float64
    accumulation, the oracle; the CPU baseline passes the reference's fp32 native GEMM)"""
    dense64_ = dense if dense is not None else dense64
    kind, u = op["kind"], op["u"]
    T, cin = sa[0], sa[1]
    G = {4: 4, 5: 3, 6: 1}[kind]
    gu = G * u
    sig = lambda z: act(z, 3)  # noqa: E731

    def run_dir(W, U, bias, backward):
        zx = dense64_(a, W, bias[:gu]).reshape(B, T, gu)
        # the fp32 recurrent weight (an int8 one dequantized once, as the reference's workspace keeps it)
        Uf = U[1] if U[0] == "f32" else (U[1].astype(np.float32) * U[2][None, :]).astype(np.float32)
        brec = bias[gu:] if kind == 5 else None
        h = np.zeros((B, u), np.float32)
        c = np.zeros((B, u), np.float32)
        outs = np.zeros((B, T, u), np.float32)
        for step in range(T):
            t = T - 1 - step if backward else step
            z = zx[:, t, :].copy()
            if step == 0:
                rec = np.tile(brec, (B, 1)).astype(np.float32) if kind == 5 else None
            elif U[0] == "i8" and (mode == "i8" or B <= INT8_MAX_ROWS):
                if kind == 5:
                    rec = qmatmul(h, U[1], U[2], brec)
                else:
                    z = qmatmul(h, U[1], U[2], None, y_old=z)
                    rec = None
            else:
                rec = dense64_(h, Uf, brec)
            if kind == 4:
                if rec is not None:
                    z = (z + rec).astype(np.float32)
                i_, f_, g_, o_ = sig(z[:, :u]), sig(z[:, u:2 * u]), act(z[:, 2 * u:3 * u], op["act"]), sig(z[:, 3 * u:])
                c = (i_ * g_).astype(np.float32) if step == 0 else (i_ * g_ + (f_ * c).astype(np.float32)).astype(np.float32)
                h = (act(c, op["act"]) * o_).astype(np.float32)
            elif kind == 5:
                zr = sig((z[:, :2 * u] + rec[:, :2 * u]).astype(np.float32))
                zg, rg = zr[:, :u], zr[:, u:]
                hh = act(((rg * rec[:, 2 * u:]).astype(np.float32) + z[:, 2 * u:]).astype(np.float32), op["act"])
                prev = np.zeros_like(h) if step == 0 else h
                h = (((prev - hh).astype(np.float32) * zg).astype(np.float32) + hh).astype(np.float32)
            else:
                if rec is not None:
                    z = (z + rec).astype(np.float32)
                h = act(z, op["act"])
            outs[:, t] = h
        return outs if op["ret"] else h[:, None, :]

    res = [run_dir(W, U, b, d == 1) for d, (W, U, b) in enumerate(op["dirs"])]
    if len(res) == 1:
        y = res[0]
    elif op["merge"] == 0:
        y = np.concatenate(res, axis=2)
    elif op["merge"] == 2:
        y = (res[0] * res[1]).astype(np.float32)
    else:
        y = (res[0] + res[1]).astype(np.float32)
        if op["merge"] == 3:
            y = (y * np.float32(0.5)).astype(np.float32)
    uo = y.shape[2]
    if op["ret"]:
        return y.reshape(B * T, uo), (T, uo)
    return y.reshape(B, uo), (uo,)
