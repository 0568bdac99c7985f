""".knx writer (numpy only): KNX1 / KNX2 sequential models and KNX3 graphs.

Byte format (little endian, u32 unless noted), as the reference documents it (reference docs/mlp-runtime-design.md
§4, docs/int8-quantization-design.md §4, docs/graph-runtime-design.md §3) and as its loader reads it:

    KNX1/KNX2: magic, n_ops, then per op: kind, args, weights            (KNX2: every weight is a dtype'd block)
    KNX3:      magic, n_ops, layout, in_nd, in_dims[in_nd], then per op: kind, n_in, in[n_in], args, weights
    weight block (KNX2/3): u32 dtype, then F32: f32[k·n] | I8_COL: f32 scale[n], i8[k·n] | I8_ROW: f32 scale[k], i8[k·n]

Weights are in×out (k×n, row-major).  Symmetric int8 quantization per output column (I8_COL) or input row (I8_ROW):
scale = float32(max|w| / 127) computed in float64 (1 when all zero), q = clip(rint(w / scale), −127, 127) with
round-half-even — the quantizer of the reference exporter (reference tools/knx_quant.py:18-25).
"""
import struct

import numpy as np

OP = dict(LINEAR=0, ACT=1, LAYERNORM=2, SOFTMAX=3, LSTM=4, GRU=5, RNN=6, CONV=7, POOL=8, GLOBAL_POOL=9, RESHAPE=10,
          PERMUTE=11, BINARY=12, CONCAT=13, EMBEDDING=14, AFFINE=15, ADD_CONST=16, ATTENTION=17, SELECT=18, PAD=19,
          UPSAMPLE=20)
ACT = dict(relu=0, gelu=1, silu=2, sigmoid=3, tanh=4, leaky_relu=5, elu=6, selu=7, softplus=8, relu6=9,
           hard_sigmoid=10, hard_swish=11, gelu_tanh=12, exp=13, mish=14, softsign=15)
BIN = dict(add=0, sub=1, mul=2, div=3, max=4, min=5)
MERGE = dict(concat=0, sum=1, mul=2, ave=3)
DT = dict(f32=0, i8_col=1, i8_row=2)
FIRST, LAST = 0, 1
GATES = dict(LSTM=4, GRU=3, RNN=1)


def u32(*v):
    return struct.pack(f"<{len(v)}I", *[int(x) for x in v])


def f32(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.float64).astype("<f4")).tobytes()


def quantize(w, axis="col"):
    """(scale float32, q int8) of a k×n weight, per column ("col") or per row ("row")."""
    w = np.asarray(w, np.float64)
    m = np.abs(w).max(axis=0 if axis == "col" else 1)
    scale = np.where(m > 0, m / 127.0, 1.0).astype(np.float32)
    s = (scale[None, :] if axis == "col" else scale[:, None]).astype(np.float64)
    q = np.clip(np.rint(w / s), -127, 127).astype(np.int8)
    return scale, q


def weight_block(w, dtype="f32", v2=True):
    """Bytes of one k×n weight; v2=False writes the bare KNX1 float32 values."""
    w = np.asarray(w, np.float64)
    if not v2:
        if dtype != "f32":
            raise ValueError("KNX1 holds float32 weights only")
        return f32(w)
    head = u32(DT[dtype])
    if dtype == "f32":
        return head + f32(w)
    scale, q = quantize(w, "col" if dtype == "i8_col" else "row")
    return head + f32(scale) + np.ascontiguousarray(q).tobytes()


class Sequential:
    """KNX1 (float32) or KNX2 (dtype'd weight blocks) sequential model: LINEAR, ACT, LAYERNORM, SOFTMAX, LSTM."""

    def __init__(self, v2=False):
        self.v2 = v2
        self.ops = []

    def linear(self, w, b=None, dtype="f32"):
        w = np.asarray(w, np.float64)
        body = u32(OP["LINEAR"], w.shape[0], w.shape[1], b is not None) + weight_block(w, dtype, self.v2)
        self.ops.append(body + (f32(b) if b is not None else b""))
        return self

    def act(self, name):
        self.ops.append(u32(OP["ACT"], ACT[name]))
        return self

    def layernorm(self, cols, eps=1e-5, gamma=None, beta=None):
        affine = gamma is not None
        body = u32(OP["LAYERNORM"], cols, affine) + struct.pack("<f", eps)
        self.ops.append(body + (f32(gamma) + f32(beta) if affine else b""))
        return self

    def softmax(self):
        self.ops.append(u32(OP["SOFTMAX"]))
        return self

    def lstm(self, w, u, b, act="tanh", ret_seq=False, seq=1, w_dtype="f32", u_dtype="f32"):
        w = np.asarray(w, np.float64)
        units = np.asarray(u).shape[0]
        body = u32(OP["LSTM"], w.shape[0], units, ACT[act], ret_seq, seq)
        body += weight_block(w, w_dtype, self.v2) + weight_block(u, u_dtype, self.v2) + f32(b)
        self.ops.append(body)
        return self

    def tobytes(self):
        return (b"KNX2" if self.v2 else b"KNX1") + u32(len(self.ops)) + b"".join(self.ops)

    def write(self, path):
        with open(path, "wb") as f:
            f.write(self.tobytes())
        return path


class Graph:
    """KNX3 graph writer.  Value ids: 0 = model input, k+1 = output of op k.  Shapes are per sample, channels-last;
    the model output is the last op's value.  quantize="int8" writes every weight of LINEAR/CONV/ATTENTION/recurrent
    weights as I8_COL and RNN input / embedding weights as I8_ROW."""

    def __init__(self, in_shape, layout=0, quantize=None):
        if quantize not in (None, "int8"):
            raise ValueError(f"unsupported quantize: {quantize}")
        self.layout, self.quantize = layout, quantize
        self.shapes = [tuple(int(d) for d in in_shape)]
        self.ops = []

    def shape(self, v):
        return self.shapes[v]

    def _dt(self, mode):
        return mode if self.quantize else "f32"

    def _add(self, kind, inp, args, payload, shape):
        shape = tuple(int(d) for d in shape)
        if not 1 <= len(shape) <= 4 or min(shape) < 1:
            raise ValueError(f"{kind}: output shape {shape} not representable")
        self.ops.append(u32(OP[kind], len(inp), *inp) + u32(*args) + payload)
        self.shapes.append(shape)
        return len(self.ops)

    def act(self, x, name, alpha=0.0):
        if name in (None, "linear"):
            return x
        if name == "softmax":
            return self.softmax(x)
        return self._add("ACT", [x], [ACT[name]], struct.pack("<f", alpha), self.shape(x))

    def linear(self, x, w, b=None, act=None, alpha=0.0):
        w = np.asarray(w, np.float64)
        s = self.shape(x)
        if s[-1] != w.shape[0]:
            raise ValueError(f"Linear input {s[-1]} != weight {w.shape}")
        payload = weight_block(w, self._dt("i8_col")) + (f32(b) if b is not None else b"")
        y = self._add("LINEAR", [x], [w.shape[0], w.shape[1], b is not None], payload, s[:-1] + (w.shape[1],))
        return self.act(y, act, alpha)

    def layernorm(self, x, gamma=None, beta=None, eps=1e-5):
        c = self.shape(x)[-1]
        affine = gamma is not None or beta is not None
        payload = struct.pack("<f", eps)
        if affine:
            payload += f32(np.ones(c) if gamma is None else gamma) + f32(np.zeros(c) if beta is None else beta)
        return self._add("LAYERNORM", [x], [c, affine], payload, self.shape(x))

    def softmax(self, x):
        return self._add("SOFTMAX", [x], [], b"", self.shape(x))

    @staticmethod
    def _hw(s):
        if len(s) not in (2, 3):
            raise ValueError(f"conv/pool input must be (T, C) or (H, W, C): {s}")
        return s[0], (s[1] if len(s) == 3 else 1)

    def conv(self, x, w, b, k, stride=(1, 1), dil=(1, 1), pads=(0, 0, 0, 0), groups=1, act=None, alpha=0.0):
        """w: (kh·kw·cin/groups) × cout, rows ordered (ky, kx, ci); pads: (top, bottom, left, right)"""
        s = self.shape(x)
        H, W = self._hw(s)
        kh, kw = k
        w = np.asarray(w, np.float64)
        cout = w.shape[1]
        oh = (H + pads[0] + pads[1] - dil[0] * (kh - 1) - 1) // stride[0] + 1
        ow = (W + pads[2] + pads[3] - dil[1] * (kw - 1) - 1) // stride[1] + 1
        out = (oh, ow, cout) if len(s) == 3 else (oh, cout)
        payload = weight_block(w, self._dt("i8_col")) + (f32(b) if b is not None else b"")
        y = self._add("CONV", [x], [s[-1], cout, kh, kw, *stride, *dil, *pads, groups, b is not None], payload, out)
        return self.act(y, act, alpha)

    def pool(self, x, kind, k, stride, pads=(0, 0, 0, 0), count_pad=False):
        s = self.shape(x)
        H, W = self._hw(s)
        oh = (H + pads[0] + pads[1] - k[0]) // stride[0] + 1
        ow = (W + pads[2] + pads[3] - k[1]) // stride[1] + 1
        out = (oh, ow, s[-1]) if len(s) == 3 else (oh, s[-1])
        return self._add("POOL", [x], [{"max": 0, "avg": 1}[kind], *k, *stride, *pads, int(count_pad)], b"", out)

    def global_pool(self, x, kind="avg"):
        return self._add("GLOBAL_POOL", [x], [{"max": 0, "avg": 1}[kind]], b"", (self.shape(x)[-1],))

    def reshape(self, x, shape):
        shape = tuple(int(d) for d in shape)
        return self._add("RESHAPE", [x], [len(shape), *shape], b"", shape)

    def permute(self, x, perm):
        s = self.shape(x)
        return self._add("PERMUTE", [x], [len(perm), *perm], b"", tuple(s[p] for p in perm))

    def binary(self, a, b, op):
        sa, sb = self.shape(a), self.shape(b)
        ra, rb = int(np.prod(sa[:-1])), int(np.prod(sb[:-1]))
        big = sa if ra * sa[-1] >= rb * sb[-1] else sb
        return self._add("BINARY", [a, b], [BIN[op]], b"", big[:-1] + (max(sa[-1], sb[-1]),))

    def concat(self, xs, axis):
        s0 = self.shape(xs[0])
        ax = 0 if axis == FIRST else len(s0) - 1
        out = list(s0)
        out[ax] = sum(self.shape(v)[ax] for v in xs)
        return self._add("CONCAT", list(xs), [axis], b"", out)

    def embedding(self, x, table):
        table = np.asarray(table, np.float64)
        return self._add("EMBEDDING", [x], [table.shape[0], table.shape[1]], weight_block(table, self._dt("i8_row")),
                         self.shape(x) + (table.shape[1],))

    def affine(self, x, scale, shift):
        c = self.shape(x)[-1]
        return self._add("AFFINE", [x], [c], f32(np.broadcast_to(scale, (c,))) + f32(np.broadcast_to(shift, (c,))),
                         self.shape(x))

    def add_const(self, x, c):
        c = np.asarray(c, np.float64).reshape(-1)
        return self._add("ADD_CONST", [x], [c.size], f32(c), self.shape(x))

    def attention(self, q, heads, wq, bq, wk, bk, wv, bv, wo, bo, v=None, k=None, causal=False):
        """w*: in channels × heads·d (head-major columns), wo: heads·dv × out"""
        inp = [q] + ([v] if v is not None else []) + ([k] if k is not None else [])
        wq, wk, wv, wo = (np.asarray(a, np.float64) for a in (wq, wk, wv, wo))
        dk, dv = wq.shape[1] // heads, wv.shape[1] // heads
        cv = self.shape(v if v is not None else q)[-1]
        ck = self.shape(k if k is not None else (v if v is not None else q))[-1]
        has_b = bq is not None
        payload = b""
        for w, b in ((wq, bq), (wk, bk), (wv, bv), (wo, bo)):
            payload += weight_block(w, self._dt("i8_col")) + (f32(b) if has_b else b"")
        return self._add("ATTENTION", inp, [heads, dk, dv, int(causal), wq.shape[0], cv, ck, wo.shape[1], int(has_b)],
                         payload, self.shape(q)[:-1] + (wo.shape[1],))

    def rnn(self, x, cell, units, dirs_w, act="tanh", ret_seq=False, merge="concat"):
        """dirs_w: per direction (W in×G·u, U u×G·u, bias) with Keras gate order (LSTM i f c o, GRU z r h); the GRU
        bias holds the input-side G·u values then the recurrent-side G·u values."""
        s = self.shape(x)
        payload = b""
        for w, u, b in dirs_w:
            payload += weight_block(w, self._dt("i8_row")) + weight_block(u, self._dt("i8_col")) + f32(b)
        uo = units * (2 if len(dirs_w) == 2 and merge == "concat" else 1)
        return self._add(cell, [x], [s[1], units, ACT[act], int(ret_seq), len(dirs_w), MERGE[merge]], payload,
                         (s[0], uo) if ret_seq else (uo,))

    def select(self, x, axis, start, length, squeeze=False):
        s = list(self.shape(x))
        ax = 0 if axis == FIRST else len(s) - 1
        s[ax] = length
        if squeeze and length == 1 and len(s) > 1:
            del s[ax]
        return self._add("SELECT", [x], [axis, start, length, int(squeeze)], b"", s)

    def pad(self, x, pads):
        s = self.shape(x)
        out = (s[0] + pads[0] + pads[1],) + ((s[1] + pads[2] + pads[3],) if len(s) == 3 else ()) + (s[-1],)
        return self._add("PAD", [x], list(pads), b"", out)

    def upsample(self, x, sh, sw=1):
        s = self.shape(x)
        out = (s[0] * sh,) + ((s[1] * sw,) if len(s) == 3 else ()) + (s[-1],)
        return self._add("UPSAMPLE", [x], [sh, sw], b"", out)

    def tobytes(self):
        s = self.shapes[0]
        return b"KNX3" + u32(len(self.ops), self.layout, len(s), *s) + b"".join(self.ops)

    def write(self, path):
        with open(path, "wb") as f:
            f.write(self.tobytes())
        return path
