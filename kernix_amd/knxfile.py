""".knx model files from numpy arrays: a small graph builder and its encoder (numpy only).

    b = ModelBuilder((784,))                        # per-sample input shape, channels-last
    h = b.linear(b.input, w1, b1, activation="relu", fmt="i8_col")
    y = b.linear(h, w2, b2)
    b.save("mlp.knx")                               # KNX2 here: a chain of Linear/activation ops with int8 weights

Values are `Value` handles (an id and a per-sample shape); every op returns the Value it writes, and the model output is
the value of the last op added.  Shapes are tracked with the runtime's rules, so a mismatch is a ValueError here rather
than a file the loader rejects.  `save`/`to_bytes` pick the oldest format that holds the graph — KNX1 for a chain of
Linear / activation / LayerNorm / Softmax / LSTM ops with float32 weights, KNX2 for such a chain with int8 weights, KNX3
otherwise — or the version asked for.

Format (little endian; u32 unless noted), as the reference documents it (docs/mlp-runtime-design.md §4,
docs/int8-quantization-design.md §4, docs/graph-runtime-design.md §3):
    KNX1/KNX2  magic, n_ops, then per op: kind, fields, weights
    KNX3       magic, n_ops, layout, in_nd, in_dims[in_nd], then per op: kind, n_in, in_ids[n_in], fields, weights
    weights    KNX1: f32[k·n];  KNX2/3: u32 dtype, then F32 f32[k·n] | I8_COL f32 scale[n] i8[k·n] | I8_ROW f32 scale[k] i8[k·n]
Weight matrices are in × out (k × n, row-major).  Value ids: 0 the model input, i + 1 the output of op i.
"""
import struct

import numpy as np

# ---------------------------------------------------------------- format ids (part of the file ABI)
OPS = ("LINEAR", "ACT", "LAYERNORM", "SOFTMAX", "LSTM", "GRU", "RNN", "CONV", "POOL", "GLOBAL_POOL", "RESHAPE", "PERMUTE",
       "BINARY", "CONCAT", "EMBEDDING", "AFFINE", "ADD_CONST", "ATTENTION", "SELECT", "PAD", "UPSAMPLE")
OP_ID = {name: i for i, name in enumerate(OPS)}
ACTIVATIONS = ("relu", "gelu", "silu", "sigmoid", "tanh", "leaky_relu", "elu", "selu", "softplus", "relu6",
               "hard_sigmoid", "hard_swish", "gelu_tanh", "exp", "mish", "softsign")
ACT_ID = {name: i for i, name in enumerate(ACTIVATIONS)}
BINARY_OPS = ("add", "sub", "mul", "div", "max", "min")
MERGES = ("concat", "sum", "mul", "ave")
POOLS = ("max", "avg")
AXES = ("first", "last")
WEIGHT_FORMATS = ("f32", "i8_col", "i8_row")
GATES = {"LSTM": 4, "GRU": 3, "RNN": 1}
LEGACY_OPS = {"LINEAR", "ACT", "LAYERNORM", "SOFTMAX", "LSTM"}  # the ops KNX1/KNX2 files can hold


def quantize(w, per="column"):
    """Symmetric int8 quantization of a k×n weight, one scale per output column (I8_COL) or per input row (I8_ROW):
    scale = float32(max|w| / 127), computed in float64 (1 for an all-zero column/row); q = clip(rint(w / scale), ±127)
    with round-half-to-even (reference tools/knx_quant.py:18-25).  Returns (scale float32, q int8)."""
    w = np.asarray(w, np.float64)
    axis = 0 if per == "column" else 1
    peak = np.max(np.abs(w), axis=axis)
    scale = np.where(peak > 0.0, peak / 127.0, 1.0).astype(np.float32)
    q = np.rint(w / np.expand_dims(scale.astype(np.float64), axis))
    return scale, np.clip(q, -127, 127).astype(np.int8)


# ---------------------------------------------------------------- encoding helpers
def _u32(*values):
    return struct.pack(f"<{len(values)}I", *(int(v) for v in values))


def _f32(a):
    return np.ascontiguousarray(np.asarray(a, np.float64), dtype="<f4").tobytes()


def _weight(w, fmt, version):
    """the bytes of one k×n weight matrix in the given format"""
    w = np.asarray(w, np.float64)
    if w.ndim != 2:
        raise ValueError(f"weight must be a k x n matrix, got shape {w.shape}")
    if version == 1:
        if fmt != "f32":
            raise ValueError("KNX1 holds float32 weights only")
        return _f32(w)
    head = _u32(WEIGHT_FORMATS.index(fmt))
    if fmt == "f32":
        return head + _f32(w)
    scale, q = quantize(w, "column" if fmt == "i8_col" else "row")
    return head + _f32(scale) + np.ascontiguousarray(q).tobytes()


class Value:
    """A value of the graph: its id (0 = the model input) and its per-sample channels-last shape."""

    __slots__ = ("id", "shape")

    def __init__(self, vid, shape):
        self.id, self.shape = vid, tuple(int(d) for d in shape)

    def __repr__(self):
        return f"Value({self.id}, {self.shape})"


class _Node:
    __slots__ = ("kind", "inputs", "fields", "parts")

    def __init__(self, kind, inputs, fields, parts):
        self.kind, self.inputs, self.fields, self.parts = kind, inputs, fields, parts


def _rows(shape):
    return int(np.prod(shape[:-1])) if len(shape) > 1 else 1


def _window(n, k, stride, dil, pad_a, pad_b):
    return (n + pad_a + pad_b - dil * (k - 1) - 1) // stride + 1


class ModelBuilder:
    """Builds a .knx graph op by op (see the module docstring)."""

    def __init__(self, input_shape, channels_first=False, int8=False):
        """input_shape: one sample's input, channels-last (H, W, C) / (T, F) / (F,).  channels_first: the model is fed
        channels-first arrays (layout 1; the binding moves the axis).  int8: default weight format — I8_COL for Linear,
        convolution, attention and recurrent matrices, I8_ROW for recurrent input and embedding matrices."""
        self._nodes = []
        self._shapes = [tuple(int(d) for d in input_shape)]
        self._check_shape(self._shapes[0], "input")
        self.channels_first = bool(channels_first)
        self.int8 = bool(int8)
        self.input = Value(0, self._shapes[0])

    # ---------------------------------------------------------------- internals
    @staticmethod
    def _check_shape(shape, what):
        if not 1 <= len(shape) <= 4 or min(shape) < 1:
            raise ValueError(f"{what}: shape {shape} cannot be stored (1 to 4 axes, each at least 1)")

    def _value(self, v):
        if isinstance(v, Value):
            vid = v.id
        else:
            vid = int(v)
        if not 0 <= vid < len(self._shapes):
            raise ValueError(f"unknown value {v!r}")
        return Value(vid, self._shapes[vid])

    def _fmt(self, fmt, default_int8):
        fmt = fmt or (default_int8 if self.int8 else "f32")
        if fmt not in WEIGHT_FORMATS:
            raise ValueError(f"unknown weight format {fmt!r}")
        return fmt

    def _add(self, kind, inputs, fields, parts, shape):
        shape = tuple(int(d) for d in shape)
        self._check_shape(shape, kind)
        self._nodes.append(_Node(kind, [v.id for v in inputs], [int(f) for f in fields], parts))
        self._shapes.append(shape)
        return Value(len(self._shapes) - 1, shape)

    # ---------------------------------------------------------------- ops
    def linear(self, x, weight, bias=None, activation=None, alpha=0.0, fmt=None):
        """x·weight + bias over the last axis; weight is in × out."""
        x = self._value(x)
        weight = np.asarray(weight, np.float64)
        if x.shape[-1] != weight.shape[0]:
            raise ValueError(f"Linear: input width {x.shape[-1]} does not match weight {weight.shape}")
        parts = [("w", weight, self._fmt(fmt, "i8_col"))] + ([("f", bias)] if bias is not None else [])
        y = self._add("LINEAR", [x], [weight.shape[0], weight.shape[1], bias is not None], parts,
                      x.shape[:-1] + (weight.shape[1],))
        return self.activation(y, activation, alpha)

    def activation(self, x, name, alpha=0.0):
        """an activation by name (None / "linear": none; "softmax": the Softmax op)"""
        x = self._value(x)
        if name in (None, "linear"):
            return x
        if name == "softmax":
            return self.softmax(x)
        if name not in ACT_ID:
            raise ValueError(f"unknown activation {name!r}")
        return self._add("ACT", [x], [ACT_ID[name]], [("alpha", float(alpha))], x.shape)

    def layer_norm(self, x, gamma=None, beta=None, eps=1e-5):
        x = self._value(x)
        c = x.shape[-1]
        affine = gamma is not None or beta is not None
        parts = [("eps", float(eps))]
        if affine:
            parts += [("f", np.ones(c) if gamma is None else gamma), ("f", np.zeros(c) if beta is None else beta)]
        return self._add("LAYERNORM", [x], [c, affine], parts, x.shape)

    def softmax(self, x):
        x = self._value(x)
        return self._add("SOFTMAX", [x], [], [], x.shape)

    def conv(self, x, weight, bias=None, kernel=(1, 1), stride=(1, 1), dilation=(1, 1), padding=(0, 0, 0, 0),
             groups=1, activation=None, alpha=0.0, fmt=None):
        """2-D (H×W×C) or 1-D (T×C, kernel (k, 1)) convolution; weight is (kh·kw·C/groups) × out with rows ordered
        (ky, kx, ci); padding (top, bottom, left, right)."""
        x = self._value(x)
        (kh, kw), (sh, sw), (dh, dw) = kernel, stride, dilation
        weight = np.asarray(weight, np.float64)
        cin, cout = x.shape[-1], weight.shape[1]
        if weight.shape[0] != kh * kw * cin // groups or cin % groups or cout % groups:
            raise ValueError(f"convolution weight {weight.shape} does not fit kernel {kernel}, {cin} inputs, "
                             f"{groups} groups")
        out = self._spatial(x, kh, kw, sh, sw, dh, dw, padding, cout)
        parts = [("w", weight, self._fmt(fmt, "i8_col"))] + ([("f", bias)] if bias is not None else [])
        y = self._add("CONV", [x], [cin, cout, kh, kw, sh, sw, dh, dw, *padding, groups, bias is not None], parts, out)
        return self.activation(y, activation, alpha)

    @staticmethod
    def _spatial(x, kh, kw, sh, sw, dh, dw, padding, channels):
        if len(x.shape) not in (2, 3):
            raise ValueError(f"windowed op on shape {x.shape}: needs (T, C) or (H, W, C)")
        pt, pb, pl, pr = padding
        h = _window(x.shape[0], kh, sh, dh, pt, pb)
        if len(x.shape) == 2:
            return (h, channels)
        return (h, _window(x.shape[1], kw, sw, dw, pl, pr), channels)

    def pool(self, x, kind, kernel, stride, padding=(0, 0, 0, 0), count_pad=False):
        x = self._value(x)
        out = self._spatial(x, kernel[0], kernel[1], stride[0], stride[1], 1, 1, padding, x.shape[-1])
        return self._add("POOL", [x], [POOLS.index(kind), *kernel, *stride, *padding, bool(count_pad)], [], out)

    def global_pool(self, x, kind="avg"):
        x = self._value(x)
        return self._add("GLOBAL_POOL", [x], [POOLS.index(kind)], [], (x.shape[-1],))

    def reshape(self, x, shape):
        x = self._value(x)
        shape = tuple(int(d) for d in shape)
        if int(np.prod(shape)) != int(np.prod(x.shape)):
            raise ValueError(f"Reshape {x.shape} -> {shape}: sizes differ")
        return self._add("RESHAPE", [x], [len(shape), *shape], [], shape)

    def permute(self, x, order):
        x = self._value(x)
        if sorted(order) != list(range(len(x.shape))):
            raise ValueError(f"Permute {order} of shape {x.shape}")
        return self._add("PERMUTE", [x], [len(order), *order], [], tuple(x.shape[i] for i in order))

    def binary(self, a, b, op):
        """elementwise a (op) b; a size-1 row count or channel count broadcasts within the sample"""
        a, b = self._value(a), self._value(b)
        big = a if _rows(a.shape) * a.shape[-1] >= _rows(b.shape) * b.shape[-1] else b
        return self._add("BINARY", [a, b], [BINARY_OPS.index(op)], [],
                         big.shape[:-1] + (max(a.shape[-1], b.shape[-1]),))

    def add(self, a, b):
        return self.binary(a, b, "add")

    def concat(self, values, axis="last"):
        values = [self._value(v) for v in values]
        ax = 0 if axis == "first" else len(values[0].shape) - 1
        out = list(values[0].shape)
        out[ax] = sum(v.shape[ax] for v in values)
        return self._add("CONCAT", values, [AXES.index(axis)], [], out)

    def embedding(self, ids, table, fmt=None):
        ids = self._value(ids)
        table = np.asarray(table, np.float64)
        return self._add("EMBEDDING", [ids], [table.shape[0], table.shape[1]], [("w", table, self._fmt(fmt, "i8_row"))],
                         ids.shape + (table.shape[1],))

    def affine(self, x, scale, shift):
        x = self._value(x)
        c = x.shape[-1]
        return self._add("AFFINE", [x], [c], [("f", np.broadcast_to(scale, (c,))), ("f", np.broadcast_to(shift, (c,)))],
                         x.shape)

    def add_const(self, x, const):
        x = self._value(x)
        const = np.asarray(const, np.float64).reshape(-1)
        return self._add("ADD_CONST", [x], [const.size], [("f", const)], x.shape)

    def attention(self, q, heads, wq, wk, wv, wo, bq=None, bk=None, bv=None, bo=None, v=None, k=None, causal=False,
                  fmt=None):
        """Multi-head attention: queries from q, values from v (default q), keys from k (default v); wq/wk: in × heads·dk,
        wv: in × heads·dv, wo: heads·dv × out (head-major columns).  Biases all given or all None."""
        q = self._value(q)
        v = self._value(v) if v is not None else q
        k = self._value(k) if k is not None else v
        wq, wk, wv, wo = (np.asarray(a, np.float64) for a in (wq, wk, wv, wo))
        dk, dv = wq.shape[1] // heads, wv.shape[1] // heads
        biases = (bq, bk, bv, bo)
        has_bias = bq is not None
        if any((b is not None) != has_bias for b in biases):
            raise ValueError("attention biases: give all four or none")
        fmt = self._fmt(fmt, "i8_col")
        parts = []
        for w, b in zip((wq, wk, wv, wo), biases):
            parts.append(("w", w, fmt))
            if has_bias:
                parts.append(("f", b))
        inputs = [q] + ([v] if v.id != q.id or k.id != v.id else []) + ([k] if k.id != v.id else [])
        fields = [heads, dk, dv, bool(causal), wq.shape[0], wv.shape[0], wk.shape[0], wo.shape[1], has_bias]
        return self._add("ATTENTION", inputs, fields, parts, q.shape[:-1] + (wo.shape[1],))

    def recurrent(self, x, cell, units, directions, activation="tanh", return_sequences=False, merge="concat",
                  fmt_input=None, fmt_recurrent=None):
        """LSTM / GRU / RNN over a T × F input.  directions: one (forward) or two (forward, backward) tuples
        (W in × G·units, U units × G·units, bias), gates in Keras order (LSTM i f c o, GRU z r h); a GRU bias holds the
        input-side G·units values then the recurrent-side ones."""
        x = self._value(x)
        if len(x.shape) != 2:
            raise ValueError(f"{cell}: input must be T x F, got {x.shape}")
        fi, fr = self._fmt(fmt_input, "i8_row"), self._fmt(fmt_recurrent, "i8_col")
        parts = []
        for w, u, b in directions:
            parts += [("w", w, fi), ("w", u, fr), ("f", b)]
        width = units * (2 if len(directions) == 2 and merge == "concat" else 1)
        out = (x.shape[0], width) if return_sequences else (width,)
        fields = [x.shape[1], units, ACT_ID[activation], bool(return_sequences), len(directions), MERGES.index(merge)]
        return self._add(cell, [x], fields, parts, out)

    def select(self, x, axis, start, length, squeeze=False):
        x = self._value(x)
        out = list(x.shape)
        ax = 0 if axis == "first" else len(out) - 1
        out[ax] = length
        if squeeze and length == 1 and len(out) > 1:
            del out[ax]
        return self._add("SELECT", [x], [AXES.index(axis), start, length, bool(squeeze)], [], out)

    def pad(self, x, padding):
        """zero padding (top, bottom, left, right) of T×C or H×W×C"""
        x = self._value(x)
        pt, pb, pl, pr = padding
        out = (x.shape[0] + pt + pb,) + ((x.shape[1] + pl + pr,) if len(x.shape) == 3 else ()) + (x.shape[-1],)
        return self._add("PAD", [x], padding, [], out)

    def upsample(self, x, factors):
        """nearest upsampling by (sh, sw) (sw must be 1 on T×C)"""
        x = self._value(x)
        sh, sw = factors
        out = (x.shape[0] * sh,) + ((x.shape[1] * sw,) if len(x.shape) == 3 else ()) + (x.shape[-1],)
        return self._add("UPSAMPLE", [x], [sh, sw], [], out)

    # ---------------------------------------------------------------- encoding
    def _legacy_ok(self):
        """KNX1/KNX2 hold a chain (op i reads op i-1's output) of legacy ops whose input shape the loader derives"""
        if not self._nodes:
            return False
        seq = None
        for i, n in enumerate(self._nodes):
            if n.kind not in LEGACY_OPS or n.inputs != [i]:
                return False
            if n.kind == "ACT" and (n.fields[0] > ACT_ID["tanh"] or n.parts[0][1] != 0.0):
                return False
            if n.kind == "LSTM" and (n.fields[4] != 1 or n.fields[2] not in (ACT_ID["relu"], ACT_ID["tanh"])):
                return False
            if n.kind == "LSTM" and seq is None:
                seq = self._shapes[n.inputs[0]][0]
        first_sized = next((n for n in self._nodes if n.kind in ("LINEAR", "LAYERNORM", "LSTM")), None)
        if first_sized is None or self.channels_first:
            return False
        in_dim = first_sized.fields[0]
        return self._shapes[0] == ((seq, in_dim) if seq else (in_dim,))

    def _uses_int8(self):
        return any(p[0] == "w" and p[2] != "f32" for n in self._nodes for p in n.parts)

    def _record(self, i, node, version):
        out = [_u32(OP_ID[node.kind])]
        if version == 3:
            out.append(_u32(len(node.inputs), *node.inputs))
        fields = node.fields
        if node.kind == "LSTM" and version < 3:  # in units act ret_seq seq (one direction)
            fields = fields[:4] + [self._shapes[node.inputs[0]][0]]
        out.append(_u32(*fields))
        for part in node.parts:
            tag = part[0]
            if tag == "w":
                out.append(_weight(part[1], part[2], version))
            elif tag == "f":
                out.append(_f32(part[1]))
            elif tag == "eps":
                out.append(_f32([part[1]]))
            elif tag == "alpha" and version == 3:
                out.append(_f32([part[1]]))
        return b"".join(out)

    def to_bytes(self, version=None):
        legacy = self._legacy_ok()
        if version is None:
            version = (2 if self._uses_int8() else 1) if legacy else 3
        if version in (1, 2) and not legacy:
            raise ValueError("this graph needs KNX3 (not a chain of Linear/activation/LayerNorm/Softmax/LSTM ops)")
        if version == 1 and self._uses_int8():
            raise ValueError("KNX1 holds float32 weights only")
        if version not in (1, 2, 3):
            raise ValueError(f"unknown version {version}")
        head = b"KNX%d" % version + _u32(len(self._nodes))
        if version == 3:
            shape = self._shapes[0]
            head += _u32(1 if self.channels_first else 0, len(shape), *shape)
        return head + b"".join(self._record(i, n, version) for i, n in enumerate(self._nodes))

    def save(self, path, version=None):
        data = self.to_bytes(version)
        with open(path, "wb") as f:
            f.write(data)
        return path

    @property
    def output(self):
        """the model output: the value of the last op"""
        return Value(len(self._shapes) - 1, self._shapes[-1])
