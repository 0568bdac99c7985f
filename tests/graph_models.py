"""Small .knx graphs that together use every op kind, activation, binary op, broadcast, merge mode and convolution
variant of the runtime, shared by the GPU graph parity tests and the loader fuzz test.

    vision     H×W×C: plain, depthwise, grouped + dilated, strided and pointwise convolutions, both poolings with and
               without padding counted, padding, upsampling, concat on the channel axis, global poolings, max/sub
    sequence   T×C: 1-D convolutions (dilated, strided, grouped), 1-D pooling, layer norm without affine, row and
               channel broadcasting (add, mul, div), select, reshape, the smooth activations
    recurrent  T×F: LSTM, GRU and simple RNN cells, one and two directions, every merge, sequences and last states
    tokens     token ids: embedding, constant add, causal self-attention with biases, cross attention with three
               inputs and S ≠ Rq, layer norm, upsampling on T×C, permute, affine, softmax, min

Written with kernix_amd.knxfile; weights N(0, 0.3) (activation-specific scales where a function would saturate)
from a seed per family."""
import numpy as np

from kernix_amd.knxfile import ModelBuilder


def _w(rng, *shape, scale=0.3):
    return rng.normal(0.0, scale, shape)


def vision(rng, int8=False):
    b = ModelBuilder((10, 9, 4), int8=int8)
    x = b.conv(b.input, _w(rng, 36, 8), _w(rng, 8), kernel=(3, 3), padding=(1, 1, 1, 1), activation="relu6")
    d = b.conv(x, _w(rng, 9, 8), None, kernel=(3, 3), padding=(1, 1, 1, 1), groups=8)                # depthwise
    g = b.conv(x, _w(rng, 12, 8), _w(rng, 8), kernel=(1, 3), dilation=(1, 2), padding=(0, 0, 2, 2), groups=2,
               activation="hard_sigmoid")                                                              # grouped, dilated
    x = b.binary(d, g, "max")                                                                          # 10×9×8
    s = b.conv(x, _w(rng, 72, 6), _w(rng, 6), kernel=(3, 3), stride=(2, 2), padding=(1, 1, 1, 1),
               activation="mish")                                                                      # 5×5×6
    p = b.pool(x, "max", (3, 3), (2, 2), (1, 1, 1, 1))                                                  # 5×5×8
    p = b.upsample(b.pad(p, (0, 1, 1, 0)), (2, 1))                                                     # 12×6×8
    p = b.pool(p, "avg", (2, 2), (2, 1), (0, 0, 1, 0), count_pad=True)                                 # 6×6×8
    p = b.pool(p, "avg", (2, 2), (1, 1), (1, 0, 0, 0), count_pad=False)                                # 6×5×8
    p = b.select(p, "first", 0, 5)                                                                     # 5×5×8
    y = b.concat([p, s], "last")                                                                       # 5×5×14
    y = b.conv(y, _w(rng, 14, 10), _w(rng, 10), activation="selu")                                     # pointwise
    hi, lo = b.global_pool(y, "max"), b.global_pool(y, "avg")
    return b, b.linear(b.binary(hi, lo, "sub"), _w(rng, 10, 5), _w(rng, 5), activation="softmax")


def sequence(rng, int8=False):
    b = ModelBuilder((16, 6), int8=int8)
    x = b.conv(b.input, _w(rng, 30, 9), _w(rng, 9), kernel=(5, 1), padding=(2, 2, 0, 0), activation="elu",
               alpha=0.5)                                                                              # 16×9
    x = b.pool(x, "avg", (3, 1), (1, 1), (1, 1, 0, 0), count_pad=True)
    x = b.conv(x, _w(rng, 9, 9), None, kernel=(3, 1), stride=(2, 1), dilation=(2, 1), padding=(2, 1, 0, 0),
               groups=3, activation="softplus")                                                        # 8×9
    x = b.pool(x, "max", (2, 1), (2, 1))                                                               # 4×9
    x = b.layer_norm(x)
    x = b.binary(x, b.global_pool(x, "max"), "add")                                                    # row broadcast
    c = b.select(x, "last", 4, 1)                                                                      # 4×1
    x = b.binary(x, b.activation(c, "sigmoid"), "mul")                                                 # channel broadcast
    x = b.binary(x, b.add_const(b.activation(c, "softsign"), np.full(4, 2.0)), "div")
    x = b.activation(b.activation(x, "gelu_tanh"), "leaky_relu", alpha=0.2)
    x = b.linear(b.reshape(x, (36,)), _w(rng, 36, 7), _w(rng, 7), activation="silu")
    x = b.activation(b.linear(x, _w(rng, 7, 7, scale=0.1), None, activation="tanh"), "exp")
    return b, b.linear(b.activation(x, "gelu"), _w(rng, 7, 3), _w(rng, 3), activation="hard_swish")


def recurrent(rng, int8=False):
    b = ModelBuilder((6, 4), int8=int8)

    def cell(cell, fin, units, dirs):
        g = {"LSTM": 4, "GRU": 3, "RNN": 1}[cell] * units
        nb = 2 * g if cell == "GRU" else g
        return [(_w(rng, fin, g), _w(rng, units, g), _w(rng, nb)) for _ in range(dirs)]

    a = b.recurrent(b.input, "LSTM", 3, cell("LSTM", 4, 3, 2), return_sequences=True)               # 6×6 (concat)
    g = b.recurrent(b.input, "GRU", 5, cell("GRU", 4, 5, 1), activation="relu", return_sequences=True)  # 6×5
    s = b.concat([a, g], "last")                                                                     # 6×11
    r = b.recurrent(s, "RNN", 4, cell("RNN", 11, 4, 2), return_sequences=True, merge="mul")           # 6×4
    l = b.recurrent(r, "LSTM", 3, cell("LSTM", 4, 3, 2), activation="relu", merge="ave")             # (3,)
    q = b.recurrent(s, "GRU", 3, cell("GRU", 11, 3, 2), merge="sum")                                 # (3,)
    t = b.select(g, "first", 5, 1, squeeze=True)                                                     # (5,)
    u = b.recurrent(b.select(s, "first", 2, 3), "RNN", 2, cell("RNN", 11, 2, 1), activation="sigmoid")  # (2,)
    return b, b.concat([l, q, t, u], "last")


def tokens(rng, int8=False):
    b = ModelBuilder((5,), int8=int8)
    e = b.add_const(b.embedding(b.input, _w(rng, 12, 6)), _w(rng, 30))                               # 5×6
    a = b.attention(e, 3, _w(rng, 6, 6), _w(rng, 6, 6), _w(rng, 6, 9), _w(rng, 9, 6), _w(rng, 6), _w(rng, 6),
                    _w(rng, 9), _w(rng, 6), causal=True)                                             # dk 2, dv 3
    h = b.layer_norm(b.add(e, a), 1.0 + _w(rng, 6, scale=0.1), _w(rng, 6, scale=0.1))
    u = b.upsample(h, (2, 1))                                                                        # 10×6
    k = b.activation(u, "relu")
    c = b.attention(h, 2, _w(rng, 6, 8), _w(rng, 6, 8), _w(rng, 6, 4), _w(rng, 4, 6), v=u, k=k)     # S = 10, Rq = 5
    c = b.permute(b.reshape(c, (5, 3, 2)), (2, 0, 1))                                                # 2×5×3
    c = b.affine(b.reshape(c, (10, 3)), _w(rng, 3), _w(rng, 3))
    c = b.softmax(b.binary(c, b.select(c, "first", 4, 1), "min"))
    return b, b.binary(c, b.concat([b.select(c, "first", 0, 5), b.select(c, "first", 5, 5)], "first"), "add")


FAMILIES = {"vision": vision, "sequence": sequence, "recurrent": recurrent, "tokens": tokens}


def make(tmp_path, family, quantize=None):
    """(path of the written .knx, its builder); quantize="int8" writes int8 weight blocks"""
    rng = np.random.default_rng(sum(map(ord, family)))
    b, _ = FAMILIES[family](rng, int8=quantize == "int8")
    p = str(tmp_path / f"{family}{'_i8' if quantize else ''}.knx")
    b.save(p)
    return p, b


def inputs(b, batch, seed=0):
    rng = np.random.default_rng(seed + batch)
    shape = b.input.shape
    if shape == (5,):  # token ids of the embedding model
        return rng.integers(0, 12, (batch,) + shape).astype(np.float32)
    return rng.standard_normal((batch,) + shape).astype(np.float32)


def random_sequence_model(rng, int8=False):
    """A random graph over one T × F sample (T 1-12, F 1-64): 3-9 ops drawn from Linear (with and without bias and
    activation), activations, layer norm, softmax, a Linear whose output is added to its input (the residual add the
    runtime fuses into the Linear), affine, constant add, self-attention (causal or not), recurrent layers (one or two
    directions, every merge, sequences or the last state), concat and select; each op reads the latest value or an
    earlier one.  Weights N(0, 1/in) so values stay of order one; layer norm eps ≥ 1e-3 (a near-constant row otherwise
    turns last-bit differences of fp32 sums into large ones).  Returns (builder, output value)."""
    T, F = int(rng.integers(1, 13)), int(rng.integers(1, 65))
    b = ModelBuilder((T, F), int8=int8)
    vals = [b.input]

    def w(i, o):
        return rng.normal(0.0, 1.0 / np.sqrt(i), (i, o))

    def maybe_bias(n):
        return rng.normal(0.0, 0.1, n) if rng.random() < 0.8 else None

    acts = [None, "relu", "gelu", "tanh", "sigmoid", "silu", "leaky_relu", "elu"]
    for _ in range(int(rng.integers(3, 10))):
        x = vals[-1] if rng.random() < 0.6 else vals[int(rng.integers(0, len(vals)))]
        seq, d = len(x.shape) == 2, x.shape[-1]
        ops = ["linear", "act", "layer_norm", "softmax", "residual", "affine", "add_const", "concat"]
        if seq:
            ops += ["attention", "attention", "recurrent", "recurrent", "select"]
        op = str(rng.choice(ops))
        if op == "linear":
            n = int(rng.integers(1, 97))
            y = b.linear(x, w(d, n), maybe_bias(n), activation=acts[int(rng.integers(0, len(acts)))], alpha=0.1)
        elif op == "act":
            y = b.activation(x, str(rng.choice(acts[1:])), alpha=0.1)
        elif op == "layer_norm":
            affine = rng.random() < 0.7
            y = b.layer_norm(x, rng.normal(1.0, 0.2, d) if affine else None, rng.normal(0.0, 0.2, d) if affine else None,
                             eps=float(rng.choice([1e-3, 1e-2])))
        elif op == "softmax":
            y = b.softmax(x)
        elif op == "residual":
            h = b.linear(x, w(d, d), maybe_bias(d), activation=str(rng.choice(["relu", "gelu"])) if rng.random() < 0.4
                         else None)
            y = b.add(h, x) if rng.random() < 0.5 else b.add(x, h)
        elif op == "affine":
            y = b.affine(x, rng.normal(1.0, 0.2, d), rng.normal(0.0, 0.2, d))
        elif op == "add_const":
            y = b.add_const(x, rng.normal(0.0, 0.2, int(np.prod(x.shape))))
        elif op == "concat":
            peers = [v for v in vals if v.shape[:-1] == x.shape[:-1]]
            y = b.concat([x, peers[int(rng.integers(0, len(peers)))]])
        elif op == "attention":
            heads, dk, dv, out = int(rng.integers(1, 5)), int(rng.integers(1, 33)), int(rng.integers(1, 33)), int(
                rng.integers(1, 97))
            bias = rng.random() < 0.5
            bs = [rng.normal(0.0, 0.1, n) if bias else None for n in (heads * dk, heads * dk, heads * dv, out)]
            y = b.attention(x, heads, w(d, heads * dk), w(d, heads * dk), w(d, heads * dv), w(heads * dv, out), *bs,
                            causal=bool(rng.random() < 0.5))
        elif op == "recurrent":
            cell = str(rng.choice(["LSTM", "GRU", "RNN"]))
            units, g = int(rng.integers(1, 65)), {"LSTM": 4, "GRU": 3, "RNN": 1}[cell]
            dirs = [(w(d, g * units), w(units, g * units), rng.normal(0.0, 0.1, (2 if cell == "GRU" else 1) * g * units))
                    for _ in range(int(rng.integers(1, 3)))]
            y = b.recurrent(x, cell, units, dirs, return_sequences=bool(rng.random() < 0.5),
                            merge=str(rng.choice(["concat", "sum", "mul", "ave"])))
        else:  # select rows of the sequence
            if x.shape[0] < 2:
                continue
            start = int(rng.integers(0, x.shape[0]))
            length = int(rng.integers(1, x.shape[0] - start + 1))
            y = b.select(x, "first", start, length, squeeze=length == 1 and bool(rng.random() < 0.5))
        vals.append(y)
    return b, vals[-1]


def _extent(n, k, stride, dil, pad_a, pad_b):
    """output length of a window of k taps (dilation dil) over n padded positions"""
    return (n + pad_a + pad_b - dil * (k - 1) - 1) // stride + 1


def random_vision_model(rng, int8=False):
    """A random graph over one H × W × C sample (H, W 1-20; C 1-16, 32 or 64): 3-8 ops drawn from convolutions (kernel
    1-3, stride, dilation, padding, groups, activation), a convolution added to its input (the residual add fused into
    the convolution), pooling (max / average, padding counted or not), padding, upsampling, concat on channels,
    binary ops against the sample's pooled channel vector (row broadcast), affine and activations; then a global pool
    and a Linear.  Half of the models take channels-first input.  Returns (builder, output value)."""
    H, W = int(rng.integers(1, 21)), int(rng.integers(1, 21))
    C = int(rng.choice([1, 2, 3, 4, 8, 16, 32, 64]))
    b = ModelBuilder((H, W, C), channels_first=bool(rng.random() < 0.5), int8=int8)
    vals = [b.input]

    def conv_w(k, cin, cout, groups):
        return rng.normal(0.0, 1.0 / np.sqrt(k * cin / groups), (k * cin // groups, cout))

    acts = [None, "relu", "relu6", "gelu", "tanh", "silu"]
    for _ in range(int(rng.integers(3, 9))):
        x = vals[-1] if rng.random() < 0.6 else vals[int(rng.integers(0, len(vals)))]
        h, w, c = x.shape
        op = str(rng.choice(["conv", "conv", "conv", "residual", "pool", "pad", "upsample", "concat", "binary",
                             "affine", "act"]))
        if op in ("conv", "residual"):
            kh, kw = (int(rng.integers(1, 4)), int(rng.integers(1, 4))) if op == "conv" else (3, 3)
            groups = int(rng.choice([g for g in (1, 1, 1, 2, 4, c) if c % g == 0]))
            co = c if op == "residual" or groups == c else groups * int(rng.choice([1, 2, 4, 8, 16, 32]))
            if op == "residual":
                y = b.conv(x, conv_w(9, c, co, groups), rng.normal(0.0, 0.1, co), kernel=(3, 3), padding=(1, 1, 1, 1),
                           groups=groups, activation="relu" if rng.random() < 0.5 else None)
                y = b.add(y, x) if rng.random() < 0.5 else b.add(x, y)
            else:
                sh, sw = int(rng.integers(1, 3)), int(rng.integers(1, 3))
                dh, dw = int(rng.integers(1, 3)), int(rng.integers(1, 3))
                pad = tuple(int(rng.integers(0, k)) for k in (kh, kh, kw, kw))
                if _extent(h, kh, sh, dh, pad[0], pad[1]) < 1 or _extent(w, kw, sw, dw, pad[2], pad[3]) < 1:
                    continue
                y = b.conv(x, conv_w(kh * kw, c, co, groups), rng.normal(0.0, 0.1, co) if rng.random() < 0.8 else None,
                           kernel=(kh, kw), stride=(sh, sw), dilation=(dh, dw), padding=pad, groups=groups,
                           activation=acts[int(rng.integers(0, len(acts)))])
        elif op == "pool":
            k, s = int(rng.integers(1, 4)), int(rng.integers(1, 3))
            pad = tuple(int(rng.integers(0, k)) for _ in range(4))
            if _extent(h, k, s, 1, pad[0], pad[1]) < 1 or _extent(w, k, s, 1, pad[2], pad[3]) < 1:
                continue
            y = b.pool(x, str(rng.choice(["max", "avg"])), (k, k), (s, s), pad, count_pad=bool(rng.random() < 0.5))
        elif op == "pad":
            y = b.pad(x, tuple(int(rng.integers(0, 3)) for _ in range(4)))
        elif op == "upsample":
            if h * w > 200:
                continue
            y = b.upsample(x, (int(rng.integers(1, 3)), int(rng.integers(1, 3))))
        elif op == "concat":
            peers = [v for v in vals if v.shape[:-1] == x.shape[:-1]]
            y = b.concat([x, peers[int(rng.integers(0, len(peers)))]])
        elif op == "binary":
            y = b.binary(x, b.global_pool(x, str(rng.choice(["avg", "max"]))), str(rng.choice(["add", "sub", "mul", "max"])))
        elif op == "affine":
            y = b.affine(x, rng.normal(1.0, 0.2, c), rng.normal(0.0, 0.2, c))
        else:
            y = b.activation(x, str(rng.choice(acts[1:])))
        vals.append(y)
    g = b.global_pool(vals[-1], str(rng.choice(["avg", "max"])))
    n = int(rng.integers(1, 17))
    return b, b.linear(g, rng.normal(0.0, 1.0 / np.sqrt(g.shape[-1]), (g.shape[-1], n)), rng.normal(0.0, 0.1, n))
