"""Small .knx graphs that together use every op kind of the runtime, one family per graph (CNN ops, 1-D convolution
and broadcasting, recurrent cells, embedding and attention), shared by the GPU graph parity tests and the loader fuzz
test.  Written with the numpy .knx writer; weights N(0, 0.3) from a seed per family."""
import numpy as np

from kernix_amd import knx_write
from kernix_amd.knx_write import FIRST, LAST


def W(rng, *s, scale=0.3):
    return rng.normal(0.0, scale, s)


def cnn_graph(rng, quantize=None):
    g = knx_write.Graph((9, 8, 3), quantize=quantize)
    x = g.conv(0, W(rng, 27, 6), W(rng, 6), (3, 3), pads=(1, 1, 1, 1), act="relu")
    y = g.conv(x, W(rng, 9, 6), None, (3, 3), pads=(1, 1, 1, 1), groups=6)                   # depthwise
    y = g.conv(y, W(rng, 27, 6), W(rng, 6), (3, 3), pads=(1, 1, 1, 1), groups=2, act="gelu")  # grouped
    x = g.binary(x, y, "add")
    z = g.conv(x, W(rng, 24, 6), W(rng, 6), (2, 2), stride=(1, 1), dil=(2, 2), pads=(1, 1, 1, 1), act="silu")
    z = g.conv(z, W(rng, 54, 5), W(rng, 5), (3, 3), stride=(2, 2), pads=(0, 1, 0, 1), act="tanh")  # 4×4×5
    x = g.upsample(g.pad(g.pool(x, "max", (2, 2), (2, 2)), (1, 0, 0, 1)), 2, 2)                  # 10×10×6
    x = g.pool(x, "avg", (3, 3), (1, 1), (1, 1, 1, 1), True)
    x = g.pool(x, "avg", (3, 3), (3, 3), (1, 1, 1, 1), False)                                   # 4×4×6
    x = g.concat([x, z], LAST)                                                                  # 4×4×11
    m = g.global_pool(x, "max")
    a = g.global_pool(x, "avg")
    v = g.binary(m, a, "sub")
    return g, g.linear(v, W(rng, 11, 4), W(rng, 4), act="softmax")


def conv1d_graph(rng, quantize=None):
    g = knx_write.Graph((20, 4), quantize=quantize)
    x = g.conv(0, W(rng, 12, 8), W(rng, 8), (3, 1), dil=(2, 1), pads=(2, 2, 0, 0), act="elu", alpha=0.7)
    x = g.pool(x, "max", (2, 1), (2, 1))                                                        # 10×8
    x = g.conv(x, W(rng, 16, 8), W(rng, 8), (4, 1), stride=(2, 1), pads=(1, 1, 0, 0), groups=2, act="leaky_relu",
               alpha=0.1)                                                                       # 5×8
    x = g.layernorm(x, 1.0 + W(rng, 8, scale=0.1), W(rng, 8, scale=0.1), 1e-5)
    r = g.global_pool(x, "avg")                                                                 # (8,)
    x = g.binary(x, r, "mul")                                                                   # row broadcast
    c = g.select(x, LAST, 0, 1)                                                                 # 5×1
    x = g.binary(x, c, "div")                                                                   # channel broadcast
    x = g.act(x, "softsign")
    return g, g.linear(g.reshape(x, (40,)), W(rng, 40, 6), W(rng, 6), act="hard_swish")


def rnn_graph(rng, quantize=None):
    g = knx_write.Graph((7, 5), quantize=quantize)
    a = g.rnn(0, "GRU", 4, [(W(rng, 5, 12), W(rng, 4, 12), W(rng, 24)), (W(rng, 5, 12), W(rng, 4, 12), W(rng, 24))],
              ret_seq=True)                                                                     # 7×8
    b = g.rnn(0, "LSTM", 3, [(W(rng, 5, 12), W(rng, 3, 12), W(rng, 12))], act="relu", ret_seq=True)  # 7×3
    c = g.concat([a, b], LAST)                                                                  # 7×11
    d = g.rnn(c, "RNN", 4, [(W(rng, 11, 4), W(rng, 4, 4), W(rng, 4)), (W(rng, 11, 4), W(rng, 4, 4), W(rng, 4))],
              ret_seq=False, merge="ave")                                                       # (4,)
    e = g.rnn(c, "LSTM", 4, [(W(rng, 11, 16), W(rng, 4, 16), W(rng, 16)), (W(rng, 11, 16), W(rng, 4, 16), W(rng, 16))],
              ret_seq=True, merge="sum")                                                        # 7×4
    f = g.rnn(e, "GRU", 4, [(W(rng, 4, 12), W(rng, 4, 12), W(rng, 24)), (W(rng, 4, 12), W(rng, 4, 12), W(rng, 24))],
              ret_seq=False, merge="mul")                                                       # (4,)
    s = g.select(a, FIRST, 6, 1, True)                                                          # (8,)
    return g, g.concat([d, s, f], LAST)


def attn_graph(rng, quantize=None):
    g = knx_write.Graph((6,), quantize=quantize)
    e = g.add_const(g.embedding(0, W(rng, 10, 8)), W(rng, 48))                                 # 6×8
    h = g.attention(e, 2, W(rng, 8, 6), W(rng, 6), W(rng, 8, 6), W(rng, 6), W(rng, 8, 4), W(rng, 4), W(rng, 4, 8),
                    W(rng, 8), causal=True)
    h = g.layernorm(g.binary(e, h, "add"), W(rng, 8), W(rng, 8), 1e-5)
    u = g.upsample(h, 2)                                                                        # 12×8
    k = g.act(u, "tanh")
    h = g.attention(h, 4, W(rng, 8, 16), None, W(rng, 8, 16), None, W(rng, 8, 8), None, W(rng, 8, 8), None,
                    v=u, k=k)                                                                   # cross, S = 12
    h = g.permute(g.reshape(h, (6, 2, 4)), (1, 0, 2))
    h = g.affine(g.reshape(h, (2, 24)), W(rng, 24), W(rng, 24))
    h = g.softmax(g.binary(h, g.select(h, FIRST, 1, 1), "max"))
    return g, g.binary(h, g.select(h, LAST, 3, 1), "min")


FAMILIES = {"cnn": cnn_graph, "conv1d": conv1d_graph, "rnn": rnn_graph, "attn": attn_graph}


def make(tmp_path, family, quantize=None):
    rng = np.random.default_rng(sum(map(ord, family)))
    g, _ = FAMILIES[family](rng, quantize)
    p = str(tmp_path / f"{family}.knx")
    g.write(p)
    return p, g


def inputs(g, batch, seed=0):
    rng = np.random.default_rng(seed + batch)
    shape = g.shapes[0]
    if shape == (6,):  # token ids of the embedding model
        return rng.integers(0, 10, (batch,) + shape).astype(np.float32)
    return rng.standard_normal((batch,) + shape).astype(np.float32)
