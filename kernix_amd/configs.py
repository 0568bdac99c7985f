"""Synthetic workloads of the KERNIX forward hot path (random weights from a seed, written as .knx files).

    int8_mlp      int8-quantized MLP 784-512-256-10 (ReLU hidden, linear out), KNX2 I8_COL, batch 64, x ~ U[0,1)
    i8gemm        standalone int8 GEMM y = relu(((float)(A·Wᵀ)·sa[m])·sw[n] + bias[n]), K = N = 4096
    fp32_mlp      fp32 MLP 4096-4096-4096-1000 (ReLU fused on the hidden layers), KNX1, batch 8192, x ~ N(0,1)
    cnn           conv3x3 3→64 → conv3x3 64→64 → residual add → conv3x3/2 64→128 → conv3x3/2 128→256 → GAP → dense 10,
                  ReLU after each conv, KNX3 layout 1 (NCHW input), batch 256 × 3×32×32, x ~ N(0,1)
    transformer   4 pre-LN encoder layers, d_model 512, 8 heads, FFN 2048 GELU, seq 128, int8 (I8_COL) weights, batch 64
    lstm          one LSTM layer over T × F (F = 128, 128 units, T = 32, last state), then a dense 10; KNX3, fp32 or int8
                  (I8_ROW input / I8_COL recurrent weights) weights, x ~ N(0,1)

Weight init: Linear W ~ N(0, 1/√fan_in) (int8 MLP) or Kaiming-normal N(0, √(2/fan_in)); biases N(0, 0.01);
conv He-normal with the BatchNorm already folded (a plain conv bias).  Every generator takes a scale divisor so the
tests can build the same architecture at reduced width / batch.
"""
import numpy as np

from .knxfile import ModelBuilder


def int8_mlp(path, seed=0, batch=64, dims=(784, 512, 256, 10)):
    rng = np.random.default_rng(seed)
    b = ModelBuilder((dims[0],))
    h = b.input
    for i in range(len(dims) - 1):
        fan_in = dims[i]
        w = rng.normal(0.0, 1.0 / np.sqrt(fan_in), (fan_in, dims[i + 1]))
        bias = rng.normal(0.0, 0.01, dims[i + 1])
        h = b.linear(h, w, bias, activation="relu" if i < len(dims) - 2 else None, fmt="i8_col")
    b.save(path, version=2)
    return rng.random((batch, dims[0]), dtype=np.float32)


def i8gemm_inputs(M, N=4096, K=4096, seed=12345):
    """A (M×K), W (N×K) int8 uniform in [−127, 127]; sa (M), sw (N) U[0.001, 0.01]; bias N(0, 0.1)."""
    rng = np.random.default_rng(seed)
    A = rng.integers(-127, 128, (M, K), dtype=np.int8)
    W = rng.integers(-127, 128, (N, K), dtype=np.int8)
    sa = rng.uniform(0.001, 0.01, M).astype(np.float32)
    sw = rng.uniform(0.001, 0.01, N).astype(np.float32)
    bias = rng.normal(0.0, 0.1, N).astype(np.float32)
    return A, W, sa, sw, bias


def fp32_mlp(path, seed=0, batch=8192, dims=(4096, 4096, 4096, 1000)):
    rng = np.random.default_rng(seed)
    b = ModelBuilder((dims[0],))
    h = b.input
    for i in range(len(dims) - 1):
        fan_in = dims[i]
        w = rng.standard_normal((fan_in, dims[i + 1]), dtype=np.float32) * np.float32(np.sqrt(2.0 / fan_in))
        bias = rng.normal(0.0, 0.01, dims[i + 1])
        h = b.linear(h, w, bias, activation="relu" if i < len(dims) - 2 else None)
    b.save(path, version=1)
    return rng.standard_normal((batch, dims[0]), dtype=np.float32)


def cnn(path, seed=0, batch=256, hw=32, widths=(64, 64, 128, 256), classes=10):
    """The residual add joins conv1 and conv2 (the only same-shape pair); returns NCHW input."""
    rng = np.random.default_rng(seed)
    b = ModelBuilder((hw, hw, 3), channels_first=True)

    def conv(x, cin, cout, stride):
        fan_in = 9 * cin
        w = rng.standard_normal((fan_in, cout), dtype=np.float32) * np.float32(np.sqrt(2.0 / fan_in))
        bias = rng.normal(0.0, 0.01, cout)
        return b.conv(x, w, bias, kernel=(3, 3), stride=(stride, stride), padding=(1, 1, 1, 1), activation="relu")

    h1 = conv(b.input, 3, widths[0], 1)
    h2 = conv(h1, widths[0], widths[1], 1)
    r = b.add(h1, h2)
    h3 = conv(r, widths[1], widths[2], 2)
    h4 = conv(h3, widths[2], widths[3], 2)
    p = b.global_pool(h4, "avg")
    w = rng.normal(0.0, 1.0 / np.sqrt(widths[3]), (widths[3], classes))
    b.linear(p, w, rng.normal(0.0, 0.01, classes))
    b.save(path)
    return rng.standard_normal((batch, 3, hw, hw), dtype=np.float32)


def transformer(path, seed=0, batch=64, seq=128, d=512, heads=8, ffn=2048, layers=4, quantize="int8"):
    rng = np.random.default_rng(seed)
    b = ModelBuilder((seq, d), int8=quantize == "int8")

    def lin(fan_in, fan_out):
        return rng.normal(0.0, 1.0 / np.sqrt(fan_in), (fan_in, fan_out)), rng.normal(0.0, 0.01, fan_out)

    x = b.input
    for _ in range(layers):
        h = b.layer_norm(x, 1.0 + rng.normal(0.0, 0.05, d), rng.normal(0.0, 0.05, d), 1e-5)
        (wq, bq), (wk, bk), (wv, bv), (wo, bo) = lin(d, d), lin(d, d), lin(d, d), lin(d, d)
        a = b.attention(h, heads, wq, wk, wv, wo, bq, bk, bv, bo)
        x = b.add(x, a)
        h = b.layer_norm(x, 1.0 + rng.normal(0.0, 0.05, d), rng.normal(0.0, 0.05, d), 1e-5)
        w1, b1 = lin(d, ffn)
        w2, b2 = lin(ffn, d)
        f = b.linear(b.linear(h, w1, b1, activation="gelu"), w2, b2)
        x = b.add(x, f)
    b.save(path)
    return rng.standard_normal((batch, seq, d), dtype=np.float32)


# Algorithmic work per unit (one forward of the whole batch / one GEMM): used for roofline fractions.
def i8gemm_work(M, N=4096, K=4096):
    ops = 2.0 * M * N * K
    bytes_ = M * K + N * K + 4 * M + 8 * N + 4 * M * N
    return ops, bytes_


def lstm(path, seed=0, batch=64, T=32, fin=128, units=128, classes=10, int8=False, cell="LSTM", directions=1):
    """Recurrent model (reference kernix_rnn_dir, include/kernix_model.h:563-632): one recurrent layer (gates in Keras
    order), W ~ N(0, 1/√fin), U ~ N(0, 1/√units), bias N(0, 0.01) (a GRU's holds the input and recurrent halves),
    then a Linear to `classes`."""
    rng = np.random.default_rng(seed)
    g = {"LSTM": 4, "GRU": 3, "RNN": 1}[cell] * units
    b = ModelBuilder((T, fin), int8=int8)
    dirs = []
    for _ in range(directions):
        w = rng.normal(0.0, 1.0 / np.sqrt(fin), (fin, g))
        u = rng.normal(0.0, 1.0 / np.sqrt(units), (units, g))
        bias = rng.normal(0.0, 0.01, 2 * g if cell == "GRU" else g)
        dirs.append((w, u, bias))
    h = b.recurrent(b.input, cell, units, dirs)
    width = units * directions
    h = b.linear(h, rng.normal(0.0, 1.0 / np.sqrt(width), (width, classes)), rng.normal(0.0, 0.01, classes))
    b.save(path)
    return rng.normal(0.0, 1.0, (batch, T, fin)).astype(np.float32)


def lstm_flops(batch=64, T=32, fin=128, units=128, classes=10, gates=4, directions=1):
    return directions * 2.0 * batch * T * gates * units * (fin + units) + 2.0 * batch * units * directions * classes


def mlp_flops(batch, dims):
    return 2.0 * batch * sum(dims[i] * dims[i + 1] for i in range(len(dims) - 1))


def cnn_flops(batch=256, hw=32, widths=(64, 64, 128, 256), classes=10):
    f, h, cin = 0.0, hw, 3
    for i, cout in enumerate(widths):
        stride = 2 if i >= 2 else 1
        h = (h + 2 - 3) // stride + 1
        f += 2.0 * batch * h * h * 9 * cin * cout
        cin = cout
    return f + 2.0 * batch * widths[-1] * classes


def transformer_flops(batch=64, seq=128, d=512, heads=8, ffn=2048, layers=4):
    rows = batch * seq
    proj = 2.0 * rows * d * d * 4
    attn = 2.0 * batch * heads * seq * seq * (d // heads) * 2
    ff = 2.0 * rows * d * ffn * 2
    return layers * (proj + attn + ff)


def transformer_ffn_flops(batch=64, seq=128, d=512, ffn=2048, layers=4):
    """The feed-forward LINEAR layers: the part of transformer_flops that runs on the int8 GEMM in `i8` mode (the
    attention projections are dequantized to fp32 at load, as the reference does)."""
    return layers * 2.0 * batch * seq * d * ffn * 2
