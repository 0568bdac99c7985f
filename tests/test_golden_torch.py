"""KNX3 semantics pinned by PyTorch: files written by the reference's own exporter from small torch models, with
torch's outputs (tests/golden/torch, made by tests/golden/make_torch_golden.py).  The CPU oracle and the GPU forward
must both reproduce torch — a wrong attention input/weight order, convolution row order, channels-first handling,
LSTM gate order or BatchNorm fold would not.  Tolerance: the reference's exporter tests' 2e-4 relative to
max(1, max|y|) (reference test/zoo_torch_test.py:33-57); int8 weights against the float torch model: 5e-2, the
reference's bound for int8 models (reference test/zoo_torch_test.py:207-208)."""
import os

import numpy as np
import pytest

from oracle import knx_ref

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "torch")
NAMES = ["bilstm", "convnet", "encoder", "encoder_int8", "mlp"]


def fixture(name):
    f = np.load(os.path.join(HERE, f"{name}.npz"), allow_pickle=False)
    return os.path.join(HERE, f"{name}.knx"), f["x"], f["y"], int(f["layout"])


def tol(name):
    return 5e-2 if name.endswith("int8") else 2e-4


def rel_err(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    return float(np.max(np.abs(got - want)) / max(1.0, float(np.max(np.abs(want)))))


def channels_last_rows(x, layout, in_dim):
    if layout == 1 and x.ndim >= 3:
        x = np.moveaxis(x, 1, -1)
    return np.ascontiguousarray(x, np.float32).reshape(-1, in_dim)


@pytest.mark.parametrize("name", NAMES)
def test_oracle_reproduces_torch(name):
    path, x, y, layout = fixture(name)
    model = knx_ref.parse(path)
    in_dim = x.shape[1] if layout == 1 else x.shape[-1]
    got, _ = knx_ref.forward(model, channels_last_rows(x, layout, in_dim))
    want = y if not (layout == 1 and y.ndim >= 3) else np.moveaxis(y, 1, -1)
    assert rel_err(got.reshape(want.shape), want) <= tol(name)


@pytest.mark.parametrize("name", NAMES)
def test_loader_shapes_match_torch(name):
    """the runtime's loader (no device work) reads the shapes torch has"""
    from kernix_amd.kernix import Model

    path, x, y, layout = fixture(name)
    m = Model(path)
    assert m.channels_first == (layout == 1)
    assert m.in_shape == x.shape[1:] and m.out_shape == y.shape[1:]
    m.close()


@pytest.mark.gpu
@pytest.mark.parametrize("name", NAMES)
@pytest.mark.parametrize("mode", ["ref", "i8"])
def test_gpu_forward_reproduces_torch(name, mode):
    from kernix_amd.kernix import INT8_I8, Model

    path, x, y, _ = fixture(name)
    m = Model(path)
    if mode == "i8":
        m.set_int8_mode(INT8_I8)
    got = m(x)
    m.close()
    limit = tol(name) if mode == "ref" or not name.endswith("int8") else 5e-2
    assert rel_err(got, y) <= limit
