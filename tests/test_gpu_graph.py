"""Every graph op kind of the runtime through the GPU forward (Python Model binding → kernix_capi_*) against the CPU
oracle's forward, beyond the five benchmark models: grouped / depthwise / dilated / strided / 1-D convolution,
max and average pooling (with and without padding counted), padding, upsampling, global pooling, every binary op with
row and channel broadcasting, concat on both axes, select, reshape, permute, embedding, affine, add_const, layer norm,
softmax, every activation, causal and cross attention (three inputs, Rq ≠ S), and the recurrent cells (LSTM, GRU,
simple RNN) in one or two directions with every merge mode, returning sequences or the last state.

The models (tests/graph_models.py) are in the spirit of the reference's loader fuzz models (reference
test/knx_fuzz_test.py:22-44): one graph per family, small enough for the oracle.  Tolerance: max|a−b| / max(1, max|ref|) ≤ 1e-4 (reference
test/model_test.c:127-142); int8 ("i8" mode, recurrences and Linear on int8 arithmetic) ≤ 1e-2 (reference
test/model_test.c:651), since fp32 ops feed the per-row quantizer.
"""
import numpy as np
import pytest

from kernix_amd.kernix import INT8_I8, Model
from oracle import knx_ref
from tests.graph_models import FAMILIES, inputs, make

pytestmark = pytest.mark.gpu


def rel_err(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    if got.shape != want.shape:
        return np.inf
    return float(np.max(np.abs(got - want)) / max(1.0, float(np.max(np.abs(want))))) if want.size else 0.0


def run(path, x, mode="ref", workspace_mb=None):
    m = Model(path, workspace_mb=workspace_mb)
    try:
        if mode == "i8":
            m.set_int8_mode(INT8_I8)
        y = m(x).reshape(len(x), -1)
        in_dim, cf = m.in_dim, m.channels_first and np.ndim(x) >= 3
    finally:
        m.close()
    rows = np.moveaxis(np.asarray(x), 1, -1) if cf else x  # the oracle reads channels-last rows
    want, _ = knx_ref.forward(knx_ref.parse(path), np.ascontiguousarray(rows).reshape(-1, in_dim), mode=mode)
    return y, want


@pytest.mark.parametrize("family", sorted(FAMILIES))
@pytest.mark.parametrize("batch", [1, 3, 64])
def test_graph_fp32(tmp_path, family, batch):
    p, g = make(tmp_path, family)
    y, want = run(p, inputs(g, batch))
    assert np.isfinite(want).all()
    assert rel_err(y, want) <= 1e-4, family


@pytest.mark.parametrize("family", sorted(FAMILIES))
@pytest.mark.parametrize("mode", ["ref", "i8"])
def test_graph_int8_weights(tmp_path, family, mode):
    """int8 (I8_COL / I8_ROW) weights: dequantized at load (conv, attention, RNN input), int8 Linear and recurrence
    at ≤ 2 rows (ref mode, the reference's dispatch) or at every M (i8 mode)"""
    p, g = make(tmp_path, family, quantize="int8")
    for batch in (1, 2, 5):
        y, want = run(p, inputs(g, batch, seed=1), mode=mode)
        tol = 1e-4 if mode == "ref" and batch > 2 else 1e-2
        assert rel_err(y, want) <= tol, (family, mode, batch)


@pytest.mark.parametrize("kind", ["sequence", "vision"])
@pytest.mark.parametrize("seed", [1, 2])
def test_random_graphs(tmp_path, monkeypatch, kind, seed):
    """random graphs (graph_models.random_sequence_model / random_vision_model), fp32 or int8 weights, ref or i8 mode,
    batch 1-40: the forward with every fusion of the runtime (residual adds in the producer's epilogue, layer norm +
    quantize, Linear chains, the one-launch recurrence and its fused Linear) against the same forward with all of them
    off (KNX_NO_FUSE=1, KNX_CHAIN=0, KNX_RNN_PERSISTENT=0) and against the oracle, also run in pieces of a few samples
    under a small workspace limit"""
    from tests.graph_models import random_sequence_model, random_vision_model

    make_graph = random_sequence_model if kind == "sequence" else random_vision_model
    rng = np.random.default_rng(seed)
    for case in range(15):
        int8 = bool(rng.random() < 0.4)
        mode = "i8" if int8 and rng.random() < 0.5 else "ref"
        b, _ = make_graph(rng, int8=int8)
        p = str(tmp_path / f"{kind}{seed}_{case}.knx")
        b.save(p)
        batch = int(np.exp(rng.uniform(0.0, np.log(41))))
        shape = (b.input.shape[-1],) + b.input.shape[:-1] if b.channels_first else b.input.shape  # what the caller gives
        x = rng.standard_normal((batch,) + shape).astype(np.float32)
        name = (f"case {case}: ops {[n.kind for n in b._nodes]} input {shape} channels-first {b.channels_first} "
                f"batch {batch} int8 {int8} mode {mode}")
        print(name, flush=True)
        for var in ("KNX_NO_FUSE", "KNX_CHAIN", "KNX_RNN_PERSISTENT"):
            monkeypatch.delenv(var, raising=False)
        y, want = run(p, x, mode)
        monkeypatch.setenv("KNX_NO_FUSE", "1")
        monkeypatch.setenv("KNX_CHAIN", "0")
        monkeypatch.setenv("KNX_RNN_PERSISTENT", "0")
        y_off, _ = run(p, x, mode)
        for var in ("KNX_NO_FUSE", "KNX_CHAIN", "KNX_RNN_PERSISTENT"):
            monkeypatch.delenv(var, raising=False)
        y_chunk, _ = run(p, x, mode, workspace_mb=0.02)  # pieces of a few samples (fusions on)
        tol = 1e-2 if int8 else 1e-4  # int8: fp32 ops feed the per-row quantizer (see the module docstring)
        assert np.isfinite(want).all(), name
        assert rel_err(y, y_off) <= tol and rel_err(y, want) <= tol and rel_err(y_off, want) <= tol, name
        # ref mode dispatches int8 weights by rows (the reference's): pieces of one or two samples run them on int8
        # arithmetic where the whole batch runs their fp32 copies, so the int8-vs-fp32 bound holds there
        # (reference test/zoo_torch_test.py:207-208)
        assert rel_err(y_chunk, want) <= (5e-2 if int8 and mode == "ref" else tol), name
    for var in ("KNX_NO_FUSE", "KNX_CHAIN", "KNX_RNN_PERSISTENT"):
        monkeypatch.delenv(var, raising=False)


@pytest.mark.parametrize("family", sorted(FAMILIES))
def test_graph_chunked(tmp_path, family):
    """a workspace limit of a few samples: the forward runs in chunks and must give the unchunked result"""
    p, g = make(tmp_path, family)
    x = inputs(g, 50, seed=2)
    y_all, want = run(p, x)
    y_chunk, _ = run(p, x, workspace_mb=0.05)
    assert rel_err(y_all, want) <= 1e-4
    assert rel_err(y_chunk, want) <= 1e-4  # chunks of other row counts may take other GEMM tilings
