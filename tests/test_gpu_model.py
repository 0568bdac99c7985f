""".knx forward parity on the GPU (through kernix_capi_* via the Python Model binding) against the CPU oracle.

Tolerance: max|a−b| / max(1, max|ref|) ≤ 1e-4 for fp32 paths (reference test/model_test.c:127-142).
int8 ("i8" mode) forward vs the oracle's int8 arithmetic: bit-exact when every int8 layer's input is itself bit-exact
(chains of int8 Linear + ReLU); when an fp32 op (LayerNorm, GELU, attention) feeds the per-row int8 quantizer, a
1-ulp difference can move rint(x/sx) across a .5 boundary (or change the row maximum) and shift an output by about
one quantization step, so those models are held to the reference's int8 bound 1e-2 (reference test/model_test.c:651).
int8 vs the dequantized fp32 path of the same model: the reference's int8-model bound 5e-2
(reference test/zoo_torch_test.py:207-208).
Full-size configurations are checked on a random subset of samples (samples are independent, so the oracle only has
to run the subset).
"""
import os

import numpy as np
import pytest

from kernix_amd import configs
from kernix_amd.kernix import INT8_I8, INT8_REF, Model
from oracle import knx_ref

pytestmark = pytest.mark.gpu


def rel_err(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want)) / max(1.0, float(np.max(np.abs(want)))))


def to_rows(m, x):
    """model input in the runtime's channels-last row layout"""
    x = np.asarray(x, np.float32)
    if m.channels_first and x.ndim >= 3:
        x = np.moveaxis(x, 1, -1)
    return np.ascontiguousarray(x).reshape(-1, m.in_dim)


def check(path, x, tol=1e-4, mode="ref", workspace_mb=None, subset=None):
    m = Model(path, workspace_mb=workspace_mb)
    if mode == "i8":
        m.set_int8_mode(INT8_I8)
    y = m(x).reshape(len(x), -1)
    ref = knx_ref.parse(path)
    idx = np.arange(len(x)) if subset is None else np.sort(np.random.default_rng(1).choice(len(x), subset, replace=False))
    xs = to_rows(m, np.asarray(x)[idx])
    want, _ = knx_ref.forward(ref, xs, mode=mode)
    err = rel_err(y[idx], want)
    m.close()
    assert err <= tol, f"{os.path.basename(path)} {mode}: rel err {err:.3e} > {tol}"
    return y


# ---------------------------------------------------------------- int8 MLP (784-512-256-10)
@pytest.mark.parametrize("batch", [1, 2, 3, 64])
def test_int8_mlp_ref_mode(tmp_path, batch):
    p = str(tmp_path / "mlp.knx")
    x = configs.int8_mlp(p, batch=batch)
    check(p, x)


@pytest.mark.parametrize("batch", [1, 64, 1000])
def test_int8_mlp_i8_mode_bit_exact(tmp_path, batch):
    """int8 arithmetic end to end: quantize → i8 MFMA → dequant/bias/ReLU epilogue is bit-exact with the oracle."""
    p = str(tmp_path / "mlp.knx")
    x = configs.int8_mlp(p, batch=batch)
    y = check(p, x, tol=0.0, mode="i8")
    y_ref = Model(p)(x)
    assert rel_err(y, y_ref) <= 5e-2  # int8 vs dequantized fp32


# ---------------------------------------------------------------- fp32 MLP
def test_fp32_mlp_small(tmp_path):
    p = str(tmp_path / "f.knx")
    x = configs.fp32_mlp(p, batch=300, dims=(256, 320, 256, 100))
    check(p, x)


def test_fp32_mlp_full_size_subset(tmp_path):
    p = str(tmp_path / "f.knx")
    x = configs.fp32_mlp(p, batch=8192)
    check(p, x, workspace_mb=0, subset=48)


# ---------------------------------------------------------------- CNN
def test_cnn_small(tmp_path):
    p = str(tmp_path / "c.knx")
    x = configs.cnn(p, batch=8, hw=16, widths=(16, 16, 32, 64))
    check(p, x)


def test_cnn_full_size_subset(tmp_path):
    p = str(tmp_path / "c.knx")
    x = configs.cnn(p, batch=256)
    check(p, x, workspace_mb=0, subset=8)


# ---------------------------------------------------------------- Transformer
def test_transformer_small_ref_and_i8(tmp_path):
    p = str(tmp_path / "t.knx")
    x = configs.transformer(p, batch=4, seq=32, d=64, heads=4, ffn=128, layers=2)
    y_ref = check(p, x)
    y_i8 = check(p, x, mode="i8", tol=1e-2)
    assert rel_err(y_i8, y_ref) <= 5e-2


def test_transformer_full_size_subset(tmp_path):
    p = str(tmp_path / "t.knx")
    x = configs.transformer(p, batch=64)
    check(p, x, workspace_mb=0, subset=4)
    check(p, x, workspace_mb=0, subset=4, mode="i8", tol=1e-2)


# ---------------------------------------------------------------- fused residual add
FUSE_CASES = {
    "cnn": lambda p: configs.cnn(p, batch=64, hw=16, widths=(64, 64, 128, 256)),  # conv2 + add: pipelined conv
    "cnn_small": lambda p: configs.cnn(p, batch=8, hw=16, widths=(16, 16, 32, 64)),  # conv2 + add: general conv
    "transformer": lambda p: configs.transformer(p, batch=8, seq=64, d=128, heads=4, ffn=256, layers=2),
}


@pytest.mark.parametrize("name", sorted(FUSE_CASES))
@pytest.mark.parametrize("mode", ["ref", "i8"])
def test_fused_residual_add_is_bit_identical(tmp_path, monkeypatch, name, mode):
    """a step followed by the BINARY add of its output runs as one pass (the add in the step's epilogue); the result
    is the same bits as the two separate steps (KNX_NO_FUSE=1), and both match the oracle"""
    p = str(tmp_path / "m.knx")
    x = FUSE_CASES[name](p)
    outs = []
    for no_fuse in ("0", "1"):
        monkeypatch.setenv("KNX_NO_FUSE", no_fuse)
        m = Model(p)
        if mode == "i8":
            m.set_int8_mode(INT8_I8)
        outs.append(np.array(m(x)))
        m.close()
    assert np.array_equal(outs[0], outs[1]), name
    want, _ = knx_ref.forward(knx_ref.parse(p), to_rows(Model(p), x), mode=mode)
    assert rel_err(outs[0].reshape(len(want), -1), want) <= (1e-4 if mode == "ref" else 1e-2)


# ---------------------------------------------------------------- runtime behaviour (reference test/model_test.c)
def test_chunking_reuse_and_trim(tmp_path):
    """chunked == unchunked (reference test/model_test.c:296-360)"""
    p = str(tmp_path / "t.knx")
    x = configs.transformer(p, batch=10, seq=16, d=32, heads=2, ffn=64, layers=1)
    m = Model(p, workspace_mb=0)
    want = m(x)
    per, fixed, batch = m.ws_info()
    assert batch == 10 * 16
    for chunk in (1, 3, 9):
        from kernix_amd import kernix as kx
        kx._lib.kernix_capi_set_workspace_limit(m._h, (fixed + per * chunk) * 4)
        got = m(x)
        assert m.ws_info()[2] == chunk * 16
        assert rel_err(got, want) <= 1e-5
    got3 = m(x[:3])  # after chunks of 3 (3,3,3,1): same buffers at the full chunk size
    assert rel_err(got3, want[:3]) <= 1e-5
    m.trim()
    assert m.ws_info()[2] == -1
    assert rel_err(m(x), want) <= 1e-5
    m.close()


def test_zero_rows_bad_input_and_own_output(tmp_path):
    p = str(tmp_path / "mlp.knx")
    x = configs.int8_mlp(p, batch=3)
    m = Model(p)
    with pytest.raises(ValueError):
        m(np.zeros((2, 783), np.float32))
    y = m(x)
    assert y.shape == (3, 10)
    m.close()


@pytest.mark.parametrize("batch,workspace_mb", [(1, None), (64, None), (256, None), (64, 0.5)])
def test_channels_first_input_moved_on_the_device(tmp_path, batch, workspace_mb):
    """A channels-first model called with NCHW samples: the binding passes them as they are to kernix_capi_forward_cf,
    which transposes them on the GPU (inputs of up to 1 MB through the pinned staging buffer, larger ones through the
    copy engine, in workspace pieces when a limit splits the batch).  The result is the bits of kernix_capi_forward on
    the channels-last rows that the binding used to make on the host."""
    from kernix_amd import kernix as kx

    p = str(tmp_path / "c.knx")
    x = configs.cnn(p, batch=batch, hw=32 if batch > 1 else 16)
    m = Model(p, workspace_mb=workspace_mb)
    assert m.channels_first
    y = m(x)
    rows = np.ascontiguousarray(np.moveaxis(x, 1, -1), np.float32).reshape(-1, m.in_dim)
    want = np.empty_like(y)
    assert kx._lib.kernix_capi_forward(m._h, rows.ctypes.data, rows.shape[0], want.ctypes.data) == 0
    assert np.array_equal(y, want)
    assert np.array_equal(m(x), want)  # again, with the staging buffer and the device copy already allocated
    m.close()


def test_workspace_identical_across_batch_sizes(tmp_path):
    """batch 37 after 4096 after 1 gives the same result (buffer reallocation, reference test/model_test.c:148)"""
    p = str(tmp_path / "f.knx")
    x = configs.fp32_mlp(p, batch=4096, dims=(64, 128, 96, 10))
    m = Model(p)
    a = m(x[:37]).copy()
    m(x)
    m(x[:1])
    b = m(x[:37])
    assert np.array_equal(a, b)
    m.close()


@pytest.mark.parametrize("name", ["cnn", "transformer"])
def test_forward_device_matches_host_forward(tmp_path, name):
    """kernix_capi_forward_device on device buffers gives the bits of the host-pointer forward: on a torch stream, on
    the model's own stream (stream=None), chunked under a small workspace limit, and interleaved with host forwards
    of another batch (the forwards share the model's workspace; the runtime orders them on the device)."""
    import torch

    p = str(tmp_path / f"{name}.knx")
    if name == "cnn":
        x = configs.cnn(p, batch=24, hw=16, widths=(32, 32, 64, 64))
    else:
        x = configs.transformer(p, batch=6, layers=2, seq=32, d=128, heads=4, ffn=256)
    m = Model(p)
    want = m(x).reshape(len(x), -1)
    other = np.asarray(x)[::-1].copy()
    want_other = m(other).reshape(len(x), -1)
    dx = torch.from_numpy(to_rows(m, x)).cuda()
    s = torch.cuda.Stream()
    outs = []
    for stream in (s, None):
        out = torch.full((len(x), m.out_dim), 7.0, dtype=torch.float32, device="cuda")
        with torch.cuda.stream(s):
            m.forward_device(dx.data_ptr(), dx.shape[0], out.data_ptr(),
                             None if stream is None else stream.cuda_stream)
        got_other = m(other).reshape(len(x), -1)  # a host forward right after, on the model's stream
        assert np.array_equal(got_other, want_other)
        torch.cuda.synchronize()
        outs.append(out.cpu().numpy())
    for got in outs:
        assert np.array_equal(got, want)
    m.close()
    # chunked: at most 5 samples per piece
    m = Model(p)
    per, fixed, _ = m.ws_info()
    m2 = Model(p, workspace_mb=((fixed + 5 * per) * 4 + 100) / (1 << 20))
    out = torch.zeros((len(x), m.out_dim), dtype=torch.float32, device="cuda")
    with torch.cuda.stream(s):
        m2.forward_device(dx.data_ptr(), dx.shape[0], out.data_ptr(), s.cuda_stream)
    s.synchronize()
    assert m2.ws_info()[2] == 5 * m2.seq_len
    got = out.cpu().numpy()
    m.close()
    m2.close()
    assert np.array_equal(got, want)



@pytest.mark.parametrize("case", ["direct", "reshape_out", "in_place"])
def test_forward_device_output_paths(tmp_path, case):
    """The device forward's output: written by the last step straight into the caller's buffer (direct), or copied
    from the workspace when the output value is a reshape view or when the output buffer is the input buffer
    (in_place): all give the host forward's bits."""
    import torch

    from kernix_amd.knxfile import ModelBuilder

    rng = np.random.default_rng(5)
    b = ModelBuilder((16,))
    h = b.linear(b.input, rng.normal(0, 0.3, (16, 32)), rng.normal(0, 0.1, 32), activation="relu")
    y = b.linear(h, rng.normal(0, 0.3, (32, 16)), rng.normal(0, 0.1, 16))
    if case == "reshape_out":
        b.reshape(y, (4, 4))
    p = b.save(str(tmp_path / "m.knx"))
    x = rng.normal(0, 1, (40, 16)).astype(np.float32)
    m = Model(p)
    want = m(x).reshape(40, -1).copy()
    s = torch.cuda.Stream()
    for _ in range(3):
        dx = torch.from_numpy(x).cuda()
        out = dx if case == "in_place" else torch.full((40, m.out_dim), 7.0, dtype=torch.float32, device="cuda")
        with torch.cuda.stream(s):
            m.forward_device(dx.data_ptr(), 40, out.data_ptr(), s.cuda_stream)
        s.synchronize()
        assert np.array_equal(out.cpu().numpy().reshape(40, -1), want)
    m.close()


# ---------------------------------------------------------------- Linear chains (one launch for consecutive Linears)
@pytest.mark.parametrize("mode", ["ref", "i8"])
@pytest.mark.parametrize("batch", [1, 2, 17, 64])
def test_linear_chain_matches_separate_steps(tmp_path, monkeypatch, mode, batch):
    """The int8 MLP's three Linear steps as one chain launch (≤ 64 rows) against the same steps launched one by one
    (KNX_CHAIN=0): the same bits wherever the layers run int8 arithmetic (i8 mode, or ≤ 2 rows), within 1e-5 where
    they run fp32 on the dequantized weights (another summation order)."""
    p = str(tmp_path / "mlp.knx")
    x = configs.int8_mlp(p, batch=batch)
    got = {}
    for chain in ("1", "0"):
        monkeypatch.setenv("KNX_CHAIN", chain)
        m = Model(p)
        if mode == "i8":
            m.set_int8_mode(INT8_I8)
        got[chain] = m(x).copy()
        got[chain + "again"] = m(x).copy()
        m.close()
    assert np.array_equal(got["1"], got["1again"])
    if mode == "i8" or batch <= 2:
        assert np.array_equal(got["1"], got["0"])
    else:
        assert rel_err(got["1"], got["0"]) <= 1e-5


@pytest.mark.parametrize("seed", [1, 2])
def test_linear_chain_sweep(tmp_path, monkeypatch, seed):
    """Random MLPs (1-5 Linear layers of widths 1-2048 log-uniform, fp32 / int8-column / int8-row weights, with or
    without bias, activations with and without transcendentals), batch 1-64, ref or i8 mode: the forward with chains
    against the layers launched one by one (KNX_CHAIN=0) — the same bits where every layer runs int8 arithmetic (int8
    column weights in i8 mode or at <= 2 rows), within 1e-5 otherwise."""
    from kernix_amd.knxfile import ModelBuilder

    rng = np.random.default_rng(seed)

    def logu(lo, hi):
        return int(np.exp(rng.uniform(np.log(lo), np.log(hi + 1))))

    for case in range(25):
        depth = int(rng.integers(1, 6))
        dims = [logu(1, 2048) for _ in range(depth + 1)]
        fmts = [str(rng.choice(["f32", "i8_col", "i8_row"])) for _ in range(depth)]
        acts = [rng.choice([None, "relu", "gelu", "leaky_relu", "tanh", "sigmoid"]) for _ in range(depth)]
        batch = logu(1, 64)
        mode = str(rng.choice(["ref", "i8"]))
        name = f"case {case}: dims {dims} formats {fmts} activations {acts} batch {batch} mode {mode}"
        print(name, flush=True)
        b = ModelBuilder((dims[0],))
        h = b.input
        for i in range(depth):
            w = rng.normal(0.0, 1.0 / np.sqrt(dims[i]), (dims[i], dims[i + 1]))
            bias = rng.normal(0.0, 0.1, dims[i + 1]) if rng.random() < 0.8 else None
            h = b.linear(h, w, bias, activation=acts[i], alpha=0.1, fmt=fmts[i])
        p = str(tmp_path / f"sweep{seed}_{case}.knx")
        b.save(p)
        x = rng.normal(0.0, 1.0, (batch, dims[0])).astype(np.float32)
        got = {}
        for chain in ("1", "0"):
            monkeypatch.setenv("KNX_CHAIN", chain)
            m = Model(p)
            if mode == "i8":
                m.set_int8_mode(INT8_I8)
            got[chain] = m(x).copy()
            m.close()
        # int8 arithmetic needs int8-column weights (an int8-row block is dequantized to fp32 when it is read)
        if all(f == "i8_col" for f in fmts) and (mode == "i8" or batch <= 2):
            assert np.array_equal(got["1"], got["0"]), name
        else:
            assert rel_err(got["1"], got["0"]) <= 1e-5, name


@pytest.mark.parametrize("batch", [1, 16])
def test_linear_chain_gave_up_is_recomputed(tmp_path, monkeypatch, capfd, batch):
    """A chain launch whose barrier stops waiting (forced from the host: KNX_GRID_SPIN=0 stops every workgroup but
    the last to arrive without polling; all accesses stay those of a normal launch) does not leave wrong outputs:
    the host forward recomputes the whole forward one launch per layer in the same call, so its result is the bits of
    KNX_CHAIN=0; a device forward reports it through device_status() (False once, then True after a normal
    forward).  i8 mode at batch 16, the reference's int8 dispatch at batch 1: every layer int8, so the chain and the
    separate launches give the same bits."""
    import torch

    p = str(tmp_path / "mlp.knx")
    x = configs.int8_mlp(p, batch=batch)
    m = Model(p)
    if batch > 2:
        m.set_int8_mode(INT8_I8)
    monkeypatch.setenv("KNX_CHAIN", "0")
    want = m(x).copy()
    monkeypatch.delenv("KNX_CHAIN")
    capfd.readouterr()
    monkeypatch.setenv("KNX_GRID_SPIN", "0")
    got = m(x).copy()
    assert "recomputed one launch per layer" in capfd.readouterr().err
    assert np.array_equal(got, want)
    dx = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    out = torch.zeros((len(x), m.out_dim), dtype=torch.float32, device="cuda")
    for _ in range(3):
        m.forward_device(dx.data_ptr(), dx.shape[0], out.data_ptr())
        assert not m.device_status()
    monkeypatch.delenv("KNX_GRID_SPIN")
    m.forward_device(dx.data_ptr(), dx.shape[0], out.data_ptr())
    assert m.device_status()
    assert np.array_equal(out.cpu().numpy(), want)
    assert np.array_equal(m(x), want)
    assert "recomputed" not in capfd.readouterr().err
    m.close()


def test_linear_chain_graph_boundaries(tmp_path):
    """Chains inside a graph: a run broken by a value that two steps read, a Linear whose output feeds a fused add,
    a layer_norm between Linears, int8 and fp32 weights mixed, pieces of ≤ 64 rows through the workspace limit;
    against the oracle in both modes."""
    from kernix_amd.knxfile import ModelBuilder

    rng = np.random.default_rng(21)

    def w(i, o):
        return rng.normal(0, 1.0 / np.sqrt(i), (i, o))

    b = ModelBuilder((48,))
    h1 = b.linear(b.input, w(48, 64), rng.normal(0, 0.1, 64), activation="relu", fmt="i8_col")
    h2 = b.linear(h1, w(64, 64), rng.normal(0, 0.1, 64), activation="gelu")
    h3 = b.linear(h2, w(64, 32), None, activation="relu", fmt="i8_col")
    h4 = b.linear(h3, w(32, 64), rng.normal(0, 0.1, 64), fmt="i8_col")
    r = b.add(h4, h1)  # h1 read twice: the run h1 → h2 stops there; h4 feeds a fused add
    n = b.layer_norm(r, np.ones(64), np.zeros(64))
    h5 = b.linear(n, w(64, 40), rng.normal(0, 0.1, 40), activation="leaky_relu", alpha=0.2, fmt="i8_col")
    h6 = b.linear(h5, w(40, 24), rng.normal(0, 0.1, 24), activation="tanh")
    b.linear(h6, w(24, 8), rng.normal(0, 0.1, 8), fmt="i8_col")
    p = b.save(str(tmp_path / "g.knx"))
    x = rng.normal(0, 1, (100, 48)).astype(np.float32)
    for mode in ("ref", "i8"):
        check(p, x[:2], mode=mode, tol=1e-4 if mode == "ref" else 1e-2)
        check(p, x[:40], mode=mode, tol=1e-4 if mode == "ref" else 1e-2)
        check(p, x, mode=mode, tol=1e-4 if mode == "ref" else 1e-2, workspace_mb=0.05)


# ---------------------------------------------------------------- host-buffer forward with overlapped copies
@pytest.mark.parametrize("case", ["fp32", "int8_i8", "int8_i8_chunked", "transformer"])
def test_overlapped_host_forward(tmp_path, monkeypatch, case):
    """Batches with ≥ 32 MB of input run as sub-pieces whose input copies (through the pinned staging ring) overlap
    the previous piece's compute (two halves of the staged input, ordered by events): against the same forward without
    overlap (KNX_OVERLAP=0), the same bits where the rows are independent of the piece size (int8 arithmetic), within
    1e-5 for fp32 GEMMs of other row counts; inside workspace chunking too; twice in a row (the halves' events carried
    over)."""
    p = str(tmp_path / "m.knx")
    mode, ws = "ref", None
    if case == "fp32":
        x = configs.fp32_mlp(p, batch=8400, dims=(1024, 512, 256, 100))
    elif case == "transformer":
        x = configs.transformer(p, batch=132, seq=128, d=512, heads=8, ffn=1024, layers=1)
    else:
        x = configs.int8_mlp(p, batch=11000)
        mode = "i8"
        if case == "int8_i8_chunked":
            ws = 24.0
    assert np.asarray(x, np.float32).nbytes >= 32 << 20
    got = {}
    for ov in ("1", "0"):
        monkeypatch.setenv("KNX_OVERLAP", ov)
        m = Model(p, workspace_mb=ws)
        if mode == "i8":
            m.set_int8_mode(INT8_I8)
        got[ov] = m(x).copy()
        got[ov + "b"] = m(x).copy()
        m.close()
    assert np.array_equal(got["1"], got["1b"])
    if case.startswith("int8"):
        assert np.array_equal(got["1"], got["0"])
    else:
        assert rel_err(got["1"], got["0"]) <= 1e-5
    ref = knx_ref.parse(p)
    xs = to_rows(Model(p), np.asarray(x)[:4])
    want, _ = knx_ref.forward(ref, xs, mode=mode)
    assert rel_err(got["1"][:4].reshape(4, -1), want) <= (1e-4 if mode == "ref" else 0.0)


def test_ffn_fusions_full_size(tmp_path, monkeypatch):
    """The Transformer at full size in i8 mode (8192 rows, d 512, FFN 2048, one layer): the fused steps (layer_norm +
    quantize, GEMM + residual add) give the same bits as every step on its own (KNX_NO_FUSE=1), forward after forward."""
    p = str(tmp_path / "t.knx")
    x = configs.transformer(p, batch=64, layers=1)
    outs = []
    for no_fuse in ("0", "1"):
        monkeypatch.setenv("KNX_NO_FUSE", no_fuse)
        m = Model(p)
        m.set_int8_mode(INT8_I8)
        outs.append(np.array(m(x)))
        outs.append(np.array(m(x)))
        m.close()
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])


_TORCH_AFTER = r"""
import sys
import numpy as np
sys.path.insert(0, sys.argv[1])
from kernix_amd import configs
from kernix_amd.kernix import Model
x = configs.int8_mlp(sys.argv[2], batch=3)
m = Model(sys.argv[2])
y1 = m(x)
assert "torch" not in sys.modules
import torch
t = torch.arange(4, dtype=torch.float32, device="cuda") * 2
assert float(t.sum()) == 12.0
y2 = m(x)
m.close()
np.save(sys.argv[3], np.stack([y1, y2]))
print("ok")
"""


def test_model_before_torch_import(tmp_path):
    """a Model created and run before `import torch` keeps working after it (the binding loads torch's HIP runtime
    before the library, so the two share one): a child process runs the forward, imports torch, uses the device
    through torch and runs the forward again; both outputs match the oracle"""
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    p, out = str(tmp_path / "m.knx"), str(tmp_path / "y.npy")
    r = subprocess.run([sys.executable, "-c", _TORCH_AFTER, root, p, out], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), r.stderr[-2000:]
    y = np.load(out)
    assert np.array_equal(y[0], y[1])
    x = configs.int8_mlp(p, batch=3)
    want, _ = knx_ref.forward(knx_ref.parse(p), x.reshape(3, -1))
    assert rel_err(y[0], want) <= 1e-4
