"""The persistent RNN recurrence (knx_hip_rnn_recurrence: every timestep of a direction in one launch; the batch
rows split over workgroups that each hold all of U where it fits, else a grid of workgroups splitting the units with a
barrier per timestep, KNX_RNN_SOLO=0 forcing the latter) against the per-timestep launches (KNX_RNN_PERSISTENT=0) and
the oracle (reference kernix_rnn_dir, include/kernix_model.h:563-632).

Where the recurrence runs int8 arithmetic (int8 recurrent weights in i8 mode, or at <= 2 rows in the reference's
dispatch) both paths quantize the same rows with the quantizer's operations and sum exactly in int32, so they give the
same bits; fp32 recurrences sum in different orders, within 1e-5 of each other.  Against the oracle: 1e-4 for fp32
(reference test/model_test.c:268-272 holds the LSTM to 1e-5 of a double loop), and for int8 recurrences the
reference's int8 bound 1e-2 (test/model_test.c:651).
"""
import numpy as np
import pytest

from kernix_amd import configs, hipabi
from kernix_amd.hipabi import ptr
from kernix_amd.kernix import INT8_I8, Model
from oracle import knx_ref

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def rel_err(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want)) / max(1.0, float(np.max(np.abs(want)))))


def forward(path, x, mode, monkeypatch, persistent, solo=True):
    monkeypatch.setenv("KNX_RNN_PERSISTENT", "1" if persistent else "0")
    monkeypatch.setenv("KNX_RNN_SOLO", "1" if solo else "0")
    m = Model(path)
    try:
        if mode == "i8":
            m.set_int8_mode(INT8_I8)
        return m(x).copy()
    finally:
        m.close()


CASES = [
    # cell, directions, units, fin, T
    ("LSTM", 1, 40, 20, 9),
    ("GRU", 2, 33, 12, 7),
    ("RNN", 2, 64, 16, 5),
    ("LSTM", 2, 128, 128, 6),
    ("GRU", 1, 200, 24, 4),
    ("LSTM", 1, 3, 5, 1),
    ("RNN", 1, 512, 8, 3),     # a row of h over 64 lanes, two float4s each (fp32 fits the LDS up to batch 17)
    ("LSTM", 1, 1000, 8, 3),   # int8 recurrences: four float4s per lane, the last row partly past u
    ("LSTM", 1, 256, 16, 4),   # past the row-split kernel (int8 and fp32): the grid
]


@pytest.mark.parametrize("case", range(len(CASES)))
@pytest.mark.parametrize("int8,mode", [(False, "ref"), (True, "ref"), (True, "i8")])
@pytest.mark.parametrize("batch", [1, 2, 17, 64])
def test_persistent_matches_per_step_and_oracle(tmp_path, monkeypatch, case, int8, mode, batch):
    cell, dirs, units, fin, T = CASES[case]
    p = str(tmp_path / "r.knx")
    x = configs.lstm(p, seed=case, batch=batch, T=T, fin=fin, units=units, int8=int8, cell=cell, directions=dirs)
    got = forward(p, x, mode, monkeypatch, True)
    per_step = forward(p, x, mode, monkeypatch, False)
    int8_rec = int8 and (mode == "i8" or batch <= 2)
    if int8_rec:
        assert np.array_equal(got, per_step), (cell, dirs, units, batch, mode)
    else:
        assert rel_err(got, per_step) <= 1e-5, (cell, dirs, units, batch, mode)
    want, _ = knx_ref.forward(knx_ref.parse(p), x.reshape(-1, fin), mode=mode)
    assert rel_err(got.reshape(want.shape), want) <= (1e-2 if int8_rec else 1e-4)
    # the grid form at the same shape (the per-timestep path where it does not fit)
    multi = forward(p, x, mode, monkeypatch, True, solo=False)
    if int8_rec:
        assert np.array_equal(multi, got)
    else:
        assert rel_err(multi, got) <= 1e-5


@pytest.mark.parametrize("int8,mode", [(False, "ref"), (True, "i8")])
def test_persistent_two_rows_per_workgroup(tmp_path, monkeypatch, int8, mode):
    """above 256 rows each workgroup of the row split takes two rows: against the per-timestep path and the oracle"""
    p = str(tmp_path / "w.knx")
    x = configs.lstm(p, seed=9, batch=300, T=5, fin=12, units=40, int8=int8)
    got = forward(p, x, mode, monkeypatch, True)
    per_step = forward(p, x, mode, monkeypatch, False)
    if int8:
        assert np.array_equal(got, per_step)
    else:
        assert rel_err(got, per_step) <= 1e-5
    want, _ = knx_ref.forward(knx_ref.parse(p), x.reshape(-1, 12), mode=mode)
    assert rel_err(got.reshape(want.shape), want) <= (1e-2 if int8 else 1e-4)


@pytest.mark.parametrize("seed", [1, 2])
def test_recurrence_sweep(tmp_path, monkeypatch, seed):
    """shapes drawn at random (cell, directions, units 1-300 log-uniform, inputs, timesteps, batch 1-300 log-uniform,
    fp32 or int8 weights, ref or i8 mode): the one-launch recurrence (the row-split kernel where it fits, with the
    Linear after a one-direction layer in the same launch) and the grid form against the per-timestep launches"""
    rng = np.random.default_rng(seed)

    def logu(lo, hi):
        return int(np.exp(rng.uniform(np.log(lo), np.log(hi + 1))))

    for case in range(20):
        cell, dirs = str(rng.choice(["LSTM", "GRU", "RNN"])), int(rng.integers(1, 3))
        units, fin, T, batch = logu(1, 300), logu(1, 64), int(rng.integers(1, 13)), logu(1, 300)
        int8 = bool(rng.random() < 0.6)
        mode = "i8" if int8 and rng.random() < 0.5 else "ref"
        name = f"case {case}: {cell} dirs {dirs} units {units} fin {fin} T {T} batch {batch} int8 {int8} mode {mode}"
        print(name, flush=True)
        p = str(tmp_path / f"sweep{seed}_{case}.knx")
        x = configs.lstm(p, seed=100 * seed + case, batch=batch, T=T, fin=fin, units=units, int8=int8, cell=cell,
                         directions=dirs)
        got = forward(p, x, mode, monkeypatch, True)
        per_step = forward(p, x, mode, monkeypatch, False)
        grid = forward(p, x, mode, monkeypatch, True, solo=False)
        if int8 and (mode == "i8" or batch <= 2):
            assert np.array_equal(got, per_step) and np.array_equal(grid, per_step), name
        else:
            assert rel_err(got, per_step) <= 1e-5 and rel_err(grid, per_step) <= 1e-5, name


def test_persistent_returns_sequences_and_nan_rows(tmp_path, monkeypatch):
    """a sequence-returning bidirectional LSTM (every timestep's state at its own position, the backward direction
    from t = T-1) feeding a GRU, int8 in i8 mode; a sample holding NaN gives a NaN output row and leaves the others
    untouched, bit for bit as the per-step path"""
    from kernix_amd.knxfile import ModelBuilder

    rng = np.random.default_rng(5)
    T, F, u1, u2 = 8, 10, 24, 16
    b = ModelBuilder((T, F), int8=True)

    def cell(kind, fin, units):
        g = {"LSTM": 4, "GRU": 3}[kind] * units
        return (rng.normal(0, 0.3, (fin, g)), rng.normal(0, 0.3, (units, g)),
                rng.normal(0, 0.1, 2 * g if kind == "GRU" else g))

    h = b.recurrent(b.input, "LSTM", u1, [cell("LSTM", F, u1), cell("LSTM", F, u1)], return_sequences=True)
    h = b.recurrent(h, "GRU", u2, [cell("GRU", 2 * u1, u2)], return_sequences=True)
    p = str(tmp_path / "s.knx")
    b.save(p)
    x = rng.normal(0, 1, (5, T, F)).astype(np.float32)
    x[3, 4, 2] = np.nan
    got = forward(p, x, "i8", monkeypatch, True)
    assert np.array_equal(got, forward(p, x, "i8", monkeypatch, False), equal_nan=True)
    assert np.isnan(got[3]).all() and np.isfinite(np.delete(got, 3, axis=0)).all()
    want, _ = knx_ref.forward(knx_ref.parse(p), x.reshape(-1, F), mode="i8")
    ok = np.isfinite(want)
    assert np.array_equal(np.isnan(got.reshape(want.shape)), ~ok)
    assert rel_err(got.reshape(want.shape)[ok], want[ok]) <= 1e-2


@pytest.mark.parametrize("kind,u", [(4, 40), (5, 36), (6, 100)])
def test_recurrence_int8_rows_of_any_word_pitch(kind, u):
    """int8 recurrent weight rows of a multiple of 4 bytes but not of 16 (the C ABI allows them; the forward's rows are
    multiples of 64 bytes) are loaded a word at a time: the bits of the same weight at a 64-byte pitch"""
    L = hipabi.lib()
    hipabi.check(L.knx_hip_init())
    rng = np.random.default_rng(kind)
    gates = {4: 4, 5: 3, 6: 1}[kind]
    gu, B, T = gates * u, 3, 5
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    zx = dev(rng.normal(0, 1, (B * T, gu)).astype(np.float32))
    q = rng.integers(-127, 128, (gu, u)).astype(np.int8)
    qs = dev(rng.uniform(0.001, 0.01, gu).astype(np.float32))
    brec = dev(rng.normal(0, 0.1, gu).astype(np.float32)) if kind == 5 else None
    u4 = (u + 3) // 4 * 4
    h0 = torch.zeros((B, u4), dtype=torch.float32, device="cuda")
    h1 = torch.zeros((B, u4), dtype=torch.float32, device="cuda")
    scratch = torch.zeros(64, dtype=torch.int64, device="cuda")
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    outs = []
    for kp in (u4, (u + 63) // 64 * 64):
        assert kp % 16 != 0 or kp % 64 == 0
        qp = np.zeros((gu, kp), np.int8)
        qp[:, :u] = q
        dq = dev(qp)
        y = torch.full((B, T, u), float("nan"), dtype=torch.float32, device="cuda")
        hipabi.check(L.knx_hip_rnn_recurrence(kind, 4, 0.0, B, T, u, 0, ptr(zx), None, 0, ptr(dq), kp, ptr(qs),
                                              ptr(brec), ptr(h0), ptr(h1), ptr(y), u, 1, ptr(scratch), 512,
                                              ptr(status), hipabi.stream()))
        torch.cuda.synchronize()
        outs.append(y.cpu().numpy())
    assert np.isfinite(outs[1]).all()
    assert np.array_equal(outs[0], outs[1])


@pytest.mark.parametrize("cell,units", [("LSTM", 128), ("GRU", 40), ("RNN", 100)])
@pytest.mark.parametrize("int8,mode", [(False, "ref"), (True, "ref"), (True, "i8")])
@pytest.mark.parametrize("batch", [1, 2, 17, 300])
def test_recurrence_runs_its_linear_in_the_same_launch(tmp_path, monkeypatch, cell, units, int8, mode, batch):
    """a one-direction recurrence whose last state only feeds a Linear runs that Linear at the end of its own launch
    (knx_hip_rnn_recurrence_dense): against the separate steps (KNX_NO_FUSE=1), an int8 Linear gives the same bits
    (the same quantizer, int32 sums and epilogue), an fp32 one is within 1e-5; with and without the Linear's bias and
    activation; and the forward against the oracle"""
    from kernix_amd.knxfile import ModelBuilder

    rng = np.random.default_rng(units + batch)
    T, F, n = 6, 24, 12
    g = {"LSTM": 4, "GRU": 3, "RNN": 1}[cell] * units
    b = ModelBuilder((T, F), int8=int8)
    h = b.recurrent(b.input, cell, units, [(rng.normal(0, 1 / np.sqrt(F), (F, g)), rng.normal(0, 1 / np.sqrt(units), (units, g)),
                                           rng.normal(0, 0.01, 2 * g if cell == "GRU" else g))])
    bias = None if cell == "GRU" else rng.normal(0, 0.1, n)
    h = b.linear(h, rng.normal(0, 1 / np.sqrt(units), (units, n)), bias, activation="relu" if cell == "LSTM" else None)
    p = str(tmp_path / "d.knx")
    b.save(p)
    x = rng.normal(0, 1, (batch, T, F)).astype(np.float32)
    L = hipabi.lib()
    kind = {"LSTM": 4, "GRU": 5, "RNN": 6}[cell]
    rec_i8 = int8 and (mode == "i8" or batch <= 2)
    assert L.knx_hip_rnn_recurrence_dense_fits(kind, batch, units, int(rec_i8), n) == 1
    got = forward(p, x, mode, monkeypatch, True)
    monkeypatch.setenv("KNX_NO_FUSE", "1")
    sep = forward(p, x, mode, monkeypatch, True)
    monkeypatch.delenv("KNX_NO_FUSE")
    if rec_i8:
        assert np.array_equal(got, sep)
    else:
        assert rel_err(got, sep) <= 1e-5
    want, _ = knx_ref.forward(knx_ref.parse(p), x.reshape(-1, F), mode=mode)
    assert rel_err(got.reshape(want.shape), want) <= (1e-2 if rec_i8 else 1e-4)


def test_recurrence_entry_point_rejects(monkeypatch):
    L = hipabi.lib()
    hipabi.check(L.knx_hip_init())
    assert L.knx_hip_rnn_recurrence_fits(4, 64, 128, 0) == 1
    assert L.knx_hip_rnn_recurrence_fits(4, 1000, 128, 0) == 1  # U fits a workgroup: the rows split, any batch
    assert L.knx_hip_rnn_recurrence_fits(4, 65, 256, 0) == 0  # neither form: the per-timestep path
    assert L.knx_hip_rnn_recurrence_fits(4, 64, 256, 0) == 1  # the grid form
    assert L.knx_hip_rnn_recurrence_dense_fits(4, 64, 256, 0, 10) == 0  # the Linear only joins the batch-split form
    assert L.knx_hip_rnn_recurrence_dense_fits(4, 1000, 128, 1, 10) == 1
    assert L.knx_hip_rnn_recurrence_fits(7, 1, 128, 0) == 0
    assert L.knx_hip_rnn_recurrence_fits(4, 64, 4096, 0) == 0  # h does not fit a workgroup's LDS


@pytest.mark.parametrize("batch,units,expect", [(1, 32, True), (64, 32, True), (65, 32, True), (65, 256, False)])
def test_forward_uses_the_persistent_recurrence(tmp_path, monkeypatch, batch, units, expect):
    """the forward takes the one-launch recurrence wherever it fits (an injected failure of that entry point fails the
    forward) and the per-timestep launches otherwise or with KNX_RNN_PERSISTENT=0"""
    p = str(tmp_path / "l.knx")
    x = configs.lstm(p, batch=batch, T=4, fin=16, units=units)
    monkeypatch.setenv("KNX_HIP_FAIL", "knx_hip_rnn_recurrence,knx_hip_rnn_recurrence_dense")
    m = Model(p)
    try:
        if expect:
            with pytest.raises(RuntimeError):
                m(x)
        else:
            m(x)
        monkeypatch.setenv("KNX_RNN_PERSISTENT", "0")
        y = m(x)
    finally:
        m.close()
    want, _ = knx_ref.forward(knx_ref.parse(p), x.reshape(-1, 16))
    assert rel_err(y, want) <= 1e-4


def test_recurrence_that_stopped_waiting_is_recomputed(tmp_path, monkeypatch):
    """with a poll limit of 0 (forced from the host) every workgroup of the grid form but the last to reach a
    timestep's barrier stops waiting and sets the model's status word; the forward is then recomputed one launch per
    timestep, so the result is the per-timestep path's, bit for bit (int8 recurrence)"""
    p = str(tmp_path / "g.knx")
    x = configs.lstm(p, seed=3, batch=16, T=6, fin=16, units=64, int8=True)
    want = forward(p, x, "i8", monkeypatch, False)
    monkeypatch.setenv("KNX_GRID_SPIN", "0")
    got = forward(p, x, "i8", monkeypatch, True, solo=False)
    assert np.array_equal(got, want)
