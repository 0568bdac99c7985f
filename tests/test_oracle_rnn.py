"""Pins the oracle's recurrent cells (oracle/knx_ref.py _rnn, restating reference include/kernix_model.h:563-648)
against an independent implementation: torch.nn.LSTM / GRU / RNN on the CPU in float64.

Mapping (Keras gate order in the .knx file, reference docs/graph-runtime-design.md): LSTM i f c o = torch i f g o;
GRU z r h (reset after, input-side then recurrent-side bias) = torch r z n with b_ih / b_hh; simple RNN h = act(x·W +
b + h·U).  Two directions: torch's output holds [forward, backward] per step (the "concat" merge), its h_n the last
state of each direction (the backward one is the state at t = 0, which a non-sequence output returns).  A wrong gate
order, a reset gate applied before the recurrent product, a missing recurrent bias or a backward pass that is not
reversed in time fails these comparisons.
"""
import numpy as np
import pytest
import torch

from oracle import knx_ref

KIND = {"LSTM": 4, "GRU": 5, "RNN": 6}
GATES = {"LSTM": 4, "GRU": 3, "RNN": 1}
ACT = {"tanh": 4, "relu": 0}


def keras_to_torch(cell, W, U, b, u):
    """per-direction torch parameters (weight_ih, weight_hh, bias_ih, bias_hh) from Keras-order W, U, bias"""
    G = GATES[cell]
    if cell == "GRU":  # z r h → r z n
        order = lambda a: np.concatenate([a[..., u:2 * u], a[..., :u], a[..., 2 * u:3 * u]], axis=-1)  # noqa: E731
        return order(W).T, order(U).T, order(b[:G * u]), order(b[G * u:])
    return W.T, U.T, b, np.zeros_like(b)


def torch_rnn(cell, act, dirs, x, B, T, u):
    cin = x.shape[1]
    kw = dict(input_size=cin, hidden_size=u, batch_first=True, bidirectional=len(dirs) == 2, dtype=torch.float64)
    mod = torch.nn.RNN(nonlinearity=act, **kw) if cell == "RNN" else getattr(torch.nn, cell)(**kw)
    with torch.no_grad():
        for d, (W, U, b) in enumerate(dirs):
            sfx = "_reverse" if d == 1 else ""
            wi, wh, bi, bh = keras_to_torch(cell, W.astype(np.float64), U.astype(np.float64), b.astype(np.float64), u)
            getattr(mod, "weight_ih_l0" + sfx).copy_(torch.from_numpy(np.ascontiguousarray(wi)))
            getattr(mod, "weight_hh_l0" + sfx).copy_(torch.from_numpy(np.ascontiguousarray(wh)))
            getattr(mod, "bias_ih_l0" + sfx).copy_(torch.from_numpy(np.ascontiguousarray(bi)))
            getattr(mod, "bias_hh_l0" + sfx).copy_(torch.from_numpy(np.ascontiguousarray(bh)))
        out, hn = mod(torch.from_numpy(x.astype(np.float64).reshape(B, T, cin)))
    if cell == "LSTM":
        hn = hn[0]
    return out.numpy(), hn.numpy()


def merged(out, hn, ndir, u, merge, ret):
    if ret:
        parts = [out[..., :u], out[..., u:]] if ndir == 2 else [out]
    else:
        parts = [hn[0], hn[1]] if ndir == 2 else [hn[0]]
    if ndir == 1 or merge == 0:
        return np.concatenate(parts, axis=-1)
    if merge == 1:
        return parts[0] + parts[1]
    if merge == 2:
        return parts[0] * parts[1]
    return (parts[0] + parts[1]) * 0.5


CASES = [(cell, act, nd, merge, ret)
         for cell in ("LSTM", "GRU", "RNN")
         for act in (("tanh", "relu") if cell == "RNN" else ("tanh",))
         for nd, merge in ((1, 0), (2, 0), (2, 1), (2, 2), (2, 3))
         for ret in (0, 1)]


@pytest.mark.parametrize("cell,act,ndir,merge,ret", CASES)
def test_rnn_cells_vs_torch(cell, act, ndir, merge, ret):
    rng = np.random.default_rng(KIND[cell] * 100 + ndir * 10 + merge + 3 * ret)
    B, T, cin, u = 3, 6, 5, 4
    G = GATES[cell]
    nb = 2 * G * u if cell == "GRU" else G * u
    dirs = [(rng.uniform(-0.6, 0.6, (cin, G * u)).astype(np.float32),
             rng.uniform(-0.6, 0.6, (u, G * u)).astype(np.float32),
             rng.uniform(-0.5, 0.5, nb).astype(np.float32)) for _ in range(ndir)]
    x = rng.normal(0, 1, (B * T, cin)).astype(np.float32)
    op = dict(kind=KIND[cell], u=u, act=ACT[act], ret=ret, dirs=[(W, ("f32", U), b) for W, U, b in dirs], merge=merge)
    y, shape = knx_ref._rnn(op, x, (T, cin), B, "ref")
    out, hn = torch_rnn(cell, act, dirs, x, B, T, u)
    want = merged(out, hn, ndir, u, merge, ret).reshape(y.shape)
    assert np.max(np.abs(y - want)) <= 2e-5, (cell, act, ndir, merge, ret)
