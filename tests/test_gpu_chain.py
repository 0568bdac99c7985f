"""knx_hip_linear_chain (a run of Linear layers over ≤ 64 rows in one launch) against the oracle, through the C ABI.

Every layer is checked on the chain's own input to that layer (the previous layer's output as the GPU wrote it):
int8 layers bit-exact against the oracle's kernix_qmatmul + activation (reference include/kernix_model.h:99-182,
:1853-1856) with no activation, ReLU or leaky ReLU, within 1e-5 with GELU (hardware exp2 / reciprocal); fp32 layers
within max|a−b| / max(1, max|ref|) ≤ 1e-4 of the float64 product.  An all-int8 chain is also
compared end to end with the oracle run layer after layer on its own outputs (bit-exact).
"""
import ctypes

import numpy as np
import pytest

from oracle import knx_ref
from kernix_amd import hipabi
from kernix_amd.hipabi import ChainLayer, ptr

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

RELU, GELU, LEAKY, NONE = 0, 1, 5, -1
EXACT_ACTS = (NONE, RELU, LEAKY)  # epilogues with no transcendental: int8 layers bit-exact


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def rel_err(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want)) / max(1.0, float(np.max(np.abs(want))))) if want.size else 0.0


@pytest.fixture(scope="module")
def L():
    lib = hipabi.lib()
    hipabi.check(lib.knx_hip_init())
    return lib


_STATUS = []


def status_word():
    """the launches' status word: one int of pinned host memory (set by a barrier that stopped waiting), held until
    the process ends"""
    if not _STATUS:
        p = ctypes.c_void_p()
        hipabi.check(hipabi.lib().knx_hip_host_malloc(ctypes.byref(p), 4))
        w = ctypes.c_int.from_address(p.value)
        w.value = 0
        _STATUS.append((p.value, w))
    return _STATUS[0][0]


def chain_status():
    """the status word after the launches so far (synchronized), then cleared"""
    torch.cuda.synchronize()
    status_word()
    w = _STATUS[0][1]
    v = w.value
    w.value = 0
    return v


class Chain:
    """Random layers (int8: weights in [-127, 127] with per-channel scales; fp32: N(0, 1/√k)) and their device
    buffers; run() calls the chain, outputs() reads every layer's output."""

    def __init__(self, rng, rows, dims, kinds, acts, alpha=0.1, bias=True):
        self.rows, self.dims, self.kinds, self.acts, self.alpha = rows, dims, kinds, acts, alpha
        self.host, self.keep, self.ys = [], [], []
        n_layers = len(kinds)
        self.layers = (ChainLayer * n_layers)()
        for l, kind in enumerate(kinds):
            k, n = dims[l], dims[l + 1]
            b = rng.normal(0, 0.1, n).astype(np.float32) if bias else None
            y = torch.full((rows, n), 7.0, dtype=torch.float32, device="cuda")
            if kind == "i8":
                kp = (k + 63) // 64 * 64
                q = rng.integers(-127, 128, (n, k), dtype=np.int8)
                sw = rng.uniform(0.001, 0.01, n).astype(np.float32)
                qp = np.zeros((n, kp), np.int8)
                qp[:, :k] = q
                dw, dsw = dev(qp), dev(sw)
                self.host.append(("i8", q, sw, b))
                self.layers[l] = ChainLayer(dw.data_ptr(), dsw.data_ptr(), None if b is None else 0, y.data_ptr(),
                                            k, kp, n, kp, n, acts[l], 1, alpha)
                self.keep += [dw, dsw]
            else:
                w = (rng.normal(0, 1, (n, k)) / np.sqrt(k)).astype(np.float32)
                dw = dev(w)
                self.host.append(("f32", w, None, b))
                self.layers[l] = ChainLayer(dw.data_ptr(), None, None, y.data_ptr(), k, k, n, k, n, acts[l], 0, alpha)
                self.keep.append(dw)
            if b is not None:
                db = dev(b)
                self.layers[l].bias = db.data_ptr()
                self.keep.append(db)
            self.ys.append(y)

    def scratch(self, L):
        nb = L.knx_hip_linear_chain_scratch(self.layers, len(self.kinds), self.rows)
        assert nb >= 256
        s = torch.zeros(nb // 4 + 64, dtype=torch.int32, device="cuda")  # zero: the barrier words start at 0
        return s, nb

    def run(self, L, x, scratch, nb):
        dx = dev(x)
        self.keep.append(dx)
        hipabi.check(L.knx_hip_linear_chain(ptr(dx), x.shape[1], self.rows, self.layers, len(self.kinds), ptr(scratch),
                                            nb, status_word(), hipabi.stream()))

    def outputs(self):
        return [host(y) for y in self.ys]

    def layer_ref(self, l, x):
        kind, w, sw, b = self.host[l]
        if kind == "i8":
            y = knx_ref.qmatmul(x, w.T.copy(), sw, b)
        else:
            y = knx_ref.dense64(x, w.T, b)
        return knx_ref.act(y, self.acts[l], self.alpha)


def check_layers(ch, x, outs):
    """each layer against the oracle on the input the GPU gave it"""
    inp = x
    for l, got in enumerate(outs):
        want = ch.layer_ref(l, inp)
        assert np.array_equal(np.isnan(got), np.isnan(want)), f"layer {l}: NaN pattern"
        ok = ~np.isnan(want)
        if ch.kinds[l] == "i8" and ch.acts[l] in EXACT_ACTS:
            assert np.array_equal(got[ok], want[ok]), f"layer {l}: int8 layer not bit-exact"
        elif ch.kinds[l] == "i8":  # GELU on the hardware exp2 / reciprocal: ≤ 1e-6 of the oracle's libm form
            assert rel_err(got[ok], want[ok]) <= 1e-5, f"layer {l}: int8 layer error {rel_err(got[ok], want[ok])}"
        else:
            assert rel_err(got[ok], want[ok]) <= 1e-4, f"layer {l}: fp32 layer error {rel_err(got[ok], want[ok])}"
        inp = got


MLP = (784, 512, 256, 10)
QUANTUM = 256  # each launch adds this to every barrier word


@pytest.mark.parametrize("rows", [1, 2, 3, 16, 17, 64])
@pytest.mark.parametrize("kind", ["i8", "f32"])
def test_chain_mlp(L, rows, kind):
    """the int8 MLP's shapes (784-512-256-10, ReLU, ReLU, none); int8 also end to end against the oracle chain"""
    rng = np.random.default_rng(rows * 3 + len(kind))
    ch = Chain(rng, rows, MLP, [kind] * 3, [RELU, RELU, NONE])
    x = rng.uniform(0, 1, (rows, MLP[0])).astype(np.float32)
    s, nb = ch.scratch(L)
    ch.run(L, x, s, nb)
    outs = ch.outputs()
    check_layers(ch, x, outs)
    if kind == "i8":
        inp = x
        for l in range(3):
            inp = ch.layer_ref(l, inp)
        assert np.array_equal(outs[-1], inp)
    assert not (host(s[:64]).view(np.uint64) % QUANTUM).any(), "barrier words not at a multiple of the quantum"
    assert chain_status() == 0


CASES = [
    # rows, dims, kinds, acts
    (5, (100, 36, 52, 8, 7), ["f32", "i8", "f32", "i8"], [LEAKY, RELU, GELU, NONE]),
    (9, (64, 128, 64), ["i8", "i8"], [GELU, LEAKY]),
    (33, (20, 400, 8, 12, 4, 1000), ["i8", "f32", "i8", "i8", "f32"], [RELU, NONE, LEAKY, RELU, NONE]),
    (64, (1024, 4, 300), ["f32", "i8"], [NONE, RELU]),
    (2, (2048, 2048, 16), ["i8", "i8"], [RELU, NONE]),
    (4, (12,) * 9, ["i8", "f32"] * 4, [RELU] * 8),
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_chain_shapes(L, case):
    """mixed int8/fp32 layers, k not a multiple of 64, n not a multiple of 16, up to 8 layers, int8 k up to the
    2048 limit"""
    rows, dims, kinds, acts = CASES[case]
    rng = np.random.default_rng(100 + case)
    ch = Chain(rng, rows, dims, kinds, acts, bias=case % 2 == 0)
    x = rng.normal(0, 1, (rows, dims[0])).astype(np.float32)
    s, nb = ch.scratch(L)
    ch.run(L, x, s, nb)
    check_layers(ch, x, ch.outputs())
    assert not (host(s[:64]).view(np.uint64) % QUANTUM).any()


@pytest.mark.parametrize("wg", ["1", "3", "7"])
def test_chain_few_workgroups(L, monkeypatch, wg):
    """a grid smaller than the items of a layer: every workgroup takes several items"""
    monkeypatch.setenv("KNX_CHAIN_WG", wg)
    rng = np.random.default_rng(int(wg))
    ch = Chain(rng, 40, (300, 96, 64, 10), ["i8", "i8", "f32"], [RELU, GELU, NONE])
    x = rng.normal(0, 1, (40, 300)).astype(np.float32)
    s, nb = ch.scratch(L)
    for _ in range(2):
        ch.run(L, x, s, nb)
    check_layers(ch, x, ch.outputs())
    assert not (host(s[:64]).view(np.uint64) % QUANTUM).any()


@pytest.mark.parametrize("target", ["1", "3", "1000"])
@pytest.mark.parametrize("rows", [1, 17, 64])
def test_chain_channel_blocks(L, monkeypatch, target, rows):
    """int8 items of 1, 2, 4 or 8 blocks of 16 channels (the launch sizes the grid for a target item count and then
    gives each layer the fewest blocks that fit it: 1 forces the most blocks, 1000 one block) over channel counts that
    leave partial blocks and partial items, k > 1024 (at most 2 blocks), 512 < k ≤ 1024 and k ≤ 512, a NaN row
    included; bit-exact against the oracle whatever the blocking"""
    monkeypatch.setenv("KNX_CHAIN_ITEMS", target)
    rng = np.random.default_rng(int(target) * 7 + rows)
    dims = (1100, 700, 100, 36, 8)
    ch = Chain(rng, rows, dims, ["i8", "i8", "f32", "i8"], [RELU, LEAKY, NONE, NONE])
    x = rng.normal(0, 1, (rows, dims[0])).astype(np.float32)
    if rows > 1:
        x[rows - 1, 33] = np.nan
    s, nb = ch.scratch(L)
    for _ in range(2):
        ch.run(L, x, s, nb)
    check_layers(ch, x, ch.outputs())
    assert not (host(s[:64]).view(np.uint64) % QUANTUM).any()
    assert chain_status() == 0


def test_chain_full_grid(L, monkeypatch):
    """the largest grid, 64 workgroups (one 16-channel block per item, 512 items in the wide layers, so eight items
    each): every item computed once, bit-exact, and the barrier words advance by one quantum per launch"""
    monkeypatch.setenv("KNX_CHAIN_ITEMS", "100000")
    rng = np.random.default_rng(11)
    dims = (64, 2048, 64, 2048, 8)
    ch = Chain(rng, 64, dims, ["i8", "i8", "i8", "i8"], [RELU, NONE, RELU, NONE])
    x = rng.normal(0, 1, (64, dims[0])).astype(np.float32)
    s, nb = ch.scratch(L)
    before = host(s[:64]).view(np.uint64).copy()
    for _ in range(3):
        ch.run(L, x, s, nb)
    check_layers(ch, x, ch.outputs())
    words = host(s[:64]).view(np.uint64)
    assert (words[:3] - before[:3] == 3 * QUANTUM).all(), words[:4]
    assert chain_status() == 0


def test_chain_special_rows(L):
    """zero rows (scale 1), a row with inf and a row with NaN (int8: the row's outputs are NaN, and through a second
    int8 layer without activation NaN again; a ReLU in between turns NaN into 0, as the reference's threshold)"""
    rng = np.random.default_rng(7)
    rows = 6
    x = rng.normal(0, 1, (rows, 200)).astype(np.float32)
    x[0] = 0.0
    x[2, 17] = np.inf
    x[4, 150] = np.nan
    for acts in ([NONE, NONE, RELU], [RELU, NONE, NONE]):
        ch = Chain(rng, rows, (200, 64, 32, 16), ["i8", "i8", "i8"], acts)
        s, nb = ch.scratch(L)
        ch.run(L, x, s, nb)
        outs = ch.outputs()
        check_layers(ch, x, outs)
        if acts[0] == NONE:
            assert np.isnan(outs[1][2]).all() and np.isnan(outs[1][4]).all()


def test_chain_repeated_and_rejected(L):
    """ten calls in a row on one scratch give the same bits; bad arguments are rejected before any launch"""
    rng = np.random.default_rng(11)
    ch = Chain(rng, 8, MLP, ["i8"] * 3, [RELU, RELU, NONE])
    x = rng.uniform(0, 1, (8, MLP[0])).astype(np.float32)
    s, nb = ch.scratch(L)
    ch.run(L, x, s, nb)
    first = ch.outputs()[-1]
    for _ in range(10):
        ch.run(L, x, s, nb)
    assert np.array_equal(ch.outputs()[-1], first)
    dx = dev(x)
    st = hipabi.stream()
    assert L.knx_hip_linear_chain(ptr(dx), MLP[0], 65, ch.layers, 3, ptr(s), nb, status_word(), st) == -1  # > 64 rows
    assert L.knx_hip_linear_chain(ptr(dx), MLP[0], 8, ch.layers, 3, ptr(s), 255, status_word(), st) == -1  # scratch too small
    assert L.knx_hip_linear_chain(ptr(dx), MLP[0], 8, ch.layers, 0, ptr(s), nb, status_word(), st) == -1
    bad = (ChainLayer * 3)(*ch.layers)
    bad[1].y = bad[0].y  # output over its own input
    assert L.knx_hip_linear_chain(ptr(dx), MLP[0], 8, bad, 3, ptr(s), nb, status_word(), st) == -1
    bad = (ChainLayer * 3)(*ch.layers)
    bad[1].k = 510  # not the previous layer's n
    assert L.knx_hip_linear_chain(ptr(dx), MLP[0], 8, bad, 3, ptr(s), nb, status_word(), st) == -1
    assert L.knx_hip_linear_chain(ptr(dx), MLP[0], 8, ch.layers, 3, ptr(s), nb, None, st) == -1  # no status word
    assert L.knx_hip_linear_chain_scratch(ch.layers, 3, 0) == 0
    assert chain_status() == 0


def test_chain_barrier_gives_up(L, monkeypatch):
    """a barrier that stops waiting sets the caller's status word and every workgroup still ends: KNX_GRID_SPIN=0
    makes every workgroup but the last to arrive stop without polling (forced from the host: all loads and stores
    stay where a normal launch puts them); the barrier words still advance by one quantum per launch, so the next
    launch with the normal wait on the same scratch is bit-exact again and leaves the word at 0"""
    rng = np.random.default_rng(21)
    ch = Chain(rng, 16, MLP, ["i8"] * 3, [RELU, RELU, NONE])
    x = rng.uniform(0, 1, (16, MLP[0])).astype(np.float32)
    s, nb = ch.scratch(L)
    monkeypatch.setenv("KNX_GRID_SPIN", "0")
    for _ in range(3):
        ch.run(L, x, s, nb)
        assert chain_status() == 1, "a barrier of more than one workgroup must stop waiting at a spin limit of 0"
    assert not (host(s[:64]).view(np.uint64) % QUANTUM).any()
    monkeypatch.delenv("KNX_GRID_SPIN")
    ch.run(L, x, s, nb)
    assert chain_status() == 0
    check_layers(ch, x, ch.outputs())
