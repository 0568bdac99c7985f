"""Kernel-level parity of the gfx950 kernels against the CPU oracle, through the C ABI (include/knx_hip.h).

int8: int32 accumulators and ReLU-epilogue outputs bit-exact; fp32 ops: max|a−b| / max(1, max|ref|) ≤ 1e-4
(the fp32 GEMM against the float64 closed form), row ops ≤ 1e-5.
"""
import ctypes

import numpy as np
import pytest

from oracle import knx_ref
from kernix_amd import hipabi
from kernix_amd.hipabi import ptr

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def dev(a):
    """Device copy of a numpy array.  Keep the returned tensor alive while a kernel may use it: a temporary would go
    back to torch's caching allocator and its memory could be handed to the next allocation."""
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


# ---------------------------------------------------------------- int8 GEMM
I8_SHAPES = [(1, 16, 64), (2, 10, 64), (5, 100, 192), (64, 256, 128), (200, 520, 320), (300, 300, 1024),
             (512, 512, 256), (1, 4096, 4096), (16, 4096, 4096), (1024, 1024, 512), (2048, 2048, 256)]


@pytest.mark.parametrize("M,N,K", I8_SHAPES)
def test_i8gemm_bit_exact(L, M, N, K):
    rng = np.random.default_rng(M * 7 + N * 13 + K)
    A = rng.integers(-127, 128, (M, K), dtype=np.int8)
    W = rng.integers(-128, 128, (N, K), dtype=np.int8)
    sa = rng.uniform(0.001, 0.01, M).astype(np.float32)
    sw = rng.uniform(0.001, 0.01, N).astype(np.float32)
    bias = rng.normal(0, 0.1, N).astype(np.float32)
    want_y, want_acc = knx_ref.i8gemm(A, W, sa, sw, bias, act_id=0)
    dA, dW, dsa, dsw, db = dev(A), dev(W), dev(sa), dev(sw), dev(bias)
    Y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    acc = torch.empty((M, N), dtype=torch.int32, device="cuda")
    hipabi.check(L.knx_hip_i8gemm(M, N, K, ptr(dA), K, ptr(dsa), ptr(dW), K, ptr(dsw), ptr(db), 0, 0.0, 0,
                                  ptr(Y), N, ptr(acc), N, hipabi.stream()))
    assert np.array_equal(host(acc), want_acc)
    assert np.array_equal(host(Y), want_y)


@pytest.mark.parametrize("M", [1, 16, 256, 4096])
def test_i8gemm_standalone_config(L, M):
    """The standalone int8 GEMM workload, K = N = 4096 at every benchmarked M, through the default dispatch (the
    skinny kernel at M <= 16, the 64x64 ring at M = 256, the three-stage 256x256 kernel at M = 4096): the config's
    inputs (A, W uniform int8 in [-127, 127], scales U[0.001, 0.01], bias N(0, 0.1), seed 12345), ReLU epilogue;
    int32 accumulators and outputs bit-exact against the oracle (reference include/kernix_model.h:143-178)."""
    from kernix_amd import configs

    A, W, sa, sw, bias = configs.i8gemm_inputs(M)
    N, K = W.shape
    want_y, want_acc = knx_ref.i8gemm(A, W, sa, sw, bias, act_id=0, threads=16)
    dA, dW, dsa, dsw, db = dev(A), dev(W), dev(sa), dev(sw), dev(bias)
    Y = torch.full((M, N), 7.0, dtype=torch.float32, device="cuda")
    acc = torch.zeros((M, N), dtype=torch.int32, device="cuda")
    # accumulators and outputs together, then the output-only path the benchmark times
    hipabi.check(L.knx_hip_i8gemm(M, N, K, ptr(dA), K, ptr(dsa), ptr(dW), K, ptr(dsw), ptr(db), 0, 0.0, 0,
                                  ptr(Y), N, ptr(acc), N, hipabi.stream()))
    assert np.array_equal(host(acc), want_acc)
    assert np.array_equal(host(Y), want_y)
    Y.fill_(7.0)
    hipabi.check(L.knx_hip_i8gemm(M, N, K, ptr(dA), K, ptr(dsa), ptr(dW), K, ptr(dsw), ptr(db), 0, 0.0, 0,
                                  ptr(Y), N, None, 0, hipabi.stream()))
    assert np.array_equal(host(Y), want_y)


# every kernel instantiation a shape can select, each forced onto every edge shape (a library built with KNX_TUNING=1
# also has the tuning-only variants: pp, k128, k128w8, k128w8ta3, k128w16, k128r, k128c, ring64s8k2, ring64s8,
# pipe256, pipe256w8, pipe256s3, pipe128, tile256, which this list can name there)
I8_VARIANTS = ["default", "k128w8t", "k128m", "k128ma3", "k128m8a3e", "k128w8ta3e", "ring64s4", "ring64g2", "pipe64", "tile64",
               "k128ms4", "k128ma3s4", "k128m8s4", "k128ms2", "k128ms8"]
# tiles moved back at the M/N edges, half k-tiles (K % 128 == 64), N % 4 != 0, one whole 256x256 tile, 2..4 k-tiles
# (every branch of the three-stage A ring's prologue and tail), an 8 x 8 tile grid split into XCD blocks, and for the
# K split between two rings: 6 k-tiles per ring, ragged tiles with 8 per ring, 13 k-tiles (no split)
I8_EDGE_SHAPES = [(300, 300, 1024), (520, 700, 320), (257, 259, 192), (256, 256, 64), (640, 384, 4096),
                  (512, 256, 256), (256, 512, 384), (384, 384, 448), (2048, 2048, 512), (192, 320, 1536),
                  (200, 260, 2048), (130, 200, 1664)]


@pytest.mark.parametrize("variant", I8_VARIANTS)
@pytest.mark.parametrize("M,N,K", I8_EDGE_SHAPES)
def test_i8gemm_variants_y_only(L, monkeypatch, variant, M, N, K):
    """every kernel variant on the output-only path (relu, no bias; none with accumulate) against the oracle"""
    monkeypatch.setenv("KNX_I8_KERNEL", variant)
    rng = np.random.default_rng(M + 3 * N + 5 * K)
    A = rng.integers(-127, 128, (M, K), dtype=np.int8)
    W = rng.integers(-128, 128, (N, K), dtype=np.int8)
    sa = rng.uniform(0.001, 0.01, M).astype(np.float32)
    sw = rng.uniform(0.001, 0.01, N).astype(np.float32)
    bias = rng.normal(0, 0.1, N).astype(np.float32)
    want_y, acc = knx_ref.i8gemm(A, W, sa, sw, bias, act_id=0)
    dA, dW, dsa, dsw, db = dev(A), dev(W), dev(sa), dev(sw), dev(bias)
    Y = torch.full((M, N), 7.0, dtype=torch.float32, device="cuda")
    hipabi.check(L.knx_hip_i8gemm(M, N, K, ptr(dA), K, ptr(dsa), ptr(dW), K, ptr(dsw), ptr(db), 0, 0.0, 0,
                                  ptr(Y), N, None, 0, hipabi.stream()))
    assert np.array_equal(host(Y), want_y)
    # no bias, no activation, accumulate into Y: every output must be added exactly once
    y0 = rng.normal(0, 1, (M, N)).astype(np.float32)
    plain = ((acc.astype(np.float32) * sa[:, None]).astype(np.float32) * sw[None, :]).astype(np.float32)
    Y2 = dev(y0)
    hipabi.check(L.knx_hip_i8gemm(M, N, K, ptr(dA), K, ptr(dsa), ptr(dW), K, ptr(dsw), None, -1, 0.0, 1,
                                  ptr(Y2), N, None, 0, hipabi.stream()))
    assert np.array_equal(host(Y2), (y0 + plain).astype(np.float32))


def test_i8gemm_ksplit_sequence(L, monkeypatch):
    """The K split across workgroups (exact int32 partial tiles, the last workgroup of a tile adds them): the
    standalone M = 256 workload (K = N = 4096, the config's inputs) bit-exact in accumulators and outputs for every
    split count, called in turn on one stream so that launches of 2, 4 and 8 splits share the arrival counters (each
    launch leaves them at the next multiple of the counter quantum), then a larger shape that grows the scratch, then
    the first again (reference include/kernix_model.h:143-178)"""
    from kernix_amd import configs

    A, W, sa, sw, bias = configs.i8gemm_inputs(256)
    M, K = A.shape
    N = W.shape[0]
    want_y, want_acc = knx_ref.i8gemm(A, W, sa, sw, bias, act_id=0, threads=16)
    dA, dW, dsa, dsw, db = dev(A), dev(W), dev(sa), dev(sw), dev(bias)
    rng = np.random.default_rng(3)
    A2 = rng.integers(-127, 128, (640, 2048), dtype=np.int8)
    W2 = rng.integers(-128, 128, (1000, 2048), dtype=np.int8)
    s2 = rng.uniform(0.001, 0.01, 640).astype(np.float32)
    w2 = rng.uniform(0.001, 0.01, 1000).astype(np.float32)
    b2 = rng.normal(0, 0.1, 1000).astype(np.float32)
    want2, acc2 = knx_ref.i8gemm(A2, W2, s2, w2, b2, act_id=0)
    d2 = [dev(a) for a in (A2, W2, s2, w2, b2)]
    for variant in ("k128ms2", "k128ms4", "k128ms8", "k128ms4", "k128m8s4", "big", "k128ms4", "k128ma3s4"):
        if variant == "big":
            monkeypatch.setenv("KNX_I8_KERNEL", "k128ms4")
            Y2 = torch.full((640, 1000), 7.0, dtype=torch.float32, device="cuda")
            C2 = torch.zeros((640, 1000), dtype=torch.int32, device="cuda")
            hipabi.check(L.knx_hip_i8gemm(640, 1000, 2048, ptr(d2[0]), 2048, ptr(d2[2]), ptr(d2[1]), 2048, ptr(d2[3]),
                                          ptr(d2[4]), 0, 0.0, 0, ptr(Y2), 1000, ptr(C2), 1000, hipabi.stream()))
            assert np.array_equal(host(C2), acc2) and np.array_equal(host(Y2), want2), variant
            continue
        monkeypatch.setenv("KNX_I8_KERNEL", variant)
        Y = torch.full((M, N), 7.0, dtype=torch.float32, device="cuda")
        acc = torch.zeros((M, N), dtype=torch.int32, device="cuda")
        hipabi.check(L.knx_hip_i8gemm(M, N, K, ptr(dA), K, ptr(dsa), ptr(dW), K, ptr(dsw), ptr(db), 0, 0.0, 0,
                                      ptr(Y), N, ptr(acc), N, hipabi.stream()))
        assert np.array_equal(host(acc), want_acc), variant
        assert np.array_equal(host(Y), want_y), variant


I8_SKINNY_VARIANTS = ["default", "skinny"]
# every row-block count (1, 2, 4 blocks of 16), a lone half k-tile (K = 64), trailing half k-tiles (K % 128 == 64)
I8_SKINNY_SHAPES = [(1, 16, 64), (3, 100, 192), (16, 4096, 4096), (17, 300, 320), (33, 64, 448), (64, 520, 1024),
                    (1, 4096, 4096)]


@pytest.mark.parametrize("variant", I8_SKINNY_VARIANTS)
@pytest.mark.parametrize("M,N,K", I8_SKINNY_SHAPES)
def test_i8gemm_skinny_variants(L, monkeypatch, variant, M, N, K):
    """the M <= 64 kernels: int32 accumulators and the ReLU epilogue bit-exact against the oracle"""
    monkeypatch.setenv("KNX_I8_KERNEL", variant)
    rng = np.random.default_rng(11 * M + N + 7 * K)
    A = rng.integers(-127, 128, (M, K), dtype=np.int8)
    W = rng.integers(-128, 128, (N, K), dtype=np.int8)
    sa = rng.uniform(0.001, 0.01, M).astype(np.float32)
    sw = rng.uniform(0.001, 0.01, N).astype(np.float32)
    bias = rng.normal(0, 0.1, N).astype(np.float32)
    want_y, want_acc = knx_ref.i8gemm(A, W, sa, sw, bias, act_id=0)
    dA, dW, dsa, dsw, db = dev(A), dev(W), dev(sa), dev(sw), dev(bias)
    Y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    acc = torch.empty((M, N), dtype=torch.int32, device="cuda")
    hipabi.check(L.knx_hip_i8gemm(M, N, K, ptr(dA), K, ptr(dsa), ptr(dW), K, ptr(dsw), ptr(db), 0, 0.0, 0,
                                  ptr(Y), N, ptr(acc), N, hipabi.stream()))
    assert np.array_equal(host(acc), want_acc)
    assert np.array_equal(host(Y), want_y)


@pytest.mark.parametrize("variant", ["default", "k128w8t", "k128w8ta3e", "k128m", "k128m8a3e", "ring64s4", "ring64g2", "pipe64", "tile64",
                                     "skinny", "k128ms4", "k128m8s4"])
@pytest.mark.parametrize("M,N,K,inplace", [(300, 300, 1024, False), (520, 700, 320, True), (2048, 2048, 2048, False),
                                           (48, 520, 192, True)])
def test_i8gemm_residual(L, monkeypatch, variant, M, N, K, inplace):
    """Y = relu(epilogue) + R (the LINEAR + BINARY add fusion), bit-exact: the float32 add of R to the oracle's output;
    R may be Y itself"""
    monkeypatch.setenv("KNX_I8_KERNEL", variant)
    rng = np.random.default_rng(M + 17 * N + K)
    A = rng.integers(-127, 128, (M, K), dtype=np.int8)
    W = rng.integers(-128, 128, (N, K), dtype=np.int8)
    sa = rng.uniform(0.001, 0.01, M).astype(np.float32)
    sw = rng.uniform(0.001, 0.01, N).astype(np.float32)
    bias = rng.normal(0, 0.1, N).astype(np.float32)
    R = rng.normal(0, 1, (M, N)).astype(np.float32)
    want_y, _ = knx_ref.i8gemm(A, W, sa, sw, bias, act_id=0)
    want = (want_y + R).astype(np.float32)
    dA, dW, dsa, dsw, db, dR = dev(A), dev(W), dev(sa), dev(sw), dev(bias), dev(R)
    Y = dR if inplace else torch.full((M, N), 7.0, dtype=torch.float32, device="cuda")
    hipabi.check(L.knx_hip_i8gemm_res(M, N, K, ptr(dA), K, ptr(dsa), ptr(dW), K, ptr(dsw), ptr(db), 0, 0.0, ptr(dR), N,
                                      ptr(Y), N, hipabi.stream()))
    assert np.array_equal(host(Y), want)


@pytest.mark.parametrize("rows", [1, 2, 3, 4, 5, 9, 16, 17, 33, 64, 65])
@pytest.mark.parametrize("k,n", [(784, 512), (4096, 4096), (64, 10), (200, 33)])
@pytest.mark.parametrize("path", ["fused", "split"])
def test_qlinear(L, monkeypatch, rows, k, n, path):
    """knx_hip_qlinear (kernix_qmatmul + act) against the oracle's kernix_qmatmul, bit-exact: one-kernel quantize-on-
    the-fly path at ≤ 16 rows for the small weights, quantizer + GEMM above and when forced; a zero row and (from 3
    rows) a row with inf"""
    if path == "split":
        monkeypatch.setenv("KNX_QLINEAR", "split")
    rng = np.random.default_rng(rows * 131 + k + n)
    kp = (k + 63) // 64 * 64
    x = rng.normal(0, 1, (rows, k)).astype(np.float32)
    x[0, :] = 0.0
    if rows >= 3:
        x[2, k // 2] = np.inf
    q = rng.integers(-127, 128, (n, k), dtype=np.int8)
    scale = rng.uniform(0.001, 0.01, n).astype(np.float32)
    bias = rng.normal(0, 0.1, n).astype(np.float32)
    want = knx_ref.qmatmul(x, q.T.copy(), scale, bias)  # no activation: the inf row must come out all NaN
    qp = np.zeros((n, kp), np.int8)
    qp[:, :k] = q
    dx, dq, ds, db = dev(x), dev(qp), dev(scale), dev(bias)
    xq = torch.empty((rows, kp), dtype=torch.int8, device="cuda")
    sx = torch.empty(rows, dtype=torch.float32, device="cuda")
    Y = torch.full((rows, n), 7.0, dtype=torch.float32, device="cuda")
    hipabi.check(L.knx_hip_qlinear(ptr(dx), k, rows, k, kp, ptr(xq), ptr(sx), ptr(dq), kp, n, ptr(ds), ptr(db), -1,
                                   0.0, 0, None, 0, ptr(Y), n, hipabi.stream()))
    got = host(Y)
    if rows >= 3:
        assert np.isnan(got[2]).all()
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(got[~np.isnan(got)], want[~np.isnan(want)])


@pytest.mark.parametrize("act", [1, 5])
@pytest.mark.parametrize("M,N,K", [(2048, 2048, 512), (1024, 1024, 2048), (520, 700, 320)])
def test_i8gemm_activation_epilogues(L, act, M, N, K):
    """GELU (its own compile-time epilogue) and leaky ReLU (the general one) on the tile kernels: the plain call is
    bit-identical to the general epilogue (forced by asking for the raw int32 accumulators too) and within the GELU
    formula's hardware-exp2/reciprocal error of the oracle"""
    rng = np.random.default_rng(M + N + K + act)
    A = rng.integers(-127, 128, (M, K), dtype=np.int8)
    W = rng.integers(-128, 128, (N, K), dtype=np.int8)
    sa = rng.uniform(0.001, 0.01, M).astype(np.float32)
    sw = rng.uniform(0.001, 0.01, N).astype(np.float32)
    bias = rng.normal(0, 0.1, N).astype(np.float32)
    want_y, want_acc = knx_ref.i8gemm(A, W, sa, sw, bias, act_id=act, alpha=0.1)
    dA, dW, dsa, dsw, db = dev(A), dev(W), dev(sa), dev(sw), dev(bias)
    Y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    Y2 = torch.empty((M, N), dtype=torch.float32, device="cuda")
    acc = torch.empty((M, N), dtype=torch.int32, device="cuda")
    hipabi.check(L.knx_hip_i8gemm(M, N, K, ptr(dA), K, ptr(dsa), ptr(dW), K, ptr(dsw), ptr(db), act, 0.1, 0,
                                  ptr(Y), N, None, 0, hipabi.stream()))
    hipabi.check(L.knx_hip_i8gemm(M, N, K, ptr(dA), K, ptr(dsa), ptr(dW), K, ptr(dsw), ptr(db), act, 0.1, 0,
                                  ptr(Y2), N, ptr(acc), N, hipabi.stream()))
    assert np.array_equal(host(acc), want_acc)
    assert np.array_equal(host(Y), host(Y2))
    assert rel_err(host(Y), want_y) <= 1e-6


def test_i8gemm_accumulate_and_no_bias(L):
    rng = np.random.default_rng(3)
    M, N, K = 37, 70, 128
    A = rng.integers(-127, 128, (M, K), dtype=np.int8)
    W = rng.integers(-127, 128, (N, K), dtype=np.int8)
    sa = rng.uniform(0.001, 0.01, M).astype(np.float32)
    sw = rng.uniform(0.001, 0.01, N).astype(np.float32)
    y0 = rng.normal(0, 1, (M, N)).astype(np.float32)
    _, acc = knx_ref.i8gemm(A, W, sa, sw, None, act_id=-1)
    want = ((acc.astype(np.float32) * sa[:, None]).astype(np.float32) * sw[None, :]).astype(np.float32)
    want = (y0 + want).astype(np.float32)
    Y, dA, dsa, dW, dsw = dev(y0), dev(A), dev(sa), dev(W), dev(sw)
    hipabi.check(L.knx_hip_i8gemm(M, N, K, ptr(dA), K, ptr(dsa), ptr(dW), K, ptr(dsw), None, -1, 0.0, 1,
                                  ptr(Y), N, None, 0, hipabi.stream()))
    assert np.array_equal(host(Y), want)


def test_i8gemm_rejects_bad_shapes(L):
    assert L.knx_hip_i8gemm(4, 4, 60, None, 60, None, None, 60, None, None, 0, 0.0, 0, None, 4, None, 0, None) != 0


# ---------------------------------------------------------------- quantize rows
@pytest.mark.parametrize("rows,k", [(1, 1), (3, 55), (32, 114), (4, 784), (2, 4096), (3, 512), (5, 2048), (4, 4100)])
def test_quantize_rows_bit_exact(L, rows, k):
    rng = np.random.default_rng(rows * 31 + k)
    x = (rng.integers(0, 2001, (rows, k)) * 0.003 - 3.0).astype(np.float32)
    if rows >= 3:
        x[1, k // 2] = np.nan
        x[2, :] = 0.0
    if rows >= 4:
        x[3, k - 1] = -np.inf
    kp = (k + 63) // 64 * 64
    xq_want, sx_want, bad = knx_ref.quantize_rows(x)
    dx = dev(x)
    xq = torch.full((rows, kp), 99, dtype=torch.int8, device="cuda")
    sx = torch.empty(rows, dtype=torch.float32, device="cuda")
    hipabi.check(L.knx_hip_quantize_rows(ptr(dx), k, rows, k, kp, ptr(xq), kp, ptr(sx), hipabi.stream()))
    got_q, got_s = host(xq), host(sx)
    for r in range(rows):
        if bad[r]:
            assert np.isnan(got_s[r])
            continue
        assert got_s[r] == sx_want[r]
        assert np.array_equal(got_q[r, :k], xq_want[r])
        assert not got_q[r, k:].any()


@pytest.mark.parametrize("rows,cols", [(5, 64), (37, 128), (64, 512), (9, 1000), (16, 2048)])
def test_layernorm_quantize_bit_exact(L, rows, cols):
    """layer_norm + quantize in one pass against knx_hip_layernorm then knx_hip_quantize_rows, bit for bit (int8 rows
    with their zero padding to kp, scales, rows that normalize to NaN), at each lanes-per-row width of the row
    kernels"""
    rng = np.random.default_rng(rows * 7 + cols)
    x = rng.normal(0, 2, (rows, cols)).astype(np.float32)
    x[1, 3] = np.inf  # a row that normalizes to NaN
    gamma = rng.normal(1, 0.2, cols).astype(np.float32)
    beta = rng.normal(0, 0.2, cols).astype(np.float32)
    kp = (cols + 63) // 64 * 64 + 64
    dx, dg, db = dev(x), dev(gamma), dev(beta)
    y = torch.empty((rows, cols), dtype=torch.float32, device="cuda")
    q1 = torch.full((rows, kp), 99, dtype=torch.int8, device="cuda")
    s1 = torch.empty(rows, dtype=torch.float32, device="cuda")
    q2 = torch.full((rows, kp), 77, dtype=torch.int8, device="cuda")
    s2 = torch.empty(rows, dtype=torch.float32, device="cuda")
    hipabi.check(L.knx_hip_layernorm(ptr(dx), ptr(y), rows, cols, ptr(dg), ptr(db), 1e-5, hipabi.stream()))
    hipabi.check(L.knx_hip_quantize_rows(ptr(y), cols, rows, cols, kp, ptr(q1), kp, ptr(s1), hipabi.stream()))
    hipabi.check(L.knx_hip_layernorm_quantize(ptr(dx), rows, cols, ptr(dg), ptr(db), 1e-5, kp, ptr(q2), ptr(s2),
                                              hipabi.stream()))
    assert np.array_equal(host(q1), host(q2))
    a, b = host(s1), host(s2)
    assert np.isnan(a[1]) and np.isnan(b[1])
    assert np.array_equal(a[~np.isnan(a)], b[~np.isnan(b)])


# ---------------------------------------------------------------- fp32 GEMM
SG_SHAPES = [(1, 1, 1), (3, 10, 7), (64, 512, 784), (37, 96, 128), (130, 1000, 256), (512, 512, 512),
             (2048, 1024, 128), (8, 3, 0)]


@pytest.mark.parametrize("M,N,K", SG_SHAPES)
@pytest.mark.parametrize("act", [-1, 0, 1])
def test_sgemm_ep(L, M, N, K, act):
    rng = np.random.default_rng(M + 3 * N + 7 * K)
    A = rng.standard_normal((M, max(K, 1))).astype(np.float32)[:, :K].copy()
    W = (rng.standard_normal((max(K, 1), N)) / np.sqrt(max(K, 1))).astype(np.float32)[:K].copy()
    b = rng.normal(0, 0.1, N).astype(np.float32)
    want = knx_ref.act(knx_ref.dense64(A, W, b), act)
    C = torch.empty((M, N), dtype=torch.float32, device="cuda")
    dA = dev(A) if K else None
    dW = dev(W) if K else None
    db = dev(b)
    hipabi.check(L.knx_hip_sgemm_ep(M, N, K, ptr(dA), K, ptr(dW), N, ptr(db), act, 0.0, ptr(C), N, hipabi.stream()))
    assert rel_err(host(C), want) <= 1e-4


# the weight-transposed entry point: pipelined kernel (K % 32 == 0, tiles inside M and N, moved back at the edges)
# and the general kernel otherwise; 8100×1500×128 has enough 128×128 tiles for the 8-wave tile by default
SGNT_SHAPES = [(256, 256, 64), (300, 200, 96), (1024, 1000, 512), (4096, 1024, 256), (128, 128, 32), (100, 77, 50),
               (512, 512, 30), (2048, 640, 2048), (8100, 1500, 128), (2048, 512, 128)]
# small GEMMs (split-K 16×16 kernel by default): the int8 MLP's layers at batch 64, ragged M/N, K % 16 ≠ 0
SGNT_SMALL = [(64, 512, 784), (64, 256, 512), (64, 10, 256), (1, 1, 16), (5, 33, 100), (17, 70, 20), (256, 10, 256),
              (3, 4000, 4096), (2, 48, 4100)]


@pytest.mark.parametrize("M,N,K", SGNT_SHAPES)
@pytest.mark.parametrize("act", [-1, 0, 1])
def test_sgemm_nt_ep(L, M, N, K, act):
    _sgemm_nt_case(L, M, N, K, act)


@pytest.mark.parametrize("M,N,K", SGNT_SMALL)
@pytest.mark.parametrize("kernel", ["", "skinny", "general"])
def test_sgemm_nt_small(L, M, N, K, kernel, monkeypatch):
    monkeypatch.setenv("KNX_SGEMM_KERNEL", kernel)
    _sgemm_nt_case(L, M, N, K, 0)


# the pipelined tiles a shape can select (KNX_TUNING=1 builds also have t128s3, t64s3, t64w2, t256x128, t256x192,
# t128x256)
SGNT_VARIANTS = ["t256", "t128", "t128w8", "t64", "t64x64"]


@pytest.mark.parametrize("kernel", SGNT_VARIANTS)
@pytest.mark.parametrize("M,N,K", [(1024, 768, 512), (520, 700, 96), (256, 384, 64)])
def test_sgemm_nt_variants(L, M, N, K, kernel, monkeypatch):
    """every forced tile of the pipelined fp32 kernel, with tiles moved back at ragged M/N edges"""
    monkeypatch.setenv("KNX_SGEMM_KERNEL", kernel)
    _sgemm_nt_case(L, M, N, K, 1)


@pytest.mark.parametrize("kernel", ["", "t128", "t128w8", "t64", "t64x64", "t256", "skinny", "general"])
@pytest.mark.parametrize("M,N,K,inplace", [(1024, 768, 512, False), (520, 700, 96, True), (64, 256, 512, True),
                                           (100, 77, 50, False)])
def test_sgemm_nt_residual(L, M, N, K, inplace, kernel, monkeypatch):
    """C = act(A·Wtᵀ + b) + R on every fp32 kernel (the LINEAR + BINARY add fusion); R may be C itself"""
    monkeypatch.setenv("KNX_SGEMM_KERNEL", kernel)
    rng = np.random.default_rng(M + 7 * N + 3 * K)
    A = rng.standard_normal((M, K)).astype(np.float32)
    W = (rng.standard_normal((K, N)) / np.sqrt(K)).astype(np.float32)
    b = rng.normal(0, 0.1, N).astype(np.float32)
    R = rng.standard_normal((M, N)).astype(np.float32)
    want = knx_ref.act(knx_ref.dense64(A, W, b), 1).astype(np.float32) + R
    dA, dWt, db, dR = dev(A), dev(np.ascontiguousarray(W.T)), dev(b), dev(R)
    C = dR if inplace else torch.full((M, N), 7.0, dtype=torch.float32, device="cuda")
    hipabi.check(L.knx_hip_sgemm_nt_ep_res(M, N, K, ptr(dA), K, ptr(dWt), K, ptr(db), 1, 0.0, ptr(dR), N, ptr(C), N,
                                           hipabi.stream()))
    assert rel_err(host(C), want) <= 1e-4


def _sgemm_nt_case(L, M, N, K, act):
    rng = np.random.default_rng(M + 5 * N + 11 * K)
    A = rng.standard_normal((M, K)).astype(np.float32)
    W = (rng.standard_normal((K, N)) / np.sqrt(K)).astype(np.float32)
    b = rng.normal(0, 0.1, N).astype(np.float32)
    want = knx_ref.act(knx_ref.dense64(A, W, b), act)
    C = torch.full((M, N), 7.0, dtype=torch.float32, device="cuda")
    dA, dWt, db = dev(A), dev(np.ascontiguousarray(W.T)), dev(b)
    hipabi.check(L.knx_hip_sgemm_nt_ep(M, N, K, ptr(dA), K, ptr(dWt), K, ptr(db), act, 0.0, ptr(C), N, hipabi.stream()))
    assert rel_err(host(C), want) <= 1e-4


# ---------------------------------------------------------------- rows / elementwise
# scalar kernels (cols % 4 != 0 or > 2048) and every register-resident shape (16/32/64 lanes per row, 1–8 float4)
@pytest.mark.parametrize("rows,cols", [(1, 1), (7, 10), (64, 512), (300, 2048), (5, 9000), (9, 12), (17, 60),
                                       (33, 128), (20, 256), (3, 1024), (6, 1000)])
def test_layernorm_softmax(L, rows, cols):
    rng = np.random.default_rng(rows + cols)
    x = rng.standard_normal((rows, cols)).astype(np.float32) * 3
    if cols >= 4:
        x[0, cols // 2:] = -np.inf if rows > 1 else x[0, cols // 2:]  # masked positions of a causal row
    g = (1 + rng.normal(0, 0.5, cols)).astype(np.float32)
    bt = rng.normal(0, 0.5, cols).astype(np.float32)
    dx, dg, dbt = dev(x), dev(g), dev(bt)
    y = torch.empty_like(dx)
    fin = np.isfinite(x).all(axis=1)  # layer_norm over finite rows only
    hipabi.check(L.knx_hip_layernorm(ptr(dx), ptr(y), rows, cols, ptr(dg), ptr(dbt), 1e-5, hipabi.stream()))
    assert rel_err(host(y)[fin], knx_ref.layernorm(x[fin], g, bt, 1e-5)) <= 1e-5
    xf = torch.from_numpy(np.ascontiguousarray(x[fin])).cuda()
    hipabi.check(L.knx_hip_layernorm(ptr(xf), ptr(xf), int(fin.sum()), cols, None, None, 1e-5, hipabi.stream()))
    assert rel_err(host(xf), knx_ref.layernorm(x[fin], None, None, 1e-5)) <= 1e-5  # in place, no affine
    hipabi.check(L.knx_hip_softmax(ptr(dx), ptr(dx), rows, cols, hipabi.stream()))  # in place
    assert rel_err(host(dx), knx_ref.softmax(x)) <= 1e-5


@pytest.mark.parametrize("act", list(range(-1, 16)))
@pytest.mark.parametrize("cols", [70, 72])  # scalar kernel, 4-wide kernel
def test_bias_act_all_activations(L, act, cols):
    rng = np.random.default_rng(act + 100 * cols)
    x = (rng.standard_normal((33, cols)) * 4).astype(np.float32)
    b = rng.normal(0, 1, cols).astype(np.float32)
    xb = (x + b).astype(np.float32)
    want = xb if act == -1 else knx_ref.act(xb, act, 0.2)
    dx, db = dev(x), dev(b)
    hipabi.check(L.knx_hip_bias_act(ptr(dx), ptr(dx), 33, cols, ptr(db), act, 0.2, hipabi.stream()))
    got = host(dx)
    assert np.allclose(got, want, rtol=2e-6, atol=2e-6, equal_nan=True)


def test_binary_broadcast_and_pool(L):
    rng = np.random.default_rng(5)
    B, R, C = 3, 6, 8
    for op in range(6):
        for (ra, ca, rb, cb) in [(R, C, R, C), (R, C, 1, C), (R, C, R, 1), (1, C, R, C)]:
            a = rng.normal(0, 1, (B * ra, ca)).astype(np.float32)
            b = rng.normal(0, 1, (B * rb, cb)).astype(np.float32) + 2.5
            want = np.zeros((B * R, C), np.float32)
            knx_ref.lib().ko_binary(op, knx_ref._p(a), ra, ca, knx_ref._p(b), rb, cb, knx_ref._p(want), B, R, C)
            y = torch.empty((B * R, C), dtype=torch.float32, device="cuda")
            da, db = dev(a), dev(b)
            hipabi.check(L.knx_hip_binary(op, ptr(da), ra, ca, ptr(db), rb, cb, ptr(y), B, R, C, hipabi.stream()))
            assert np.array_equal(host(y), want)
    # whole groups of 32 and of eight rows, remainders, a single row; channel counts a multiple of 64 and not
    for R, C in ((64, 256), (13, 256), (1, 256), (130, 128), (64, 72), (13, 72)):
        x = rng.normal(0, 1, (4 * R, C)).astype(np.float32)
        for t in (0, 1):
            want = np.zeros((4, C), np.float32)
            knx_ref.lib().ko_global_pool(t, knx_ref._p(x), 4, R, C, knx_ref._p(want))
            y = torch.empty((4, C), dtype=torch.float32, device="cuda")
            dx = dev(x)
            hipabi.check(L.knx_hip_global_pool(t, ptr(dx), 4, R, C, ptr(y), hipabi.stream()))
            assert np.array_equal(host(y), want), (R, C, t)


# ---------------------------------------------------------------- convolution
CONV_CASES = [
    # B, H, W, C, Co, k, stride, pad, groups, dil
    (2, 8, 8, 3, 64, 3, 1, 1, 1, 1),
    (2, 8, 8, 64, 64, 3, 1, 1, 1, 1),
    (2, 16, 16, 64, 128, 3, 2, 1, 1, 1),
    (1, 9, 7, 6, 6, 3, 1, 1, 6, 1),
    (1, 9, 7, 6, 6, 3, 1, 1, 2, 2),
    (3, 5, 5, 8, 12, 1, 1, 0, 1, 1),
    (2, 11, 13, 5, 7, 2, 3, 0, 1, 1),
    # enough output pixels for the 256 × 64 tile (≥ 512 tiles of 128 on 256 CUs), channel-vector and scalar gathers
    (64, 32, 32, 64, 64, 3, 1, 1, 1, 1),
    (65, 32, 32, 3, 64, 3, 1, 1, 1, 1),
    # few taps: stride 2 with dilation 2 and ragged edges, 1×1 taps
    (4, 17, 15, 3, 32, 3, 2, 1, 1, 2),
    (3, 9, 9, 16, 8, 1, 1, 0, 1, 1),
    # shapes for the pipelined implicit GEMM (channels per group % 32 == 0, enough tiles): 256×64 tiles with groups,
    # dilation 2, 128×128 tiles, stride 2
    (128, 16, 16, 128, 128, 3, 1, 1, 2, 1),
    (64, 32, 32, 64, 64, 3, 1, 2, 1, 2),
    (128, 16, 16, 64, 128, 3, 1, 1, 1, 1),
    (256, 16, 16, 128, 256, 3, 2, 1, 1, 1),
    # the register-operand MFMA kernel (one group, K ≤ 32, Co ∈ {32, 64, 96, 128}): K = 25, 18 (even), 16 and 32
    # (1×1 over 32 channels), Co = 32, 96, 128, stride 3 with dilation 3; pixel counts not a multiple of 32
    (3, 7, 5, 1, 32, 5, 1, 2, 1, 1),
    (2, 9, 11, 2, 96, 3, 2, 1, 1, 1),
    (2, 6, 6, 4, 128, 2, 1, 0, 1, 1),
    (3, 5, 5, 32, 32, 1, 1, 0, 1, 1),
    (2, 10, 10, 3, 64, 3, 3, 2, 1, 3),
]
SMALL_CONV_CASES = [c for c in CONV_CASES if c[8] == 1 and c[5] * c[5] * c[3] <= 32 and c[4] in (32, 64, 96, 128)]


@pytest.mark.parametrize("case", [(64, 32, 32, 64, 64, 3, 1, 1, 1, 1), (2, 8, 8, 3, 64, 3, 1, 1, 1, 1),
                                  (128, 16, 16, 128, 128, 3, 1, 1, 2, 1), (2, 11, 13, 5, 7, 2, 3, 0, 1, 1),
                                  (2, 9, 11, 2, 96, 3, 2, 1, 1, 1), (3, 7, 5, 1, 32, 5, 1, 2, 1, 1),
                                  (2, 6, 6, 4, 128, 2, 1, 0, 1, 1)])
def test_conv_residual(L, case):
    """y = relu(conv(x) + b) + R on the pipelined and the general kernel (the CONV + BINARY add fusion)"""
    B, H, W, C, Co, k, s, p, g, dil = case
    rng = np.random.default_rng(sum(case) + 1)
    Ho = (H + 2 * p - dil * (k - 1) - 1) // s + 1
    Wo = (W + 2 * p - dil * (k - 1) - 1) // s + 1
    x = rng.standard_normal((B * H * W, C)).astype(np.float32)
    w = (rng.standard_normal((k * k * (C // g), Co)) / np.sqrt(k * k * C / g)).astype(np.float32)
    b = rng.normal(0, 0.1, Co).astype(np.float32)
    R = rng.standard_normal((B * Ho * Wo, Co)).astype(np.float32)
    op = dict(cin=C, cout=Co, k=(k, k), s=(s, s), d=(dil, dil), p=(p, p, p, p), g=g, w=w, b=b)
    want, _ = knx_ref._conv(x, B, H, W, op, act_id=0)
    want = want.astype(np.float32) + R
    geom = hipabi.ConvGeom(B, H, W, C, Ho, Wo, Co, k, k, s, s, dil, dil, p, p, g)
    y = torch.empty((B * Ho * Wo, Co), dtype=torch.float32, device="cuda")
    dx, dwt, db, dR = dev(x), dev(np.ascontiguousarray(w.T)), dev(b), dev(R)
    hipabi.check(L.knx_hip_conv_t_res(ctypes.byref(geom), ptr(dx), ptr(dwt), ptr(db), 0, 0.0, ptr(dR), ptr(y),
                                      hipabi.stream()))
    assert rel_err(host(y), want) <= 1e-4
    # in place (R is y), as the fused forward runs an in-place residual add: the same bits
    hipabi.check(L.knx_hip_conv_t_res(ctypes.byref(geom), ptr(dx), ptr(dwt), ptr(db), 0, 0.0, ptr(dR), ptr(dR),
                                      hipabi.stream()))
    assert np.array_equal(host(dR), host(y))


CONV_TILES = ["256x256", "256x128", "128x128", "128x128w8", "64x128", "256x64", "128x64"]
# the tap mask of the pipelined gather: 1 tap, 25 taps, 49 (bits past 32), and 81 taps (more than the mask holds:
# the general kernel); output pixels not a multiple of the tile
CONV_TILE_CASES = [(64, 32, 32, 64, 64, 3, 1, 1, 1, 1), (128, 16, 16, 64, 128, 3, 1, 1, 1, 1),
                   (256, 16, 16, 128, 256, 3, 2, 1, 1, 1), (128, 16, 16, 128, 128, 3, 1, 1, 2, 1),
                   (4, 15, 13, 64, 128, 1, 1, 0, 1, 1), (4, 12, 12, 64, 64, 5, 1, 2, 1, 1),
                   (4, 14, 14, 32, 64, 7, 1, 3, 1, 1), (3, 11, 12, 32, 128, 7, 2, 2, 1, 1),
                   (2, 12, 12, 32, 64, 9, 1, 4, 1, 1)]


@pytest.mark.parametrize("tile", ["128x128w8", "64x128", "128x64", "256x128"])
def test_conv_residual_tiles(L, tile, monkeypatch):
    """the residual epilogue on the 8-wave tiles (and one 4-wave tile), pixels not a multiple of the tile"""
    monkeypatch.setenv("KNX_CONV_TILE", tile)
    test_conv_residual(L, (17, 15, 15, 64, 128, 3, 1, 1, 1, 1))


@pytest.mark.parametrize("tile", CONV_TILES)
@pytest.mark.parametrize("case", CONV_TILE_CASES)
def test_conv_tiles(L, case, tile, monkeypatch):
    """every forced tile of the pipelined convolution (where the shape allows it) against the direct convolution"""
    monkeypatch.setenv("KNX_CONV_TILE", tile)
    test_conv(L, case, True)


@pytest.mark.parametrize("case", SMALL_CONV_CASES)
def test_conv_small_off(L, case, monkeypatch):
    """the shapes of the direct small-K kernel on the implicit-GEMM tile kernel instead (KNX_CONV_SMALL=0)"""
    monkeypatch.setenv("KNX_CONV_SMALL", "0")
    test_conv(L, case, True)
    test_conv(L, case, False)


@pytest.mark.parametrize("act", [-1, 1, 6])
@pytest.mark.parametrize("case", [(2, 8, 8, 3, 64, 3, 1, 1, 1, 1), (2, 9, 11, 2, 96, 3, 2, 1, 1, 1)])
def test_conv_small_act(L, case, act):
    """small-K shapes without activation (the register-operand kernel) and with GELU and ELU (alpha 0.1, the tile
    kernel)"""
    B, H, W, C, Co, k, s, p, g, dil = case
    rng = np.random.default_rng(sum(case) + act)
    Ho = (H + 2 * p - dil * (k - 1) - 1) // s + 1
    Wo = (W + 2 * p - dil * (k - 1) - 1) // s + 1
    x = rng.standard_normal((B * H * W, C)).astype(np.float32)
    w = (rng.standard_normal((k * k * C, Co)) / np.sqrt(k * k * C)).astype(np.float32)
    b = rng.normal(0, 0.1, Co).astype(np.float32)
    op = dict(cin=C, cout=Co, k=(k, k), s=(s, s), d=(dil, dil), p=(p, p, p, p), g=g, w=w, b=b)
    want, _ = knx_ref._conv(x, B, H, W, op, act_id=act, alpha=0.1)
    geom = hipabi.ConvGeom(B, H, W, C, Ho, Wo, Co, k, k, s, s, dil, dil, p, p, g)
    y = torch.empty((B * Ho * Wo, Co), dtype=torch.float32, device="cuda")
    dx, dwt, db = dev(x), dev(np.ascontiguousarray(w.T)), dev(b)
    hipabi.check(L.knx_hip_conv_t(ctypes.byref(geom), ptr(dx), ptr(dwt), ptr(db), act, 0.1, ptr(y), hipabi.stream()))
    assert rel_err(host(y), want) <= 1e-4


@pytest.mark.parametrize("case", CONV_CASES)
@pytest.mark.parametrize("wt", [False, True])  # weight as in the file (K × Co) or transposed (Co × K)
def test_conv(L, case, wt):
    B, H, W, C, Co, k, s, p, g, dil = case
    rng = np.random.default_rng(sum(case))
    Ho = (H + 2 * p - dil * (k - 1) - 1) // s + 1
    Wo = (W + 2 * p - dil * (k - 1) - 1) // s + 1
    x = rng.standard_normal((B * H * W, C)).astype(np.float32)
    w = (rng.standard_normal((k * k * (C // g), Co)) / np.sqrt(k * k * C / g)).astype(np.float32)
    b = rng.normal(0, 0.1, Co).astype(np.float32)
    op = dict(cin=C, cout=Co, k=(k, k), s=(s, s), d=(dil, dil), p=(p, p, p, p), g=g, w=w, b=b)
    want, _ = knx_ref._conv(x, B, H, W, op, act_id=0)
    geom = hipabi.ConvGeom(B, H, W, C, Ho, Wo, Co, k, k, s, s, dil, dil, p, p, g)
    y = torch.empty((B * Ho * Wo, Co), dtype=torch.float32, device="cuda")
    dx, dw, db = dev(x), dev(w), dev(b)
    if wt:
        dwt = dev(np.ascontiguousarray(w.T))
        hipabi.check(L.knx_hip_conv_t(ctypes.byref(geom), ptr(dx), ptr(dwt), ptr(db), 0, 0.0, ptr(y), hipabi.stream()))
    else:
        hipabi.check(L.knx_hip_conv(ctypes.byref(geom), ptr(dx), ptr(dw), ptr(db), 0, 0.0, ptr(y), hipabi.stream()))
    assert rel_err(host(y), want) <= 1e-4


# ---------------------------------------------------------------- attention core
# fused: one kernel with K, Vᵀ in LDS (dk = dv ∈ {32, 64, 128}, S ≤ 256); unfused: scores GEMM, softmax, P·V GEMM
# (the last two shapes of the list reach the pipelined GEMM there, with ragged tiles in the first); unfused_vt: P·V
# against a transposed copy of V
ATTN_SHAPES = [(2, 2, 5, 5, 4, 4, 1), (2, 8, 128, 128, 64, 64, 0), (1, 3, 7, 9, 16, 8, 0), (3, 4, 33, 33, 32, 32, 1),
               (2, 2, 5, 5, 64, 64, 1), (2, 4, 200, 200, 32, 32, 1), (3, 2, 50, 70, 128, 128, 1),
               (2, 2, 130, 300, 64, 64, 1), (2, 3, 140, 256, 64, 64, 1), (1, 2, 64, 128, 128, 128, 0),
               (16, 8, 160, 224, 32, 64, 1), (64, 8, 128, 128, 64, 64, 0)]


@pytest.mark.parametrize("B,H,Rq,S,dk,dv,causal", ATTN_SHAPES)
@pytest.mark.parametrize("mode", ["fused", "fused_d2", "fused_all", "unfused", "unfused_vt"])
def test_attention_core(L, B, H, Rq, S, dk, dv, causal, mode, monkeypatch):
    """fused: K and V staged three 32-key tiles ahead (the default), fused_d2 / fused_all: two ahead / all up front"""
    if mode.startswith("unfused"):
        monkeypatch.setenv("KNX_ATTN_KERNEL", "unfused")
    if mode == "fused_d2":
        monkeypatch.setenv("KNX_ATTN_DEPTH", "2")
    if mode == "fused_all":
        monkeypatch.setenv("KNX_ATTN_DEPTH", "all")
    vt = mode == "unfused_vt"
    rng = np.random.default_rng(B + H + Rq + S)
    Q = rng.standard_normal((B * Rq, H * dk)).astype(np.float32)
    K = rng.standard_normal((B * S, H * dk)).astype(np.float32)
    V = rng.standard_normal((B * S, H * dv)).astype(np.float32)
    scale = np.float32(1.0) / np.sqrt(np.float32(dk))
    want = np.zeros((B * Rq, H * dv), np.float32)
    knx_ref.lib().ko_attention_core(knx_ref._p(Q), knx_ref._p(K), knx_ref._p(V), knx_ref._p(want), B, H, Rq, S, dk, dv,
                                    float(scale), causal)
    ctx = torch.empty((B * Rq, H * dv), dtype=torch.float32, device="cuda")
    sc = torch.empty((B * H * Rq, S), dtype=torch.float32, device="cuda")
    dQ, dK, dV = dev(Q), dev(K), dev(V)
    if vt:
        dvt = torch.full((H * dv, B * S), float("nan"), dtype=torch.float32, device="cuda")
        hipabi.check(L.knx_hip_attention_core_ex(ptr(dQ), H * dk, ptr(dK), H * dk, ptr(dV), H * dv, ptr(dvt), ptr(ctx),
                                                 ptr(sc), B, H, Rq, S, dk, dv, float(scale), causal, hipabi.stream()))
        assert np.array_equal(host(dvt), V.T)
    else:
        hipabi.check(L.knx_hip_attention_core(ptr(dQ), ptr(dK), ptr(dV), ptr(ctx), ptr(sc), B, H, Rq, S, dk, dv,
                                              float(scale), causal, hipabi.stream()))
    assert rel_err(host(ctx), want) <= 1e-4


@pytest.mark.parametrize("B,H,Rq,dk,dv,causal", [(4, 8, 128, 64, 64, 1), (2, 3, 40, 32, 32, 0), (2, 2, 20, 16, 8, 1),
                                                 (3, 2, 300, 64, 64, 0)])
@pytest.mark.parametrize("mode", ["fused", "unfused", "unfused_vt"])
def test_attention_core_strided(L, B, H, Rq, dk, dv, causal, mode, monkeypatch):
    """Q, K, V as column slices of one (B·S) × (2·H·dk + H·dv) matrix (the output of a stacked Q|K|V projection)"""
    if mode != "fused":
        monkeypatch.setenv("KNX_ATTN_KERNEL", "unfused")
    S, n = Rq, 2 * H * dk + H * dv
    rng = np.random.default_rng(7 * B + H + Rq)
    qkv = rng.standard_normal((B * S, n)).astype(np.float32)
    Q, K, V = (np.ascontiguousarray(qkv[:, a:b]) for a, b in ((0, H * dk), (H * dk, 2 * H * dk), (2 * H * dk, n)))
    scale = np.float32(1.0) / np.sqrt(np.float32(dk))
    want = np.zeros((B * Rq, H * dv), np.float32)
    knx_ref.lib().ko_attention_core(knx_ref._p(Q), knx_ref._p(K), knx_ref._p(V), knx_ref._p(want), B, H, Rq, S, dk, dv,
                                    float(scale), causal)
    d = dev(qkv)
    at = lambda off: ctypes.c_void_p(d.data_ptr() + 4 * off)  # noqa: E731
    ctx = torch.empty((B * Rq, H * dv), dtype=torch.float32, device="cuda")
    sc = torch.empty((B * H * Rq, S), dtype=torch.float32, device="cuda")
    dvt = torch.empty((H * dv, B * S), dtype=torch.float32, device="cuda") if mode == "unfused_vt" else None
    hipabi.check(L.knx_hip_attention_core_ex(at(0), n, at(H * dk), n, at(2 * H * dk), n, ptr(dvt), ptr(ctx), ptr(sc),
                                             B, H, Rq, S, dk, dv, float(scale), causal, hipabi.stream()))
    assert rel_err(host(ctx), want) <= 1e-4
