"""knx_hip_qlinear_noalloc (the entry point that allocates nothing) against knx_hip_qlinear with caller scratch.

Both run the same kernels, so the outputs must be the same bits; the existing entry point is itself checked against
the oracle's kernix_qmatmul in the kernel tests, and the first case here is also checked against the oracle directly.
Two calls in a row, the second smaller, so the second reads a scratch array that still holds the first call's rows.
"""
import numpy as np
import pytest

from oracle import knx_ref
from kernix_amd import hipabi
from kernix_amd.hipabi import ptr

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.fixture(scope="module")
def L():
    lib = hipabi.lib()
    hipabi.check(lib.knx_hip_init())
    return lib


def _case(rng, rows, k, n):
    kp = (k + 63) // 64 * 64
    x = rng.normal(0, 1, (rows, k)).astype(np.float32)
    x[0, :] = 0.0
    if rows >= 3:
        x[2, k // 3] = np.inf
    q = rng.integers(-127, 128, (n, k), dtype=np.int8)
    qp = np.zeros((n, kp), np.int8)
    qp[:, :k] = q
    scale = rng.uniform(0.001, 0.01, n).astype(np.float32)
    bias = rng.normal(0, 0.1, n).astype(np.float32)
    return x, q, qp, scale, bias, kp


def _both(L, x, qp, scale, bias, kp, act, R=None):
    """(no-alloc output, output of knx_hip_qlinear with torch-allocated scratch) for the same arguments"""
    rows, k = x.shape
    n = qp.shape[0]
    dx, dq, ds, db = dev(x), dev(qp), dev(scale), dev(bias)
    dR = dev(R) if R is not None else None
    xq = torch.empty((rows, kp), dtype=torch.int8, device="cuda")
    sx = torch.empty(rows, dtype=torch.float32, device="cuda")
    Y0 = torch.full((rows, n), 7.0, dtype=torch.float32, device="cuda")
    Y1 = torch.full((rows, n), -3.0, dtype=torch.float32, device="cuda")
    s = hipabi.stream()
    hipabi.check(L.knx_hip_qlinear(ptr(dx), k, rows, k, kp, ptr(xq), ptr(sx), ptr(dq), kp, n, ptr(ds), ptr(db), act,
                                   0.0, 0, ptr(dR), n if R is not None else 0, ptr(Y0), n, s))
    hipabi.check(L.knx_hip_qlinear_noalloc(ptr(dx), k, rows, k, kp, ptr(dq), kp, n, ptr(ds), ptr(db), act, 0.0, 0,
                                           ptr(dR), n if R is not None else 0, ptr(Y1), n, s))
    return host(Y1), host(Y0)


def _same(a, b):
    return np.array_equal(np.isnan(a), np.isnan(b)) and np.array_equal(a[~np.isnan(a)], b[~np.isnan(b)])


def test_noalloc_matches_qlinear_twice_then_smaller(L):
    rng = np.random.default_rng(2024)
    # first call: 300 rows through the quantizer + GEMM, no activation; also against the oracle
    x, q, qp, scale, bias, kp = _case(rng, 300, 1000, 520)
    got, want = _both(L, x, qp, scale, bias, kp, -1)
    assert _same(got, want)
    ref = knx_ref.qmatmul(x, q.T.copy(), scale, bias)
    assert _same(got, ref)
    assert np.isnan(got[2]).all()
    # second call, smaller, ReLU: the scratch still holds the first call's rows and scales
    x, q, qp, scale, bias, kp = _case(rng, 37, 256, 100)
    got, want = _both(L, x, qp, scale, bias, kp, 0)
    assert _same(got, want)


def test_noalloc_residual_and_few_rows(L):
    rng = np.random.default_rng(77)
    x, q, qp, scale, bias, kp = _case(rng, 96, 512, 256)
    R = rng.normal(0, 1, (96, 256)).astype(np.float32)
    got, want = _both(L, x, qp, scale, bias, kp, 0, R)
    assert _same(got, want)
    # 3 rows of 784 -> 512 (rows <= 16 and rows*k*n <= 2^23): the quantizer runs inside the GEMM, no scratch
    x, q, qp, scale, bias, kp = _case(rng, 3, 784, 512)
    got, want = _both(L, x, qp, scale, bias, kp, 0)
    assert _same(got, want)


def test_noalloc_at_the_limit_and_beyond(L):
    # 8000 rows of 4096 int8 values and their scales: 32.8 MB, below the 32 MiB (33.55 MB) limit
    rng = np.random.default_rng(5)
    rows, k, n = 8000, 4096, 64
    x = rng.normal(0, 1, (rows, k)).astype(np.float32)
    qp = rng.integers(-127, 128, (n, k), dtype=np.int8)
    scale = rng.uniform(0.001, 0.01, n).astype(np.float32)
    bias = rng.normal(0, 0.1, n).astype(np.float32)
    got, want = _both(L, x, qp, scale, bias, k, 0)
    assert _same(got, want)
    # 8192 rows of 4096 need 32 KiB more than the limit: rejected before any launch, the output untouched
    rows = 8192
    dx = torch.zeros((rows, k), dtype=torch.float32, device="cuda")
    dq, ds = dev(qp), dev(scale)
    Y = torch.full((rows, n), 5.0, dtype=torch.float32, device="cuda")
    rc = L.knx_hip_qlinear_noalloc(ptr(dx), k, rows, k, k, ptr(dq), k, n, ptr(ds), None, -1, 0.0, 0, None, 0,
                                   ptr(Y), n, hipabi.stream())
    assert rc == -1  # KNX_EINVAL
    assert b"limit" in L.knx_hip_last_error()
    assert bool((host(Y) == 5.0).all())


def test_noalloc_allocates_nothing(L):
    """after one warm-up call, further calls leave the device's free memory unchanged (hipMemGetInfo)"""
    rng = np.random.default_rng(11)
    x, q, qp, scale, bias, kp = _case(rng, 512, 2048, 1024)
    rows, k = x.shape
    n = qp.shape[0]
    dx, dq, ds, db = dev(x), dev(qp), dev(scale), dev(bias)
    Y = torch.empty((rows, n), dtype=torch.float32, device="cuda")
    s = hipabi.stream()

    def call(r):
        hipabi.check(L.knx_hip_qlinear_noalloc(ptr(dx), k, r, k, kp, ptr(dq), kp, n, ptr(ds), ptr(db), 0, 0.0, 0,
                                               None, 0, ptr(Y), n, s))

    call(rows)
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    for r in (rows, 7, 300, 1, rows):
        call(r)
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    assert free1 == free0, (free0, free1)
