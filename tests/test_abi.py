"""The drop-in boundary: libkernix.so exports every entry point declared in include/*.h, the Python binding keeps the
reference's API (reference python/kernix.py), failures are loud, and injected device failures propagate as -1/NULL."""
import ctypes
import os
import subprocess
import sys

import numpy as np
import pytest

from kernix_amd import configs, hipabi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _has_gpu():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:  # pragma: no cover
        return False


def test_every_declared_symbol_is_exported():
    lib = ctypes.CDLL(hipabi.LIB_PATH)
    names = hipabi.declared_symbols()
    assert {"kernix_capi_load", "kernix_capi_forward", "kernix_capi_shapes", "knx_hip_i8gemm", "kernix_qmatmul"} <= names
    missing = sorted(n for n in names if not hasattr(lib, n))
    assert not missing, missing


def test_reference_capi_signatures_bind(tmp_path):
    """this repository's binding (kernix_amd/kernix.py), whose ctypes table gives the ten reference exports the argument
    types of the reference binding's table (reference python/kernix.py:21-40), drives the reference's Model API; the
    reference binding itself is not loaded"""
    from kernix_amd import kernix as kx

    p = str(tmp_path / "c.knx")
    configs.cnn(p, batch=1, hw=8, widths=(4, 4, 8, 8))
    m = kx.Model(p)
    assert m.channels_first and m.in_shape == (3, 8, 8) and m.out_shape == (10,)
    assert m.in_dim == 3 and m.seq_len == 64 and m.out_dim == 10
    assert m.ane_info() == dict(segments=0, compiles=0, ane_runs=0, failures=0)
    assert m._ane_dump(0, 1, str(tmp_path / "x.mlmodel")) == -1
    with pytest.warns(RuntimeWarning):
        kx.Model(p, ane=True).close()
    with pytest.raises(ValueError):
        kx.Model(p, workspace_mb=-1)
    with pytest.raises(ValueError):
        kx.Model(str(tmp_path / "missing.knx"))
    with pytest.raises(ValueError):
        m(np.zeros((2, 5), np.float32))  # wrong width
    m.trim()
    m.close()
    m.close()  # idempotent


def test_missing_library_fails_loudly():
    """the binding opens the library on first use: a missing library is an OSError there, not a fallback"""
    code = "import sys; sys.path.insert(0, %r); import kernix_amd.kernix as k; k.Model('any.knx')" % ROOT
    r = subprocess.run([sys.executable, "-c", code], env=dict(os.environ, KERNIX_LIB="/nonexistent/libkernix.so"),
                       capture_output=True, text=True)
    assert r.returncode != 0 and "OSError" in r.stderr


@pytest.mark.skipif(_has_gpu(), reason="checks the behaviour without a GPU")
def test_forward_without_gpu_is_an_error_not_a_fallback(tmp_path):
    from kernix_amd import kernix as kx

    p = str(tmp_path / "m.knx")
    x = configs.int8_mlp(p, batch=2)
    m = kx.Model(p)
    with pytest.raises(RuntimeError):
        m(x)
    m.close()


@pytest.mark.gpu
@pytest.mark.parametrize("batch,entry", [(32, "knx_hip_sgemm_nt_ep"), (3, "knx_hip_linear_chain")])
def test_injected_device_failure_propagates(tmp_path, batch, entry):
    """KNX_HIP_FAIL makes the kernel entry point the forward uses fail (fp32 Linears over 32 rows: one GEMM each; over
    3 rows: one chain launch): forward returns -1 (RuntimeError in Python), then recovers"""
    code = f"""
import os, sys
sys.path.insert(0, {ROOT!r})
import numpy as np
from kernix_amd import configs
from kernix_amd.kernix import Model
x = configs.fp32_mlp({str(tmp_path / 'f.knx')!r}, batch={batch}, dims=(16, 32, 8))
m = Model({str(tmp_path / 'f.knx')!r})
good = m(x)
os.environ["KNX_HIP_FAIL"] = {entry!r}
try:
    m(x)
    print("no error")
except RuntimeError:
    print("raised")
del os.environ["KNX_HIP_FAIL"]
print("recovered", bool(np.array_equal(m(x), good)))
"""
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert "raised" in r.stdout and "recovered True" in r.stdout, r.stdout + r.stderr
    assert "injected failure" in r.stderr


@pytest.mark.gpu
def test_runs_on_the_current_device(tmp_path):
    """the library checks and uses the calling thread's current device (one process per GPU selects it), and a model
    keeps running on the device current at its first forward; a device that does not exist is an error"""
    import ctypes as C

    L = hipabi.lib()
    hipabi.check(L.knx_hip_init())
    d = C.c_int(-1)
    hipabi.check(L.knx_hip_get_device(C.byref(d)))
    assert d.value >= 0
    assert L.knx_hip_set_device(d.value) == 0
    assert L.knx_hip_set_device(1 << 20) == -2  # KNX_EHIP
    from kernix_amd.kernix import Model

    p = str(tmp_path / "m.knx")
    x = configs.int8_mlp(p, batch=3)
    m = Model(p)
    y = m(x).copy()
    assert np.array_equal(m(x), y)
    m.close()
