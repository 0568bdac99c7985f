"""Python binding of the KERNIX model runtime (ctypes + numpy) for the MI355X build of libkernix.so.

API contract kept from the reference binding (reference python/kernix.py:43-115): the class `Model(path,
workspace_mb=None, ane=False)`, the attributes `in_dim, out_dim, seq_len, in_shape, out_shape, channels_first`, calling
a model on a batch, `trim()`, `ane_info()`, `_ane_dump()`, `close()`; ValueError for a file that does not load or an
input of the wrong shape, RuntimeError for a failed forward.

    m = Model("model.knx")
    y = m(x)   # x: (batch, *m.in_shape) float32 -> (batch, *m.out_shape); also accepts (rows, in_dim)

Models whose file says layout 1 (PyTorch convolution models) take and return channels-first arrays; the runtime itself
is channels-last, and the binding moves the axis both ways.  Calls on one Model are serialized by a lock: they share
the model's device workspace.  Use one Model per thread to run concurrently.

The shared library is kernix_amd/libkernix.so, or the file named by $KERNIX_LIB.  It is opened on first use (the first
Model, or the first call of an extension), not at import; opening fails with OSError when the library is missing or
was built for another target — there is no CPU fallback.  Where PyTorch is installed, its own HIP runtime is loaded
first (without importing torch), so that the library and torch share one runtime whichever is imported first.
"""
import ctypes
import importlib.util
import os
import sys
import threading
import warnings

import numpy as np

INT8_REF, INT8_I8 = 0, 1  # kernix_capi_set_int8_mode: reference dispatch / int8 arithmetic at every batch size

_VOID, _INT, _SIZE = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
_PINT, _PSIZE, _STR = ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_size_t), ctypes.c_char_p

# The C ABI (include/kernix_capi.h): name -> (argument types, result type)
_ABI = {
    "kernix_capi_load": ((_STR,), _VOID),
    "kernix_capi_free": ((_VOID,), None),
    "kernix_capi_trim": ((_VOID,), None),
    "kernix_capi_set_workspace_limit": ((_VOID, _SIZE), None),
    "kernix_capi_dims": ((_VOID, _PINT, _PINT, _PINT), None),
    "kernix_capi_forward": ((_VOID, _VOID, _INT, _VOID), _INT),
    "kernix_capi_set_ane": ((_VOID, _INT), _INT),
    "kernix_capi_ane_info": ((_VOID, _PINT), None),
    "kernix_capi_ane_dump": ((_VOID, _INT, _INT, _STR), _INT),
    "kernix_capi_shapes": ((_VOID, _PINT, _PINT, _PINT, _PINT, _PINT), None),
    # extensions of this build
    "kernix_capi_set_int8_mode": ((_VOID, _INT), _INT),
    "kernix_capi_forward_device": ((_VOID, _VOID, _INT, _VOID, _VOID), _INT),
    "kernix_capi_forward_cf": ((_VOID, _VOID, _INT, _VOID), _INT),
    "kernix_capi_device_status": ((_VOID,), _INT),
    "kernix_capi_ws_info": ((_VOID, _PSIZE, _PSIZE, _PINT), None),
}

_ANE_FIELDS = ("segments", "compiles", "ane_runs", "failures")


def library_path():
    """the shared library the binding opens"""
    return os.environ.get("KERNIX_LIB") or os.path.join(os.path.dirname(os.path.abspath(__file__)), "libkernix.so")


def _share_torch_runtime():
    """PyTorch-ROCm wheels ship their own HIP runtime (torch/lib/libamdhip64.so, the soname libkernix.so links).  When
    torch is installed but not imported yet, load its copy before the library (without importing torch): the library
    then binds to it, and a later `import torch` uses the same one instead of loading a second runtime, which would
    leave the library without a device.  Nothing to do when torch is already imported (its runtime is loaded) or not
    installed (the system runtime); KNX_SYSTEM_HIP=1 keeps the system runtime."""
    if "torch" in sys.modules or os.environ.get("KNX_SYSTEM_HIP", "") not in ("", "0"):
        return
    try:
        spec = importlib.util.find_spec("torch")
    except (ImportError, ValueError):
        return
    for d in (spec.submodule_search_locations or []) if spec is not None else []:
        path = os.path.join(d, "lib", "libamdhip64.so")
        if os.path.exists(path):
            try:
                ctypes.CDLL(path, mode=ctypes.RTLD_GLOBAL)
            except OSError:
                pass
            return


class _Library:
    """libkernix.so with its entry points typed, opened once on first attribute access."""

    def __init__(self):
        self._dll = None
        self._opening = threading.Lock()

    def _open(self):
        with self._opening:
            if self._dll is None:
                _share_torch_runtime()
                dll = ctypes.CDLL(library_path())
                for name, (args, res) in _ABI.items():
                    fn = getattr(dll, name)
                    fn.argtypes, fn.restype = list(args), res
                self._dll = dll
        return self._dll

    def __getattr__(self, name):
        if name not in _ABI:
            raise AttributeError(name)
        return getattr(self._dll or self._open(), name)


_lib = _Library()


def _channels_first_view(cl_shape):
    """(…, C) -> (C, …): how a channels-first model shows a per-sample shape of two or more axes"""
    return (cl_shape[-1],) + cl_shape[:-1] if len(cl_shape) >= 2 else cl_shape


class Model:
    """A loaded .knx model (see the module docstring)."""

    def __init__(self, path, workspace_mb=None, ane=False):
        """workspace_mb: bound of the device workspace in MB (None: the library default; 0: no bound).  A batch
        larger than the bound allows runs in pieces.  ane: accepted for compatibility; this platform has no Neural
        Engine, so asking for it warns and the model runs on the GPU path."""
        self._lock = threading.Lock()  # before anything that can fail: close() takes it
        self._h = None
        handle = _lib.kernix_capi_load(os.fsencode(path))
        if not handle:
            raise ValueError(f"cannot load KERNIX model: {path}")
        self._h = handle
        if workspace_mb is not None:
            if workspace_mb < 0:
                raise ValueError("workspace_mb must be >= 0")
            _lib.kernix_capi_set_workspace_limit(handle, int(workspace_mb * (1 << 20)))
        if ane and _lib.kernix_capi_set_ane(handle, 1) != 0:
            warnings.warn("no Neural Engine on this platform: the model runs on the KERNIX GPU path", RuntimeWarning,
                          stacklevel=2)
        self._describe()

    def _describe(self):
        ints = [ctypes.c_int() for _ in range(6)]
        in_dim, out_dim, seq_len, in_nd, out_nd, layout = ints
        _lib.kernix_capi_dims(self._h, ctypes.byref(in_dim), ctypes.byref(out_dim), ctypes.byref(seq_len))
        in4, out4 = (ctypes.c_int * 4)(), (ctypes.c_int * 4)()
        _lib.kernix_capi_shapes(self._h, ctypes.byref(in_nd), in4, ctypes.byref(out_nd), out4, ctypes.byref(layout))
        self.in_dim, self.out_dim, self.seq_len = in_dim.value, out_dim.value, seq_len.value
        self._in_cl = tuple(in4[: in_nd.value])    # channels-last, as the runtime stores values
        self._out_cl = tuple(out4[: out_nd.value])
        self.channels_first = layout.value == 1
        view = _channels_first_view if self.channels_first else tuple
        self.in_shape, self.out_shape = view(self._in_cl), view(self._out_cl)

    # ---- forward ----
    def _rows_of(self, x):
        """x as contiguous float32 values, the row count (of in_dim values) and whether the samples are channels-first:
        a batched input of a channels-first model keeps its layout (the library moves the axis on the device, the
        reference binding's host-side move), anything else is channels-last rows"""
        x = np.asarray(x)
        batched = x.ndim >= 2 and tuple(x.shape[1:]) == self.in_shape
        cf = batched and self.channels_first and x.ndim >= 3
        if not batched and not (x.ndim == 2 and x.shape[1] == self.in_dim):
            want = ", ".join(str(d) for d in self.in_shape)
            raise ValueError(f"input shape {x.shape}: expected (batch, {want}) or (rows, {self.in_dim})")
        x = np.ascontiguousarray(x, dtype=np.float32)
        rows = x.size // self.in_dim
        if rows == 0 or rows % self.seq_len != 0:
            raise ValueError(f"{rows} input rows: must be a positive multiple of seq_len {self.seq_len}")
        return x, rows, cf

    def __call__(self, x):
        x, rows, cf = self._rows_of(x)
        y = np.empty((rows // self.seq_len,) + self._out_cl, dtype=np.float32)
        forward = _lib.kernix_capi_forward_cf if cf else _lib.kernix_capi_forward
        with self._lock:
            ok = forward(self._h, x.ctypes.data, rows, y.ctypes.data) == 0
        if not ok:
            raise RuntimeError("KERNIX forward failed (see stderr)")
        if self.channels_first and y.ndim >= 3:
            y = np.moveaxis(y, -1, 1)
        return y

    # ---- reference API ----
    def trim(self):
        """Release the device workspace; the weights stay on the device and the next call allocates it again."""
        with self._lock:
            _lib.kernix_capi_trim(self._h)

    def ane_info(self):
        """Neural Engine counters (all zero here)."""
        counts = (ctypes.c_int * 4)()
        with self._lock:
            _lib.kernix_capi_ane_info(self._h, counts)
        return {name: counts[i] for i, name in enumerate(_ANE_FIELDS)}

    def _ane_dump(self, seg, batch, path):
        """Core ML export of a segment: unavailable here, returns -1."""
        with self._lock:
            return _lib.kernix_capi_ane_dump(self._h, seg, batch, os.fsencode(path))

    def close(self):
        handle = getattr(self, "_h", None)
        if handle:
            with self._lock:
                self._h = None
                _lib.kernix_capi_free(handle)

    def __del__(self):
        self.close()

    # ---- extensions of this build ----
    def set_int8_mode(self, mode):
        """INT8_REF (default): int8 arithmetic at <= 2 rows and the dequantized fp32 weights above, as the reference
        dispatches; INT8_I8: int8 arithmetic (i8 MFMA) at every batch size."""
        with self._lock:
            if _lib.kernix_capi_set_int8_mode(self._h, int(mode)) != 0:
                raise ValueError(f"unknown int8 mode {mode!r}")

    def forward_device(self, x_ptr, rows, out_ptr, stream=None):
        """Enqueue a forward on device buffers (e.g. torch tensors' data_ptr(); rows x in_dim in, rows/seq_len x
        out_dim out) on a hipStream_t handle (None: the model's own stream).  Returns without waiting; forwards on
        different streams still run in call order on the device."""
        with self._lock:
            if _lib.kernix_capi_forward_device(self._h, x_ptr, int(rows), out_ptr, stream) != 0:
                raise RuntimeError("KERNIX device forward failed (see stderr)")

    def device_status(self):
        """Wait for the last forward; True if every device forward since the previous check computed correctly,
        False if one ran a Linear chain whose workgroups could not all be resident at once (more chains running
        than the GPU holds): its outputs are wrong and it must be run again.  Host forwards (__call__) recompute such
        a forward themselves."""
        with self._lock:
            return _lib.kernix_capi_device_status(self._h) == 0

    def ws_info(self):
        """(workspace floats per sample, batch-independent floats, rows the workspace holds or -1)"""
        per, fixed, rows = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_int()
        with self._lock:
            _lib.kernix_capi_ws_info(self._h, ctypes.byref(per), ctypes.byref(fixed), ctypes.byref(rows))
        return per.value, fixed.value, rows.value
