"""KERNIX model runtime — Python binding (ctypes + numpy only) for the MI355X build.

Same API as the reference binding (reference python/kernix.py:43-115):

    from kernix_amd.kernix import Model
    m = Model("model.knx")        # workspace_mb=None → library default, 0 → unlimited
    y = m(x)                      # x: (batch, *m.in_shape) float32 → (batch, *m.out_shape)
                                  # PyTorch conv models (layout 1): (batch, C, H, W); the legacy (rows, in_dim) too

One Model may be called from several threads: calls on one model are serialized (they share its device workspace).
The library is kernix_amd/libkernix.so, or the path in the KERNIX_LIB environment variable; importing this module
fails with OSError when it cannot be loaded — there is no CPU fallback.
"""
import ctypes
import os
import threading
import warnings

import numpy as np

_LIB_PATH = os.environ.get("KERNIX_LIB", os.path.join(os.path.dirname(os.path.abspath(__file__)), "libkernix.so"))
_lib = ctypes.CDLL(_LIB_PATH)

_P = ctypes.c_void_p
_I = ctypes.c_int
_IP = ctypes.POINTER(ctypes.c_int)
for _name, _args, _res in (
    ("kernix_capi_load", [ctypes.c_char_p], _P),
    ("kernix_capi_free", [_P], None),
    ("kernix_capi_dims", [_P, _IP, _IP, _IP], None),
    ("kernix_capi_forward", [_P, _P, _I, _P], _I),
    ("kernix_capi_trim", [_P], None),
    ("kernix_capi_set_workspace_limit", [_P, ctypes.c_size_t], None),
    ("kernix_capi_shapes", [_P, _IP, _IP, _IP, _IP, _IP], None),
    ("kernix_capi_set_ane", [_P, _I], _I),
    ("kernix_capi_ane_info", [_P, _IP], None),
    ("kernix_capi_ane_dump", [_P, _I, _I, ctypes.c_char_p], _I),
    ("kernix_capi_set_int8_mode", [_P, _I], _I),
    ("kernix_capi_forward_device", [_P, _P, _I, _P, _P], _I),
    ("kernix_capi_ws_info", [_P, ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t), _IP], None),
):
    _f = getattr(_lib, _name)
    _f.argtypes = _args
    _f.restype = _res

INT8_REF, INT8_I8 = 0, 1


class Model:
    def __init__(self, path, workspace_mb=None, ane=False):
        """workspace_mb: device workspace bound in MB; larger batches run in chunks.  None = library default,
        0 = unlimited.  ane: accepted for compatibility; there is no Neural Engine here (a RuntimeWarning is issued)."""
        self._lock = threading.Lock()  # first: close() must work even if __init__ fails below
        self._h = _lib.kernix_capi_load(os.fsencode(path))
        if not self._h:
            raise ValueError(f"cannot load KERNIX model: {path}")
        if workspace_mb is not None:
            if workspace_mb < 0:
                raise ValueError("workspace_mb must be >= 0")
            _lib.kernix_capi_set_workspace_limit(self._h, int(workspace_mb * (1 << 20)))
        if ane and _lib.kernix_capi_set_ane(self._h, 1) != 0:
            warnings.warn("Neural Engine assist unavailable on this platform: running the KERNIX GPU path",
                          RuntimeWarning, stacklevel=2)
        dims = [ctypes.c_int() for _ in range(3)]
        _lib.kernix_capi_dims(self._h, *dims)
        self.in_dim, self.out_dim, self.seq_len = (d.value for d in dims)
        in_nd, out_nd, layout = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        in_s, out_s = (ctypes.c_int * 4)(), (ctypes.c_int * 4)()
        _lib.kernix_capi_shapes(self._h, ctypes.byref(in_nd), in_s, ctypes.byref(out_nd), out_s, ctypes.byref(layout))
        self._in_cl, self._out_cl = tuple(in_s[:in_nd.value]), tuple(out_s[:out_nd.value])  # channels-last
        self.channels_first = layout.value == 1
        cf = (lambda s: s[-1:] + s[:-1] if self.channels_first and len(s) >= 2 else s)  # noqa: E731
        self.in_shape, self.out_shape = cf(self._in_cl), cf(self._out_cl)
        self._forward = _lib.kernix_capi_forward

    def __call__(self, x):
        x = np.asarray(x)
        if x.ndim >= 2 and tuple(x.shape[1:]) == self.in_shape:
            if self.channels_first and x.ndim >= 3:
                x = np.moveaxis(x, 1, -1)  # (B, C, ...) → (B, ..., C)
        elif not (x.ndim == 2 and x.shape[1] == self.in_dim):  # legacy (rows, in_dim)
            raise ValueError(f"input shape {x.shape}: expected (batch, {', '.join(map(str, self.in_shape))}) "
                             f"or (rows, {self.in_dim})")
        x = np.ascontiguousarray(x, dtype=np.float32)
        rows = x.size // self.in_dim
        if rows == 0 or rows % self.seq_len:
            raise ValueError(f"input rows {rows} must be a positive multiple of seq_len {self.seq_len}")
        out = np.empty((rows // self.seq_len,) + self._out_cl, np.float32)
        with self._lock:
            status = self._forward(self._h, x.ctypes.data, rows, out.ctypes.data)
        if status != 0:
            raise RuntimeError("KERNIX forward failed")
        return np.moveaxis(out, -1, 1) if self.channels_first and out.ndim >= 3 else out

    # ---- extensions of this build ----
    def set_int8_mode(self, mode):
        """INT8_REF (default): int8 arithmetic only at <= 2 rows, the fp32 copy above (the reference's dispatch);
        INT8_I8: int8 arithmetic on i8 MFMA at every batch size."""
        with self._lock:
            if _lib.kernix_capi_set_int8_mode(self._h, int(mode)) != 0:
                raise ValueError(f"bad int8 mode {mode}")

    def forward_device(self, x_ptr, rows, out_ptr, stream=None):
        """Enqueue a forward on device buffers (e.g. torch tensors' data_ptr()); stream: hipStream_t handle or None."""
        with self._lock:
            if _lib.kernix_capi_forward_device(self._h, x_ptr, int(rows), out_ptr, stream) != 0:
                raise RuntimeError("KERNIX device forward failed")

    def ws_info(self):
        """(workspace floats per sample, batch-independent floats, rows the workspace is allocated for or -1)"""
        per, fixed, batch = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_int()
        with self._lock:
            _lib.kernix_capi_ws_info(self._h, ctypes.byref(per), ctypes.byref(fixed), ctypes.byref(batch))
        return per.value, fixed.value, batch.value

    # ---- reference API ----
    def ane_info(self):
        out = (ctypes.c_int * 4)()
        with self._lock:
            _lib.kernix_capi_ane_info(self._h, out)
        return dict(zip(("segments", "compiles", "ane_runs", "failures"), out))

    def _ane_dump(self, seg, batch, path):
        with self._lock:
            return _lib.kernix_capi_ane_dump(self._h, seg, batch, os.fsencode(path))

    def trim(self):
        """Release the device workspace (weights stay on the device); the next call allocates it again."""
        with self._lock:
            _lib.kernix_capi_trim(self._h)

    def close(self):
        if getattr(self, "_h", None):
            with self._lock:
                _lib.kernix_capi_free(self._h)
                self._h = None

    __del__ = close
