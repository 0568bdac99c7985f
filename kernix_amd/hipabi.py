"""ctypes bindings of the kernel-level C ABI (include/knx_hip.h) of libkernix.so.

Used by the benchmark and the kernel tests to call the gfx950 kernels on device buffers that the caller owns (for
example torch tensors: pass ptr(tensor) and stream()).  Loading fails with OSError when the library is missing.
"""
import ctypes
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.environ.get("KERNIX_LIB", os.path.join(ROOT, "kernix_amd", "libkernix.so"))

P, I, F, Z = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_size_t


class ConvGeom(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in
                ("B", "H", "W", "C", "Ho", "Wo", "Co", "kh", "kw", "sh", "sw", "dh", "dw", "pt", "pl", "groups")]


class ChainLayer(ctypes.Structure):
    """knx_chain_layer (include/knx_hip.h)"""
    _fields_ = [("w", P), ("sw", P), ("bias", P), ("y", P), ("k", I), ("kp", I), ("n", I), ("ldw", I), ("ldy", I),
                ("act", I), ("i8", I), ("alpha", F)]


SIGS = {
    "knx_hip_init": ([], I),
    "knx_hip_get_device": ([ctypes.POINTER(ctypes.c_int)], I),
    "knx_hip_set_device": ([I], I),
    "knx_hip_host_malloc": ([ctypes.POINTER(ctypes.c_void_p), Z], I),
    "knx_hip_host_free": ([P], I),
    "knx_hip_last_error": ([], ctypes.c_char_p),
    "knx_hip_quantize_rows": ([P, I, I, I, I, P, I, P, P], I),
    "knx_hip_i8gemm": ([I, I, I, P, I, P, P, I, P, P, I, F, I, P, I, P, I, P], I),
    "knx_hip_dequant": ([P, I, P, I, I, P, P], I),
    "knx_hip_dequant_t": ([P, I, P, I, I, P, P], I),
    "knx_hip_sgemm_ep": ([I, I, I, P, I, P, I, P, I, F, P, I, P], I),
    "knx_hip_sgemm_nt_ep": ([I, I, I, P, I, P, I, P, I, F, P, I, P], I),
    "knx_hip_conv": ([ctypes.POINTER(ConvGeom), P, P, P, I, F, P, P], I),
    "knx_hip_conv_t": ([ctypes.POINTER(ConvGeom), P, P, P, I, F, P, P], I),
    "knx_hip_conv_t_res": ([ctypes.POINTER(ConvGeom), P, P, P, I, F, P, P, P], I),
    "knx_hip_sgemm_nt_ep_res": ([I, I, I, P, I, P, I, P, I, F, P, I, P, I, P], I),
    "knx_hip_i8gemm_res": ([I, I, I, P, I, P, P, I, P, P, I, F, P, I, P, I, P], I),
    "knx_hip_qlinear": ([P, I, I, I, I, P, P, P, I, I, P, P, I, F, I, P, I, P, I, P], I),
    "knx_hip_qlinear_noalloc": ([P, I, I, I, I, P, I, I, P, P, I, F, I, P, I, P, I, P], I),
    "knx_hip_layernorm": ([P, P, I, I, P, P, F, P], I),
    "knx_hip_layernorm_quantize": ([P, I, I, P, P, F, I, P, P, P], I),
    "knx_hip_softmax": ([P, P, I, I, P], I),
    "knx_hip_bias_act": ([P, P, I, I, P, I, F, P], I),
    "knx_hip_binary": ([I, P, I, I, P, I, I, P, I, I, I, P], I),
    "knx_hip_global_pool": ([I, P, I, I, I, P, P], I),
    "knx_hip_affine": ([P, P, I, I, P, P, P], I),
    "knx_hip_add_const": ([P, P, I, I, P, P], I),
    "knx_hip_attention_core": ([P, P, P, P, P, I, I, I, I, I, I, F, I, P], I),
    "knx_hip_attention_core_ex": ([P, I, P, I, P, I, P, P, P, I, I, I, I, I, I, F, I, P], I),
    "knx_hip_linear_chain_scratch": ([ctypes.POINTER(ChainLayer), I, I], Z),
    "knx_hip_linear_chain": ([P, I, I, ctypes.POINTER(ChainLayer), I, P, Z, P, P], I),
    "knx_hip_memset": ([P, I, Z, P], I),
    "knx_hip_rnn_recurrence_fits": ([I, I, I, I], I),
    "knx_hip_rnn_recurrence_dense_fits": ([I, I, I, I, I], I),
    "knx_hip_rnn_recurrence": ([I, I, F, I, I, I, I, P, P, I, P, I, P, P, P, P, P, I, I, P, Z, P, P], I),
}

_lib = None


def lib():
    global _lib
    if _lib is None:
        L = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in SIGS.items():
            f = getattr(L, name)
            f.argtypes, f.restype = args, res
        _lib = L
    return _lib


def check(rc):
    if rc != 0:
        raise RuntimeError(f"knx_hip call failed ({rc}): {lib().knx_hip_last_error().decode()}")


def declared_symbols():
    """Every function declared in include/*.h (the ABI surface the library must export)."""
    names = set()
    for h in ("kernix.h", "kernix_model.h", "kernix_capi.h", "knx_hip.h"):
        text = open(os.path.join(ROOT, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"(?:KERNIX_API|KNX_API)\s+[\w\s\*]+?\b(\w+)\s*\(", text):
            names.add(m.group(1))
    return names


def ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream():
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
