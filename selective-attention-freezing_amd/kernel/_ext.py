"""ctypes binding of libsafattn.so (C-ABI declared in include/saf_attn.h).

The library is built in-tree by ``build_ext.build()`` and loaded from this
directory.  There is no fallback: if the library is missing, every entry point
that needs it raises ``RuntimeError`` naming the build step.
"""
import ctypes
import os

import torch

LIB_NAME = "libsafattn.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

SAF_OK, SAF_EINVAL, SAF_EUNSUPPORTED, SAF_EALIGN, SAF_ELAUNCH, SAF_EWORKSPACE = 0, -1, -2, -3, -4, -5
SAF_F32, SAF_F16, SAF_BF16, SAF_I32 = 0, 1, 2, 3
SAF_MAX_HEADS = 128

_DTYPE_CODE = {torch.float32: SAF_F32, torch.float16: SAF_F16,
               torch.bfloat16: SAF_BF16, torch.int32: SAF_I32}

# Exported symbols, in header order (checked by the CPU test suite).
EXPORTS = ("saf_mixed_attn_fwd", "saf_mixed_attn_fwd_noalloc", "saf_flash_fwd", "saf_frozen_dense_pv_fwd",
           "saf_frozen_decomp_fwd", "saf_frozen_scan_fwd", "saf_mixed_attn_bwd",
           "saf_mixed_attn_bwd_workspace_bytes", "saf_decomp_param_bwd", "saf_decomp_param_bwd_workspace_bytes",
           "saf_frozen_pv_fwd", "saf_frozen_pv_bwd",
           "saf_rope_qk_inplace", "saf_qk_rmsnorm_rope_inplace", "saf_add_layernorm",
           "saf_add_rmsnorm", "saf_linear_gelu", "saf_gelu_inplace", "saf_linear_swiglu", "saf_linear_rope", "saf_decomposed_logz",
           "saf_decomposed_logz_bwd", "saf_workspace_bytes", "saf_mixed_attn_workspace_bytes", "saf_workspace_error",
           "saf_time_next_kernel", "saf_last_error", "saf_version")


class SafTensor(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("dtype", ctypes.c_int32),
                ("ndim", ctypes.c_int32), ("size", ctypes.c_int64 * 4),
                ("stride", ctypes.c_int64 * 4)]


class SafMixedAttnArgs(ctypes.Structure):
    _fields_ = [("q", SafTensor), ("k", SafTensor), ("v", SafTensor),
                ("out", SafTensor), ("lse", SafTensor), ("patt", SafTensor),
                ("alpha", SafTensor), ("rho", SafTensor), ("z", SafTensor),
                ("n_heads", ctypes.c_int32),
                ("frozen", ctypes.POINTER(ctypes.c_int32)),
                ("hidx", ctypes.POINTER(ctypes.c_int32)),
                ("pidx", ctypes.POINTER(ctypes.c_int32)),
                ("kvidx", ctypes.POINTER(ctypes.c_int32)),
                ("closed_kind", ctypes.POINTER(ctypes.c_int32)),
                ("closed_param", ctypes.POINTER(ctypes.c_float)),
                ("sm_scale", ctypes.c_float),
                ("workspace", ctypes.c_void_p),
                ("workspace_bytes", ctypes.c_int64),
                ("flash_qtiles", ctypes.c_int32),
                ("scan_spin_limit", ctypes.c_int32),
                ("decomp_unsplit", ctypes.c_int32)]


_lib = None


def available():
    """True if libsafattn.so has been built next to this module."""
    return os.path.exists(LIB_PATH)


def lib():
    """The loaded library (loaded once per process)."""
    global _lib
    if _lib is None:
        if not available():
            raise RuntimeError(
                f"{LIB_NAME} is not built ({LIB_PATH} missing): run "
                "__graft_entry__.build() (or build_ext.build()) first; the SAF "
                "operators have no non-HIP fallback")
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.POINTER
        for name in ("saf_mixed_attn_fwd", "saf_mixed_attn_fwd_noalloc", "saf_flash_fwd", "saf_frozen_dense_pv_fwd",
                     "saf_frozen_decomp_fwd", "saf_frozen_scan_fwd"):
            fn = getattr(L, name)
            fn.argtypes = [P(SafMixedAttnArgs), ctypes.c_void_p]
            fn.restype = ctypes.c_int
        L.saf_mixed_attn_bwd.argtypes = [P(SafMixedAttnArgs)] + [P(SafTensor)] * 4 + [ctypes.c_void_p]
        L.saf_mixed_attn_bwd.restype = ctypes.c_int
        L.saf_mixed_attn_bwd_workspace_bytes.argtypes = [P(SafMixedAttnArgs)]
        L.saf_mixed_attn_bwd_workspace_bytes.restype = ctypes.c_int64
        L.saf_decomp_param_bwd.argtypes = [P(SafMixedAttnArgs)] + [P(SafTensor)] * 3 + [ctypes.c_void_p]
        L.saf_decomp_param_bwd.restype = ctypes.c_int
        L.saf_decomp_param_bwd_workspace_bytes.argtypes = [P(SafMixedAttnArgs)]
        L.saf_decomp_param_bwd_workspace_bytes.restype = ctypes.c_int64
        L.saf_frozen_pv_fwd.argtypes = [P(SafTensor), P(SafTensor), P(ctypes.c_int32),
                                        ctypes.c_int32, ctypes.c_int32, P(SafTensor),
                                        ctypes.c_void_p]
        L.saf_frozen_pv_fwd.restype = ctypes.c_int
        L.saf_frozen_pv_bwd.argtypes = L.saf_frozen_pv_fwd.argtypes
        L.saf_frozen_pv_bwd.restype = ctypes.c_int
        L.saf_rope_qk_inplace.argtypes = [P(SafTensor)] * 4 + [ctypes.c_void_p]
        L.saf_rope_qk_inplace.restype = ctypes.c_int
        L.saf_qk_rmsnorm_rope_inplace.argtypes = [P(SafTensor)] * 4 + [ctypes.c_float] + \
            [P(SafTensor)] * 2 + [ctypes.c_void_p]
        L.saf_qk_rmsnorm_rope_inplace.restype = ctypes.c_int
        L.saf_add_layernorm.argtypes = [P(SafTensor)] * 4 + [ctypes.c_float, P(SafTensor), ctypes.c_void_p]
        L.saf_add_layernorm.restype = ctypes.c_int
        L.saf_add_rmsnorm.argtypes = [P(SafTensor)] * 3 + [ctypes.c_float, P(SafTensor), ctypes.c_void_p]
        L.saf_add_rmsnorm.restype = ctypes.c_int
        L.saf_linear_gelu.argtypes = [P(SafTensor)] * 3 + [ctypes.c_void_p]
        L.saf_linear_gelu.restype = ctypes.c_int
        L.saf_gelu_inplace.argtypes = [P(SafTensor), ctypes.c_void_p]
        L.saf_gelu_inplace.restype = ctypes.c_int
        L.saf_linear_swiglu.argtypes = [P(SafTensor)] * 3 + [ctypes.c_void_p]
        L.saf_linear_swiglu.restype = ctypes.c_int
        L.saf_linear_rope.argtypes = [P(SafTensor)] * 3 + [ctypes.c_int32] * 3 + [P(SafTensor)] * 2 + [ctypes.c_void_p]
        L.saf_linear_rope.restype = ctypes.c_int
        L.saf_decomposed_logz.argtypes = [P(SafTensor)] * 3 + [ctypes.c_void_p]
        L.saf_decomposed_logz.restype = ctypes.c_int
        L.saf_decomposed_logz_bwd.argtypes = [P(SafTensor)] * 6 + [ctypes.c_void_p]
        L.saf_decomposed_logz_bwd.restype = ctypes.c_int
        L.saf_workspace_bytes.argtypes = [ctypes.c_int32] * 4
        L.saf_workspace_bytes.restype = ctypes.c_int64
        L.saf_mixed_attn_workspace_bytes.argtypes = [P(SafMixedAttnArgs)]
        L.saf_mixed_attn_workspace_bytes.restype = ctypes.c_int64
        L.saf_workspace_error.argtypes = [ctypes.c_void_p, ctypes.c_void_p, P(ctypes.c_int32)]
        L.saf_workspace_error.restype = ctypes.c_int
        L.saf_time_next_kernel.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        L.saf_time_next_kernel.restype = ctypes.c_int
        L.saf_last_error.argtypes = []
        L.saf_last_error.restype = ctypes.c_char_p
        L.saf_version.argtypes = []
        L.saf_version.restype = ctypes.c_char_p
        _lib = L
    return _lib


def tensor_desc(t):
    """saf_tensor_t for a torch tensor (None -> an absent descriptor)."""
    d = SafTensor()
    if t is None:
        return d
    if t.dim() > 4:
        raise ValueError("SAF tensors have at most 4 dimensions")
    if t.dtype not in _DTYPE_CODE:
        raise NotImplementedError(f"unsupported dtype {t.dtype}")
    d.data = t.data_ptr()
    d.dtype = _DTYPE_CODE[t.dtype]
    d.ndim = t.dim()
    for i, (s, st) in enumerate(zip(t.shape, t.stride())):
        d.size[i] = s
        d.stride[i] = st
    return d


def check(rc):
    """Raise the Python exception matching a C-ABI status."""
    if rc == SAF_OK:
        return
    msg = lib().saf_last_error().decode(errors="replace")
    if rc == SAF_EUNSUPPORTED:
        raise NotImplementedError(msg)
    if rc in (SAF_EINVAL, SAF_EALIGN, SAF_EWORKSPACE):
        raise ValueError(msg)
    raise RuntimeError(msg)


def host_i32(values):
    """ctypes int32 array from a host sequence / numpy array (None passes)."""
    if values is None:
        return None
    arr = (ctypes.c_int32 * len(values))(*[int(x) for x in values])
    return arr


def host_f32(values):
    if values is None:
        return None
    return (ctypes.c_float * len(values))(*[float(x) for x in values])


def current_stream_ptr(device):
    return torch.cuda.current_stream(device).cuda_stream
