"""ctypes binding of libvmonarch_gfx950.so (the C ABI declared in include/vmonarch_amd.h).

torch is imported before the library is loaded so that the process has one HIP runtime:
the library asks for libamdhip64.so.7 by soname and the dynamic loader hands it the copy torch
already mapped.  There is no fallback: if the library is missing or does not load, every call
raises.
"""
import ctypes
import os
import threading

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libvmonarch_gfx950.so")
ABI_VERSION = 13
FEA_FWD_SCRATCH_BYTES = 32 << 20   # VMO_FEA_FWD_SCRATCH_BYTES: scratch of vmo_fea_fwd_noalloc per GPU
DTYPES = {torch.bfloat16: 0, torch.float16: 1}

c_int32, c_int64, c_float, c_void_p, c_size_t = ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p, ctypes.c_size_t


class View(ctypes.Structure):
    _fields_ = [("data", c_void_p), ("stride_b", c_int64), ("stride_h", c_int64), ("stride_n", c_int64)]


class FeaFwdArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", c_int32), ("batch", c_int32), ("heads", c_int32), ("frames", c_int32),
        ("nq", c_int32), ("nk", c_int32), ("d", c_int32), ("dw0", c_int32), ("dw1", c_int32),
        ("q", View), ("k", View), ("w0", View), ("w1", View), ("o", View),
        ("lse", c_void_p), ("ent", c_void_p), ("stat_stride_b", c_int64), ("stat_stride_h", c_int64),
        ("sm_scale", c_float), ("num_splits", c_int32), ("workspace", c_void_p), ("workspace_bytes", c_size_t),
        ("qk_fp8", c_int32),
    ]


class FeaBwdArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", c_int32), ("batch", c_int32), ("heads", c_int32),
        ("nq", c_int32), ("nk", c_int32), ("d", c_int32), ("dv", c_int32),
        ("q", View), ("k", View), ("v", View), ("o", View), ("grad_o", View),
        ("grad_q", View), ("grad_k", View), ("grad_v", View),
        ("lse", c_void_p), ("ent", c_void_p), ("grad_ent", c_void_p),
        ("stat_stride_b", c_int64), ("stat_stride_h", c_int64),
        ("grad_ent_stride_b", c_int64), ("grad_ent_stride_h", c_int64),
        ("sm_scale", c_float), ("workspace", c_void_p), ("workspace_bytes", c_size_t), ("flags", c_int32),
        ("v1", View), ("dv1", c_int32), ("grad_k_base", View), ("grad_v_base", View), ("frames", c_int32),
        ("grad_q_base", View), ("delta", c_void_p), ("delta_stride_b", c_int64), ("delta_stride_h", c_int64),
    ]


BWD_ACCUM_Q, BWD_ACCUM_K, BWD_ACCUM_V = 1, 2, 4
BWD_F32_Q, BWD_F32_K, BWD_F32_V = 8, 16, 32
BWD_FOLD_K = 64   # values k or [k | v1]: k's value-role gradient into grad_k, grad_v holds v1's
BWD_SUM_K, BWD_SUM_V = 128, 256   # grad (dtype) = fp32 base + this call's gradient
BWD_RECOMPUTE_DQ, BWD_DS_DQ = 512, 1024   # grad_q route: recompute S and dP / GEMM over a stored dS^T
BWD_SUM_Q = 2048   # grad_q (dtype) = fp32 base + this call's gradient
LSTEP_BWD_OVERWRITE_Q = 1


class LstepArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", c_int32), ("batch", c_int32), ("heads", c_int32), ("num_blocks", c_int32),
        ("block_size", c_int32), ("d", c_int32), ("dv", c_int32), ("last", c_int32), ("skip_tokens", c_int32),
        ("q", View), ("out", View), ("ent", c_void_p), ("ent_stride_b", c_int64), ("ent_stride_h", c_int64),
        ("res", View), ("scale", c_float), ("min_col_mass", c_float),
    ]


class LstepBwdArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", c_int32), ("batch", c_int32), ("heads", c_int32), ("num_blocks", c_int32),
        ("block_size", c_int32), ("d", c_int32), ("dv", c_int32), ("last", c_int32), ("skip_tokens", c_int32),
        ("q", View), ("out", View), ("ent", c_void_p), ("ent_stride_b", c_int64), ("ent_stride_h", c_int64),
        ("grad_res", View), ("grad_q", View), ("grad_out", View), ("scale", c_float), ("min_col_mass", c_float),
        ("flags", c_int32), ("delta", c_void_p), ("delta_stride_b", c_int64), ("delta_stride_h", c_int64),
    ]


_lock = threading.Lock()
_lib = None


def lib():
    """The loaded library (loaded once; raises if it is missing or from another ABI)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"vmonarch_amd: {LIB_PATH} is not built (run `python -m vmonarch_amd.build`)")
        L = ctypes.CDLL(LIB_PATH)
        L.vmo_abi_version.restype = ctypes.c_int
        L.vmo_last_error.restype = ctypes.c_char_p
        L.vmo_fea_fwd_workspace_size.restype = c_size_t
        L.vmo_fea_fwd_workspace_size.argtypes = [ctypes.POINTER(FeaFwdArgs)]
        L.vmo_fea_fwd.restype = ctypes.c_int
        L.vmo_fea_fwd.argtypes = [ctypes.POINTER(FeaFwdArgs), c_void_p]
        L.vmo_fea_fwd_noalloc.restype = ctypes.c_int
        L.vmo_fea_fwd_noalloc.argtypes = [ctypes.POINTER(FeaFwdArgs), c_void_p]
        L.vmo_lstep_fwd.restype = ctypes.c_int
        L.vmo_lstep_fwd.argtypes = [ctypes.POINTER(LstepArgs), c_void_p]
        L.vmo_lstep_bwd.restype = ctypes.c_int
        L.vmo_lstep_bwd.argtypes = [ctypes.POINTER(LstepBwdArgs), c_void_p]
        L.vmo_fea_bwd_workspace_size.restype = c_size_t
        L.vmo_fea_bwd_workspace_size.argtypes = [ctypes.POINTER(FeaBwdArgs)]
        L.vmo_fea_bwd.restype = ctypes.c_int
        L.vmo_fea_bwd.argtypes = [ctypes.POINTER(FeaBwdArgs), c_void_p]
        v = L.vmo_abi_version()
        if v != ABI_VERSION:
            raise RuntimeError(f"vmonarch_amd: library ABI {v}, bindings expect {ABI_VERSION}")
        _lib = L
        return L


def check(rc, what):
    if rc != 0:
        msg = lib().vmo_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (code {rc}): {msg}")


def view(t):
    """(B, H, N, F) tensor -> View (element strides, feature dim contiguous)."""
    assert t.dim() == 4 and t.stride(3) == 1, "feature dimension must be contiguous"
    return View(t.data_ptr(), t.stride(0), t.stride(1), t.stride(2))


def row_aligned(t):
    """t itself when its rows are 16-byte aligned with a contiguous feature dim, else a contiguous copy."""
    ok = (t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and all(s % 8 == 0 for s in t.stride()[:-1]))
    return t if ok else t.contiguous()


def layout_order(t):
    """Order of t's (B, H, N) dims in memory, outermost first (by stride)."""
    return tuple(sorted(range(3), key=lambda d: (-t.stride(d), d)))


def empty_in_order(order, shape3, feat, dtype, device):
    """An uninitialised (B, H, N, feat) tensor whose (B, H, N) dims lie in memory in `order`, feature dim
    innermost."""
    buf = torch.empty([shape3[d] for d in order] + [feat], device=device, dtype=dtype)
    return buf.permute(*[order.index(d) for d in range(3)], 3)


def empty_in_layout(ref, feat, dtype):
    """An uninitialised (B, H, N, feat) tensor laid out like ref: for q given as a (B, N, H, D) buffer
    viewed as (B, H, N, D) (a DiT block's layout) the result is a (B, N, H, feat) buffer viewed the same
    way, so the caller needs no permute copy afterwards."""
    return empty_in_order(layout_order(ref), ref.shape[:3], feat, dtype, ref.device)


def stream_of(t):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)
