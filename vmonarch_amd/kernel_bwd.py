"""Backward of the flash-entropy attention through the C ABI (vmo_fea_bwd).

Mirrors _FlashEntropyAttention.backward of the reference (kernel.py:360-381): given the saved
q, k, v, o, lse, ent and the upstream grads (do, de) it returns (dq, dk, dv) in q.dtype.  Rows
>= n_valid are padding: their gradients are zero.
"""
import torch

from . import _lib


def _pad_features(t, width):
    return t if t.shape[-1] == width else torch.nn.functional.pad(t, (0, width - t.shape[-1]))


def fea_backward_raw(q, k, v, o, lse, ent, do, de, sm_scale, dq=None, dk=None, dv=None, overwrite="", v1=None,
                     fold_k=False, dk_base=None, dv_base=None, frames=1, dq_route=None, dq_base=None, delta=None):
    """q: (B, H, F*nq, D); k: (B, H, F*nk, D); v: (B, H, F*nk, Dv); o, do: (B, H, F*nq, Dv);
    lse, ent, de: (B, H, F*nq) fp32 with unit token stride.  Returns (dq, dk, dv).

    `frames` = F splits every (b, h) into F independent problems of nq queries and nk keys (frame f:
    rows [f nq, (f + 1) nq) and [f nk, (f + 1) nk)), read in place whatever the memory order.

    With `v1` (same shape and strides as v) the values are [v | v1], 2 Dv wide, read in place.

    A gradient passed in as a float32 view is accumulated into (+= in the kernels), or overwritten
    when its letter ("q", "k", "v") is in `overwrite`; one passed in q's dtype (a 16-bit view, any
    strides with a contiguous feature dim) is written; one not passed is returned as a new tensor of
    q's dtype.

    `fold_k` (v is k, as the VMonarch R-steps pass it): dk receives k's whole gradient, as key and
    as the first value columns, and dv only v1's (None without v1).

    `dq_base` / `dk_base` / `dv_base` (float32, shaped like dq / dk / dv): dq / dk / dv, in q's dtype, are
    that base plus this call's gradient (the last of several calls summing one gradient).

    `delta` ((B, H, F*nq) fp32, unit token stride): rowsum(o * do) when the caller has it (the L-step
    backward forms it); otherwise the kernels form it from o and do.

    `dq_route` ("recompute" or "ds"; None lets the library choose) picks how dq is formed: a pass that
    recomputes S and dP, or a GEMM over dS^T stored by the dk / dv pass (the workspace then holds nk x nq
    16-bit values per problem)."""
    L = _lib.lib()
    B, H, NQ, D = q.shape
    NK, Dv = k.shape[2], v.shape[-1] * (2 if v1 is not None else 1)
    flags = (_lib.BWD_FOLD_K if fold_k else 0) | {None: 0, "recompute": _lib.BWD_RECOMPUTE_DQ,
                                                   "ds": _lib.BWD_DS_DQ}[dq_route]
    for t, name, acc_bit, f32_bit, base in ((dq, "q", _lib.BWD_ACCUM_Q, _lib.BWD_F32_Q, dq_base),
                                            (dk, "k", _lib.BWD_ACCUM_K, _lib.BWD_F32_K, dk_base),
                                            (dv, "v", _lib.BWD_ACCUM_V, _lib.BWD_F32_V, dv_base)):
        if base is not None:
            assert base.dtype == torch.float32 and (t is None or t.dtype == q.dtype), "base fp32, result q.dtype"
            flags |= {"q": _lib.BWD_SUM_Q, "k": _lib.BWD_SUM_K, "v": _lib.BWD_SUM_V}[name]
        elif t is not None and t.dtype != q.dtype:
            assert t.dtype == torch.float32, "a gradient passed in must be float32 or q's dtype"
            flags |= f32_bit if name in overwrite else acc_bit
    if dq is None:
        dq = torch.empty((B, H, NQ, D), device=q.device, dtype=q.dtype)
    if dk is None:
        dk = torch.empty((B, H, NK, D), device=q.device, dtype=q.dtype)
    if dv is None and not (fold_k and v1 is None):
        dv = torch.empty((B, H, NK, v1.shape[-1] if fold_k else Dv), device=q.device, dtype=q.dtype)
    a = _lib.FeaBwdArgs()
    a.flags = flags
    a.dtype = _lib.DTYPES[q.dtype]
    assert NQ % frames == 0 and NK % frames == 0
    a.batch, a.heads, a.nq, a.nk, a.d, a.dv = B, H, NQ // frames, NK // frames, D, Dv
    a.frames = frames
    a.q, a.k, a.v, a.o, a.grad_o = (_lib.view(t) for t in (q, k, v, o, do))
    a.grad_q, a.grad_k = _lib.view(dq), _lib.view(dk)
    a.grad_v = _lib.view(dv) if dv is not None else _lib.View()
    if dq_base is not None:
        assert dq_base.shape == dq.shape
        a.grad_q_base = _lib.view(dq_base)
    if dk_base is not None:
        assert dk_base.shape == dk.shape
        a.grad_k_base = _lib.view(dk_base)
    if dv_base is not None:
        assert dv_base.shape == dv.shape
        a.grad_v_base = _lib.view(dv_base)
    assert lse.stride() == ent.stride() and lse.stride(2) == 1 and de.stride(2) == 1
    a.lse, a.ent, a.grad_ent = lse.data_ptr(), ent.data_ptr(), de.data_ptr()
    a.stat_stride_b, a.stat_stride_h = lse.stride(0), lse.stride(1)
    a.grad_ent_stride_b, a.grad_ent_stride_h = de.stride(0), de.stride(1)
    a.sm_scale = float(sm_scale)
    if v1 is not None:
        assert v1.shape == v.shape and v1.stride() == v.stride() and v1.dtype == v.dtype
        a.v1, a.dv1 = _lib.view(v1), v1.shape[-1]
    if delta is not None:
        assert delta.dtype == torch.float32 and delta.stride(2) == 1
        a.delta, a.delta_stride_b, a.delta_stride_h = delta.data_ptr(), delta.stride(0), delta.stride(1)
    nbytes = L.vmo_fea_bwd_workspace_size(a)
    ws = torch.empty(nbytes, device=q.device, dtype=torch.uint8)
    a.workspace, a.workspace_bytes = ws.data_ptr(), nbytes
    _lib.check(L.vmo_fea_bwd(a, _lib.stream_of(q)), "vmo_fea_bwd")
    return dq, dk, dv


def fea_backward(q, k, v, o, lse, ent, do, de, sm_scale, n_valid):
    B, H, N, D = q.shape
    Dv = v.shape[-1]
    n = int(n_valid)
    from .kernel import _kernel_widths
    Dk, Dvk = _kernel_widths(D, Dv)
    if not ((Dk in (32, 64, 128) and Dvk in (32, 64, 128, 256)) or (Dk == 16 and Dvk in (16, 32, 64, 128, 256))
            or (Dk == 256 and Dvk == 256)):
        raise NotImplementedError(f"vmonarch_amd: backward for head dims ({D}, {Dv}) is not built")
    if de is None:
        de = torch.zeros((B, H, N), device=q.device, dtype=torch.float32)
    if do is None:
        do = torch.zeros_like(o)
    do = do.to(q.dtype)
    de = de.float()
    if de.stride(2) != 1:
        de = de.contiguous()
    if n == N and Dk == D and Dvk == Dv:
        # no padding rows, no padded features: the kernels write the gradients once, in the memory order
        # of the caller's q, k, v (a DiT block's (B, N, H, D) buffers need no copy afterwards)
        grads = [_lib.empty_in_layout(t, t.shape[-1], q.dtype) for t in (q, k, v)]
        args = [_lib.row_aligned(t) for t in (q, k, v, o, do)]
        fea_backward_raw(*args[:4], lse, ent, args[4], de, sm_scale, dq=grads[0], dk=grads[1], dv=grads[2])
        return tuple(grads)
    dq = torch.zeros_like(q)
    dk = torch.zeros_like(k)
    dv = torch.zeros_like(v)
    if n == 0:
        return dq, dk, dv
    sl = slice(0, n)
    qx, kx = (_lib.row_aligned(_pad_features(t[:, :, sl], Dk)) for t in (q, k))
    vx, ox, dox = (_lib.row_aligned(_pad_features(t[:, :, sl], Dvk)) for t in (v, o, do))
    lse_x, ent_x = lse[:, :, sl], ent[:, :, sl]
    de_x = de[:, :, sl]
    gq, gk, gv = fea_backward_raw(qx, kx, vx, ox, lse_x, ent_x, dox, de_x, sm_scale)
    dq[:, :, sl] = gq[..., :D]
    dk[:, :, sl] = gk[..., :D]
    dv[:, :, sl] = gv[..., :Dv]
    return dq, dk, dv
