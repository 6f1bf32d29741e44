"""FlashEntropyAttention: attention that also returns the entropy of every attention row.

Drop-in for video_monarch_attention/kernel.py (reference).  Same public function and autograd
contract; the body calls the gfx950 HIP kernels through the C ABI (vmonarch_amd/_lib.py).

Differences from the reference that callers can observe: none in values (within bf16
tolerance).  Internally there is no padding to a multiple of 128 (kernel.py:399-400): tails are
masked in the kernel, so no padded copies of q / k / v are made.
"""
import torch

from . import _lib

SEQ_ALIGN = 128  # kept for API parity with the reference (kernel.py:12); no padding happens
_HEAD_DIMS = {16, 32, 64, 128, 256}  # accepted by the reference (kernel.py:324)


def _pad_features(t, width):
    """Zero-pad the feature dim to `width` (a zero feature changes neither q.k nor P.v)."""
    if t.shape[-1] == width:
        return t
    return torch.nn.functional.pad(t, (0, width - t.shape[-1]))


def _kernel_widths(d, dv):
    """Head dims of the flash-entropy kernels (forward and backward) that serve (d, dv): every pair the reference
    accepts (dv a multiple of d) as it is, 16-wide heads included (their kernels hold 16-wide rows in 32-wide LDS
    tiles); a 16-wide value head under wider q / k (beyond the reference) runs 32 wide, zero-padded."""
    return d, (32 if dv < 32 <= d else dv)


def fea_forward(q, k, w0, w1, sm_scale, frames=1, o=None, lse=None, ent=None, want_ent=True, want_lse=True,
                num_splits=1, qk_fp8=False):
    """Launch the flash-entropy forward.

    q: (B, H, F*nq, D); k, w0: (B, H, F*nk, .); w1: optional second value tensor (requires w0 is k).
    Returns (o, lse, ent): o (B, H, F*nq, Dw0 + Dw1) in q.dtype; lse (log2 units) and ent (nats)
    (B, H, F*nq) fp32, or None when not wanted.  o / lse / ent may be passed in as (strided) views
    to write into; lse / ent views need a unit token stride.  `qk_fp8`: S = q k^T in fp8 (the VMonarch
    R-step variants only; vmo_fea_fwd_args.qk_fp8).
    """
    L = _lib.lib()
    B, H, NQ, D = q.shape
    NK = k.shape[2]
    assert NQ % frames == 0 and NK % frames == 0
    dw0 = w0.shape[-1]
    dw1 = 0 if w1 is None else w1.shape[-1]
    dev = q.device
    if o is None:
        o = torch.empty((B, H, NQ, dw0 + dw1), device=dev, dtype=q.dtype)
    if lse is None and want_lse:
        lse = torch.empty((B, H, NQ), device=dev, dtype=torch.float32)
    if ent is None and want_ent:
        ent = torch.empty((B, H, NQ), device=dev, dtype=torch.float32)
    st = lse if lse is not None else ent
    if lse is not None and ent is not None:
        assert lse.stride()[:2] == ent.stride()[:2]
    a = _lib.FeaFwdArgs()
    a.dtype = _lib.DTYPES[q.dtype]
    a.batch, a.heads, a.frames = B, H, frames
    a.nq, a.nk = NQ // frames, NK // frames
    a.d, a.dw0, a.dw1 = D, dw0, dw1
    a.q, a.k, a.w0, a.o = _lib.view(q), _lib.view(k), _lib.view(w0), _lib.view(o)
    a.w1 = _lib.view(w1) if w1 is not None else _lib.View(0, 0, 0, 0)
    a.lse = lse.data_ptr() if lse is not None else None
    a.ent = ent.data_ptr() if ent is not None else None
    if st is not None:
        assert st.stride(2) == 1
        a.stat_stride_b, a.stat_stride_h = st.stride(0), st.stride(1)
    a.sm_scale = float(sm_scale)
    a.num_splits = int(num_splits)
    a.qk_fp8 = int(bool(qk_fp8))
    ws = None
    nbytes = L.vmo_fea_fwd_workspace_size(a)
    if nbytes:
        ws = torch.empty(nbytes, device=dev, dtype=torch.uint8)
        a.workspace, a.workspace_bytes = ws.data_ptr(), nbytes
    _lib.check(L.vmo_fea_fwd(a, _lib.stream_of(q)), "vmo_fea_fwd")
    return o, lse, ent


class _FlashEntropyAttention(torch.autograd.Function):
    """Autograd contract of the reference (kernel.py:316-381):
    forward(ctx, q, k, v, sm_scale, n_valid, warp_specialize) -> (o, E);
    backward(ctx, do, de) -> (dq, dk, dv, None, None, None).
    Rows >= n_valid are padding: they are masked as keys and their outputs are zero
    (kernel.py:352-353)."""

    @staticmethod
    def forward(ctx, q, k, v, sm_scale, n_valid, warp_specialize):
        B, H, N, D = q.shape
        Dv = v.shape[-1]
        assert q.dtype in _lib.DTYPES, f"unsupported dtype {q.dtype}"
        assert k.shape == q.shape and v.shape[:-1] == q.shape[:-1]
        assert D in _HEAD_DIMS and Dv in _HEAD_DIMS
        if D == 256 and Dv != 256:
            raise NotImplementedError("vmonarch_amd: head dim 256 for q/k is built with 256-wide values only")
        if not q.is_cuda:
            raise RuntimeError("vmonarch_amd: flash_entropy_attention needs GPU tensors (no CPU path)")
        n = int(n_valid)
        Dk, Dvk = _kernel_widths(D, Dv)
        qx, kx, vx = (_lib.row_aligned(_pad_features(t[:, :, :n], w)) for t, w in ((q, Dk), (k, Dk), (v, Dvk)))
        ent = torch.empty((B, H, N), device=q.device, dtype=torch.float32)
        lse = torch.empty((B, H, N), device=q.device, dtype=torch.float32)
        if Dvk == Dv:
            o = _lib.empty_in_layout(q, Dv, q.dtype)   # o in the caller's layout (e.g. (B, N, H, Dv))
            if n > 0:
                fea_forward(qx, kx, vx, None, sm_scale, o=o[:, :, :n], lse=lse[:, :, :n], ent=ent[:, :, :n])
        else:
            o_k = torch.empty((B, H, N, Dvk), device=q.device, dtype=q.dtype)
            if n > 0:
                fea_forward(qx, kx, vx, None, sm_scale, o=o_k[:, :, :n], lse=lse[:, :, :n], ent=ent[:, :, :n])
            o = _lib.empty_in_layout(q, Dv, q.dtype).copy_(o_k[..., :Dv])   # the caller's layout, as above
        if n < N:   # padding rows (kernel.py:352-353)
            o[:, :, n:] = 0
            ent[:, :, n:] = 0
            lse[:, :, n:] = 0
        ctx.save_for_backward(q, k, v, o, lse, ent)
        ctx.sm_scale = sm_scale
        ctx.n_valid = n
        return o, ent

    @staticmethod
    def backward(ctx, do, de):
        from .kernel_bwd import fea_backward
        q, k, v, o, lse, ent = ctx.saved_tensors
        dq, dk, dv = fea_backward(q, k, v, o, lse, ent, do, de, ctx.sm_scale, ctx.n_valid)
        return dq, dk, dv, None, None, None


def flash_entropy_attention(q, k, v, sm_scale=None, warp_specialize=True):
    """
    Non-causal attention that also returns the entropy of every attention row
    (reference: kernel.py:384-402; `warp_specialize` is accepted and ignored).

    Args:
        q, k: (B, H, N, D)
        v: (B, H, N, Dv)
        sm_scale: softmax scale, defaults to 1 / sqrt(D)
    Returns:
        o: (B, H, N, Dv) = softmax(sm_scale * q k^T) v, in q.dtype
        e: (B, H, N) float32, e_i = -sum_j P_ij log P_ij
    """
    n = q.shape[-2]
    if sm_scale is None:
        sm_scale = q.shape[-1] ** -0.5
    return _FlashEntropyAttention.apply(q, k, v, sm_scale, n, warp_specialize)
