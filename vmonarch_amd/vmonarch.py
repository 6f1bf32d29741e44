"""
VMonarch attention (drop-in for video_monarch_attention/vmonarch.py of the reference).

The N = m * b tokens are laid out on an (m, b) grid, token n -> (n // b, n % b).  The attention
map is approximated by a Monarch matrix built from
  - R: m dense (b x b) blocks, mixing tokens inside each grid row (a batched flash-entropy
    attention, the R-step);
  - L: b dense (m x m) blocks, mixing tokens inside each grid column (the L-step);
fitted by a few steps of alternating minimisation (reference: vmonarch.py:1-11, :29-69).

Execution paths, with identical results within bf16 tolerance:
  * fused (forward without autograd): every step is a gfx950 HIP kernel -- the R-step reads the
    (B, H, m*b, D) tensors in place as m frames per head (no flatten copy, no torch.cat of
    [k | v]), the L-step is one fused kernel per iteration (one MFMA tile per grid column for
    m <= 32, a general kernel beyond), and the recompute of the first tokens is a split-KV flash
    kernel writing straight into z;
  * _VMonarchFunction (autograd): the same forward keeping its activations, and a HIP backward;
  * head-dim mixes the kernels do not take as they are (16 with 32; D != Dv with autograd; neither
    is a shape the reference's VMonarch runs) run either of the above on q, k, v zero-padded to one
    kernel width;
  * composed: the reference's structure step by step (R-step through the `_row_block_attention`
    seam, L-step as torch tensor ops), used when a caller replaced `_row_block_attention`
    (tests/test_vmonarch.py:59 does), and -- with a RuntimeWarning -- for shapes no HIP path takes.
"""
import warnings

import torch
import torch.nn as nn

from . import _lib
from .kernel import fea_forward, flash_entropy_attention
from .kernel_bwd import fea_backward_raw

# number of CUs on an MI355X; the recompute picks its split-KV count to fill them
_NUM_CUS = 256


def _row_block_attention(x, k, w):
    """Attention inside every grid row (reference vmonarch.py:19-26).

    x, k: (B, H, m, b, D); w: (B, H, m, b, Dw).
    Returns softmax(x k^T) w and sum_j P_ij log P_ij (= -entropy) for every row of P.
    """
    out, ent = flash_entropy_attention(*(t.flatten(1, 2) for t in (x, k, w)), sm_scale=1.0)
    return out.view(*w.shape[:-1], -1), -ent.view(x.shape[:-1]).detach()


_ROW_BLOCK_ATTENTION = _row_block_attention   # the seam as shipped; patched seams use the composed path


def _recompute_splits(problems, nq, nk):
    """Key splits of the recompute: the fewest that fill ~80% of one round of workgroup slots (two 128-query
    workgroups per CU), each split keeping >= 512 keys.  Fewer splits write fewer fp32 partials; a split count
    whose workgroups spill a little into another round leaves that round mostly idle (measured at cfg4, 156
    query tiles: 3 splits 0.300 ms, 8 splits 0.309 ms, 16 splits 0.336 ms)."""
    base = problems * ((nq + 127) // 128)
    want = -(-int(0.8 * 2 * _NUM_CUS) // base)
    return max(1, min(16, want, nk // 512))


def _lstep_launch(q, out, ent, res, m, b, scale, last, skip, min_col_mass):
    L = _lib.lib()
    B, H, N, D = q.shape
    a = _lib.LstepArgs()
    a.dtype = _lib.DTYPES[q.dtype]
    a.batch, a.heads, a.num_blocks, a.block_size = B, H, m, b
    a.d = D
    a.dv = out.shape[-1] - D if last else 0
    a.last, a.skip_tokens = int(last), int(skip)
    a.q, a.out, a.res = _lib.view(q), _lib.view(out), _lib.view(res)
    a.ent = ent.data_ptr()
    a.ent_stride_b, a.ent_stride_h = ent.stride(0), ent.stride(1)
    a.scale, a.min_col_mass = float(scale), float(min_col_mass)
    _lib.check(L.vmo_lstep_fwd(a, _lib.stream_of(q)), "vmo_lstep_fwd")


def _lstep_one_tile(m, d, dv, last):
    """Whether the one-tile L-step kernels take this grid (csrc/lstep.hip one_tile_built)."""
    return m <= 32 and d in (64, 128) and (not last or dv in (64, 128))


def _lstep_bwd_launch(q, out, ent, grad_res, grad_q, grad_out, m, b, scale, last, skip, min_col_mass,
                      overwrite_q=False, delta=None):
    """Backward of one L-step (vmo_lstep_bwd): grad_q (fp32) += dL/dq (= with overwrite_q),
    grad_out = dL/d out; with `delta` ((B, H, N) fp32, one-tile grids only) also rowsum(out * grad_out)."""
    L = _lib.lib()
    B, H, N, D = q.shape
    a = _lib.LstepBwdArgs()
    a.dtype = _lib.DTYPES[q.dtype]
    a.batch, a.heads, a.num_blocks, a.block_size = B, H, m, b
    a.d = D
    a.dv = out.shape[-1] - D if last else 0
    a.last, a.skip_tokens = int(last), int(skip)
    a.q, a.out, a.grad_res = _lib.view(q), _lib.view(out), _lib.view(grad_res)
    a.grad_q, a.grad_out = _lib.view(grad_q), _lib.view(grad_out)
    a.ent = ent.data_ptr()
    a.ent_stride_b, a.ent_stride_h = ent.stride(0), ent.stride(1)
    a.scale, a.min_col_mass = float(scale), float(min_col_mass)
    a.flags = _lib.LSTEP_BWD_OVERWRITE_Q if overwrite_q else 0
    if delta is not None:
        assert delta.dtype == torch.float32 and delta.stride(2) == 1
        a.delta, a.delta_stride_b, a.delta_stride_h = delta.data_ptr(), delta.stride(0), delta.stride(1)
    _lib.check(L.vmo_lstep_bwd(a, _lib.stream_of(q)), "vmo_lstep_bwd")


_LDS_BYTES = 160 * 1024   # per CU on gfx950


def _lstep_general_lds(m, d, dv, last, bwd):
    """LDS bytes per grid column of the general L-step kernels (csrc/lstep.hip lw_layout): 16-bit rows of q,
    kr (and the upstream gradient, y) padded by 16 bytes, one or two fp32 m x (m + 1) matrices, 4 m floats."""
    r16 = lambda b: (b + 15) // 16 * 16   # noqa: E731
    ldq, ldy, ldm = d + 8, dv + 8, m + 1
    total = 2 * r16(m * ldq * 2) + r16(m * ldm * 4) + r16(4 * m * 4)
    if bwd:
        total += r16(m * (ldy if last else ldq) * 2) + r16(m * ldm * 4)
    if last:
        total += r16(m * ldy * 2)
    return total


_MB_MAX_FRAMES = 128
_MB_BWD = True    # the multi-block backward kernels


def _lstep_mb_lds(m, d, dv, last, bwd):
    """LDS bytes per grid column of the multi-block L-step kernels (csrc/lstep_mb.hip mb_layout with whole tiles):
    q and kr tiles (and y, and the upstream gradient) of M = 32 ceil(m / 32) 16-bit rows, M-float vectors, at least
    the four row-store patches.  (The two-block last step up to 40 frames stages compact tiles, which take less:
    this is the bound the host checks.)"""
    M = 32 * ((m + 31) // 32)
    r = lambda b: (b + 255) // 256 * 256   # noqa: E731
    d, dv = max(d, 32), max(dv, 32)   # 16-wide heads sit in 32-wide tiles
    total = 2 * r(M * d * 2) + (r(M * dv * 2) if last else 0) + 2 * r(M * 4) + r(4 * M * 4)
    if bwd:   # the upstream gradient rows, three more vectors, the backward's own row-store patches (half-size
        # ones for the last step up to 64 frames)
        total += r(M * (dv if last else d) * 2) + 3 * r(M * 4) + 4 * (2048 if last and M <= 64 else 4096)
    return max(total, 4 * 4096)


def _lstep_mb(m, d, dv, bwd):
    """Whether the multi-block MFMA L-step kernels take this grid: up to 128 frames, head dims 32 / 64 / 128 in
    any pair, or 16 / 16."""
    dims = (d in (32, 64, 128) and dv in (32, 64, 128)) or d == dv == 16
    return ((_MB_BWD or not bwd) and 1 <= m <= _MB_MAX_FRAMES and dims
            and all(_lstep_mb_lds(m, d, dv, last, bwd) <= _LDS_BYTES for last in (False, True)))


def _lstep_supported(m, d, dv, bwd):
    """Whether the HIP L-steps run this grid: the one-tile MFMA kernels (m <= 32, d and dv in {64, 128}), the
    multi-block MFMA kernels (m <= 128, head dims 32 / 64 / 128, or 16 / 16), or the general kernels (any m whose
    per-column tiles fit the LDS)."""
    if m <= 32 and d in (64, 128) and dv in (64, 128):
        return True
    if _lstep_mb(m, d, dv, bwd):
        return True
    return all(_lstep_general_lds(m, d, dv, last, bwd) <= _LDS_BYTES for last in (False, True))


def _fused_supported(q, k, v, num_blocks):
    D, Dv = q.shape[-1], v.shape[-1]
    # flash-entropy kernels at 64 / 128 (either dim), 32 / 32 or 16 / 16
    return (q.is_cuda and q.dtype in _lib.DTYPES and k.dtype == q.dtype and v.dtype == q.dtype
            and ((D in (64, 128) and Dv in (64, 128)) or D == Dv == 32 or D == Dv == 16)
            and _lstep_supported(num_blocks, D, Dv, False)
            and k.shape == q.shape and v.shape[:-1] == q.shape[:-1])


# Where the exact recompute of the first rt queries starts on its own stream: it reads q, k, v only
# and writes rows [0, rt) of z, which the L-steps never write, so it can run beside the R/L chain
# ("start": with R-step 0, "after_r0": beside L-step 0 onwards, "after_r1": beside the last L-step,
# "off": after the chain on the caller's stream).  Measured at cfg4 (four interleaved rounds of 100
# steps on one box): start 1.126-1.128 ms, after_r0 1.131-1.137 ms with the same 3 key splits.
_RECOMPUTE_OVERLAP = "start"
_side_streams = {}


def _side_stream(dev):
    s = _side_streams.get(dev)
    if s is None:
        s = _side_streams[dev] = torch.cuda.Stream(device=dev)   # default priority
    return s


def _vmonarch_fused(q, k, v, m, b, num_iters, recompute_tokens, min_col_mass, stage_hook=None, scale=None,
                    qk_fp8=False):
    """All-HIP forward.  `stage_hook(name, phase, stream)`, when given, is called on the host right
    before ("begin") and after ("end") each launch group ("rstep0", "lstep0", ..., "recompute") with
    the stream it goes to -- used by bench.py to bracket every kernel with events.  `scale` overrides
    D ** -0.5 (q / k zero-padded past their head dim).  `qk_fp8`: the R-steps' S in fp8 (the recompute
    stays exact)."""
    B, H, N, D = q.shape
    Dv = v.shape[-1]
    scale = D ** -0.5 if scale is None else scale
    q, k, v = (_lib.row_aligned(t) for t in (q, k, v))
    dev, dt = q.device, q.dtype
    main = torch.cuda.current_stream(dev)
    hook = stage_hook or (lambda name, phase, stream: None)
    ent = torch.empty((B, H, N), device=dev, dtype=torch.float32)
    z = _lib.empty_in_layout(q, Dv, dt)   # z in the caller's layout (a DiT block's (B, N, H, Dv))
    rt = min(int(recompute_tokens), N)
    side = None

    def recompute(stream):
        # exact attention for the first rt queries (vmonarch.py:66-68), written into z
        with torch.cuda.stream(stream):
            hook("recompute", "begin", stream)
            splits = _recompute_splits(B * H, rt, N)
            fea_forward(q[:, :, :rt], k, v, None, scale, o=z[:, :, :rt], want_ent=False, want_lse=False,
                        num_splits=splits)
            hook("recompute", "end", stream)

    def fork():
        nonlocal side
        side = _side_stream(dev)
        side.wait_stream(main)   # q, k, v and z are ready on the caller's stream
        recompute(side)

    if rt > 0 and _RECOMPUTE_OVERLAP == "start":
        fork()
    u = None
    for it in range(num_iters):
        last = it == num_iters - 1
        # R-step (vmonarch.py:50): iteration 0 folds u = q * scale into the softmax scale
        x, s = (q, scale) if it == 0 else (u, 1.0)
        hook(f"rstep{it}", "begin", main)
        out, _, _ = fea_forward(x, k, k, v if last else None, s, frames=m, ent=ent, want_lse=False, qk_fp8=qk_fp8)
        hook(f"rstep{it}", "end", main)
        if rt > 0 and side is None and ((_RECOMPUTE_OVERLAP == "after_r0" and it == 0) or
                                        (_RECOMPUTE_OVERLAP == "after_r1" and last)):
            fork()
        # L-step (vmonarch.py:51-63)
        hook(f"lstep{it}", "begin", main)
        if last:
            _lstep_launch(q, out, ent, z, m, b, scale, True, rt, min_col_mass)
        else:
            if u is None:
                u = torch.empty((B, H, N, D), device=dev, dtype=dt)
            _lstep_launch(q, out, ent, u, m, b, scale, False, 0, min_col_mass)
        hook(f"lstep{it}", "end", main)
    if rt > 0:
        if side is None:
            recompute(main)
        else:
            main.wait_stream(side)   # z is complete on the caller's stream
    return z


def _hip_backward_supported(q, k, v, num_blocks):
    # the last R-step's backward takes the values [k | v] as two equal halves of 64 or 128
    return (_fused_supported(q, k, v, num_blocks) and q.shape[-1] == v.shape[-1]
            and _lstep_supported(num_blocks, q.shape[-1], v.shape[-1], True))


class _VMonarchFunction(torch.autograd.Function):
    """VMonarch attention with a HIP backward (the gradient autograd takes through vmonarch.py:41-69).

    The forward is the all-HIP pipeline of _vmonarch_fused, keeping what the backward needs: every
    R-step's input u, output, LSE and entropy, and the recompute's LSE.  The backward walks the
    iterations in reverse, each as the fused L-step backward (vmo_lstep_bwd) and the R-step's
    flash-entropy backward (vmo_fea_bwd on the m frames of each head, values k or [k | v]; the
    entropy enters the L-step detached, vmonarch.py:26, so its gradient is zero), then the
    recompute rows through vmo_fea_bwd (rt queries against all N keys).  Gradients of q, k, v
    collect in fp32.
    """

    @staticmethod
    def forward(ctx, q, k, v, m, b, num_iters, recompute_tokens, min_col_mass, scale=None):
        B, H, N, D = q.shape
        Dv = v.shape[-1]
        scale = D ** -0.5 if scale is None else scale
        z = _lib.empty_in_layout(q, Dv, q.dtype)
        ctx.orders = tuple(_lib.layout_order(t) for t in (q, k, v))
        # read in place in any memory order (the backward, like the forward, takes each head's m frames
        # as m problems of the (B, H, m*b) tensors): no contiguous copies of a DiT block's (B, N, H, D)
        q, k, v = (_lib.row_aligned(t) for t in (q, k, v))
        if k.stride() != v.stride():   # the backward reads the values [k | v] as two parts with one set of strides
            k, v = k.contiguous(), v.contiguous()
        dev, dt = q.device, q.dtype
        rt = min(int(recompute_tokens), N)
        saved = []
        lse_rt = None
        main, side = torch.cuda.current_stream(dev), None

        def recompute():
            return fea_forward(q[:, :, :rt], k, v, None, scale, o=z[:, :, :rt], want_ent=False,
                               num_splits=_recompute_splits(B * H, rt, N))[1]

        if rt > 0 and _RECOMPUTE_OVERLAP != "off":
            # the exact recompute of rows [0, rt) beside the R/L chain, as in _vmonarch_fused (it reads q, k, v
            # only and writes rows of z that the last L-step leaves alone)
            side = _side_stream(dev)
            side.wait_stream(main)
            with torch.cuda.stream(side):
                lse_rt = recompute()
        u = None
        for it in range(num_iters):
            last = it == num_iters - 1
            x, s = (q, scale) if it == 0 else (u, 1.0)
            out, lse, ent = fea_forward(x, k, k, v if last else None, s, frames=m)
            if last:
                _lstep_launch(q, out, ent, z, m, b, scale, True, rt, min_col_mass)
            else:
                u = torch.empty((B, H, N, D), device=dev, dtype=dt)
                _lstep_launch(q, out, ent, u, m, b, scale, False, 0, min_col_mass)
            saved += [x, out, lse, ent]
        if side is not None:
            main.wait_stream(side)       # z and lse_rt are complete on the caller's stream
            lse_rt.record_stream(main)   # allocated on the side stream, read by the backward on this one
        elif rt > 0:
            lse_rt = recompute()
        ctx.dims = (m, b, num_iters, rt, float(min_col_mass), float(scale))
        ctx.save_for_backward(q, k, v, z, lse_rt if lse_rt is not None else z.new_empty(0), *saved)
        return z

    @staticmethod
    def backward(ctx, dz):
        m, b, num_iters, rt, min_col_mass, scale = ctx.dims
        q, k, v, z, lse_rt, *saved = ctx.saved_tensors
        B, H, N, D = q.shape
        Dv = v.shape[-1]
        dev, dt = q.device, q.dtype
        dz = _lib.row_aligned(dz.to(dt))
        f32 = torch.float32
        # Call order: the L- and R-step backwards from the last iteration down, R-step 0's last of all and the
        # recompute's (rows [0, rt), vmonarch.py:66-68) just before it.  Every gradient is written once, in
        # the caller's dtype and memory order, by the last call that contributes to it: the fp32 sum of the
        # earlier contributions plus its own (VMO_BWD_SUM_*), so no conversion pass follows.  dq: the
        # L-steps (the first overwrites, the rest add), the recompute, then R-step 0 (x = q).  dk: every
        # R-step (values start with k: the kernels fold k's value-role gradient into dk, as autograd's sum
        # over k's uses at vmonarch.py:50 does), the recompute, R-step 0 last.  dv: the last R-step (values
        # [k | v]) and the recompute.
        gq, gk, gv = (_lib.empty_in_order(o, (B, H, N), f, dt, dev) for o, f in zip(ctx.orders, (D, D, Dv)))
        dq = torch.empty((B, H, N, D), device=dev, dtype=f32)
        partial = {"k": torch.empty((B, H, N, D), device=dev, dtype=f32),
                   "v": torch.empty((B, H, N, Dv), device=dev, dtype=f32)}
        started = {"k": False, "v": False}
        final = {"k": gk, "v": gv}
        v_writers = ([num_iters - 1] if num_iters > 1 else []) + (["rt"] if rt > 0 else []) + ([0] if num_iters == 1 else [])

        def grad_args(x, last_writer):
            """fea_backward_raw arguments for gradient x ("k" or "v") of one call: into the fp32 partial sum
            (overwriting it on the first call), or, from its last writer, into the dtype result."""
            if last_writer:
                return ({f"d{x}": final[x], f"d{x}_base": partial[x]} if started[x] else {f"d{x}": final[x]}), ""
            first = not started[x]
            started[x] = True
            return {f"d{x}": partial[x]}, (x if first else "")

        de = torch.zeros((B, H, N), device=dev, dtype=f32)
        # rowsum(out * d out), formed by the L-step backward that writes d out (one-tile grids), read by the
        # R-step backward in place of another pass over both
        delta = torch.empty((B, H, N), device=dev, dtype=f32) if _lstep_one_tile(m, D, Dv, True) else None
        g = dz
        for it in reversed(range(num_iters)):
            last = it == num_iters - 1
            x, out, lse, ent = saved[4 * it: 4 * it + 4]
            dout = torch.empty_like(out)
            _lstep_bwd_launch(q, out, ent, g, dq, dout, m, b, scale, last, rt if last else 0, min_col_mass,
                              overwrite_q=last, delta=delta)
            if it == 0 and rt > 0:
                # the exact attention of the first rt queries; it reads every key and value
                zeros = torch.zeros((B, H, rt), device=dev, dtype=f32)
                kw, ow = grad_args("k", False)
                kv, ov = grad_args("v", v_writers[-1] == "rt")
                fea_backward_raw(q[:, :, :rt], k, v, z[:, :, :rt], lse_rt, zeros, _lib.row_aligned(dz[:, :, :rt]), zeros,
                                 scale, dq=dq[:, :, :rt], overwrite=ow + ov, **kw, **kv)
            # values k, or [k | v] read from the two tensors in place (vmonarch.py:50); m frames per head
            kw, ow = grad_args("k", it == 0)
            if last:
                kv, ov = grad_args("v", v_writers[-1] == it)
                kw.update(kv)
                ow += ov
            if it == 0:   # R-step 0 reads q itself: dq's last contribution
                kw.update(dq=gq, dq_base=dq)
            gx, _, _ = fea_backward_raw(x, k, k, out, lse, ent, dout, de, scale if it == 0 else 1.0, overwrite=ow,
                                        v1=v if last else None, fold_k=True, frames=m, delta=delta, **kw)
            if it > 0:
                g = gx                      # dL/du of the previous L-step's output
        return gq, gk, gv, None, None, None, None, None, None


def _vmonarch_composed(q, k, v, num_blocks, block_size, num_iters, recompute_tokens, min_col_mass):
    """Step-by-step restatement of vmonarch.py:41-69 on GPU tensors (autograd-capable)."""
    B, H, N, D = q.shape
    scale = D ** -0.5
    qg, kg, vg = (t.unflatten(2, (num_blocks, block_size)) for t in (q, k, v))
    u = qg * scale
    z = None
    for it in range(num_iters):
        last = it == num_iters - 1
        out, neg_ent = _row_block_attention(u, kg, torch.cat([kg, vg], -1) if last else kg)
        kr = out[..., :D] * scale
        logits = torch.einsum("bhijd,bhkjd->bhjik", qg, kr).float()
        attn = (logits - neg_ent.transpose(-1, -2).unsqueeze(-2)).softmax(-1)
        if last:
            y = out[..., D:]
            z = torch.einsum("bhjik,bhkjd->bhijd", attn.to(y.dtype), y)
        else:
            col_mass = attn.sum(-2).transpose(-1, -2).clamp_min(min_col_mass)
            u = torch.einsum("bhjik,bhijd->bhkjd", attn.to(q.dtype), qg)
            u = u * (scale / col_mass.unsqueeze(-1)).to(q.dtype)
    z = z.reshape(B, H, N, -1)
    if recompute_tokens > 0:
        exact = torch.nn.functional.scaled_dot_product_attention(q[:, :, :recompute_tokens], k, v)
        z = torch.cat([exact, z[:, :, recompute_tokens:]], dim=2)
    return z


def _padded_width(D, Dv):
    """The kernel width (32, 64 or 128) that q, k and v can all be zero-padded to, or None."""
    if D <= 32 and Dv <= 32:
        return 32
    w = max(64, D, Dv)
    return w if w in (64, 128) else None


def _pad_to(t, w):
    return t if t.shape[-1] == w else torch.nn.functional.pad(t, (0, w - t.shape[-1]))


def vmonarch_attention(q, k, v, num_blocks, block_size, num_iters=2, recompute_tokens=0, min_col_mass=0.01,
                       qk_fp8=False):
    """
    Args:
        q, k: (B, H, N, D); v: (B, H, N, Dv), with N == num_blocks * block_size.
        num_blocks: m, number of grid rows (keep it small).
        block_size: b, number of tokens per grid row.
        num_iters: alternating-minimization steps.
        recompute_tokens: the first `recompute_tokens` queries use exact attention.
        min_col_mass: lower bound of the column mass of L, for stability.
        qk_fp8: (beyond the reference) the R-steps' q k^T in fp8 e4m3, forward only, D = 128; the
            recompute stays exact.  An approximation: logits off by ~1% of their spread.  D = Dv = 128.
    Returns:
        (B, H, N, Dv)
    """
    B, H, N, D = q.shape
    assert N == num_blocks * block_size, f"N={N} != {num_blocks} * {block_size}"
    if num_iters < 1:
        raise UnboundLocalError("local variable 'z' referenced before assignment")  # as the reference (vmonarch.py:65)
    needs_graph = torch.is_grad_enabled() and any(t.requires_grad for t in (q, k, v))
    Dv = v.shape[-1]
    if qk_fp8:
        if needs_graph:
            raise NotImplementedError("vmonarch_amd: qk_fp8 is forward-only (the backward recomputes S in the "
                                      "16-bit type); run under torch.no_grad() or without it")
        if not (_row_block_attention is _ROW_BLOCK_ATTENTION and D == 128 and Dv == 128
                and _fused_supported(q, k, v, num_blocks)):
            raise NotImplementedError(f"vmonarch_amd: qk_fp8 is built for the fused HIP path with head dim 128 "
                                      f"(got D={D}, Dv={Dv}, num_blocks={num_blocks}, {q.dtype})")
        return _vmonarch_fused(q, k, v, num_blocks, block_size, num_iters, recompute_tokens, min_col_mass,
                               qk_fp8=True)
    if _row_block_attention is _ROW_BLOCK_ATTENTION:
        args = (num_blocks, block_size, num_iters, recompute_tokens, min_col_mass)
        if not needs_graph and _fused_supported(q, k, v, num_blocks):
            return _vmonarch_fused(q, k, v, *args)
        if needs_graph and _hip_backward_supported(q, k, v, num_blocks):
            return _VMonarchFunction.apply(q, k, v, *args)
        # Head dims the kernels do not take as they are (mixes of 16 and 32, or D != Dv with autograd): zero columns
        # change neither q.k nor P.v, so q, k and v padded to one kernel width give z with zero columns
        # past Dv, with the softmax scale of the true D; autograd slices the padded gradients back.
        w = _padded_width(D, Dv)
        if (w is not None and q.is_cuda and q.dtype in _lib.DTYPES and k.dtype == q.dtype and v.dtype == q.dtype
                and k.shape == q.shape and v.shape[:-1] == q.shape[:-1]
                and _lstep_supported(num_blocks, w, w, needs_graph)):
            qp, kp, vp = (_pad_to(t, w) for t in (q, k, v))
            if needs_graph:
                z = _VMonarchFunction.apply(qp, kp, vp, *args, D ** -0.5)
            else:
                z = _vmonarch_fused(qp, kp, vp, *args, scale=D ** -0.5)
            if w == Dv:
                return z
            # the first Dv columns, in the caller's memory order like every other path's z (a DiT block's
            # (B, N, H, Dv) buffer needs no permute copy afterwards); copy_ keeps the autograd graph
            return _lib.empty_in_layout(q, Dv, q.dtype).copy_(z[..., :Dv])
        if q.is_cuda:
            warnings.warn(f"vmonarch_amd: no HIP path for num_blocks={num_blocks}, head dims ({D}, {Dv}), {q.dtype}"
                          f"{' with autograd' if needs_graph else ''}; running the composed path (flash-entropy "
                          "R-steps in HIP, L-steps and recompute as torch ops)", RuntimeWarning, stacklevel=2)
    if not q.is_cuda:
        raise RuntimeError("vmonarch_amd: vmonarch_attention needs GPU tensors (no CPU path)")
    return _vmonarch_composed(q, k, v, num_blocks, block_size, num_iters, recompute_tokens, min_col_mass)


class VMonarchAttention(nn.Module):
    """Module wrapper (reference vmonarch.py:72-85); holds no parameters."""

    def __init__(self, num_blocks, block_size, num_iters=2, min_col_mass=0.01, qk_fp8=False):
        super().__init__()
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.num_iters = num_iters
        self.min_col_mass = min_col_mass
        self.qk_fp8 = qk_fp8   # beyond the reference: fp8 q k^T in the R-steps (vmonarch_attention)

    def forward(self, q, k, v, recompute_tokens=0):
        return vmonarch_attention(q, k, v, self.num_blocks, self.block_size, self.num_iters,
                                  recompute_tokens, self.min_col_mass, qk_fp8=self.qk_fp8)

    def extra_repr(self):
        return f"num_blocks={self.num_blocks}, block_size={self.block_size}, num_iters={self.num_iters}"
