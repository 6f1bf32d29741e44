"""VMonarch alternating minimisation restated on the CPU with numpy (test infrastructure only).

Restates /root/reference/video_monarch_attention/vmonarch.py:19-69 with the R-step taken by
the fp32 oracle exactly as the reference's own test does (tests/test_vmonarch.py:55-61), i.e.
no bf16 rounding anywhere: this is the fp32 reference the GPU path is judged against.

``vmonarch_attention_lowp`` restates the same glue with the roundings the reference's own bf16 run
makes (the einsums and products of vmonarch.py:47-67 return bf16 tensors), around an exact R-step:
it tells how far the reference's bf16 path itself lands from the fp32 reference on given inputs.
"""
import numpy as np

from .fea import entropy_attention, entropy_attention_grad, exact_attention, kernel_rounding_attention


def row_block_attention(x, k, w, dtype=np.float64):
    """R-step seam, vmonarch.py:19-26 with the oracle of tests/test_vmonarch.py:55-57.

    x, k: (B, H, m, b, D); w: (B, H, m, b, Dw).  Returns (softmax(x k^T) w, -entropy) per
    grid row; the scale is 1 (vmonarch.py:25 passes sm_scale=1.0).
    """
    out, ent = entropy_attention(x, k, w, 1.0, dtype)
    return out, -ent


def _softmax(x, axis=-1):
    m = x.max(axis, keepdims=True)
    e = np.exp(x - m)
    return e / e.sum(axis, keepdims=True)


def lstep(qg, out, neg_ent, scale, last, min_col_mass=0.01):
    """One L-step, vmonarch.py:51-63.

    qg: (B, H, m, b, D) queries; out: (B, H, m, b, Dw) R-step output; neg_ent: (B, H, m, b).
    Returns z (B, H, m, b, Dw-D) when ``last`` else the next R-step queries u (B, H, m, b, D).
    """
    D = qg.shape[-1]
    kr = out[..., :D] * scale                                            # vmonarch.py:51
    logits = np.einsum("bhijd,bhkjd->bhjik", qg, kr)                     # vmonarch.py:55
    attn = _softmax(logits - np.swapaxes(neg_ent, -1, -2)[..., None, :])  # vmonarch.py:56
    if last:
        y = out[..., D:]                                                 # vmonarch.py:58
        return np.einsum("bhjik,bhkjd->bhijd", attn, y)                  # vmonarch.py:59
    col_mass = np.maximum(np.swapaxes(attn.sum(-2), -1, -2), min_col_mass)  # vmonarch.py:61
    u = np.einsum("bhjik,bhijd->bhkjd", attn, qg)                        # vmonarch.py:62
    return u * (scale / col_mass)[..., None]                             # vmonarch.py:63


def vmonarch_attention(q, k, v, num_blocks, block_size, num_iters=2, recompute_tokens=0,
                       min_col_mass=0.01, dtype=np.float64, record=None, frozen_neg_ent=None):
    """vmonarch.py:29-69.  q, k: (B, H, N, D); v: (B, H, N, Dv); N == num_blocks*block_size.

    ``record``: a list that receives (u, w, out, neg_ent) of every iteration (for the backward).
    ``frozen_neg_ent``: per-iteration entropy biases used instead of the computed ones -- the
    reference detaches them (vmonarch.py:26), so a finite-difference check of the gradient holds
    them at their values at the base point.
    """
    q, k, v = (np.asarray(t, dtype=dtype) for t in (q, k, v))
    B, H, N, D = q.shape
    if N != num_blocks * block_size:                                     # vmonarch.py:42
        raise AssertionError(f"N={N} != {num_blocks} * {block_size}")
    if num_iters < 1:
        # the reference leaves z unbound here (vmonarch.py:65 raises UnboundLocalError)
        raise UnboundLocalError("num_iters must be >= 1")
    scale = D ** -0.5                                                    # vmonarch.py:43
    m, b = num_blocks, block_size
    qg, kg, vg = (t.reshape(B, H, m, b, t.shape[-1]) for t in (q, k, v))  # vmonarch.py:44
    u = qg * scale                                                       # vmonarch.py:47
    z = None
    for it in range(num_iters):                                          # vmonarch.py:48
        last = it == num_iters - 1
        w = np.concatenate([kg, vg], -1) if last else kg                 # vmonarch.py:50
        out, neg_ent = row_block_attention(u, kg, w, dtype)
        if frozen_neg_ent is not None:
            neg_ent = frozen_neg_ent[it]
        if record is not None:
            record.append((u, w, out, neg_ent))
        res = lstep(qg, out, neg_ent, scale, last, min_col_mass)
        if last:
            z = res
        else:
            u = res
    z = z.reshape(B, H, N, -1)                                           # vmonarch.py:65
    if recompute_tokens > 0:                                             # vmonarch.py:66-68
        rt = recompute_tokens
        z = z.copy()
        z[:, :, :rt] = exact_attention(q[:, :, :rt], k, v, None, dtype)
    return z


def round_bf16(x):
    """Round to the nearest bf16 value (ties to even), returned as float64: what storing an fp32
    result in a bfloat16 tensor does."""
    b = np.ascontiguousarray(np.asarray(x, dtype=np.float32)).view(np.uint32).astype(np.uint64)
    b = (b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFF0000
    return b.astype(np.uint32).view(np.float32).astype(np.float64)


def vmonarch_attention_lowp(q, k, v, num_blocks, block_size, num_iters=2, recompute_tokens=0,
                            min_col_mass=0.01, rnd=round_bf16, keep_fp32=(), kernel_p=False):
    """vmonarch.py:29-69 as the reference runs it on bf16 tensors: every tensor the glue stores in the
    input dtype is rounded by ``rnd`` where the reference makes it (einsum / product results rounded once,
    accumulation in float64 here), the softmaxes and col_mass in float, and the R-step exact (its output o
    rounded as a bf16 kernel stores it, the entropy kept in float).  Cast points:
      u = q * scale                          (vmonarch.py:47)  rounded
      out = R-step(u, k, w)                  (vmonarch.py:50)  o rounded, entropy float
      kr = out[..., :D] * scale              (vmonarch.py:51)  rounded
      logits = einsum(q, kr).float()         (vmonarch.py:55)  rounded, then float
      z = einsum(attn.to(dtype), y)          (vmonarch.py:59)  attn rounded, z rounded
      u = einsum(attn.to(dtype), q)          (vmonarch.py:62)  attn rounded, u rounded
      u = u * (scale / col_mass).to(dtype)   (vmonarch.py:63)  factor rounded, product rounded
      SDPA(q[:, :, :rt], k, v)               (vmonarch.py:67)  exact, rounded
    ``keep_fp32`` names cast points to skip ("u0": the first u, "kr", "logits"; "u": the u update rounded
    once, as the product of the fp32 einsum and the fp32 factor, instead of three times): with all four the
    glue rounds where this build's HIP kernels round (they fold q * scale and out * scale into their fp32
    softmax factors, keep the L-step logits in fp32 and round u once when they store it).  ``kernel_p`` takes
    the R-steps and the recompute as the flash-entropy kernels round them (fea.kernel_rounding_attention:
    P rounded where it enters P.W) instead of exactly.  Both are emulations of this build, not of the
    reference: the reference's own bf16 path is the default (no keep_fp32, kernel_p False).
    """
    q, k, v = (rnd(t) for t in (q, k, v))
    B, H, N, D = q.shape
    if N != num_blocks * block_size:
        raise AssertionError(f"N={N} != {num_blocks} * {block_size}")
    scale = D ** -0.5
    m, b = num_blocks, block_size
    qg, kg, vg = (t.reshape(B, H, m, b, t.shape[-1]) for t in (q, k, v))
    unknown = set(keep_fp32) - {"u0", "kr", "logits", "u"}
    if unknown:
        raise ValueError(f"keep_fp32: unknown cast points {sorted(unknown)}")
    keep = lambda name, x: x if name in keep_fp32 else rnd(x)   # noqa: E731
    u = keep("u0", qg * scale)
    z = None
    for it in range(num_iters):
        last = it == num_iters - 1
        w = np.concatenate([kg, vg], -1) if last else kg
        if kernel_p:
            out, ent = kernel_rounding_attention(u, kg, w, 1.0, rnd)
        else:
            out, ent = entropy_attention(u, kg, w, 1.0)
        out = rnd(out)
        kr = keep("kr", out[..., :D] * scale)
        logits = keep("logits", np.einsum("bhijd,bhkjd->bhjik", qg, kr))
        attn = _softmax(logits + np.swapaxes(ent, -1, -2)[..., None, :])   # - neg_ent
        if last:
            z = rnd(np.einsum("bhjik,bhkjd->bhijd", rnd(attn), out[..., D:]))
        else:
            col_mass = np.maximum(np.swapaxes(attn.sum(-2), -1, -2), min_col_mass)
            u = keep("u", np.einsum("bhjik,bhijd->bhkjd", rnd(attn), qg))
            u = rnd(u * keep("u", scale / col_mass)[..., None])
    z = z.reshape(B, H, N, -1)
    if recompute_tokens > 0:
        rt = recompute_tokens
        z = z.copy()
        if kernel_p:
            z[:, :, :rt] = rnd(kernel_rounding_attention(q[:, :, :rt], k, v, D ** -0.5, rnd, entropy_from_pk=False)[0])
        else:
            z[:, :, :rt] = rnd(exact_attention(q[:, :, :rt], k, v))
    return z


def lstep_grad(qg, out, neg_ent, scale, last, grad, min_col_mass=0.01):
    """Backward of ``lstep`` (vmonarch.py:51-63) with the entropy bias held constant (vmonarch.py:26
    detaches it).  ``grad`` is dL/dz (B, H, m, b, Dv) when ``last``, else dL/du (B, H, m, b, D).
    Returns (dL/dqg, dL/dout).  Derived by hand, step by step backwards through lstep:
      z = attn y               -> d attn = dz y^T, dy = attn^T dz
      u = (attn^T q) f, f = scale / max(c, mcm), c = sum_i attn
                               -> dv = du f, df = du . v, dc = -df scale / cm^2 where c >= mcm,
                                  d attn = dv q^T + dc, dq = attn dv
      attn = softmax_k(logits + ent)  -> d logits = attn (d attn - sum_k attn d attn)
      logits = q kr^T, kr = out[:D] scale  -> dq += d logits kr, d out[:D] = scale d logits^T q
    """
    D = qg.shape[-1]
    kr = out[..., :D] * scale
    logits = np.einsum("bhijd,bhkjd->bhjik", qg, kr)
    attn = _softmax(logits - np.swapaxes(neg_ent, -1, -2)[..., None, :])
    dout = np.zeros_like(out)
    if last:
        y = out[..., D:]
        dattn = np.einsum("bhijd,bhkjd->bhjik", grad, y)
        dout[..., D:] = np.einsum("bhjik,bhijd->bhkjd", attn, grad)
        dqg = np.zeros_like(qg)
    else:
        c = np.swapaxes(attn.sum(-2), -1, -2)                     # (B, H, k, j)
        cm = np.maximum(c, min_col_mass)
        f = scale / cm
        vsum = np.einsum("bhjik,bhijd->bhkjd", attn, qg)
        dv = grad * f[..., None]
        df = (grad * vsum).sum(-1)
        dc = np.where(c >= min_col_mass, -df * scale / (cm * cm), 0.0)
        dattn = np.einsum("bhkjd,bhijd->bhjik", dv, qg) + np.swapaxes(dc, -1, -2)[..., None, :]
        dqg = np.einsum("bhjik,bhkjd->bhijd", attn, dv)
    dlogits = attn * (dattn - (attn * dattn).sum(-1, keepdims=True))
    dqg = dqg + np.einsum("bhjik,bhkjd->bhijd", dlogits, kr)
    dout[..., :D] = scale * np.einsum("bhjik,bhijd->bhkjd", dlogits, qg)
    return dqg, dout


def vmonarch_attention_grad(q, k, v, grad_z, num_blocks, block_size, num_iters=2, recompute_tokens=0,
                            min_col_mass=0.01, dtype=np.float64):
    """Gradient of sum(z * grad_z) w.r.t. (q, k, v) for z = vmonarch_attention(...), with the
    R-step entropies detached as in the reference (vmonarch.py:26).  Reverse pass over the
    recorded forward: recompute rows through entropy_attention_grad (exact attention,
    vmonarch.py:66-68; the L-path rows < rt get no gradient, they are overwritten), then each
    iteration's lstep_grad and R-step entropy_attention_grad (sm_scale 1, values w = k or [k|v]).
    """
    q, k, v, grad_z = (np.asarray(t, dtype=dtype) for t in (q, k, v, grad_z))
    B, H, N, D = q.shape
    Dv = v.shape[-1]
    m, b = num_blocks, block_size
    scale = D ** -0.5
    rec = []
    vmonarch_attention(q, k, v, m, b, num_iters, 0, min_col_mass, dtype, record=rec)
    dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
    gz = grad_z.copy()
    rt = recompute_tokens
    if rt > 0:
        gq, gk, gv = entropy_attention_grad(q[:, :, :rt], k, v, grad_z[:, :, :rt],
                                            np.zeros(grad_z.shape[:2] + (rt,)), None, dtype)
        dq[:, :, :rt] += gq
        dk += gk
        dv += gv
        gz[:, :, :rt] = 0.0
    qg = q.reshape(B, H, m, b, D)
    dqg = np.zeros_like(qg)
    dkg = np.zeros((B, H, m, b, D), dtype)
    dvg = np.zeros((B, H, m, b, Dv), dtype)
    kg = k.reshape(B, H, m, b, D)
    g = gz.reshape(B, H, m, b, Dv)
    for it in reversed(range(num_iters)):
        last = it == num_iters - 1
        u, w, out, neg_ent = rec[it]
        dq_l, dout = lstep_grad(qg, out, neg_ent, scale, last, g, min_col_mass)
        dqg += dq_l
        du, dk_key, dw = entropy_attention_grad(u, kg, w, dout, np.zeros(u.shape[:-1]), 1.0, dtype)
        dkg += dk_key
        if last:
            dkg += dw[..., :D]
            dvg += dw[..., D:]
        else:
            dkg += dw
        if it > 0:
            g = du
        else:
            dqg += du * scale
    dq += dqg.reshape(B, H, N, D)
    dk += dkg.reshape(B, H, N, D)
    dv += dvg.reshape(B, H, N, Dv)
    return dq, dk, dv
