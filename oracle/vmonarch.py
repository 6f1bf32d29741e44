"""VMonarch alternating minimisation restated on the CPU with numpy (test infrastructure only).

Restates /root/reference/video_monarch_attention/vmonarch.py:19-69 with the R-step taken by
the fp32 oracle exactly as the reference's own test does (tests/test_vmonarch.py:55-61), i.e.
no bf16 rounding anywhere: this is the fp32 reference the GPU path is judged against.
"""
import numpy as np

from .fea import entropy_attention, exact_attention


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
                       min_col_mass=0.01, dtype=np.float64):
    """vmonarch.py:29-69.  q, k: (B, H, N, D); v: (B, H, N, Dv); N == num_blocks*block_size."""
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
