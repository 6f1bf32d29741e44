"""FlashEntropyAttention restated on the CPU with numpy (test infrastructure only).

Reference behaviour being restated:
  * /root/reference/tests/test_vmonarch.py:12-15 -- fp32 oracle: log_softmax(sm_scale*q k^T),
    p = exp(logp), returns (p v, -sum p logp)
  * /root/reference/video_monarch_attention/kernel.py:384-402 -- public API: default
    sm_scale = D**-0.5, entropy in nats (kernel.py:145-146, docstring :393-394), padding
    invisible to the caller
  * /root/reference/video_monarch_attention/kernel.py:154-167, :202, :241 -- backward:
    dS = P*(dP - delta) + dE*P*(-E - ln P), delta_i = sum_d o_id dO_id
"""
import numpy as np


def _f(x, dtype):
    return np.asarray(x, dtype=dtype)


def _log_softmax(s):
    m = s.max(-1, keepdims=True)
    z = s - m
    return z - np.log(np.exp(z).sum(-1, keepdims=True))


def entropy_attention(q, k, v, sm_scale=None, dtype=np.float64):
    """(o, e): o = softmax(sm_scale q k^T) v, e_i = -sum_j P_ij ln P_ij (nats).

    q, k: (..., Nq|Nk, D); v: (..., Nk, Dv).  Follows tests/test_vmonarch.py:12-15 and the
    default scale of kernel.py:397-398.
    """
    q, k, v = _f(q, dtype), _f(k, dtype), _f(v, dtype)
    if sm_scale is None:
        sm_scale = q.shape[-1] ** -0.5
    logp = _log_softmax(sm_scale * (q @ np.swapaxes(k, -1, -2)))
    p = np.exp(logp)
    return p @ v, -(p * logp).sum(-1)


def exact_attention(q, k, v, sm_scale=None, dtype=np.float64):
    """softmax(sm_scale q k^T) v -- the recompute path (vmonarch.py:66-68 calls
    F.scaled_dot_product_attention with its default scale D**-0.5, non-causal)."""
    return entropy_attention(q, k, v, sm_scale, dtype)[0]


def entropy_attention_grad(q, k, v, do, de, sm_scale=None, dtype=np.float64):
    """Analytic gradient of L = sum(o*do) + sum(e*de) w.r.t. (q, k, v).

    Restates the reference backward (kernel.py:154-167 preprocess delta = rowsum(o*dO);
    kernel.py:202 / :241 dS = P(dP - delta) + dE P(-E - ln P); dV = P^T dO (kernel.py:199);
    dK = sm_scale dS^T Q (kernel.py:205, :296); dQ = sm_scale dS K (kernel.py:244, :313)).
    """
    q, k, v, do, de = (_f(t, dtype) for t in (q, k, v, do, de))
    if sm_scale is None:
        sm_scale = q.shape[-1] ** -0.5
    logp = _log_softmax(sm_scale * (q @ np.swapaxes(k, -1, -2)))
    p = np.exp(logp)
    o = p @ v
    e = -(p * logp).sum(-1)
    dp = do @ np.swapaxes(v, -1, -2)
    delta = (o * do).sum(-1, keepdims=True)
    ds = p * (dp - delta) + de[..., None] * p * (-e[..., None] - logp)
    dq = sm_scale * (ds @ k)
    dk = sm_scale * (np.swapaxes(ds, -1, -2) @ q)
    dv = np.swapaxes(p, -1, -2) @ do
    return dq, dk, dv


def kernel_rounding_attention(q, k, w, sm_scale, rnd, entropy_from_pk=True, first_keys=32, dtype=np.float64):
    """Where the gfx950 flash-entropy kernels round (not the reference's algorithm: an emulation of this
    build's kernels, used to tell their rounding apart from the reference's in tests).  Relative to the max m
    of the row's first `first_keys` logits, p = exp(s - m) is rounded once (``rnd``) where it enters P.W as
    the MFMA operand p~.  With ``entropy_from_pk`` (the VMonarch R-step, values starting with k) the row sum is
    l~ = sum p~, o = sum p~ w / l~ and e = m + ln l~ - sum p~ s / l~; otherwise (the recompute) l = sum p,
    o = sum p~ w / l.  With an identity ``rnd`` both are exactly softmax(s) w and -sum P ln P.
    Returns (o, e); e is None without ``entropy_from_pk``."""
    q, k, w = _f(q, dtype), _f(k, dtype), _f(w, dtype)
    s = sm_scale * (q @ np.swapaxes(k, -1, -2))
    m = s[..., :first_keys].max(-1, keepdims=True)
    p = np.exp(s - m)
    pt = rnd(p)
    if entropy_from_pk:
        l = pt.sum(-1, keepdims=True)
        e = m[..., 0] + np.log(l[..., 0]) - (pt * s).sum(-1) / l[..., 0]
        return (pt @ w) / l, e
    return (pt @ w) / p.sum(-1, keepdims=True), None

