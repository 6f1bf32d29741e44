"""The two routes of the flash-entropy backward (vmo_fea_bwd) against the oracle and against each other.

* dS route (VMO_BWD_DS_DQ; the default for d = 128, dv = 256): fea_bwd_prep forms the per-row scalars, the
  dkdv kernel stores dS^T in the workspace, fea_bwd_dq_ds forms dq = sm_scale dS k from it.
* recompute route (VMO_BWD_RECOMPUTE_DQ; the default elsewhere): the dq kernel recomputes S and dP.

The shapes cover what the dS route has to get right: query counts that are not multiples of 8 / 32 / 128 (the
padded dS^T rows and the last query tile reading past a row), key counts that are not multiples of 64 / 128
(masked keys of the last stage), frames (problems inside one (b, h)), nq != nk with key splits of dq, values k,
[k | v1] and values in two parts, fp16.  Gradients: the reference metric of tests/test_vmonarch.py:42 (3e-2)
and elementwise 2e-2 + 1e-2 |ref| against the float64 oracle; the two routes within 1e-2 of each other's
maximum (they differ only in the rounding of the row scalar delta and the order of the dq sums).
"""
import numpy as np
import pytest
import torch

from conftest import assert_grad_close, hip_library_loaded, randn_lp
from oracle import entropy_attention_grad

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

CASES = [
    # nq, nk, frames, heads, D, values, Dv, dtype
    (200, 200, 1, 2, 64, "plain", 64, torch.bfloat16),
    (77, 333, 1, 2, 128, "plain", 128, torch.bfloat16),
    (1557, 1557, 2, 1, 128, "k_v1", 256, torch.bfloat16),
    (1000, 1000, 3, 1, 128, "k", 128, torch.float16),
    (130, 4100, 1, 2, 128, "plain", 128, torch.bfloat16),
    (96, 250, 1, 2, 64, "two_parts", 128, torch.bfloat16),
    (33, 33, 1, 2, 64, "k", 64, torch.bfloat16),
    (520, 520, 4, 1, 64, "k_v1", 128, torch.float16),
]


def _run(case, route):
    from vmonarch_amd.kernel import fea_forward
    from vmonarch_amd.kernel_bwd import fea_backward_raw
    nq, nk, F, H, D, kind, Dv, dt = case
    g = torch.Generator().manual_seed(nq + 7 * nk + F + D + Dv)
    q = randn_lp(g, 1, H, F * nq, D, dtype=dt)
    k = randn_lp(g, 1, H, F * nk, D, dtype=dt)
    v0 = randn_lp(g, 1, H, F * nk, Dv // 2 if kind in ("k_v1", "two_parts") else Dv, dtype=dt)
    do = randn_lp(g, 1, H, F * nq, Dv, dtype=dt)
    de = torch.randn(1, H, F * nq, generator=g)
    qd, kd, vd, dod, ded = (t.to(DEV) for t in (q, k, v0, do, de))
    sc = D ** -0.5
    if kind == "plain":
        w_parts, bwd_v, v1 = (vd, None), vd, None
    elif kind == "k":
        w_parts, bwd_v, v1 = (kd, None), kd, None
    elif kind == "k_v1":
        w_parts, bwd_v, v1 = (kd, vd), kd, vd
    else:   # two_parts: values [v0 | v1] with v1 a second tensor of v0's shape and strides
        v1 = randn_lp(g, 1, H, F * nk, Dv // 2, dtype=dt).to(DEV)
        w_parts, bwd_v = (torch.cat([vd, v1], -1), None), vd
    o, lse, ent = fea_forward(qd, kd, w_parts[0], w_parts[1], sc, frames=F)
    print(f"fea_bwd route={route} case={case[:7]}", flush=True)
    grads = fea_backward_raw(qd, kd, bwd_v, o, lse, ent, dod, ded, sc, v1=v1, frames=F, dq_route=route)
    torch.cuda.synchronize()
    w = {"plain": vd, "k": kd}.get(kind)
    if w is None:
        w = torch.cat([kd if kind == "k_v1" else vd, v1], -1)
    return grads, (q, k, w.cpu(), do, de)


def _oracle(inputs, case):
    nq, nk, F, H, D = case[:5]
    q, k, w, do, de = inputs

    def per_problem(t, n):   # (1, H, F n, X) -> (1, H F, n, X): frame f is rows [f n, (f + 1) n)
        return t.float().numpy().reshape(1, H * F, n, -1)
    refs = entropy_attention_grad(per_problem(q, nq), per_problem(k, nk), per_problem(w, nk), per_problem(do, nq),
                                  de.numpy().reshape(1, H * F, nq), D ** -0.5)
    return [r.reshape(1, H, F * r.shape[2], -1) for r in refs]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"nq{c[0]}-nk{c[1]}-f{c[2]}-d{c[4]}-{c[5]}{c[6]}-{str(c[7])[6:]}")
def test_backward_routes_match_oracle_and_each_other(case):
    (dq, dk, dv), inputs = _run(case, "ds")
    (dq_r, dk_r, dv_r), _ = _run(case, "recompute")
    refs = _oracle(inputs, case)
    for (a, b, ref, name) in ((dq, dq_r, refs[0], "dq"), (dk, dk_r, refs[1], "dk"), (dv, dv_r, refs[2], "dv")):
        a, b = a.float().cpu().numpy(), b.float().cpu().numpy()
        assert np.isfinite(a).all() and np.isfinite(b).all(), name
        assert_grad_close(a, ref, 3e-2, f"{name} (dS route)")
        assert_grad_close(b, ref, 3e-2, f"{name} (recompute route)")
        assert np.abs(a - b).max() <= 1e-2 * np.abs(b).max(), name
    assert hip_library_loaded()


@pytest.mark.parametrize("route", ["ds", "recompute"])
def test_backward_with_given_delta(route):
    """vmo_fea_bwd_args.delta: rowsum(o * do) handed in (as the L-step backward forms it) instead of formed
    from o and do -- the same gradients up to the order of that sum."""
    from vmonarch_amd.kernel import fea_forward
    from vmonarch_amd.kernel_bwd import fea_backward_raw
    g = torch.Generator().manual_seed(77)
    F, n, D = 3, 300, 128
    q, k = randn_lp(g, 1, 2, F * n, D).to(DEV), randn_lp(g, 1, 2, F * n, D).to(DEV)
    v1 = randn_lp(g, 1, 2, F * n, D).to(DEV)
    o, lse, ent = fea_forward(q, k, k, v1, D ** -0.5, frames=F)
    do = randn_lp(g, 1, 2, F * n, 2 * D).to(DEV)
    de = torch.randn(1, 2, F * n, generator=g).to(DEV)
    delta = (o.float() * do.float()).sum(-1)
    args = (q, k, k, o, lse, ent, do, de, D ** -0.5)
    ref = fea_backward_raw(*args, v1=v1, frames=F, dq_route=route)
    got = fea_backward_raw(*args, v1=v1, frames=F, dq_route=route, delta=delta)
    for a, b, name in zip(got, ref, ("dq", "dk", "dv")):
        a, b = a.float().cpu().numpy(), b.float().cpu().numpy()
        assert np.abs(a - b).max() <= 1e-2 * np.abs(b).max(), name
