"""Seeded random VMonarch shapes against the CPU oracle: frames m (one-tile and multi-block L-steps, 2-128), block
sizes, head dims 16 / 32 / 64 / 128 (and D != Dv), 1-3 iterations, recompute rows, bf16 and fp16, contiguous and
(B, N, H, D)-strided inputs; z, and with autograd the gradients, through the HIP path (no composed-path
warning).  Tolerances as tests/test_vmonarch.py:64-66 (z 3e-2, gradients 5e-2) beside elementwise
2e-2 + 1e-2 |ref| for z."""
import warnings

import numpy as np
import pytest
import torch

from conftest import assert_close_elementwise, assert_close_ref, assert_grad_close, hip_library_loaded, randn_lp
from oracle import vmonarch_attention as vmonarch_oracle
from oracle import vmonarch_attention_grad

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
DIMS = [(32, 32), (64, 64), (128, 128), (64, 128), (128, 64), (16, 16)]


def _case(seed):
    rng = np.random.default_rng(seed)
    D, Dv = DIMS[seed % len(DIMS)]
    m = int(rng.choice([2, 3, 5, 8, 13, 21, 32, 40, 64, 97, 128]))
    b = int(rng.integers(8, 97))
    iters = int(rng.integers(1, 4))
    rt = int(rng.choice([0, b, int(rng.integers(1, b + 1))]))
    dtype = torch.float16 if rng.random() < 0.3 else torch.bfloat16
    dit = bool(rng.random() < 0.4)
    return D, Dv, m, b, iters, rt, dtype, dit


@pytest.mark.parametrize("seed", range(20))
def test_fuzz_vmonarch(seed):
    from vmonarch_amd import vmonarch_attention
    D, Dv, m, b, iters, rt, dtype, dit = _case(seed)
    g = torch.Generator().manual_seed(seed)
    B, H, N = 1, 2, m * b

    def tensor(d):
        t = randn_lp(g, B, N, H, d, dtype=dtype) if dit else randn_lp(g, B, H, N, d, dtype=dtype)
        t = t.to(DEV)
        return t.transpose(1, 2) if dit else t

    q, k, v = tensor(D), tensor(D), tensor(Dv)
    do = torch.randn(B, H, N, Dv, generator=g)
    print(f"fuzz vmonarch seed={seed} D={D} Dv={Dv} m={m} b={b} iters={iters} rt={rt} {dtype} dit={dit}", flush=True)
    qn, kn, vn = (t.float().cpu().numpy() for t in (q, k, v))
    z_ref = vmonarch_oracle(qn, kn, vn, m, b, iters, rt)
    with warnings.catch_warnings():
        warnings.simplefilter("error", RuntimeWarning)   # the composed path warns: it must not be taken
        with torch.no_grad():
            z = vmonarch_attention(q, k, v, m, b, iters, recompute_tokens=rt)
        zz = z.float().cpu().numpy()
        assert np.isfinite(zz).all()
        assert_close_ref(zz, z_ref, 3e-2)
        assert_close_elementwise(zz, z_ref)
        leaves = [t.detach().requires_grad_() for t in (q, k, v)]
        zg = vmonarch_attention(*leaves, m, b, iters, recompute_tokens=rt)
    if D == Dv:   # the same kernels with and without autograd (D != Dv pads to one width for the backward)
        assert torch.equal(zg.detach(), z)
    grads = torch.autograd.grad((zg.float() * do.to(DEV)).sum(), leaves)
    refs = vmonarch_attention_grad(qn, kn, vn, do.numpy(), m, b, iters, rt)
    for gd, gr, t, name in zip(grads, refs, leaves, ("dq", "dk", "dv")):
        assert gd.shape == t.shape and gd.dtype == t.dtype
        assert_grad_close(gd.float().cpu().numpy(), gr, 5e-2, name)
    assert hip_library_loaded()


@pytest.mark.parametrize("m, b, rt, D", [(4, 48, 100, 64), (8, 40, 320, 128), (21, 24, 61, 128), (40, 16, 47, 64),
                                         (6, 32, 192, 32)])
def test_vmonarch_recompute_spans_frames(m, b, rt, D):
    """recompute_tokens past one frame's block (rt > b, up to all N tokens): vmonarch.py:66-68 recomputes rows
    [0, rt) exactly whatever frames they cover, and the last L-step leaves exactly those rows to it."""
    from vmonarch_amd import vmonarch_attention
    g = torch.Generator().manual_seed(m * 1000 + rt)
    B, H, N = 1, 2, m * b
    q, k, v = (randn_lp(g, B, H, N, D).to(DEV) for _ in range(3))
    do = torch.randn(B, H, N, D, generator=g)
    print(f"vmonarch recompute spanning frames m={m} b={b} rt={rt} D={D}", flush=True)
    qn, kn, vn = (t.float().cpu().numpy() for t in (q, k, v))
    z_ref = vmonarch_oracle(qn, kn, vn, m, b, 2, rt)
    with warnings.catch_warnings():
        warnings.simplefilter("error", RuntimeWarning)
        with torch.no_grad():
            z = vmonarch_attention(q, k, v, m, b, 2, recompute_tokens=rt)
        leaves = [t.detach().requires_grad_() for t in (q, k, v)]
        zg = vmonarch_attention(*leaves, m, b, 2, recompute_tokens=rt)
    zz = z.float().cpu().numpy()
    assert_close_ref(zz, z_ref, 3e-2)
    assert_close_elementwise(zz, z_ref)
    assert torch.equal(zg.detach(), z)
    grads = torch.autograd.grad((zg.float() * do.to(DEV)).sum(), leaves)
    refs = vmonarch_attention_grad(qn, kn, vn, do.numpy(), m, b, 2, rt)
    for gd, gr, name in zip(grads, refs, ("dq", "dk", "dv")):
        assert_grad_close(gd.float().cpu().numpy(), gr, 5e-2, name)
    assert hip_library_loaded()


@pytest.mark.parametrize("m, b, D, dit", [(4, 48, 64, False), (21, 24, 128, True), (40, 16, 128, False),
                                          (40, 16, 64, True), (97, 8, 32, False)])
def test_vmonarch_batch_of_two(m, b, D, dit):
    """B = 2 through every kernel (one-tile and multi-block L-steps, forward and backward; (B, H, N, D) and
    (B, N, H, D) inputs): each batch entry must match the oracle run on its own."""
    from vmonarch_amd import vmonarch_attention
    g = torch.Generator().manual_seed(m * 100 + D + dit)
    B, H, N, rt = 2, 2, m * b, b

    def tensor():
        t = randn_lp(g, B, N, H, D) if dit else randn_lp(g, B, H, N, D)
        t = t.to(DEV)
        return t.transpose(1, 2) if dit else t

    q, k, v = tensor(), tensor(), tensor()
    do = torch.randn(B, H, N, D, generator=g)
    print(f"vmonarch batch 2 m={m} b={b} D={D} dit={dit}", flush=True)
    with warnings.catch_warnings():
        warnings.simplefilter("error", RuntimeWarning)
        leaves = [t.detach().requires_grad_() for t in (q, k, v)]
        zg = vmonarch_attention(*leaves, m, b, 2, recompute_tokens=rt)
    grads = torch.autograd.grad((zg.float() * do.to(DEV)).sum(), leaves)
    qn, kn, vn = (t.float().cpu().numpy() for t in (q, k, v))
    for bi in range(B):
        sl = slice(bi, bi + 1)
        z_ref = vmonarch_oracle(qn[sl], kn[sl], vn[sl], m, b, 2, rt)
        assert_close_ref(zg[sl].detach().float().cpu().numpy(), z_ref, 3e-2)
        refs = vmonarch_attention_grad(qn[sl], kn[sl], vn[sl], do[sl].numpy(), m, b, 2, rt)
        for gd, gr, name in zip(grads, refs, ("dq", "dk", "dv")):
            assert_grad_close(gd[sl].float().cpu().numpy(), gr, 5e-2, f"{name} batch {bi}")
    assert hip_library_loaded()


@pytest.mark.parametrize("m, b, rt", [(1, 64, 0), (1, 64, 64), (16, 1, 0), (16, 1, 1), (48, 1, 5), (1, 1, 0)])
def test_vmonarch_degenerate_grids(m, b, rt):
    """One frame (m = 1: the L-step attends over a single row) and one token per frame (b = 1: the R-steps attend
    over a single key), forward and gradients against the oracle."""
    from vmonarch_amd import vmonarch_attention
    g = torch.Generator().manual_seed(m * 10 + b + rt)
    B, H, N, D = 1, 2, m * b, 64
    q, k, v = (randn_lp(g, B, H, N, D).to(DEV) for _ in range(3))
    do = torch.randn(B, H, N, D, generator=g)
    print(f"vmonarch degenerate m={m} b={b} rt={rt}", flush=True)
    with warnings.catch_warnings():
        warnings.simplefilter("error", RuntimeWarning)
        leaves = [t.detach().requires_grad_() for t in (q, k, v)]
        zg = vmonarch_attention(*leaves, m, b, 2, recompute_tokens=rt)
    grads = torch.autograd.grad((zg.float() * do.to(DEV)).sum(), leaves)
    qn, kn, vn = (t.float().cpu().numpy() for t in (q, k, v))
    z_ref = vmonarch_oracle(qn, kn, vn, m, b, 2, rt)
    zz = zg.detach().float().cpu().numpy()
    assert np.isfinite(zz).all()
    assert_close_ref(zz, z_ref, 3e-2)
    refs = vmonarch_attention_grad(qn, kn, vn, do.numpy(), m, b, 2, rt)
    for gd, gr, name in zip(grads, refs, ("dq", "dk", "dv")):
        gn = gd.float().cpu().numpy()
        assert np.isfinite(gn).all()
        if not np.abs(gr).max() > 0:   # a softmax over one element passes no gradient: zero up to fp32 rounding
            assert np.abs(gn).max() < 1e-5, name
            continue
        assert_grad_close(gn, gr, 5e-2, name)
    assert hip_library_loaded()
