"""Seeded random shapes through the flash-entropy kernels against the CPU oracle: head dims from every built
pair (narrow, mixed, wide), ragged N, several frames with nq != nk (the C ABI's `frames` problems, as the
VMonarch R-steps and the recompute use them), bf16 and fp16, strided (B, N, H, D) views, forward and
backward.  Tolerances as tests/test_fea_gpu.py: the reference metric and elementwise 2e-2 + 1e-2 |ref|
(gradients: reference metric 3e-2)."""
import numpy as np
import pytest
import torch

from conftest import assert_close_elementwise, assert_close_ref, assert_grad_close, hip_library_loaded, randn_lp
from oracle import entropy_attention, entropy_attention_grad

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
PAIRS = [(16, 16), (32, 32), (32, 64), (64, 32), (32, 128), (128, 32), (64, 64), (64, 128), (128, 64),
         (128, 128), (64, 256), (128, 256), (256, 256), (16, 32), (16, 64), (16, 128), (16, 256), (32, 256)]


def _case(seed):
    rng = np.random.default_rng(seed)
    D, Dv = PAIRS[rng.integers(len(PAIRS))]
    frames = int(rng.integers(1, 4))
    nq, nk = int(rng.integers(1, 400)), int(rng.integers(1, 400))
    dtype = torch.float16 if rng.random() < 0.3 else torch.bfloat16
    dit = bool(rng.random() < 0.4)   # (B, N, H, D) buffers viewed as (B, H, N, D)
    return D, Dv, frames, nq, nk, dtype, dit


def _tensor(g, B, H, N, D, dtype, dit):
    t = randn_lp(g, B, N, H, D, dtype=dtype) if dit else randn_lp(g, B, H, N, D, dtype=dtype)
    t = t.to(DEV)
    return t.transpose(1, 2) if dit else t


@pytest.mark.parametrize("seed", range(24))
def test_fuzz_forward_frames(seed):
    """fea_forward over `frames` problems of nq queries and nk keys (C ABI), against the oracle per frame."""
    from vmonarch_amd.kernel import fea_forward, _kernel_widths
    D, Dv, F, nq, nk, dtype, dit = _case(seed)
    if (D, Dv) != _kernel_widths(D, Dv):
        pytest.skip("padded dims go through the autograd path (test_fuzz_autograd)")
    g = torch.Generator().manual_seed(seed)
    B, H = 1, 2
    q, k, v = _tensor(g, B, H, F * nq, D, dtype, dit), _tensor(g, B, H, F * nk, D, dtype, dit), \
        _tensor(g, B, H, F * nk, Dv, dtype, dit)
    sm = D ** -0.5
    print(f"fuzz fwd seed={seed} D={D} Dv={Dv} F={F} nq={nq} nk={nk} {dtype} dit={dit}", flush=True)
    o, lse, ent = fea_forward(q, k, v, None, sm, frames=F)
    for f in range(F):
        qs = q[:, :, f * nq:(f + 1) * nq].float().cpu().numpy()
        ks = k[:, :, f * nk:(f + 1) * nk].float().cpu().numpy()
        vs = v[:, :, f * nk:(f + 1) * nk].float().cpu().numpy()
        o_ref, e_ref = entropy_attention(qs, ks, vs, sm)
        o_f = o[:, :, f * nq:(f + 1) * nq].float().cpu().numpy()
        e_f = ent[:, :, f * nq:(f + 1) * nq].cpu().numpy()
        assert np.isfinite(o_f).all() and np.isfinite(e_f).all()
        assert_close_elementwise(o_f, o_ref)
        assert_close_elementwise(e_f, e_ref)
        if np.abs(o_ref).max() > 0:
            assert_close_ref(o_f, o_ref, 2e-2)
    assert hip_library_loaded()


@pytest.mark.parametrize("seed", range(100, 112))
def test_fuzz_autograd(seed):
    """flash_entropy_attention forward and gradients (the loss of tests/test_vmonarch.py:35) at a random shape."""
    from vmonarch_amd import flash_entropy_attention
    D, Dv, _, n, _, dtype, dit = _case(seed)
    g = torch.Generator().manual_seed(seed)
    B, H = 1, 2
    q, k, v = (_tensor(g, B, H, n, d, dtype, dit) for d in (D, D, Dv))
    do, de = torch.randn(B, H, n, Dv, generator=g), torch.randn(B, H, n, generator=g)
    print(f"fuzz autograd seed={seed} D={D} Dv={Dv} N={n} {dtype} dit={dit}", flush=True)
    leaves = [t.detach().requires_grad_() for t in (q, k, v)]
    o, e = flash_entropy_attention(*leaves)
    qn, kn, vn = (t.detach().float().cpu().numpy() for t in (q, k, v))
    o_ref, e_ref = entropy_attention(qn, kn, vn, D ** -0.5)
    assert_close_elementwise(o.detach().float().cpu().numpy(), o_ref)
    assert_close_elementwise(e.detach().cpu().numpy(), e_ref)
    grads = torch.autograd.grad((o.float() * do.to(DEV)).sum() + (e * de.to(DEV)).sum(), leaves)
    refs = entropy_attention_grad(qn, kn, vn, do.to(dtype).float().numpy(), de.numpy(), D ** -0.5)
    for gd, gr, t, name in zip(grads, refs, leaves, ("dq", "dk", "dv")):
        assert gd.shape == t.shape and gd.dtype == t.dtype
        assert_grad_close(gd.float().cpu().numpy(), gr, 3e-2, name)
