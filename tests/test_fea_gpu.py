"""GPU parity of the flash-entropy forward (HIP kernel through the C ABI) against the CPU oracle.

Mirrors the reference's tests/test_vmonarch.py:27-42 parameters (N in {128, 200, 1024},
(D, Dv) in {(64, 64), (128, 128), (64, 128), (128, 256)}, B=2, H=3) plus the BASELINE cfg2 shape,
fp16, padding semantics, split-KV, strided inputs and entropy closed forms.
Tolerances: reference metric max|x - ref| <= 2e-2 * max|ref| (tests/test_vmonarch.py:22-24, :39-40)
AND elementwise |x - ref| <= 2e-2 + 1e-2 |ref|.
"""
import numpy as np
import pytest
import torch

from conftest import (assert_close_elementwise, elementwise_margin, assert_close_ref, assert_grad_close, golden_names, hip_library_loaded,
                      load_golden, randn_lp)
from oracle import entropy_attention

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _check(o, e, o_ref, e_ref):
    o, e = o.float().cpu().numpy(), e.float().cpu().numpy()
    assert np.isfinite(o).all() and np.isfinite(e).all()
    assert_close_ref(o, o_ref, 2e-2)
    assert_close_ref(e, e_ref, 2e-2)
    assert_close_elementwise(o, o_ref)
    assert_close_elementwise(e, e_ref)


@pytest.mark.parametrize("name", golden_names("fea_"))
def test_fea_forward_matches_reference_golden(name):
    from vmonarch_amd import flash_entropy_attention
    g = load_golden(name)
    q, k, v = (torch.from_numpy(g[x]).to(torch.bfloat16).to(DEV) for x in "qkv")
    o, e = flash_entropy_attention(q, k, v, float(g["sm_scale"]))
    _check(o, e, g["o"], g["e"])
    assert hip_library_loaded()


@pytest.mark.parametrize("N", [128, 200, 1024])
@pytest.mark.parametrize("D, Dv", [(64, 64), (128, 128), (64, 128), (128, 256)])
def test_fea_forward_reference_params(N, D, Dv):
    from vmonarch_amd import flash_entropy_attention
    g = torch.Generator().manual_seed(0)
    q, k, v = randn_lp(g, 2, 3, N, D), randn_lp(g, 2, 3, N, D), randn_lp(g, 2, 3, N, Dv)
    o, e = flash_entropy_attention(q.to(DEV), k.to(DEV), v.to(DEV))
    assert o.shape == (2, 3, N, Dv) and o.dtype == torch.bfloat16 and e.shape == (2, 3, N) and e.dtype == torch.float32
    o_ref, e_ref = entropy_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), D ** -0.5)
    _check(o, e, o_ref, e_ref)


@pytest.mark.parametrize("D, Dv", [(64, 64), (128, 128)])
def test_fea_forward_fp16(D, Dv):
    from vmonarch_amd import flash_entropy_attention
    g = torch.Generator().manual_seed(1)
    q, k, v = (randn_lp(g, 1, 2, 333, d, dtype=torch.float16) for d in (D, D, Dv))
    o, e = flash_entropy_attention(q.to(DEV), k.to(DEV), v.to(DEV))
    assert o.dtype == torch.float16
    o_ref, e_ref = entropy_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), D ** -0.5)
    _check(o, e, o_ref, e_ref)


def test_fea_forward_cfg2_sampled_rows():
    """BASELINE cfg2: B=2, H=4, N=4096, D=128, bf16; oracle on 384 query rows per head (all keys)."""
    from vmonarch_amd import flash_entropy_attention
    g = torch.Generator().manual_seed(0)
    q, k, v = (randn_lp(g, 2, 4, 4096, 128) for _ in range(3))
    o, e = flash_entropy_attention(q.to(DEV), k.to(DEV), v.to(DEV))
    rows = torch.randperm(4096, generator=g)[:384].sort().values.numpy()
    o_ref, e_ref = entropy_attention(q.float().numpy()[:, :, rows], k.float().numpy(), v.float().numpy(), 128 ** -0.5)
    _check(o[:, :, rows], e[:, :, rows], o_ref, e_ref)


@pytest.mark.parametrize("N", [1, 2, 63, 64, 65, 127, 129, 1560])
def test_fea_entropy_uniform_rows_is_log_n(N):
    """Identical keys make every row uniform: e = ln N exactly in math, o = mean(v)."""
    from vmonarch_amd import flash_entropy_attention
    g = torch.Generator().manual_seed(N)
    q = randn_lp(g, 1, 1, N, 64).to(DEV)
    k = randn_lp(g, 1, 1, 1, 64).expand(1, 1, N, 64).contiguous().to(DEV)
    v = randn_lp(g, 1, 1, N, 64).to(DEV)
    o, e = flash_entropy_attention(q, k, v)
    np.testing.assert_allclose(e.cpu().numpy(), np.full((1, 1, N), np.log(N)), atol=2e-3 * max(1.0, np.log(N)))
    assert_close_elementwise(o.float().cpu().numpy(), np.broadcast_to(v.float().cpu().numpy().mean(2, keepdims=True), (1, 1, N, 64)))


def test_fea_padding_rows_follow_reference_semantics():
    """_FlashEntropyAttention.apply with n_valid < N: keys >= n_valid masked, rows >= n_valid zero
    (kernel.py:352-353)."""
    from vmonarch_amd.kernel import _FlashEntropyAttention
    g = torch.Generator().manual_seed(3)
    q, k, v = (randn_lp(g, 1, 2, 256, 64) for _ in range(3))
    o, e = _FlashEntropyAttention.apply(q.to(DEV), k.to(DEV), v.to(DEV), 0.125, 200, True)
    assert (o[:, :, 200:] == 0).all() and (e[:, :, 200:] == 0).all()
    o_ref, e_ref = entropy_attention(*(t.float().numpy()[:, :, :200] for t in (q, k, v)), 0.125)
    _check(o[:, :, :200], e[:, :, :200], o_ref, e_ref)


def test_fea_strided_inputs():
    """q / k / v as (B, N, H, D) permuted views (DiT layout) are read in place."""
    from vmonarch_amd import flash_entropy_attention
    g = torch.Generator().manual_seed(4)
    q, k, v = (randn_lp(g, 2, 300, 3, 128).to(DEV).transpose(1, 2) for _ in range(3))
    assert not q.is_contiguous()
    o, e = flash_entropy_attention(q, k, v)
    o_ref, e_ref = entropy_attention(*(t.float().cpu().numpy() for t in (q, k, v)), 128 ** -0.5)
    _check(o, e, o_ref, e_ref)
    # o comes back in the caller's layout: a (B, N, H, Dv) buffer viewed as (B, H, N, Dv)
    assert o.shape == (2, 3, 300, 128) and o.stride() == (300 * 3 * 128, 128, 3 * 128, 1)


@pytest.mark.parametrize("D, Dv", [(16, 16), (32, 64), (64, 32)])
def test_fea_narrow_head_dims(D, Dv):
    from vmonarch_amd import flash_entropy_attention
    g = torch.Generator().manual_seed(5)
    q, k, v = randn_lp(g, 1, 2, 150, D), randn_lp(g, 1, 2, 150, D), randn_lp(g, 1, 2, 150, Dv)
    o, e = flash_entropy_attention(q.to(DEV), k.to(DEV), v.to(DEV))
    assert o.shape[-1] == Dv
    o_ref, e_ref = entropy_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), D ** -0.5)
    _check(o, e, o_ref, e_ref)


@pytest.mark.parametrize("N", [77, 256, 1000])
def test_fea_head_dim_256(N):
    """D = Dv = 256, the widest head the reference accepts (kernel.py:324, Dv a multiple of D)."""
    from vmonarch_amd import flash_entropy_attention
    g = torch.Generator().manual_seed(N)
    q, k, v = (randn_lp(g, 1, 2, N, 256) for _ in range(3))
    print(f"fea D=256 N={N}", flush=True)
    o, e = flash_entropy_attention(q.to(DEV), k.to(DEV), v.to(DEV))
    o_ref, e_ref = entropy_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), 256 ** -0.5)
    _check(o, e, o_ref, e_ref)


@pytest.mark.parametrize("N", [77, 300])
def test_fea_head_dim_256_backward(N):
    """D = Dv = 256 gradients (q, k, v) against the oracle, tests/test_vmonarch.py:27-42's loss."""
    from oracle import entropy_attention_grad
    g = torch.Generator().manual_seed(30 + N)
    q, k, v = (randn_lp(g, 1, 2, N, 256) for _ in range(3))
    do, de = torch.randn(1, 2, N, 256, generator=g), torch.randn(1, 2, N, generator=g)
    print(f"fea bwd D=256 N={N}", flush=True)
    grads = _grads(q, k, v, do, de)
    refs = entropy_attention_grad(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                  do.bfloat16().float().numpy(), de.numpy(), 256 ** -0.5)
    _check_grads(grads, refs)


def test_fea_head_dim_256_with_narrower_values_is_not_built():
    from vmonarch_amd import flash_entropy_attention
    q = torch.zeros(1, 1, 64, 256, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError):
        flash_entropy_attention(q, q, q[..., :128])


@pytest.mark.parametrize("splits", [1, 2, 4, 7])
def test_fea_split_kv_cross_attention(splits):
    """Nq != Nk with split-KV (the recompute path): o and lse against the oracle."""
    from vmonarch_amd.kernel import fea_forward
    g = torch.Generator().manual_seed(6)
    q, k, v = randn_lp(g, 2, 3, 300, 128), randn_lp(g, 2, 3, 3000, 128), randn_lp(g, 2, 3, 3000, 128)
    o, lse, _ = fea_forward(q.to(DEV), k.to(DEV), v.to(DEV), None, 128 ** -0.5, want_ent=False, num_splits=splits)
    o_ref, _ = entropy_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), 128 ** -0.5)
    assert_close_ref(o.float().cpu().numpy(), o_ref, 2e-2)
    assert_close_elementwise(o.float().cpu().numpy(), o_ref)
    s = (q.double() @ k.double().transpose(-1, -2)).numpy() * 128 ** -0.5 / np.log(2)
    lse_ref = np.log2(np.exp2(s - s.max(-1, keepdims=True)).sum(-1)) + s.max(-1)
    np.testing.assert_allclose(lse.cpu().numpy(), lse_ref, atol=2e-2, rtol=1e-3)


def test_fea_two_value_tensors_alias_k():
    """w0 = k, w1 = v writes [P k | P v] (replaces torch.cat([k, v], -1) of vmonarch.py:50)."""
    from vmonarch_amd.kernel import fea_forward
    g = torch.Generator().manual_seed(7)
    q, k, v = (randn_lp(g, 1, 2, 3 * 100, 128) for _ in range(3))
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    o, _, ent = fea_forward(qd, kd, kd, vd, 0.09, frames=3)
    qn, kn, vn = (t.float().numpy().reshape(1, 2, 3, 100, 128) for t in (q, k, v))
    o_ref, e_ref = entropy_attention(qn, kn, np.concatenate([kn, vn], -1), 0.09)
    _check(o.view(1, 2, 3, 100, 256), ent.view(1, 2, 3, 100), o_ref, e_ref)


def test_fea_forward_is_deterministic():
    from vmonarch_amd import flash_entropy_attention
    g = torch.Generator().manual_seed(8)
    q, k, v = (randn_lp(g, 1, 4, 777, 128).to(DEV) for _ in range(3))
    o1, e1 = flash_entropy_attention(q, k, v)
    o2, e2 = flash_entropy_attention(q, k, v)
    assert torch.equal(o1, o2) and torch.equal(e1, e2)


# ----------------------------------------------------------------------------------- backward
def _grads(q, k, v, do, de, sm_scale=None):
    from vmonarch_amd import flash_entropy_attention
    qd, kd, vd = (t.to(DEV).requires_grad_() for t in (q, k, v))
    o, e = flash_entropy_attention(qd, kd, vd, sm_scale)
    loss = (o.float() * do.to(DEV)).sum() + (e * de.to(DEV)).sum()   # tests/test_vmonarch.py:35
    return torch.autograd.grad(loss, (qd, kd, vd))


def _check_grads(grads, refs, tol=3e-2):
    for g, r, name in zip(grads, refs, ("dq", "dk", "dv")):
        assert_grad_close(g.float().cpu().numpy(), r, tol, name)


@pytest.mark.parametrize("N", [128, 200, 1024])
@pytest.mark.parametrize("D, Dv", [(64, 64), (128, 128), (64, 128), (128, 64), (128, 256), (64, 256)])
def test_fea_backward_reference_params(N, D, Dv):
    """tests/test_vmonarch.py:27-42: loss = sum(o * do) + sum(e * de); grads within 3e-2."""
    from oracle import entropy_attention_grad
    g = torch.Generator().manual_seed(0)
    q, k, v = randn_lp(g, 2, 3, N, D), randn_lp(g, 2, 3, N, D), randn_lp(g, 2, 3, N, Dv)
    do, de = torch.randn(2, 3, N, Dv, generator=g), torch.randn(2, 3, N, generator=g)
    grads = _grads(q, k, v, do, de)
    # the bf16 output o receives do rounded to bf16 (the .float() of the loss casts its grad back)
    refs = entropy_attention_grad(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                  do.bfloat16().float().numpy(), de.numpy(), D ** -0.5)
    _check_grads(grads, refs)


@pytest.mark.parametrize("N", [1, 2, 33, 65, 97])
@pytest.mark.parametrize("D, Dv", [(64, 64), (128, 128), (128, 256)])
def test_fea_backward_tiny_and_ragged_lengths(N, D, Dv):
    """Lengths below one stage and one key / query past a stage boundary (the peeled, masked stages)."""
    from oracle import entropy_attention_grad
    g = torch.Generator().manual_seed(N + D + Dv)
    q, k, v = randn_lp(g, 1, 2, N, D), randn_lp(g, 1, 2, N, D), randn_lp(g, 1, 2, N, Dv)
    do, de = torch.randn(1, 2, N, Dv, generator=g), torch.randn(1, 2, N, generator=g)
    print(f"fea bwd N={N} D={D} Dv={Dv}", flush=True)
    grads = _grads(q, k, v, do, de)
    refs = entropy_attention_grad(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                  do.bfloat16().float().numpy(), de.numpy(), D ** -0.5)
    if N == 1:   # one key: P = 1, so dq = dk = 0 (up to the fp32 rounding of dP - delta) and dv = do
        assert float(grads[0].abs().max()) < 1e-4 and float(grads[1].abs().max()) < 1e-4
    _check_grads(grads if N > 1 else grads[2:], refs if N > 1 else refs[2:])


def test_fea_backward_entropy_term_only():
    """do = 0: the gradient is the entropy term alone (dS = dE P (-E - ln P))."""
    from oracle import entropy_attention_grad
    g = torch.Generator().manual_seed(11)
    q, k, v = (randn_lp(g, 1, 2, 300, 64) for _ in range(3))
    do, de = torch.zeros(1, 2, 300, 64), torch.randn(1, 2, 300, generator=g)
    grads = _grads(q, k, v, do, de)
    refs = entropy_attention_grad(q.float().numpy(), k.float().numpy(), v.float().numpy(), do.numpy(), de.numpy(), 0.125)
    _check_grads(grads[:2], refs[:2])
    assert float(grads[2].abs().max()) == 0.0


def test_fea_backward_padding_rows_get_zero_grad():
    from vmonarch_amd.kernel import _FlashEntropyAttention
    from oracle import entropy_attention_grad
    g = torch.Generator().manual_seed(12)
    q, k, v = (randn_lp(g, 1, 1, 256, 64).to(DEV).requires_grad_() for _ in range(3))
    o, e = _FlashEntropyAttention.apply(q, k, v, 0.125, 200, True)
    do, de = torch.randn(1, 1, 256, 64, generator=g), torch.randn(1, 1, 256, generator=g)
    dq, dk, dv = torch.autograd.grad((o.float() * do.to(DEV)).sum() + (e * de.to(DEV)).sum(), (q, k, v))
    for t in (dq, dk, dv):
        assert (t[:, :, 200:] == 0).all()
    refs = entropy_attention_grad(*(t.detach().float().cpu().numpy()[:, :, :200] for t in (q, k, v)),
                                  do.bfloat16().float().numpy()[:, :, :200], de.numpy()[:, :, :200], 0.125)
    _check_grads([t[:, :, :200] for t in (dq, dk, dv)], refs)


def test_fea_backward_cfg5_head_sample():
    """BASELINE cfg5: B=1, H=24, N=16384, D=128 fwd+bwd on the GPU; heads 0 and 23 against the oracle.  With
    dO, dE ~ N(0,1) the gradients over 16384 soft keys are ~1e-2, below the elementwise class's 2e-2 atol;
    the gradients are linear in (dO, dE), so both are scaled by 128 (a power of two: exact in bf16 and fp32,
    and every rounding in the kernels commutes with it) to bring them to O(1), where the elementwise
    2e-2 / 1e-2 class binds beside the reference metric."""
    from oracle import entropy_attention_grad
    g = torch.Generator().manual_seed(0)
    q, k, v = (randn_lp(g, 1, 24, 16384, 128) for _ in range(3))
    do, de = torch.randn(1, 24, 16384, 128, generator=g) * 128, torch.randn(1, 24, 16384, generator=g) * 128
    grads = _grads(q, k, v, do, de)
    for h in (0, 23):
        sl = slice(h, h + 1)
        refs = entropy_attention_grad(q[:, sl].float().numpy(), k[:, sl].float().numpy(), v[:, sl].float().numpy(),
                                      do[:, sl].bfloat16().float().numpy(), de[:, sl].numpy(), 128 ** -0.5,
                                      dtype=np.float32)
        for gd, gr, name in zip(grads, refs, ("dq", "dk", "dv")):
            print(f"  cfg5 head {h} {name}: max|ref| {np.abs(gr).max():.3f}, elementwise margin "
                  f"{elementwise_margin(gd[:, sl].float().cpu().numpy(), gr):.3f} (<= 1 passes)", flush=True)
        _check_grads([t[:, sl] for t in grads], refs)


@pytest.mark.parametrize("nq, nk, D, Dv", [(200, 8192, 64, 64), (130, 16000, 128, 128), (64, 4096, 128, 256),
                                          (40, 4096, 256, 256)])
def test_fea_backward_few_queries_many_keys(nq, nk, D, Dv):
    """nq != nk with few query tiles (the shape of VMonarch's recompute backward): the dq kernel
    splits the keys and sums fp32 partials; dE = 0 and ent = 0 as that caller passes them."""
    from oracle import entropy_attention_grad
    from vmonarch_amd.kernel import fea_forward
    from vmonarch_amd.kernel_bwd import fea_backward_raw
    g = torch.Generator().manual_seed(nq + nk)
    q, k = randn_lp(g, 1, 2, nq, D, scale=0.5), randn_lp(g, 1, 2, nk, D, scale=0.5)
    v, do = randn_lp(g, 1, 2, nk, Dv), randn_lp(g, 1, 2, nq, Dv)
    qd, kd, vd, dod = (t.to(DEV) for t in (q, k, v, do))
    o, lse, _ = fea_forward(qd, kd, vd, None, D ** -0.5)
    zeros = torch.zeros(1, 2, nq, device=DEV)
    print(f"fea_bwd nq={nq} nk={nk} D={D} Dv={Dv}", flush=True)
    grads = fea_backward_raw(qd, kd, vd, o, lse, zeros, dod, zeros, D ** -0.5)
    refs = entropy_attention_grad(q.float().numpy(), k.float().numpy(), v.float().numpy(), do.float().numpy(),
                                  np.zeros((1, 2, nq)), D ** -0.5)
    _check_grads(grads, refs)


def test_fea_backward_accumulates_into_fp32_gradients():
    """With float32 gradient views passed in, the kernels add into them (VMO_BWD_ACCUM_*): result =
    prefill + the gradients the plain call returns, for a split-KV dq and strided column slices; or
    overwrite them (VMO_BWD_F32_*)."""
    from vmonarch_amd.kernel import fea_forward
    from vmonarch_amd.kernel_bwd import fea_backward_raw
    g = torch.Generator().manual_seed(11)
    nq, nk, D, Dv = 96, 8192, 128, 128
    q, k = randn_lp(g, 1, 2, nq, D, scale=0.5).to(DEV), randn_lp(g, 1, 2, nk, D, scale=0.5).to(DEV)
    v, do = randn_lp(g, 1, 2, nk, Dv).to(DEV), randn_lp(g, 1, 2, nq, Dv).to(DEV)
    de = torch.randn(1, 2, nq, generator=g).to(DEV)
    o, lse, ent = fea_forward(q, k, v, None, D ** -0.5)
    plain = fea_backward_raw(q, k, v, o, lse, ent, do, de, D ** -0.5)
    dq0 = torch.randn(1, 2, nq, D, generator=g).to(DEV)
    kv0 = torch.randn(1, 2, nk, D + Dv + 32, generator=g).to(DEV)   # dk | dv | spare columns
    dq, kv = dq0.clone(), kv0.clone()
    fea_backward_raw(q, k, v, o, lse, ent, do, de, D ** -0.5, dq=dq, dk=kv[..., :D], dv=kv[..., D:D + Dv])
    torch.cuda.synchronize()
    torch.testing.assert_close(dq - dq0, plain[0].float(), rtol=2e-2, atol=2e-2 * plain[0].float().abs().max().item())
    torch.testing.assert_close(kv[..., :D] - kv0[..., :D], plain[1].float(), rtol=2e-2,
                               atol=2e-2 * plain[1].float().abs().max().item())
    torch.testing.assert_close(kv[..., D:D + Dv] - kv0[..., D:D + Dv], plain[2].float(), rtol=2e-2,
                               atol=2e-2 * plain[2].float().abs().max().item())
    assert torch.equal(kv[..., D + Dv:], kv0[..., D + Dv:])
    # overwrite mode (VMO_BWD_F32_*): the prefill is replaced, the spare columns stay untouched
    dq, kv = dq0.clone(), kv0.clone()
    fea_backward_raw(q, k, v, o, lse, ent, do, de, D ** -0.5, dq=dq, dk=kv[..., :D], dv=kv[..., D:D + Dv],
                     overwrite="qkv")
    torch.cuda.synchronize()
    for got, want in ((dq, plain[0]), (kv[..., :D], plain[1]), (kv[..., D:D + Dv], plain[2])):
        torch.testing.assert_close(got, want.float(), rtol=2e-2, atol=2e-2 * want.float().abs().max().item())
    assert torch.equal(kv[..., D + Dv:], kv0[..., D + Dv:])


@pytest.mark.parametrize("D, Dv", [(64, 64), (128, 128), (128, 256), (256, 256)])
def test_fea_backward_fp16(D, Dv):
    """fp16 inputs (kernel.py:13 accepts float16): gradients within the reference's 3e-2."""
    from oracle import entropy_attention_grad
    g = torch.Generator().manual_seed(D + Dv)
    q, k = randn_lp(g, 1, 2, 300, D, dtype=torch.float16), randn_lp(g, 1, 2, 300, D, dtype=torch.float16)
    v = randn_lp(g, 1, 2, 300, Dv, dtype=torch.float16)
    do, de = torch.randn(1, 2, 300, Dv, generator=g), torch.randn(1, 2, 300, generator=g)
    grads = _grads(q, k, v, do, de)
    assert all(t.dtype == torch.float16 for t in grads)
    refs = entropy_attention_grad(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                  do.half().float().numpy(), de.numpy(), D ** -0.5)
    _check_grads(grads, refs)


@pytest.mark.parametrize("nq, nk, D", [(300, 300, 64), (300, 300, 128), (40, 4096, 128), (200, 1000, 64)])
def test_fea_backward_values_in_two_parts(nq, nk, D):
    """Values given as [v0 | v1] (vmo_fea_bwd_args.v1, VMonarch's last R-step [k | v]) read in place
    give the gradients of the concatenated tensor bit for bit."""
    from vmonarch_amd.kernel import fea_forward
    from vmonarch_amd.kernel_bwd import fea_backward_raw
    g = torch.Generator().manual_seed(nq + nk + D)
    q, k = randn_lp(g, 1, 2, nq, D).to(DEV), randn_lp(g, 1, 2, nk, D).to(DEV)
    v0, v1 = randn_lp(g, 1, 2, nk, D).to(DEV), randn_lp(g, 1, 2, nk, D).to(DEV)
    w = torch.cat([v0, v1], -1)
    do = randn_lp(g, 1, 2, nq, 2 * D).to(DEV)
    de = torch.randn(1, 2, nq, generator=g).to(DEV)
    o, lse, ent = fea_forward(q, k, w, None, D ** -0.5)
    print(f"fea_bwd two-part values nq={nq} nk={nk} D={D}", flush=True)
    ref = fea_backward_raw(q, k, w, o, lse, ent, do, de, D ** -0.5)
    got = fea_backward_raw(q, k, v0, o, lse, ent, do, de, D ** -0.5, v1=v1)
    for a, b, name in zip(got, ref, ("dq", "dk", "dv")):
        assert torch.equal(a, b), name
    # values [k | v1] with the first part k itself: the kernels reuse the K operands for dP's k half,
    # accumulating in the same order, so again bit for bit
    w = torch.cat([k, v1], -1)
    o, lse, ent = fea_forward(q, k, w, None, D ** -0.5)
    ref = fea_backward_raw(q, k, w, o, lse, ent, do, de, D ** -0.5)
    got = fea_backward_raw(q, k, k, o, lse, ent, do, de, D ** -0.5, v1=v1)
    for a, b, name in zip(got, ref, ("dq", "dk", "dv")):
        assert torch.equal(a, b), "k-first " + name


@pytest.mark.parametrize("nq, nk, D, two_parts, dt", [(300, 300, 64, False, torch.bfloat16),
                                                      (300, 300, 128, False, torch.bfloat16),
                                                      (40, 4096, 128, False, torch.bfloat16),
                                                      (300, 300, 64, True, torch.bfloat16),
                                                      (200, 1000, 128, True, torch.bfloat16),
                                                      (300, 300, 128, False, torch.float16),
                                                      (200, 1000, 128, True, torch.float16)])
def test_fea_backward_fold_k(nq, nk, D, two_parts, dt):
    """VMO_BWD_FOLD_K (values k, or [k | v1]): dk holds k's key-role plus value-role gradient, dv only
    v1's.  Bit for bit the sum of the unfolded fp32 stores (one rounding each for the product and
    the sum), in the inputs' dtype the rounding of that sum, and added into an fp32 buffer within
    float32 rounding of the unfolded additions -- except for [k | v1] at d = 128, whose folded launch
    accumulates both gradients of k in one set of registers with dS rounded after its sm_scale factor
    (and stores dS^T that way for the dq GEMM): there dk and dq agree with the unfolded results within
    1e-2 of their largest element (measured ~1e-3), and v1's gradient stays bit for bit."""
    from vmonarch_amd.kernel import fea_forward
    from vmonarch_amd.kernel_bwd import fea_backward_raw
    g = torch.Generator().manual_seed(11 * nq + nk + D + two_parts)
    q, k = randn_lp(g, 1, 2, nq, D, dtype=dt).to(DEV), randn_lp(g, 1, 2, nk, D, dtype=dt).to(DEV)
    v1 = randn_lp(g, 1, 2, nk, D, dtype=dt).to(DEV) if two_parts else None
    w = torch.cat([k, v1], -1) if two_parts else k
    do = randn_lp(g, 1, 2, nq, w.shape[-1], dtype=dt).to(DEV)
    de = torch.randn(1, 2, nq, generator=g).to(DEV)
    o, lse, ent = fea_forward(q, k, w, None, D ** -0.5)
    print(f"fea_bwd fold_k nq={nq} nk={nk} D={D} two_parts={two_parts} {dt}", flush=True)
    f32 = dict(device=DEV, dtype=torch.float32)
    args = (q, k, k, o, lse, ent, do, de, D ** -0.5)
    exact = not (two_parts and D == 128)

    def same(x, ref, name):
        if exact:
            assert torch.equal(x, ref), name
        else:
            err = float((x.float() - ref.float()).abs().max())
            assert err <= 1e-2 * float(ref.float().abs().max()), f"{name}: {err}"

    # unfolded, fp32 stores
    dk_ref, dv_ref = torch.empty(1, 2, nk, D, **f32), torch.empty(1, 2, nk, w.shape[-1], **f32)
    dq_ref, _, _ = fea_backward_raw(*args, dk=dk_ref, dv=dv_ref, overwrite="kv", v1=v1)
    k_sum = dk_ref + dv_ref[..., :D]
    # folded, fp32 stores
    dk, dv = torch.full((1, 2, nk, D), 7.0, **f32), (torch.full((1, 2, nk, D), 7.0, **f32) if two_parts else None)
    dq, _, dv_out = fea_backward_raw(*args, dk=dk, dv=dv, overwrite="kv", v1=v1, fold_k=True)
    same(dq, dq_ref, "dq")
    same(dk, k_sum, "dk")
    if two_parts:
        assert torch.equal(dv_out, dv_ref[..., D:])
    else:
        assert dv_out is None
    # folded, stored in the inputs' dtype
    _, dk_lp, dv_lp = fea_backward_raw(*args, v1=v1, fold_k=True)
    assert dk_lp.dtype == q.dtype
    same(dk_lp, k_sum.to(q.dtype), "dk in the inputs' dtype")
    if two_parts:
        assert dv_lp.shape[-1] == D and torch.equal(dv_lp, dv_ref[..., D:].to(q.dtype))
    # folded, added into fp32 buffers that already hold a gradient
    base_k = torch.randn(1, 2, nk, D, generator=g).to(DEV)
    base_v = torch.randn(1, 2, nk, D, generator=g).to(DEV)
    dk_acc, dv_acc = base_k.clone(), (base_v.clone() if two_parts else None)
    fea_backward_raw(*args, dk=dk_acc, dv=dv_acc, v1=v1, fold_k=True)
    if exact:
        torch.testing.assert_close(dk_acc, base_k + k_sum, rtol=1e-6, atol=1e-6)
    else:
        torch.testing.assert_close(dk_acc, base_k + dk, rtol=1e-6, atol=1e-6)   # the folded fp32 store above
    if two_parts:
        torch.testing.assert_close(dv_acc, base_v + dv_ref[..., D:], rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("nq, nk, D, Dv, fold, dt", [(300, 300, 128, 128, False, torch.bfloat16),
                                                    (40, 4096, 128, 128, False, torch.bfloat16),
                                                    (200, 700, 128, 256, False, torch.bfloat16),
                                                    (77, 300, 64, 64, False, torch.bfloat16),
                                                    (200, 700, 128, 256, True, torch.bfloat16),
                                                    (40, 4096, 128, 128, False, torch.float16),
                                                    (200, 700, 128, 256, True, torch.float16)])
def test_fea_backward_sum_into_dtype(nq, nk, D, Dv, fold, dt):
    """VMO_BWD_SUM_Q / _K / _V: dq, dk, dv in the inputs' dtype = fp32 base + this call's gradient, bit for
    bit the dtype rounding of the base plus the call's fp32 store (dq from one key range or summed over key
    splits, both dq routes; the dV columns split over two launches at Dv = 256 included; with
    VMO_BWD_FOLD_K the folded dk and v1's dv)."""
    from vmonarch_amd.kernel import fea_forward
    from vmonarch_amd.kernel_bwd import fea_backward_raw
    g = torch.Generator().manual_seed(13 * nq + nk + D + Dv + fold)
    q, k = randn_lp(g, 1, 2, nq, D, dtype=dt).to(DEV), randn_lp(g, 1, 2, nk, D, dtype=dt).to(DEV)
    if fold:
        v, v1 = k, randn_lp(g, 1, 2, nk, Dv - D, dtype=dt).to(DEV)
        w = torch.cat([k, v1], -1)
    else:
        v = v1 = None
        w = randn_lp(g, 1, 2, nk, Dv, dtype=dt).to(DEV)
    do = randn_lp(g, 1, 2, nq, Dv, dtype=dt).to(DEV)
    de = torch.randn(1, 2, nq, generator=g).to(DEV)
    o, lse, ent = fea_forward(q, k, w, None, D ** -0.5)
    print(f"fea_bwd sum into dtype nq={nq} nk={nk} D={D} Dv={Dv} fold={fold} {dt}", flush=True)
    args = (q, k, v if fold else w, o, lse, ent, do, de, D ** -0.5)
    f32 = dict(device=DEV, dtype=torch.float32)
    dvw = Dv - D if fold else Dv
    base_k, base_v = torch.randn(1, 2, nk, D, generator=g).to(DEV), torch.randn(1, 2, nk, dvw, generator=g).to(DEV)
    base_q = torch.randn(1, 2, nq, D, generator=g).to(DEV)
    for route in ("recompute", "ds"):
        dq32, dk32, dv32 = (torch.empty(1, 2, n, w, **f32) for n, w in ((nq, D), (nk, D), (nk, dvw)))
        fea_backward_raw(*args, dq=dq32, dk=dk32, dv=dv32, overwrite="qkv", v1=v1, fold_k=fold, dq_route=route)
        dq, dk, dv = fea_backward_raw(*args, v1=v1, fold_k=fold, dq_base=base_q, dk_base=base_k, dv_base=base_v,
                                      dq_route=route)
        assert dq.dtype == q.dtype and dk.dtype == q.dtype and dv.dtype == q.dtype
        assert torch.equal(dq, (base_q + dq32).to(q.dtype)), route
        assert torch.equal(dk, (base_k + dk32).to(q.dtype)), route
        assert torch.equal(dv, (base_v + dv32).to(q.dtype)), route


@pytest.mark.parametrize("nq, nk, D", [(300, 300, 64), (300, 300, 128), (40, 4096, 128)])
def test_fea_backward_values_are_keys(nq, nk, D):
    """Values that are k itself (VMonarch's R-steps before the last, vmonarch.py:50): the kernels
    take dP's operand from the K fragments they already read, bit for bit the result for a copy of k."""
    from vmonarch_amd.kernel import fea_forward
    from vmonarch_amd.kernel_bwd import fea_backward_raw
    g = torch.Generator().manual_seed(7 * nq + nk + D)
    q, k = randn_lp(g, 1, 2, nq, D).to(DEV), randn_lp(g, 1, 2, nk, D).to(DEV)
    do = randn_lp(g, 1, 2, nq, D).to(DEV)
    de = torch.randn(1, 2, nq, generator=g).to(DEV)
    o, lse, ent = fea_forward(q, k, k, None, D ** -0.5)
    print(f"fea_bwd values = keys nq={nq} nk={nk} D={D}", flush=True)
    ref = fea_backward_raw(q, k, k.clone(), o, lse, ent, do, de, D ** -0.5)
    got = fea_backward_raw(q, k, k, o, lse, ent, do, de, D ** -0.5)
    for a, b, name in zip(got, ref, ("dq", "dk", "dv")):
        assert torch.equal(a, b), name
