"""The narrow flash-entropy kernels (heads of 32, and of 16 held as 32-wide LDS tiles with each row twice)
against the CPU oracle: the reference's narrow head dims (kernel.py:324), ragged N, fp16, frames, the
no-entropy variant called through the C ABI, the exact two-pass path of the fixed reference point, and the
gradients (dq with key splits at N = 4096).  Tolerances as tests/test_fea_gpu.py: the reference metric
(2e-2 * max|ref|, gradients 3e-2) and elementwise 2e-2 + 1e-2 |ref|."""
import numpy as np
import pytest
import torch

from conftest import assert_close_elementwise, assert_close_ref, assert_grad_close, hip_library_loaded, randn_lp
from oracle import entropy_attention, entropy_attention_grad, vmonarch_attention as vmonarch_oracle
from oracle import vmonarch_attention_grad

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
LOG2E = 1.4426950408889634


def _check(o, e, o_ref, e_ref):
    o, e = o.float().cpu().numpy(), e.float().cpu().numpy()
    assert np.isfinite(o).all() and np.isfinite(e).all()
    for x, ref in ((o, o_ref), (e, e_ref)):
        if np.abs(ref).max() > 0:   # (one key: every entropy is 0, and the relative metric has no scale)
            assert_close_ref(x, ref, 2e-2)
        assert_close_elementwise(x, ref)


@pytest.mark.parametrize("D, Dv", [(32, 32), (16, 16), (16, 32), (32, 16)])
@pytest.mark.parametrize("N", [1, 77, 300, 1024])
def test_narrow_heads_forward(D, Dv, N):
    from vmonarch_amd import flash_entropy_attention
    g = torch.Generator().manual_seed(1000 + 10 * D + Dv + N)
    q, k, v = randn_lp(g, 2, 3, N, D), randn_lp(g, 2, 3, N, D), randn_lp(g, 2, 3, N, Dv)
    print(f"narrow forward D={D} Dv={Dv} N={N}", flush=True)
    o, e = flash_entropy_attention(q.to(DEV), k.to(DEV), v.to(DEV))
    assert o.shape == (2, 3, N, Dv)
    o_ref, e_ref = entropy_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), D ** -0.5)
    _check(o, e, o_ref, e_ref)
    assert hip_library_loaded()


def test_narrow_heads_forward_fp16():
    from vmonarch_amd import flash_entropy_attention
    g = torch.Generator().manual_seed(7)
    q, k, v = (randn_lp(g, 1, 2, 500, 32, dtype=torch.float16) for _ in range(3))
    o, e = flash_entropy_attention(q.to(DEV), k.to(DEV), v.to(DEV))
    assert o.dtype == torch.float16
    o_ref, e_ref = entropy_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), 32 ** -0.5)
    _check(o, e, o_ref, e_ref)


@pytest.mark.parametrize("want_ent", [True, False])
def test_32_wide_kernel_through_the_c_abi(want_ent):
    """fea_forward on 32-wide tensors (no padding: the library rejects widths it has no kernel for), three
    frames of 200 queries and 170 keys, with and without the entropy output."""
    from vmonarch_amd.kernel import fea_forward
    g = torch.Generator().manual_seed(11)
    F, nq, nk = 3, 200, 170
    q, k, v = randn_lp(g, 1, 2, F * nq, 32), randn_lp(g, 1, 2, F * nk, 32), randn_lp(g, 1, 2, F * nk, 32)
    o, lse, ent = fea_forward(q.to(DEV), k.to(DEV), v.to(DEV), None, 0.2, frames=F, want_ent=want_ent)
    assert (ent is not None) == want_ent
    for f in range(F):
        qs, ks, vs = (t[:, :, f * n:(f + 1) * n].float().numpy() for t, n in ((q, nq), (k, nk), (v, nk)))
        o_ref, e_ref = entropy_attention(qs, ks, vs, 0.2)
        o_f = o[:, :, f * nq:(f + 1) * nq].float().cpu().numpy()
        assert_close_ref(o_f, o_ref, 2e-2)
        assert_close_elementwise(o_f, o_ref)
        s = np.einsum("bhqd,bhkd->bhqk", qs.astype(np.float64), ks.astype(np.float64)) * 0.2 * LOG2E
        lse_ref = np.log2(np.exp2(s - s.max(-1, keepdims=True)).sum(-1)) + s.max(-1)
        np.testing.assert_allclose(lse[:, :, f * nq:(f + 1) * nq].cpu().numpy(), lse_ref, atol=2e-2, rtol=1e-3)
        if want_ent:
            e_f = ent[:, :, f * nq:(f + 1) * nq].cpu().numpy()
            assert_close_elementwise(e_f, e_ref)


def test_narrow_heads_reference_point_overflow():
    """Keys 70+ log2 units above the max of the first 32 keys take the exact two-pass path (bf16)."""
    from vmonarch_amd import flash_entropy_attention
    g = torch.Generator().manual_seed(12)
    N, D = 300, 32
    q = torch.randn(1, 2, N, D, generator=g)
    q[:, :, : N // 2] += 1.0
    k = torch.randn(1, 2, N, D, generator=g)
    for j in (40, 290):   # one in the first stage, one in the last partial stage
        k[:, :, j] = 4.0 + 0.05 * torch.randn(1, 2, D, generator=g)
    v = torch.randn(1, 2, N, D, generator=g)
    q, k, v = q.bfloat16(), k.bfloat16(), v.bfloat16()
    sm = 1.0
    s = (q.double() @ k.double().transpose(-1, -2)) * sm * LOG2E
    assert float((s.amax(-1) - s[..., :32].amax(-1)).max()) > 70.0, "inputs do not reach the fallback"
    o, e = flash_entropy_attention(q.to(DEV), k.to(DEV), v.to(DEV), sm)
    o_ref, e_ref = entropy_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), sm)
    _check(o, e, o_ref, e_ref)


@pytest.mark.parametrize("D, Dv, N", [(32, 32, 77), (32, 32, 300), (32, 32, 4096), (16, 32, 300), (32, 16, 300),
                                      (16, 16, 129)])
def test_narrow_heads_backward(D, Dv, N):
    """Gradients of the loss of tests/test_vmonarch.py:35 through the 32-wide dq and dk/dv kernels (N = 4096:
    the dq kernel splits the keys four ways and reduces the partials)."""
    from vmonarch_amd import flash_entropy_attention
    g = torch.Generator().manual_seed(2000 + 10 * D + Dv + N)
    q, k, v = randn_lp(g, 1, 2, N, D), randn_lp(g, 1, 2, N, D), randn_lp(g, 1, 2, N, Dv)
    do, de = torch.randn(1, 2, N, Dv, generator=g), torch.randn(1, 2, N, generator=g)
    print(f"narrow backward D={D} Dv={Dv} N={N}", flush=True)
    leaves = [t.to(DEV).requires_grad_() for t in (q, k, v)]
    o, e = flash_entropy_attention(*leaves)
    grads = torch.autograd.grad((o.float() * do.to(DEV)).sum() + (e * de.to(DEV)).sum(), leaves)
    refs = entropy_attention_grad(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                  do.bfloat16().float().numpy(), de.numpy(), D ** -0.5)
    for gd, gr, t, name in zip(grads, refs, leaves, ("dq", "dk", "dv")):
        assert gd.shape == t.shape and gd.dtype == t.dtype
        assert_grad_close(gd.float().cpu().numpy(), gr, 3e-2, name)
    assert hip_library_loaded()


@pytest.mark.parametrize("m, b, rt", [(21, 100, 100), (8, 77, 30)])
def test_vmonarch_head_dim_32_native(m, b, rt):
    """VMonarch at D = Dv = 32 on the 32-wide flash-entropy kernels (R-steps with values k and [k | v], the
    split-KV recompute) and the general L-step kernels, no padding: z and the gradients against the oracle
    (reference metric 3e-2 / 5e-2 as tests/test_vmonarch.py:64-66, and elementwise)."""
    import vmonarch_amd.vmonarch as vm
    from vmonarch_amd import vmonarch_attention
    g = torch.Generator().manual_seed(3000 + m + b)
    q, k, v = (randn_lp(g, 1, 2, m * b, 32) for _ in range(3))
    do = torch.randn(1, 2, m * b, 32, generator=g)
    assert vm._fused_supported(q.to(DEV), k.to(DEV), v.to(DEV), m)
    print(f"vmonarch D=32 m={m} b={b} rt={rt}", flush=True)
    with torch.no_grad():
        z = vmonarch_attention(q.to(DEV), k.to(DEV), v.to(DEV), m, b, 2, recompute_tokens=rt)
    qn, kn, vn = (t.float().numpy() for t in (q, k, v))
    z_ref = vmonarch_oracle(qn, kn, vn, m, b, 2, rt)
    zz = z.float().cpu().numpy()
    assert np.isfinite(zz).all()
    assert_close_ref(zz, z_ref, 3e-2)
    assert_close_elementwise(zz, z_ref)
    leaves = [t.to(DEV).requires_grad_() for t in (q, k, v)]
    zg = vmonarch_attention(*leaves, m, b, 2, recompute_tokens=rt)
    assert type(zg.grad_fn).__name__ == "_VMonarchFunctionBackward"
    grads = torch.autograd.grad((zg.float() * do.to(DEV)).sum(), leaves)
    refs = vmonarch_attention_grad(qn, kn, vn, do.numpy(), m, b, 2, rt)
    for gd, gr, name in zip(grads, refs, ("dq", "dk", "dv")):
        assert_grad_close(gd.float().cpu().numpy(), gr, 5e-2, name)
    assert hip_library_loaded()


@pytest.mark.parametrize("D, Dv", [(32, 64), (32, 128), (64, 32), (128, 32), (16, 64), (16, 256), (32, 256)])
def test_narrow_and_wide_head_mixes(D, Dv):
    """A 32-wide (or 16-wide) dim with a wider one: the 32 / 64, 32 / 128, 32 / 256, 64 / 32, 128 / 32, 16 / 64 and
    16 / 256 kernels; o, e and the gradients against the oracle."""
    from vmonarch_amd import flash_entropy_attention
    g = torch.Generator().manual_seed(4000 + D + 3 * Dv)
    N = 333
    q, k, v = randn_lp(g, 1, 2, N, D), randn_lp(g, 1, 2, N, D), randn_lp(g, 1, 2, N, Dv)
    do, de = torch.randn(1, 2, N, Dv, generator=g), torch.randn(1, 2, N, generator=g)
    print(f"head mix D={D} Dv={Dv}", flush=True)
    leaves = [t.to(DEV).requires_grad_() for t in (q, k, v)]
    o, e = flash_entropy_attention(*leaves)
    qn, kn, vn = (t.float().numpy() for t in (q, k, v))
    o_ref, e_ref = entropy_attention(qn, kn, vn, D ** -0.5)
    _check(o.detach(), e.detach(), o_ref, e_ref)
    grads = torch.autograd.grad((o.float() * do.to(DEV)).sum() + (e * de.to(DEV)).sum(), leaves)
    refs = entropy_attention_grad(qn, kn, vn, do.bfloat16().float().numpy(), de.numpy(), D ** -0.5)
    for gd, gr, t, name in zip(grads, refs, leaves, ("dq", "dk", "dv")):
        assert gd.shape == t.shape
        assert_grad_close(gd.float().cpu().numpy(), gr, 3e-2, name)


@pytest.mark.parametrize("D, Dv", [(32, 32), (32, 64), (64, 32)])
def test_narrow_heads_backward_fp16(D, Dv):
    """fp16 through the 32-wide dq and dk/dv kernels (and a mix with a 64-wide dim)."""
    from vmonarch_amd import flash_entropy_attention
    g = torch.Generator().manual_seed(5000 + D + Dv)
    N = 300
    q, k, v = (randn_lp(g, 1, 2, N, d, dtype=torch.float16) for d in (D, D, Dv))
    do, de = torch.randn(1, 2, N, Dv, generator=g), torch.randn(1, 2, N, generator=g)
    leaves = [t.to(DEV).requires_grad_() for t in (q, k, v)]
    o, e = flash_entropy_attention(*leaves)
    assert o.dtype == torch.float16
    grads = torch.autograd.grad((o.float() * do.to(DEV)).sum() + (e * de.to(DEV)).sum(), leaves)
    refs = entropy_attention_grad(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                  do.half().float().numpy(), de.numpy(), D ** -0.5)
    for gd, gr, t, name in zip(grads, refs, leaves, ("dq", "dk", "dv")):
        assert gd.dtype == torch.float16
        assert_grad_close(gd.float().cpu().numpy(), gr, 3e-2, name)


def test_vmonarch_head_dim_32_fp16():
    """VMonarch at D = Dv = 32 in fp16, forward and gradients."""
    from vmonarch_amd import vmonarch_attention
    g = torch.Generator().manual_seed(5100)
    m, b, rt = 8, 100, 100
    q, k, v = (randn_lp(g, 1, 2, m * b, 32, dtype=torch.float16) for _ in range(3))
    do = torch.randn(1, 2, m * b, 32, generator=g)
    leaves = [t.to(DEV).requires_grad_() for t in (q, k, v)]
    z = vmonarch_attention(*leaves, m, b, 2, recompute_tokens=rt)
    assert z.dtype == torch.float16 and type(z.grad_fn).__name__ == "_VMonarchFunctionBackward"
    qn, kn, vn = (t.float().numpy() for t in (q, k, v))
    zz = z.detach().float().cpu().numpy()
    z_ref = vmonarch_oracle(qn, kn, vn, m, b, 2, rt)
    assert_close_ref(zz, z_ref, 3e-2)
    assert_close_elementwise(zz, z_ref)
    grads = torch.autograd.grad((z.float() * do.to(DEV)).sum(), leaves)
    refs = vmonarch_attention_grad(qn, kn, vn, do.numpy(), m, b, 2, rt)
    for gd, gr, name in zip(grads, refs, ("dq", "dk", "dv")):
        assert_grad_close(gd.float().cpu().numpy(), gr, 5e-2, name)


@pytest.mark.parametrize("D, Dv", [(32, 256), (32, 64), (128, 32), (64, 256), (16, 16), (16, 32), (16, 64), (16, 256)])
def test_head_mixes_make_no_padded_copies(D, Dv, monkeypatch):
    """Pairs with a native kernel run on the caller's tensors: forward and backward never zero-pad a feature dim
    (torch.nn.functional.pad is made to raise for the duration of the call), with o and the gradients checked
    against the oracle."""
    from vmonarch_amd import flash_entropy_attention

    def no_pad(*args, **kwargs):
        raise AssertionError("a zero-padded copy was made")

    g = torch.Generator().manual_seed(4100 + D + Dv)
    N = 200
    q, k, v = randn_lp(g, 1, 2, N, D), randn_lp(g, 1, 2, N, D), randn_lp(g, 1, 2, N, Dv)
    do, de = torch.randn(1, 2, N, Dv, generator=g), torch.randn(1, 2, N, generator=g)
    leaves = [t.to(DEV).requires_grad_() for t in (q, k, v)]
    print(f"head mix without padding D={D} Dv={Dv}", flush=True)
    monkeypatch.setattr(torch.nn.functional, "pad", no_pad)
    o, e = flash_entropy_attention(*leaves)
    grads = torch.autograd.grad((o.float() * do.to(DEV)).sum() + (e * de.to(DEV)).sum(), leaves)
    monkeypatch.undo()
    qn, kn, vn = (t.float().numpy() for t in (q, k, v))
    o_ref, e_ref = entropy_attention(qn, kn, vn, D ** -0.5)
    _check(o.detach(), e.detach(), o_ref, e_ref)
    refs = entropy_attention_grad(qn, kn, vn, do.bfloat16().float().numpy(), de.numpy(), D ** -0.5)
    for gd, gr, name in zip(grads, refs, ("dq", "dk", "dv")):
        assert_grad_close(gd.float().cpu().numpy(), gr, 3e-2, name)


@pytest.mark.parametrize("m, b, rt, dtype", [(21, 100, 100, torch.bfloat16), (8, 77, 30, torch.bfloat16),
                                             (40, 24, 24, torch.bfloat16), (8, 100, 100, torch.float16)])
def test_vmonarch_head_dim_16_native(m, b, rt, dtype, monkeypatch):
    """VMonarch at D = Dv = 16 (the reference runs it: kernel.py:324 takes 16-wide heads) on the 16-wide kernels --
    R-steps with values k and [k | v], the split-KV recompute, the multi-block L-steps, and their backward --
    with no zero-padded copy (torch.nn.functional.pad raises for the duration of the calls): z and the gradients
    against the oracle (reference metric 3e-2 / 5e-2 as tests/test_vmonarch.py:64-66, and z elementwise)."""
    import vmonarch_amd.vmonarch as vm
    from vmonarch_amd import vmonarch_attention

    def no_pad(*args, **kwargs):
        raise AssertionError("a zero-padded copy was made")

    g = torch.Generator().manual_seed(3100 + m + b)
    q, k, v = (randn_lp(g, 1, 2, m * b, 16, dtype=dtype) for _ in range(3))
    do = torch.randn(1, 2, m * b, 16, generator=g)
    assert vm._fused_supported(q.to(DEV), k.to(DEV), v.to(DEV), m)
    print(f"vmonarch D=16 m={m} b={b} rt={rt} {dtype}", flush=True)
    leaves = [t.to(DEV).requires_grad_() for t in (q, k, v)]
    monkeypatch.setattr(torch.nn.functional, "pad", no_pad)
    with torch.no_grad():
        z = vmonarch_attention(*(t.detach() for t in leaves), m, b, 2, recompute_tokens=rt)
    zg = vmonarch_attention(*leaves, m, b, 2, recompute_tokens=rt)
    grads = torch.autograd.grad((zg.float() * do.to(DEV)).sum(), leaves)
    monkeypatch.undo()
    assert type(zg.grad_fn).__name__ == "_VMonarchFunctionBackward"
    assert z.shape == (1, 2, m * b, 16) and z.dtype == dtype and torch.equal(zg.detach(), z)
    qn, kn, vn = (t.float().numpy() for t in (q, k, v))
    z_ref = vmonarch_oracle(qn, kn, vn, m, b, 2, rt)
    zz = z.float().cpu().numpy()
    assert np.isfinite(zz).all()
    assert_close_ref(zz, z_ref, 3e-2)
    assert_close_elementwise(zz, z_ref)
    refs = vmonarch_attention_grad(qn, kn, vn, do.numpy(), m, b, 2, rt)
    for gd, gr, t, name in zip(grads, refs, leaves, ("dq", "dk", "dv")):
        assert gd.shape == t.shape and gd.dtype == dtype
        assert_grad_close(gd.float().cpu().numpy(), gr, 5e-2, name)
    assert hip_library_loaded()
