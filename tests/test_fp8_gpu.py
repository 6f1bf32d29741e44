"""The opt-in fp8 S of the VMonarch R-steps (beyond the reference): S = q k^T on v_mfma_f32_32x32x64_f8f6f4 with
e4m3 operands (q rows scaled by their own max |q| / 448 in the kernel, k by one max |k| / 448 per 64-key tile in a
pass before it), everything after S as on the 16-bit path (vmo_fea_fwd_args.qk_fp8, vmonarch_attention(...,
qk_fp8=True)).

Tolerances, from a study against the float64 oracle (three 520-token frames, values [k | v], D = 128):
* logits of std 0.25 (the cfg4 synthetic inputs, q and k x 0.5): the bf16 class of the rest of the suite holds --
  elementwise |x - ref| <= 2e-2 + 1e-2 |ref| for o and e, reference metric 3e-2 (measured: o 0.0022, e 0.0016);
* logits of std 1: an fp8 class, |o - ref| <= 6e-2 + 3e-2 |ref| and |e - ref| <= 5e-2 (measured: o 0.027,
  e 0.031 -- the entropy's LSE is the fp8 one, its mean logit q . sum p k / l the exact one; the bf16 class
  misses 9 of 798720 elements);
* sharper rows (std 2-4) are outside both: e4m3's 3-bit mantissa moves each logit by ~4% of its size (measured o
  0.34-1.36, e 0.15-0.53), which is why the mode is opt-in and the 16-bit path stays the default.  The entropy
  there also mixes the fp8 LSE with the exact mean logit (the R-steps' P.K form), so a one-hot row's e is the
  fp8 error of its dominant logit rather than 0.
"""
import numpy as np
import pytest
import torch

from conftest import assert_close_elementwise, assert_close_ref, hip_library_loaded, randn_lp
from oracle import entropy_attention, vmonarch_attention as vmonarch_oracle

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _rstep(q, k, v, F, fp8, sm=None):
    from vmonarch_amd.kernel import fea_forward
    kd = k.to(DEV)   # one tensor as keys and first values (the library checks w0 == k by address)
    sm = q.shape[-1] ** -0.5 if sm is None else sm
    o, _, e = fea_forward(q.to(DEV), kd, kd, v.to(DEV) if v is not None else None, sm, frames=F, qk_fp8=fp8)
    torch.cuda.synchronize()
    return o, e


def _oracle(q, k, v, F, sm=None):
    B, H, N, D = q.shape
    n = N // F
    per = lambda t: t.float().numpy().reshape(B, H * F, n, -1)   # noqa: E731
    w = per(k) if v is None else np.concatenate([per(k), per(v)], -1)
    o_ref, e_ref = entropy_attention(per(q), per(k), w, D ** -0.5 if sm is None else sm)
    return o_ref.reshape(B, H, N, -1), e_ref.reshape(B, H, N)


@pytest.mark.parametrize("mult", [0.5, 1.0])
@pytest.mark.parametrize("two_values", [False, True])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_fp8_rstep_against_oracle(mult, two_values, dtype):
    g = torch.Generator().manual_seed(int(10 * mult) + two_values + (dtype == torch.float16))
    F, n, D = 3, 520, 128
    q, k = randn_lp(g, 1, 2, F * n, D, scale=mult, dtype=dtype), randn_lp(g, 1, 2, F * n, D, scale=mult, dtype=dtype)
    v = randn_lp(g, 1, 2, F * n, D, dtype=dtype) if two_values else None
    print(f"fp8 rstep mult={mult} two_values={two_values} {dtype}", flush=True)
    o, e = _rstep(q, k, v, F, True)
    o_ref, e_ref = _oracle(q, k, v, F)
    oo, ee = o.float().cpu().numpy(), e.cpu().numpy()
    assert np.isfinite(oo).all() and np.isfinite(ee).all()
    if mult == 0.5:   # (with values k and soft rows o averages ~1500 keys: |o| <= ~0.1, so the metric is 3e-2)
        for x, ref in ((oo, o_ref), (ee, e_ref)):
            assert_close_ref(x, ref, 3e-2)
            assert_close_elementwise(x, ref)
    else:
        assert_close_elementwise(oo, o_ref, atol=6e-2, rtol=3e-2)
        assert_close_elementwise(ee, e_ref, atol=5e-2, rtol=0.0)
    o16, _ = _rstep(q, k, v, F, False)
    assert not torch.equal(o, o16), "the fp8 path gave the 16-bit path's bits"
    assert hip_library_loaded()


def test_fp8_vmonarch_cfg4_head_sample():
    """cfg4 (21 frames x 1560 tokens, H = 12, D = 128, q, k ~ 0.5 N(0,1)) with fp8 S in both R-steps: heads 0 and
    11 against the oracle at the suite's z tolerance (3e-2 reference metric, elementwise 2e-2 + 1e-2 |ref|)."""
    from vmonarch_amd import VMonarchAttention
    g = torch.Generator().manual_seed(0)
    q = randn_lp(g, 1, 12, 32760, 128, scale=0.5)
    k = randn_lp(g, 1, 12, 32760, 128, scale=0.5)
    v = randn_lp(g, 1, 12, 32760, 128)
    with torch.no_grad():
        z = VMonarchAttention(21, 1560, 2, qk_fp8=True)(q.to(DEV), k.to(DEV), v.to(DEV), recompute_tokens=1560)
    for h in (0, 11):
        sl = slice(h, h + 1)
        z_ref = vmonarch_oracle(q[:, sl].float().numpy(), k[:, sl].float().numpy(), v[:, sl].float().numpy(),
                                21, 1560, 2, 1560, dtype=np.float32)
        zz = z[:, sl].float().cpu().numpy()
        assert np.isfinite(zz).all()
        assert_close_ref(zz, z_ref, 3e-2)
        assert_close_elementwise(zz, z_ref)


@pytest.mark.parametrize("two_values", [False, True])
def test_fp8_overflow_fallback(two_values):
    """One key per frame ~110 log2 units above the first 32 keys of the shifted rows: the fp8 variants take the
    exact two-pass fallback (the max pass with each tile's k scale); those rows then put all their weight on the
    planted key, so o is its value row whatever the logits' fp8 error.  (Their entropy, from the fp8 LSE against
    the exact mean logit, carries that error -- these are the sharp rows outside the mode's domain -- and is
    only required to be finite.)"""
    g = torch.Generator().manual_seed(31 + two_values)
    F, n, D = 3, 260, 128
    N = F * n
    q = torch.randn(1, 2, N, D, generator=g)
    q[:, :, : N // 2] += 1.0
    k = torch.randn(1, 2, N, D, generator=g)
    keys = (50, n + 100, 2 * n + 200)
    for j in keys:
        k[:, :, j] = 2.0 + 0.05 * torch.randn(1, 2, D, generator=g)
    v = torch.randn(1, 2, N, D, generator=g)
    q, k, v = (t.bfloat16() for t in (q, k, v))
    sm = 0.3
    s = (q.float().view(1, 2, F, n, D) @ k.float().view(1, 2, F, n, D).transpose(-1, -2)) * sm * 1.4426950408889634
    gap = s.max(-1).values - s[..., :32].max(-1).values   # log2 units above the first 32 keys
    assert float(gap.max()) > 70.0, "inputs do not reach the fallback"
    print(f"fp8 overflow fallback two_values={two_values}", flush=True)
    o, e = _rstep(q, k, v if two_values else None, F, True, sm)
    o_ref, e_ref = _oracle(q, k, v if two_values else None, F, sm)
    oo, ee = o.float().cpu().numpy(), e.cpu().numpy()
    assert np.isfinite(oo).all() and np.isfinite(ee).all()
    rows = np.arange(N // 2)   # the shifted rows: each frame's rows see their frame's planted key
    assert_close_elementwise(oo[:, :, rows], o_ref[:, :, rows])


def test_fp8_rejections():
    from vmonarch_amd import vmonarch_attention
    from vmonarch_amd.kernel import fea_forward
    g = torch.Generator().manual_seed(5)
    q, k, v = (randn_lp(g, 1, 2, 4 * 128, 128).to(DEV) for _ in range(3))
    with pytest.raises(NotImplementedError, match="forward-only"):
        vmonarch_attention(q.requires_grad_(), k, v, 4, 128, qk_fp8=True)
    q64 = randn_lp(g, 1, 2, 4 * 128, 64).to(DEV)
    with pytest.raises(NotImplementedError, match="head dim 128"):
        with torch.no_grad():
            vmonarch_attention(q64, q64, q64, 4, 128, qk_fp8=True)
    with pytest.raises(RuntimeError, match="qk_fp8"):   # values that are not k: no fp8 variant
        fea_forward(q.detach(), k, v, None, 0.1, qk_fp8=True)
