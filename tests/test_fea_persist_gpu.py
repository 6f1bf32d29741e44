"""GPU tests of the flash-entropy forward's tile schedule: a launch with fewer workgroups than query tiles.

When a problem has more query tiles than the GPU holds workgroups at once, each workgroup runs several tiles
in turn, and the next tile's first K / W stages and q rows load while the current tile's outputs are written.
vmo_fea_fwd_args.max_blocks caps the launch, so these tests drive every forward variant through that
schedule at small sizes -- tail tiles whose last waves have no queries, split-KV ranges of unequal length
(down to one stage), the fp8-S variants, fp16, and tiles that take the exact two-pass overflow fallback in
the middle of a workgroup's run -- and require results bit-identical to one workgroup per tile (whose parity
with the oracle the other forward tests establish; one case here checks the oracle too).
"""
import numpy as np
import pytest
import torch

from conftest import assert_close_elementwise, randn_lp
from oracle import entropy_attention

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _run(q, k, w0, w1, sm, frames=1, want_ent=True, num_splits=1, qk_fp8=False, max_blocks=0):
    from vmonarch_amd.kernel import fea_forward
    o, lse, ent = fea_forward(q, k, w0, w1, sm, frames=frames, want_ent=want_ent, num_splits=num_splits,
                              qk_fp8=qk_fp8, max_blocks=max_blocks)
    torch.cuda.synchronize()
    return o, lse, ent


def _assert_same(a, b, what):
    for x, y, name in zip(a, b, ("o", "lse", "ent")):
        if x is None:
            assert y is None
            continue
        assert torch.equal(x, y), f"{what}: {name} differs (max |diff| {float((x.float() - y.float()).abs().max())})"


def _both(label, q, k, w0, w1, sm, blocks=(8, 16), **kw):
    print(label, flush=True)
    ref = _run(q, k, w0, w1, sm, **kw)
    assert torch.isfinite(ref[0].float()).all()
    for mb in blocks:
        _assert_same(ref, _run(q, k, w0, w1, sm, max_blocks=mb, **kw), f"{label} max_blocks={mb}")
    return ref


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D, Dv", [(64, 64), (128, 128), (64, 128), (128, 256), (256, 256)])
def test_online_entropy_tiles_carried(D, Dv, dtype):
    """flash_entropy_attention (online entropy): 2 x 3 heads of 300 queries = 18 tiles (tails of 44 queries:
    two waves without queries) over 8 or 16 workgroups."""
    g = torch.Generator().manual_seed(D + Dv)
    q, k = (randn_lp(g, 2, 3, 300, D, dtype=dtype).to(DEV) for _ in range(2))
    v = randn_lp(g, 2, 3, 300, Dv, dtype=dtype).to(DEV)
    _both(f"online D={D} Dv={Dv} {dtype}", q, k, v, None, D ** -0.5)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D, Dv1", [(128, 0), (128, 128), (128, 64), (64, 0), (64, 64), (64, 128)])
def test_rstep_tiles_carried(D, Dv1, dtype):
    """VMonarch R-step variants (values k or [k | v1], P.K entropy): 2 heads x 5 frames of 200 queries = 20
    tiles, frames of 200 keys (4 stages, the last partial)."""
    g = torch.Generator().manual_seed(7 * D + Dv1)
    m, b = 5, 200
    q, k = (randn_lp(g, 1, 2, m * b, D, dtype=dtype).to(DEV) for _ in range(2))
    v = randn_lp(g, 1, 2, m * b, Dv1, dtype=dtype).to(DEV) if Dv1 else None
    _both(f"rstep D={D} Dv1={Dv1} {dtype}", q, k, k, v, D ** -0.5, frames=m)


def test_rstep_tiles_carried_matches_oracle():
    """The [k | v] R-step with 8 workgroups for 20 tiles against the oracle (elementwise 2e-2 / 1e-2)."""
    g = torch.Generator().manual_seed(11)
    m, b, D = 5, 200, 128
    q, k, v = (randn_lp(g, 1, 2, m * b, D) for _ in range(3))
    kd = k.to(DEV)
    o, _, ent = _run(q.to(DEV), kd, kd, v.to(DEV), D ** -0.5, frames=m, max_blocks=8)
    qn, kn, vn = (t.float().numpy().reshape(1, 2, m, b, D) for t in (q, k, v))
    o_ref, e_ref = entropy_attention(qn, kn, np.concatenate([kn, vn], -1), D ** -0.5)
    assert_close_elementwise(o.float().cpu().numpy().reshape(o_ref.shape), o_ref)
    assert_close_elementwise(ent.cpu().numpy().reshape(e_ref.shape), e_ref)


@pytest.mark.parametrize("D, Dv, nk, splits", [(128, 128, 3000, 4), (64, 64, 788, 4), (64, 64, 788, 1),
                                               (128, 64, 1000, 3), (64, 128, 2000, 2)])
def test_no_entropy_and_split_kv_tiles_carried(D, Dv, nk, splits):
    """The recompute variant (no entropy; split-KV with an LSE merge); 788 keys in 4 splits leave a last
    range of one stage."""
    g = torch.Generator().manual_seed(D + Dv + nk + splits)
    q = randn_lp(g, 2, 2, 330, D).to(DEV)
    k = randn_lp(g, 2, 2, nk, D).to(DEV)
    v = randn_lp(g, 2, 2, nk, Dv).to(DEV)
    _both(f"no-entropy D={D} Dv={Dv} nk={nk} splits={splits}", q, k, v, None, D ** -0.5, want_ent=False,
          num_splits=splits)


@pytest.mark.parametrize("Dv1", [0, 128])
def test_fp8_s_tiles_in_turn(Dv1):
    """fp8 S (the R-step variants) with fewer workgroups than tiles."""
    g = torch.Generator().manual_seed(5 + Dv1)
    m, b, D = 4, 200, 128
    q, k = (randn_lp(g, 1, 2, m * b, D, scale=0.5).to(DEV) for _ in range(2))
    v = randn_lp(g, 1, 2, m * b, Dv1).to(DEV) if Dv1 else None
    _both(f"fp8 S Dv1={Dv1}", q, k, k, v, D ** -0.5, frames=m, qk_fp8=True)


def _planted(g, B, H, N, D, Dv, amp, keys, dtype=torch.bfloat16):
    q = torch.randn(B, H, N, D, generator=g)
    q[:, :, : N // 2] += 1.0
    k = torch.randn(B, H, N, D, generator=g)
    for j in keys:
        k[:, :, j] = amp + 0.05 * torch.randn(B, H, D, generator=g)
    v = torch.randn(B, H, N, Dv, generator=g)
    return q.to(dtype), k.to(dtype), v.to(dtype)


@pytest.mark.parametrize("variant", ["online", "rstep_k", "rstep_kv", "split"])
def test_overflow_fallback_in_a_carried_run(variant):
    """Planted keys 70+ log2 units above the first 32 keys of their range send some tiles of a workgroup's
    run through the exact two-pass fallback; the tiles before and after run normally."""
    g = torch.Generator().manual_seed({"online": 1, "rstep_k": 2, "rstep_kv": 3, "split": 4}[variant])
    D = 128
    if variant == "online":
        q, k, v = _planted(g, 2, 2, 300, D, D, 2.0, (40, 290))
        args, kw = (q.to(DEV), k.to(DEV), v.to(DEV), None, 0.3), {}
    elif variant.startswith("rstep"):
        m, b = 4, 260
        q, k, v = _planted(g, 1, 2, m * b, D, D, 2.0, (50, 2 * b + 100, 2 * b + 255))
        kd = k.to(DEV)
        args, kw = (q.to(DEV), kd, kd, v.to(DEV) if variant == "rstep_kv" else None, 0.3), {"frames": m}
    else:
        q = torch.randn(1, 2, 330, D, generator=g)
        q[:, :, :165] += 1.0
        _, k, v = _planted(g, 1, 2, 3000, D, D, 2.0, (800, 2990), dtype=torch.float32)
        q, k, v = (t.bfloat16() for t in (q, k, v))
        args, kw = (q.to(DEV), k.to(DEV), v.to(DEV), None, 0.3), {"want_ent": False, "num_splits": 4}
    _both(f"overflow in a carried run: {variant}", *args, **kw)


def test_many_tiles_any_block_count():
    """More tiles than the GPU holds workgroups (the default launch then runs several per workgroup too): the R-step
    [k | v] at 8 heads x 21 frames of 520 queries (5 tiles each, 840 tiles) with the default launch, 64 and
    24 workgroups."""
    g = torch.Generator().manual_seed(3)
    m, b, D = 21, 520, 128
    q, k, v = (randn_lp(g, 1, 8, m * b, D, scale=0.5).to(DEV) for _ in range(3))
    _both("many tiles", q, k, k, v, D ** -0.5, blocks=(64, 24), frames=m)
