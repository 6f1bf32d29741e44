"""GPU parity of the VMonarch shapes outside the one-tile L-step kernels (m <= 32 frames, head dims 64 /
128): the general L-step kernels (csrc/lstep.hip, lstep_wide_kernel / lstep_wide_bwd_kernel) for more
frames and other head dims, head dims 16 / 32 (16-wide rows held in 32-wide LDS tiles) and the zero-padded route for
D != Dv with autograd,
and the flash-entropy backward at narrow head dims -- all against the CPU oracle, with the same
tolerances as the rest of the suite: elementwise 2e-2 + 1e-2 |ref| beside the reference's metric (3e-2 for
z, 5e-2 for VMonarch gradients as tests/test_vmonarch.py:64-66, 2e-2 for one L-step's gradients, 3e-2 for
flash-entropy gradients as tests/test_vmonarch.py:42).  Each test asserts that the HIP path ran: no
composed-path warning, and the autograd node of the HIP Function.
"""
import warnings

import numpy as np
import pytest
import torch

from conftest import assert_close_elementwise, assert_close_ref, assert_grad_close, hip_library_loaded, randn_lp
from oracle import entropy_attention_grad, lstep, lstep_grad, vmonarch_attention as vmonarch_oracle
from oracle import vmonarch_attention_grad

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
BF16, FP16 = torch.bfloat16, torch.float16


def _r5(t, m, b):
    B, H, N, F = t.shape
    return t.float().cpu().numpy().reshape(B, H, m, b, F)


def _grids(ms, dims, lasts, bwd):
    """(m, d, dv, last) for the grids some HIP L-step kernel takes (the others are refused on the host: the LDS of a
    CU bounds a column's tiles; a non-last step has no value width of its own)."""
    from vmonarch_amd.vmonarch import _lstep_supported
    return [(m, d, dv, last) for m in ms for d, dv in dims for last in lasts
            if _lstep_supported(m, d, dv, bwd) and (last or not bwd or d == dv)]


# m = 140: past the multi-block kernels (the general ones)
@pytest.mark.parametrize("m, d, dv, last", _grids([7, 33, 40, 41, 48, 64, 65, 96, 128, 140],
                                                  [(64, 64), (128, 128), (32, 32), (128, 64), (32, 128), (256, 256),
                                                   (16, 16)], [False, True], False))
def test_general_lstep_forward_matches_oracle(m, d, dv, last):
    from vmonarch_amd.vmonarch import _lstep_launch
    g = torch.Generator().manual_seed(7 * m + d + dv + last)
    B, H, b = 1, 2, 24
    N = m * b
    q = randn_lp(g, B, H, N, d)
    out = randn_lp(g, B, H, N, d + (dv if last else 0), scale=0.5)
    ent = torch.rand(B, H, N, generator=g) * 3.0
    res = torch.zeros(B, H, N, dv if last else d, dtype=torch.bfloat16, device=DEV)
    skip = b if last else 0
    print(f"general lstep m={m} d={d} dv={dv} last={last}", flush=True)
    _lstep_launch(q.to(DEV), out.to(DEV), ent.to(DEV), res, m, b, d ** -0.5, last, skip, 0.01)
    torch.cuda.synchronize()
    ref = lstep(_r5(q, m, b), _r5(out, m, b), -ent.numpy().reshape(B, H, m, b), d ** -0.5, last, 0.01)
    got = _r5(res, m, b)
    if last:   # tokens < skip belong to the recompute: left untouched
        assert (got[:, :, 0] == 0).all()
        got, ref = got[:, :, 1:], ref[:, :, 1:]
    assert_close_ref(got, ref, 2e-2)
    assert_close_elementwise(got, ref)
    assert hip_library_loaded()


# m = 129: the general kernel (fits at 16 / 16); mcm 0.6 keeps the column-mass clamp active
@pytest.mark.parametrize("m, d, dv, last, mcm",
                         [(m, d, dv, last, mcm) for m, d, dv, last in
                          _grids([7, 33, 40, 41, 48, 64, 65, 96, 128, 129], [(64, 64), (128, 128), (32, 32), (64, 128), (128, 32),
                                                                      (128, 64), (16, 16)], [False, True], True)
                          for mcm in ((0.01,) if last else (0.01, 0.6))])
def test_general_lstep_backward_matches_oracle(m, d, dv, last, mcm):
    from vmonarch_amd.vmonarch import _lstep_bwd_launch
    g = torch.Generator().manual_seed(11 * m + d + dv + last + int(10 * mcm))
    B, H, b = 1, 2, 20
    N = m * b
    wout = d + (dv if last else 0)
    q = randn_lp(g, B, H, N, d)
    out = randn_lp(g, B, H, N, wout, scale=0.5)
    ent = torch.rand(B, H, N, generator=g) * 3.0
    grad = randn_lp(g, B, H, N, dv if last else d)
    skip = b if last else 0
    dq0 = torch.randn(B, H, N, d, generator=g)
    dq = dq0.to(DEV)
    dout = torch.empty((B, H, N, wout), device=DEV, dtype=q.dtype)
    print(f"general lstep_bwd m={m} d={d} dv={dv} last={last} mcm={mcm}", flush=True)
    _lstep_bwd_launch(q.to(DEV), out.to(DEV), ent.to(DEV), grad.to(DEV), dq, dout, m, b, d ** -0.5, last, skip, mcm)
    torch.cuda.synchronize()
    gg = _r5(grad, m, b)
    if last:
        gg[:, :, 0] = 0.0
    dq_ref, dout_ref = lstep_grad(_r5(q, m, b), _r5(out, m, b), -ent.numpy().reshape(B, H, m, b), d ** -0.5, last, gg,
                                  mcm)
    assert_grad_close((dq.cpu() - dq0).numpy(), dq_ref.reshape(B, H, N, d), 2e-2, "dq")
    assert_grad_close(dout.float().cpu().numpy(), dout_ref.reshape(B, H, N, wout), 2e-2, "dout")
    # overwrite mode gives the increment itself, bit for bit
    dq_ow = torch.full_like(dq, 5.0)
    _lstep_bwd_launch(q.to(DEV), out.to(DEV), ent.to(DEV), grad.to(DEV), dq_ow, dout, m, b, d ** -0.5, last, skip, mcm,
                      overwrite_q=True)
    dq_inc = torch.zeros_like(dq)
    _lstep_bwd_launch(q.to(DEV), out.to(DEV), ent.to(DEV), grad.to(DEV), dq_inc, dout, m, b, d ** -0.5, last, skip, mcm)
    torch.cuda.synchronize()
    assert torch.equal(dq_ow, dq_inc)


def _no_composed_warning(fn):
    with warnings.catch_warnings():
        warnings.simplefilter("error", RuntimeWarning)
        return fn()


@pytest.mark.parametrize("m, b, D, dt", [(33, 24, 64, BF16), (48, 16, 64, BF16), (64, 12, 64, BF16), (65, 8, 64, BF16),
                                         (96, 6, 64, BF16), (128, 4, 64, BF16), (33, 20, 128, BF16), (65, 6, 128, BF16),
                                         (96, 4, 128, BF16), (128, 3, 128, BF16),
                                         # the two-block kernels on compact tiles (up to 40 frames) and past them
                                         (33, 20, 128, FP16), (40, 16, 128, FP16), (41, 16, 128, FP16), (40, 16, 128, BF16)],
                         ids=lambda x: str(x).replace("torch.", "") if isinstance(x, torch.dtype) else None)
def test_vmonarch_many_frames_forward_and_grad(m, b, D, dt):
    """More than 32 frames (HunyuanVideo's 129 frames are 33 latent frames; 128 latent frames are ~512 video
    frames) through the HIP path -- no composed-path warning -- forward without autograd and forward + backward
    with it, against the oracle."""
    from vmonarch_amd import vmonarch_attention
    g = torch.Generator().manual_seed(m + b + D)
    q, k, v = (randn_lp(g, 1, 2, m * b, D, dtype=dt) for _ in range(3))
    do = torch.randn(1, 2, m * b, D, generator=g)
    print(f"vmonarch many frames m={m} b={b}", flush=True)
    with torch.no_grad():
        z = _no_composed_warning(lambda: vmonarch_attention(q.to(DEV), k.to(DEV), v.to(DEV), m, b, 2, recompute_tokens=b))
    qn, kn, vn = (t.float().numpy() for t in (q, k, v))
    z_ref = vmonarch_oracle(qn, kn, vn, m, b, 2, b)
    zz = z.float().cpu().numpy()
    assert_close_ref(zz, z_ref, 3e-2)
    assert_close_elementwise(zz, z_ref)
    leaves = [t.to(DEV).requires_grad_() for t in (q, k, v)]
    zg = _no_composed_warning(lambda: vmonarch_attention(*leaves, m, b, 2, recompute_tokens=b))
    assert type(zg.grad_fn).__name__ == "_VMonarchFunctionBackward"
    assert torch.equal(zg.detach(), z)
    grads = torch.autograd.grad((zg.float() * do.to(DEV)).sum(), leaves)
    refs = vmonarch_attention_grad(qn, kn, vn, do.numpy(), m, b, 2, b)
    for gd, gr, name in zip(grads, refs, ("dq", "dk", "dv")):
        assert_grad_close(gd.float().cpu().numpy(), gr, 5e-2, name)


@pytest.mark.parametrize("D, Dv", [(64, 128), (128, 64), (32, 32), (16, 16), (32, 64), (16, 32)])
def test_vmonarch_other_head_dims_forward_and_grad(D, Dv):
    """Head dims the kernels do not take as they are run on q, k, v zero-padded to one kernel width (32, 64 or
    128) with the softmax scale of the true D (32 / 32 and 16 / 16 themselves run unpadded); z and the gradients
    against the oracle."""
    from vmonarch_amd import vmonarch_attention
    g = torch.Generator().manual_seed(D + 3 * Dv)
    m, b = 4, 64
    q, k, v = randn_lp(g, 1, 2, m * b, D), randn_lp(g, 1, 2, m * b, D), randn_lp(g, 1, 2, m * b, Dv)
    do = torch.randn(1, 2, m * b, Dv, generator=g)
    print(f"vmonarch head dims D={D} Dv={Dv}", flush=True)
    with torch.no_grad():
        z = _no_composed_warning(lambda: vmonarch_attention(q.to(DEV), k.to(DEV), v.to(DEV), m, b, 2, recompute_tokens=b))
    assert z.shape == (1, 2, m * b, Dv)
    qn, kn, vn = (t.float().numpy() for t in (q, k, v))
    z_ref = vmonarch_oracle(qn, kn, vn, m, b, 2, b)
    zz = z.float().cpu().numpy()
    assert_close_ref(zz, z_ref, 3e-2)
    assert_close_elementwise(zz, z_ref)
    leaves = [t.to(DEV).requires_grad_() for t in (q, k, v)]
    zg = _no_composed_warning(lambda: vmonarch_attention(*leaves, m, b, 2, recompute_tokens=b))
    grads = torch.autograd.grad((zg.float() * do.to(DEV)).sum(), leaves)
    refs = vmonarch_attention_grad(qn, kn, vn, do.numpy(), m, b, 2, b)
    for gd, gr, t, name in zip(grads, refs, leaves, ("dq", "dk", "dv")):
        assert gd.shape == t.shape
        assert_grad_close(gd.float().cpu().numpy(), gr, 5e-2, name)


def test_vmonarch_composed_path_warns_and_matches():
    """A grid no HIP L-step takes (200 frames: beyond the LDS of a CU) still runs, on the composed path,
    with a RuntimeWarning naming the shape."""
    from vmonarch_amd import vmonarch_attention
    g = torch.Generator().manual_seed(200)
    m, b = 200, 2
    q, k, v = (randn_lp(g, 1, 1, m * b, 64) for _ in range(3))
    with pytest.warns(RuntimeWarning, match="num_blocks=200"):
        with torch.no_grad():
            z = vmonarch_attention(q.to(DEV), k.to(DEV), v.to(DEV), m, b, 2, recompute_tokens=b)
    z_ref = vmonarch_oracle(*(t.float().numpy() for t in (q, k, v)), m, b, 2, b)
    assert_close_ref(z.float().cpu().numpy(), z_ref, 3e-2)


@pytest.mark.parametrize("D, Dv", [(16, 16), (32, 32), (16, 64), (32, 128), (64, 32)])
def test_fea_backward_narrow_head_dims(D, Dv):
    """flash_entropy_attention gradients at head dims 16 / 32 (kernel.py:324 accepts them), the loss of
    tests/test_vmonarch.py:35, against the oracle."""
    from vmonarch_amd import flash_entropy_attention
    g = torch.Generator().manual_seed(50 + D + Dv)
    N = 200
    q, k, v = randn_lp(g, 1, 2, N, D), randn_lp(g, 1, 2, N, D), randn_lp(g, 1, 2, N, Dv)
    do, de = torch.randn(1, 2, N, Dv, generator=g), torch.randn(1, 2, N, generator=g)
    print(f"fea bwd narrow D={D} Dv={Dv}", flush=True)
    leaves = [t.to(DEV).requires_grad_() for t in (q, k, v)]
    o, e = flash_entropy_attention(*leaves)
    grads = torch.autograd.grad((o.float() * do.to(DEV)).sum() + (e * de.to(DEV)).sum(), leaves)
    refs = entropy_attention_grad(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                  do.bfloat16().float().numpy(), de.numpy(), D ** -0.5)
    for gd, gr, t, name in zip(grads, refs, leaves, ("dq", "dk", "dv")):
        assert gd.shape == t.shape
        assert_grad_close(gd.float().cpu().numpy(), gr, 3e-2, name)
