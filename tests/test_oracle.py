"""Pins the CPU oracle (oracle/) before anything is judged against it.

Each check is chosen so that a plausible slip in the oracle (a dropped term, a wrong sign, a
transposed operand, a wrong einsum index) fails at least one of them:
  * brute-force pure-Python loops on tiny inputs (independent restatement of the formulas);
  * closed forms of the entropy (uniform -> ln n, two keys -> binary entropy, dominant -> 0);
  * central finite differences for the analytic backward;
  * golden vectors written by the reference's own code (tests/golden/make_golden.py), including its
    bf16 run, which pins every rounding point of the reduced-precision restatement;
  * reductions of VMonarch to exact attention (m=1, b=1, rt=N), permutation equivariance
    within a frame, linearity in v.
"""
import math

import numpy as np
import pytest

from conftest import assert_close_ref, golden_names, load_golden
from oracle import (entropy_attention, entropy_attention_grad, exact_attention, lstep, lstep_grad, round_bf16,
                    vmonarch_attention, vmonarch_attention_grad, vmonarch_attention_lowp)


def brute_entropy_attention(q, k, v, scale):
    """Pure-Python loops: o_i = sum_j P_ij v_j, e_i = -sum_j P_ij ln P_ij."""
    nq, nk = len(q), len(k)
    o, e = [], []
    for i in range(nq):
        s = [scale * sum(q[i][d] * k[j][d] for d in range(len(q[i]))) for j in range(nk)]
        mx = max(s)
        w = [math.exp(x - mx) for x in s]
        tot = sum(w)
        p = [x / tot for x in w]
        o.append([sum(p[j] * v[j][c] for j in range(nk)) for c in range(len(v[0]))])
        e.append(-sum(pj * math.log(pj) for pj in p if pj > 0))
    return np.array(o), np.array(e)


def test_fea_matches_brute_force_loops():
    rng = np.random.default_rng(0)
    q, k, v = rng.normal(size=(5, 3)), rng.normal(size=(7, 3)), rng.normal(size=(7, 4))
    o, e = entropy_attention(q, k, v, 0.7)
    o_b, e_b = brute_entropy_attention(q.tolist(), k.tolist(), v.tolist(), 0.7)
    np.testing.assert_allclose(o, o_b, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(e, e_b, rtol=1e-12, atol=1e-12)


def test_fea_default_scale_is_inverse_sqrt_d():
    rng = np.random.default_rng(1)
    q, k, v = rng.normal(size=(1, 2, 9, 16)), rng.normal(size=(1, 2, 9, 16)), rng.normal(size=(1, 2, 9, 8))
    o1, e1 = entropy_attention(q, k, v)
    o2, e2 = entropy_attention(q, k, v, 16 ** -0.5)
    np.testing.assert_array_equal(o1, o2)
    np.testing.assert_array_equal(e1, e2)


@pytest.mark.parametrize("n", [1, 2, 17, 1560])
def test_entropy_uniform_is_log_n(n):
    rng = np.random.default_rng(n)
    q = rng.normal(size=(3, 8))
    k = np.tile(rng.normal(size=(1, 8)), (n, 1))          # identical keys -> uniform rows
    v = rng.normal(size=(n, 5))
    o, e = entropy_attention(q, k, v, 1.0)
    np.testing.assert_allclose(e, np.full(3, math.log(n)), atol=1e-12)
    np.testing.assert_allclose(o, np.tile(v.mean(0), (3, 1)), atol=1e-12)
    o0, e0 = entropy_attention(np.zeros((2, 8)), rng.normal(size=(n, 8)), v, 1.0)  # q = 0 -> uniform
    np.testing.assert_allclose(e0, np.full(2, math.log(n)), atol=1e-12)


def test_entropy_two_keys_is_binary_entropy():
    q = np.array([[1.0, 0.0]])
    for delta in [-3.0, -0.5, 0.0, 0.25, 2.0]:
        k = np.array([[0.0, 0.0], [delta, 0.0]])
        _, e = entropy_attention(q, k, np.eye(2), 1.0)
        p = 1.0 / (1.0 + math.exp(-delta))
        h = -(p * math.log(p) + (1 - p) * math.log(1 - p))
        assert abs(e[0] - h) < 1e-12


def test_entropy_dominant_logit_goes_to_zero():
    q = np.array([[1.0]])
    k = np.array([[0.0], [0.0], [60.0], [0.0]])
    v = np.arange(8.0).reshape(4, 2)
    o, e = entropy_attention(q, k, v, 1.0)
    assert 0.0 <= e[0] < 1e-20
    np.testing.assert_allclose(o[0], v[2], atol=1e-20)


@pytest.mark.parametrize("nq,nk,d,dv", [(4, 6, 3, 2), (3, 3, 5, 4)])
def test_fea_grad_matches_finite_differences(nq, nk, d, dv):
    rng = np.random.default_rng(nq * 100 + nk)
    q, k, v = rng.normal(size=(nq, d)), rng.normal(size=(nk, d)), rng.normal(size=(nk, dv))
    do, de = rng.normal(size=(nq, dv)), rng.normal(size=(nq,))
    scale = 0.8

    def loss(q_, k_, v_):
        o, e = entropy_attention(q_, k_, v_, scale)
        return (o * do).sum() + (e * de).sum()

    grads = entropy_attention_grad(q, k, v, do, de, scale)
    eps = 1e-6
    for x, g in zip((q, k, v), grads):
        num = np.zeros_like(x)
        for idx in np.ndindex(x.shape):
            xp, xm = x.copy(), x.copy()
            xp[idx] += eps
            xm[idx] -= eps
            args_p = [xp if a is x else a for a in (q, k, v)]
            args_m = [xm if a is x else a for a in (q, k, v)]
            num[idx] = (loss(*args_p) - loss(*args_m)) / (2 * eps)
        np.testing.assert_allclose(g, num, rtol=1e-6, atol=1e-7)


def _numeric_grads(loss, xs, eps=1e-6):
    """Central differences of the scalar loss(*xs) with respect to every element of every x."""
    out = []
    for n, x in enumerate(xs):
        num = np.zeros_like(x)
        for idx in np.ndindex(x.shape):
            xp, xm = x.copy(), x.copy()
            xp[idx] += eps
            xm[idx] -= eps
            num[idx] = (loss(*xs[:n], xp, *xs[n + 1:]) - loss(*xs[:n], xm, *xs[n + 1:])) / (2 * eps)
        out.append(num)
    return out


@pytest.mark.parametrize("last", [False, True])
@pytest.mark.parametrize("min_col_mass", [0.01, 0.7])
def test_lstep_grad_matches_finite_differences(last, min_col_mass):
    # m = 4 frames: with min_col_mass 0.7 some columns of attn sum below it (clamp active), some above
    rng = np.random.default_rng(7 + last)
    B, H, m, b, D, Dv = 1, 2, 4, 3, 3, 2
    qg = rng.normal(size=(B, H, m, b, D))
    out = rng.normal(size=(B, H, m, b, D + (Dv if last else 0)))
    neg_ent = rng.normal(size=(B, H, m, b))
    grad = rng.normal(size=(B, H, m, b, Dv if last else D))
    scale = 0.7
    if not last and min_col_mass > 0.5:
        attn_sums = []
        kr = out[..., :D] * scale
        logits = np.einsum("bhijd,bhkjd->bhjik", qg, kr) - np.swapaxes(neg_ent, -1, -2)[..., None, :]
        a = np.exp(logits - logits.max(-1, keepdims=True))
        a /= a.sum(-1, keepdims=True)
        attn_sums = a.sum(-2)
        assert (attn_sums < min_col_mass).any() and (attn_sums > min_col_mass).any()

    def loss(qg_, out_):
        return (lstep(qg_, out_, neg_ent, scale, last, min_col_mass) * grad).sum()

    dq, dout = lstep_grad(qg, out, neg_ent, scale, last, grad, min_col_mass)
    nq, nout = _numeric_grads(loss, [qg, out])
    np.testing.assert_allclose(dq, nq, rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(dout, nout, rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("iters,rt,min_col_mass", [(1, 0, 0.01), (2, 4, 0.01), (3, 0, 0.6), (2, 0, 0.6)])
def test_vmonarch_grad_matches_finite_differences(iters, rt, min_col_mass):
    rng = np.random.default_rng(iters * 10 + rt)
    B, H, m, b, D, Dv = 1, 1, 3, 4, 3, 2
    q, k = rng.normal(size=(B, H, m * b, D)), rng.normal(size=(B, H, m * b, D))
    v, gz = rng.normal(size=(B, H, m * b, Dv)), rng.normal(size=(B, H, m * b, Dv))
    rec = []
    vmonarch_attention(q, k, v, m, b, iters, rt, min_col_mass, record=rec)
    frozen = [r[3] for r in rec]   # the reference detaches the entropy bias (vmonarch.py:26)

    def loss(q_, k_, v_):
        z = vmonarch_attention(q_, k_, v_, m, b, iters, rt, min_col_mass, frozen_neg_ent=frozen)
        return (z * gz).sum()

    grads = vmonarch_attention_grad(q, k, v, gz, m, b, iters, rt, min_col_mass)
    for g, n in zip(grads, _numeric_grads(loss, [q, k, v])):
        np.testing.assert_allclose(g, n, rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("name", golden_names("fea_"))
def test_fea_oracle_matches_reference_golden(name):
    g = load_golden(name)
    o, e = entropy_attention(g["q"], g["k"], g["v"], float(g["sm_scale"]))
    assert_close_ref(o, g["o"], 1e-5)
    assert_close_ref(e, g["e"], 1e-5)
    np.testing.assert_allclose(o, g["o"], atol=2e-5, rtol=1e-4)
    np.testing.assert_allclose(e, g["e"], atol=2e-5, rtol=1e-4)


@pytest.mark.parametrize("name", golden_names("vmonarch_"))
def test_vmonarch_oracle_matches_reference_golden(name):
    g = load_golden(name)
    z = vmonarch_attention(g["q"], g["k"], g["v"], int(g["num_blocks"]), int(g["block_size"]),
                           int(g["num_iters"]), int(g["recompute_tokens"]))
    assert_close_ref(z, g["z"], 1e-5)
    np.testing.assert_allclose(z, g["z"], atol=5e-5, rtol=1e-4)


def _qkv(seed, B, H, N, D, Dv=None):
    rng = np.random.default_rng(seed)
    return rng.normal(size=(B, H, N, D)), rng.normal(size=(B, H, N, D)), rng.normal(size=(B, H, N, Dv or D))


@pytest.mark.parametrize("iters", [1, 2, 3])
def test_vmonarch_single_frame_is_exact_attention(iters):
    q, k, v = _qkv(3, 1, 2, 24, 8)
    z = vmonarch_attention(q, k, v, 1, 24, iters)
    np.testing.assert_allclose(z, exact_attention(q, k, v), atol=1e-12)


@pytest.mark.parametrize("iters", [1, 2, 3])
def test_vmonarch_single_token_frames_is_exact_attention(iters):
    q, k, v = _qkv(4, 1, 2, 10, 8, 6)
    z = vmonarch_attention(q, k, v, 10, 1, iters)
    np.testing.assert_allclose(z, exact_attention(q, k, v), atol=1e-12)


def test_vmonarch_full_recompute_is_exact_attention():
    q, k, v = _qkv(5, 1, 1, 4 * 6, 8)
    z = vmonarch_attention(q, k, v, 4, 6, 2, recompute_tokens=24)
    np.testing.assert_allclose(z, exact_attention(q, k, v), atol=1e-12)
    z2 = vmonarch_attention(q, k, v, 4, 6, 2, recompute_tokens=6)
    np.testing.assert_allclose(z2[:, :, :6], exact_attention(q[:, :, :6], k, v), atol=1e-12)


def test_vmonarch_permutation_equivariant_within_frames():
    m, b = 3, 7
    q, k, v = _qkv(6, 1, 1, m * b, 8)
    perm = np.random.default_rng(9).permutation(b)
    full = (np.arange(m)[:, None] * b + perm[None, :]).reshape(-1)
    z = vmonarch_attention(q, k, v, m, b, 2, recompute_tokens=b)
    zp = vmonarch_attention(q[:, :, full], k[:, :, full], v[:, :, full], m, b, 2, recompute_tokens=b)
    np.testing.assert_allclose(zp, z[:, :, full], atol=1e-12)


def test_vmonarch_linear_in_v():
    q, k, v = _qkv(7, 1, 1, 4 * 5, 8)
    v2 = np.random.default_rng(8).normal(size=v.shape)
    za = vmonarch_attention(q, k, 2.0 * v - 3.0 * v2, 4, 5, 2, recompute_tokens=5)
    zb = 2.0 * vmonarch_attention(q, k, v, 4, 5, 2, recompute_tokens=5) - 3.0 * vmonarch_attention(q, k, v2, 4, 5, 2, recompute_tokens=5)
    np.testing.assert_allclose(za, zb, atol=1e-10)


def test_vmonarch_rejects_bad_shape_and_zero_iters():
    q, k, v = _qkv(8, 1, 1, 12, 4)
    with pytest.raises(AssertionError):
        vmonarch_attention(q, k, v, 5, 3)
    with pytest.raises(UnboundLocalError):
        vmonarch_attention(q, k, v, 4, 3, 0)


def test_round_bf16_is_nearest_even():
    # 1 + 2^-8 lies halfway between the bf16 neighbours 1 and 1 + 2^-7: the tie goes to the even one (1);
    # 1 + 3 * 2^-8 is the tie between 1 + 2^-7 and 1 + 2^-6 (even: 1 + 2^-6); past a tie, up
    x = np.array([1.0, 1 + 2.0 ** -8, 1 + 3 * 2.0 ** -8, 1 + 2.0 ** -8 + 2.0 ** -20, -2.5])
    np.testing.assert_array_equal(round_bf16(x), [1.0, 1.0, 1 + 2.0 ** -6, 1 + 2.0 ** -7, -2.5])


@pytest.mark.parametrize("name", golden_names("lowp_vmonarch_"))
def test_lowp_oracle_matches_reference_bf16_golden(name):
    """vmonarch_attention_lowp against the reference's own vmonarch_attention run on bf16 tensors: almost
    every element bit for bit, the rest within about one bf16 step at |z| ~ 1 (the reference's CPU
    einsums accumulate in another order, which moves a rounding now and then).  Leaving out any one rounding point makes the
    3-iteration fixture drop from all-exact to at most ~61% exact."""
    g = load_golden(name)
    z_ref = g["z"].astype(np.uint16).astype(np.uint32) << 16
    z_ref = z_ref.view(np.float32).astype(np.float64)
    args = [int(g[x]) for x in ("num_blocks", "block_size", "num_iters", "recompute_tokens")]
    z = vmonarch_attention_lowp(g["q"], g["k"], g["v"], *args)
    exact = float((z == z_ref).mean())
    assert exact >= (0.99 if args[2] == 3 else 0.9), exact
    assert np.abs(z - z_ref).max() <= 1e-2   # about one bf16 step at |z| ~ 1
    # and the fp32 restatement is visibly elsewhere (the roundings matter on these inputs)
    assert float((vmonarch_attention(g["q"], g["k"], g["v"], *args) == z_ref).mean()) < 0.05


def test_lowp_oracle_without_rounding_is_the_fp32_oracle():
    rng = np.random.default_rng(5)
    q, k, v = (rng.normal(size=(1, 2, 4 * 24, 32)) for _ in range(3))
    z = vmonarch_attention_lowp(q, k, v, 4, 24, 2, 24, rnd=lambda x: np.asarray(x, dtype=np.float64))
    np.testing.assert_allclose(z, vmonarch_attention(q, k, v, 4, 24, 2, 24), rtol=1e-12, atol=1e-12)


def test_lowp_oracle_keep_fp32_drops_exactly_the_named_roundings():
    """keep_fp32 skips the named cast points: with rounding switched off everywhere else and the three named
    points kept in fp32 the result is the fp32 oracle; each of the three, rounded on its own beside the others
    kept, moves z visibly; and on sharp inputs the variant without them (the HIP rounding points) is nearer to
    the fp32 result than the reference's full bf16 path (golden-pinned above)."""
    rng = np.random.default_rng(7)
    q, k, v = (rng.normal(size=(1, 2, 4 * 24, 32)) * s for s in (3.0, 3.0, 1.0))
    args = (4, 24, 2, 24)
    z32 = vmonarch_attention(q, k, v, *args)
    names = ("u0", "kr", "logits")

    ident = lambda x: np.asarray(x, dtype=np.float64)   # noqa: E731
    z_keep = vmonarch_attention_lowp(q, k, v, *args, rnd=ident, keep_fp32=names + ("u",), kernel_p=True)
    np.testing.assert_allclose(z_keep, z32, rtol=1e-12, atol=1e-12)
    base = np.abs(vmonarch_attention_lowp(q, k, v, *args) - z32).max()
    hip = np.abs(vmonarch_attention_lowp(q, k, v, *args, keep_fp32=names) - z32).max()
    assert hip < base
    for name in names:   # each of the three, rounded on its own, moves z
        others = tuple(n for n in names if n != name)
        z_one = vmonarch_attention_lowp(q, k, v, *args, keep_fp32=others)
        assert np.abs(z_one - vmonarch_attention_lowp(q, k, v, *args, keep_fp32=names)).max() > 1e-3, name
    with pytest.raises(ValueError):
        vmonarch_attention_lowp(q, k, v, *args, keep_fp32=("scale",))


@pytest.mark.parametrize("from_pk", [True, False])
def test_kernel_rounding_attention(from_pk):
    """The emulation of the kernels' P rounding: exactly the fp32 oracle with an identity rounding (any
    reference point m), and with bf16 rounding of p within the bounds the rounding allows: o moves by at most
    ~2 x 2^-8 max|w| (the weights p~ / sum p~ of the R-step are perturbed by <= 2^-8 relative) or 2^-9 max|w|
    (the recompute's sum p~ w / sum p), and the R-step entropy by at most ~2^-8 (max s - min s)."""
    from oracle import kernel_rounding_attention, round_bf16
    rng = np.random.default_rng(11)
    q, k = rng.normal(size=(2, 3, 40, 16)) * 1.5, rng.normal(size=(2, 3, 70, 16)) * 1.5
    w = rng.normal(size=(2, 3, 70, 24))
    o_ref, e_ref = entropy_attention(q, k, w, 0.5)
    ident = lambda x: x   # noqa: E731
    for first in (1, 32, 70):
        o, e = kernel_rounding_attention(q, k, w, 0.5, ident, entropy_from_pk=from_pk, first_keys=first)
        np.testing.assert_allclose(o, o_ref, rtol=1e-10, atol=1e-10)
        if from_pk:
            np.testing.assert_allclose(e, e_ref, rtol=1e-10, atol=1e-10)
    o, e = kernel_rounding_attention(q, k, w, 0.5, round_bf16, entropy_from_pk=from_pk)
    err = np.abs(o - o_ref).max()
    assert 0 < err <= (2 * 2.0 ** -8 if from_pk else 2.0 ** -9) * np.abs(w).max(), err
    if from_pk:
        s = 0.5 * (q @ np.swapaxes(k, -1, -2))
        spread = (s.max(-1) - s.min(-1)).max()
        assert 0 < np.abs(e - e_ref).max() <= 2.0 ** -8 * spread
