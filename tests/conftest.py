import glob
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def bf16_bits_to_f32(bits):
    """uint16 bf16 bit patterns -> float32 values (exact)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def load_golden(name):
    """Load a fixture written by tests/golden/make_golden.py; inputs come back as float32."""
    with np.load(os.path.join(GOLDEN, name), allow_pickle=False) as f:
        d = {k: f[k] for k in f.files}
    for key in ("q", "k", "v"):
        d[key] = bf16_bits_to_f32(d[key])
    return d


def golden_names(prefix):
    return sorted(os.path.basename(p) for p in glob.glob(os.path.join(GOLDEN, prefix + "*.npz")))


def assert_close_ref(x, ref, tol):
    """Reference metric (tests/test_vmonarch.py:22-24): max|x - ref| <= tol * max|ref|."""
    x = np.asarray(x, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    err = np.abs(x - ref).max()
    bound = tol * np.abs(ref).max()
    assert err <= bound, f"max abs err {err:.3e} > {tol} * max|ref| = {bound:.3e}"


def randn_lp(g, *shape, scale=1.0, dtype=None):
    """Seeded N(0, 1) * scale drawn on the CPU and rounded to a 16-bit float (bf16 by default)."""
    import torch
    return (torch.randn(*shape, generator=g) * scale).to(dtype or torch.bfloat16)


def assert_close_elementwise(x, ref, atol=2e-2, rtol=1e-2):
    """Stated bf16 tolerance: |x - ref| <= atol + rtol * |ref| elementwise."""
    np.testing.assert_allclose(np.asarray(x, dtype=np.float64), np.asarray(ref, dtype=np.float64), atol=atol, rtol=rtol)


def elementwise_margin(x, ref, atol=2e-2, rtol=1e-2):
    """max |x - ref| / (atol + rtol |ref|): the elementwise class holds where this is <= 1."""
    x = np.asarray(x, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float((np.abs(x - ref) / (atol + rtol * np.abs(ref))).max())


def assert_grad_close(g, ref, ref_tol, name=""):
    """Gradient parity: the reference metric (tests/test_vmonarch.py:22-24) with the reference's own
    gradient tolerance `ref_tol` AND the stated bf16 class elementwise, |g - ref| <= 2e-2 + 1e-2 |ref|
    (the same class as o and e)."""
    g = np.asarray(g, dtype=np.float64)
    assert np.isfinite(g).all(), f"non-finite gradient {name}"
    assert_close_ref(g, ref, ref_tol)
    assert_close_elementwise(g, ref)


def hip_library_loaded():
    import os
    from vmonarch_amd import _lib
    maps = open("/proc/self/maps").read()
    return os.path.realpath(_lib.LIB_PATH) in maps or _lib.LIB_PATH in maps
