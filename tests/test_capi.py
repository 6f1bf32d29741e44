"""CPU-side checks of the C ABI: the library loads, exports every symbol include/vmonarch_amd.h
declares, and rejects bad arguments with an error code before touching the GPU."""
import ctypes
import os
import re

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "vmonarch_amd.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vmo_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def L():
    from vmonarch_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail(f"{_lib.LIB_PATH} not built; run python -m vmonarch_amd.build")
    return _lib.lib()


def test_header_declares_the_entry_points():
    names = _declared_functions()
    for n in ("vmo_abi_version", "vmo_last_error", "vmo_fea_fwd", "vmo_fea_fwd_workspace_size", "vmo_lstep_fwd",
              "vmo_fea_bwd", "vmo_fea_bwd_workspace_size", "vmo_lstep_bwd", "vmo_fea_fwd_noalloc"):
        assert n in names


def test_library_exports_every_declared_symbol(L):
    for n in _declared_functions():
        assert hasattr(L, n), f"{n} declared in the header but not exported"


def test_abi_version(L):
    from vmonarch_amd import _lib
    assert L.vmo_abi_version() == _lib.ABI_VERSION


def test_single_hip_runtime_in_process(L):
    maps = open("/proc/self/maps").read().splitlines()
    hip = {ln.split()[-1] for ln in maps if "libamdhip64" in ln}
    assert len(hip) <= 1, hip


_DEVICE_BUFFER = []


def _addr(offset=0):
    """Base address for the views of the rejection tests below.  With a GPU visible it lies inside a real
    64 MiB device buffer that covers every view these tests describe, so a launch that slipped past the
    host checks would read valid memory and fail an assertion rather than fault the GPU; without a GPU
    (nothing can launch) it is a made-up page-aligned address."""
    import torch
    if not torch.cuda.is_available():
        return 4096 + offset
    if not _DEVICE_BUFFER:
        _DEVICE_BUFFER.append(torch.zeros(64 << 20, dtype=torch.uint8, device="cuda:0"))
    return _DEVICE_BUFFER[0].data_ptr() + 4096 + offset


def _fwd_args(**kw):
    from vmonarch_amd import _lib
    a = _lib.FeaFwdArgs()
    a.dtype, a.batch, a.heads, a.frames, a.nq, a.nk, a.d, a.dw0, a.dw1 = 0, 1, 1, 1, 128, 128, 128, 128, 0
    v = _lib.View(_addr(), 128, 128 * 128, 128)
    a.q = a.k = a.w0 = a.o = v
    a.sm_scale = 0.1
    a.num_splits = 1
    for k, x in kw.items():
        setattr(a, k, x)
    return a


@pytest.mark.parametrize("field,value,code", [
    ("dtype", 7, 1), ("d", 48, 2), ("dw0", 96, 2), ("nk", 0, 1), ("sm_scale", -1.0, 1),
])
def test_fea_fwd_rejects_bad_arguments_without_launching(L, field, value, code):
    a = _fwd_args(**{field: value})
    rc = L.vmo_fea_fwd(ctypes.byref(a), None)
    assert rc == code
    assert L.vmo_last_error().decode()


def test_fea_fwd_rejects_misaligned_rows(L):
    from vmonarch_amd import _lib
    a = _fwd_args()
    a.q = _lib.View(_addr() + 2, 128, 128 * 128, 128)
    assert L.vmo_fea_fwd(ctypes.byref(a), None) == 1
    a = _fwd_args()
    a.k = _lib.View(_addr(), 128, 128 * 128, 100)
    assert L.vmo_fea_fwd(ctypes.byref(a), None) == 1


def test_fea_fwd_split_needs_workspace(L):
    a = _fwd_args(num_splits=4, nk=4096)
    need = L.vmo_fea_fwd_workspace_size(ctypes.byref(a))
    assert need >= 4 * 128 * 128 * 4
    assert L.vmo_fea_fwd(ctypes.byref(a), None) == 3


def test_fea_fwd_empty_problem_is_a_no_op(L):
    a = _fwd_args(nq=0)
    assert L.vmo_fea_fwd(ctypes.byref(a), None) == 0


def test_lstep_rejects_too_many_blocks(L):
    """m = 200 frames: the one-tile kernels stop at 32, the multi-block ones at 128, and the general ones need
    more LDS per grid column than a CU has, so the call is refused on the host (the addresses are never
    dereferenced)."""
    from vmonarch_amd import _lib
    a = _lib.LstepArgs()
    a.dtype, a.batch, a.heads, a.num_blocks, a.block_size, a.d, a.dv = 0, 1, 1, 200, 4, 128, 128
    v = _lib.View(_addr(), 128, 128, 128)
    a.q = a.out = a.res = v
    a.ent = _addr()
    assert L.vmo_lstep_fwd(ctypes.byref(a), None) == 2
    assert b"LDS" in L.vmo_last_error()
    a.num_blocks, a.d = 40, 100   # head dim not a multiple of 8
    assert L.vmo_lstep_fwd(ctypes.byref(a), None) != 0


def test_lstep_bwd_rejects_too_many_blocks_and_null_args(L):
    from vmonarch_amd import _lib
    a = _lib.LstepBwdArgs()
    a.dtype, a.batch, a.heads, a.num_blocks, a.block_size, a.d, a.dv = 0, 1, 1, 200, 4, 128, 128
    v = _lib.View(_addr(), 128, 128, 128)
    a.q = a.out = a.grad_res = a.grad_q = a.grad_out = v
    a.ent = _addr()
    assert L.vmo_lstep_bwd(ctypes.byref(a), None) == 2   # 200 frames: beyond the multi-block kernels and the LDS
    assert b"LDS" in L.vmo_last_error()
    assert L.vmo_lstep_bwd(None, None) != 0
    a.num_blocks, a.delta = 40, _addr()                  # delta from a general (m > 32) kernel: not built
    assert L.vmo_lstep_bwd(ctypes.byref(a), None) == 2
    assert b"delta" in L.vmo_last_error()


def test_fea_bwd_rejects_unknown_and_conflicting_flags(L):
    from vmonarch_amd import _lib
    a = _lib.FeaBwdArgs()
    a.dtype, a.batch, a.heads, a.nq, a.nk, a.d, a.dv = 0, 1, 1, 128, 128, 128, 128
    v = _lib.View(_addr(), 128, 128 * 128, 128)
    a.q = a.k = a.v = a.o = a.grad_o = a.grad_q = a.grad_k = a.grad_v = v
    a.lse = a.ent = a.grad_ent = _addr()
    a.sm_scale = 0.1
    for flags in (_lib.BWD_ACCUM_K | _lib.BWD_F32_K, _lib.BWD_ACCUM_Q | _lib.BWD_F32_Q, 4096,
                  _lib.BWD_RECOMPUTE_DQ | _lib.BWD_DS_DQ):
        a.flags = flags
        assert L.vmo_fea_bwd(ctypes.byref(a), None) == 1
        assert b"flags" in L.vmo_last_error()


def test_lstep_bwd_rejects_unknown_flags(L):
    from vmonarch_amd import _lib
    a = _lib.LstepBwdArgs()
    a.dtype, a.batch, a.heads, a.num_blocks, a.block_size, a.d, a.dv = 0, 1, 1, 4, 4, 128, 128
    v = _lib.View(_addr(), 128, 128, 128)
    a.q = a.out = a.grad_res = a.grad_q = a.grad_out = v
    a.ent = _addr()
    a.flags = 2
    assert L.vmo_lstep_bwd(ctypes.byref(a), None) == 1
    assert b"flags" in L.vmo_last_error()


def test_fea_bwd_rejects_bad_value_parts(L):
    from vmonarch_amd import _lib
    a = _lib.FeaBwdArgs()
    a.dtype, a.batch, a.heads, a.nq, a.nk, a.d, a.dv = 0, 1, 1, 128, 128, 128, 256
    v = _lib.View(_addr(), 128, 128 * 128, 128)
    a.q = a.k = a.v = a.o = a.grad_o = a.grad_q = a.grad_k = a.grad_v = v
    a.lse = a.ent = a.grad_ent = _addr()
    a.sm_scale = 0.1
    a.v1, a.dv1 = _lib.View(_addr(4096), 128, 128 * 128, 256), 128    # token stride differs from v's
    assert L.vmo_fea_bwd(ctypes.byref(a), None) == 1
    assert b"v1" in L.vmo_last_error()
    a.v1, a.dv1 = _lib.View(_addr(4096), 128, 128 * 128, 128), 64     # parts of unequal width
    assert L.vmo_fea_bwd(ctypes.byref(a), None) == 2
    a.dv1 = 256                                                 # no first part left
    assert L.vmo_fea_bwd(ctypes.byref(a), None) == 1


def test_fea_bwd_fold_k_needs_values_that_start_with_k(L):
    """VMO_BWD_FOLD_K is rejected for values other than k, and for shapes without a fold kernel,
    before anything is launched."""
    from vmonarch_amd import _lib
    a = _lib.FeaBwdArgs()
    a.dtype, a.batch, a.heads, a.nq, a.nk, a.d, a.dv = 0, 1, 1, 128, 128, 128, 128
    v = _lib.View(_addr(), 128, 128 * 128, 128)
    a.q = a.k = a.o = a.grad_o = a.grad_q = a.grad_k = v
    a.v = _lib.View(_addr(4096), 128, 128 * 128, 128)          # not k
    a.grad_v = _lib.View()                              # values k alone write no grad_v
    a.lse = a.ent = a.grad_ent = _addr()
    a.sm_scale = 0.1
    a.flags = _lib.BWD_FOLD_K
    assert L.vmo_fea_bwd(ctypes.byref(a), None) == 1
    assert b"FOLD_K" in L.vmo_last_error()
    a.v = _lib.View(_addr(), 128, 128 * 128, 256)          # k's address with another token stride
    assert L.vmo_fea_bwd(ctypes.byref(a), None) == 1
    # values k at d = dv = 256: a valid request this build has no fold kernel for, rejected by the host
    # checks (no workspace is passed, so a call that got past them would still stop at the workspace
    # check and never launch)
    a.d = a.dv = 256
    a.q = a.k = a.v = a.o = a.grad_o = a.grad_q = a.grad_k = _lib.View(_addr(), 256, 256 * 128, 256)
    assert L.vmo_fea_bwd(ctypes.byref(a), None) == 2
    assert b"FOLD_K" in L.vmo_last_error()


def test_fea_bwd_sum_needs_a_base_and_no_fp32_bits(L):
    """VMO_BWD_SUM_Q / _K / _V write the gradient in the inputs' dtype from an fp32 base: together with
    ACCUM / F32 of the same gradient, or without the base view, they are rejected."""
    from vmonarch_amd import _lib
    a = _lib.FeaBwdArgs()
    a.dtype, a.batch, a.heads, a.nq, a.nk, a.d, a.dv = 0, 1, 1, 128, 128, 128, 128
    v = _lib.View(_addr(), 128, 128 * 128, 128)
    a.q = a.k = a.v = a.o = a.grad_o = a.grad_q = a.grad_k = a.grad_v = v
    a.lse = a.ent = a.grad_ent = _addr()
    a.sm_scale = 0.1
    a.grad_q_base = a.grad_k_base = a.grad_v_base = _lib.View(_addr(1 << 16), 128, 128 * 128, 128)
    for flags in (_lib.BWD_SUM_K | _lib.BWD_ACCUM_K, _lib.BWD_SUM_V | _lib.BWD_F32_V, _lib.BWD_SUM_Q | _lib.BWD_F32_Q,
                  _lib.BWD_SUM_Q | _lib.BWD_ACCUM_Q):
        a.flags = flags
        assert L.vmo_fea_bwd(ctypes.byref(a), None) == 1
        assert b"flags" in L.vmo_last_error()
    for flag, field in ((_lib.BWD_SUM_V, "grad_v_base"), (_lib.BWD_SUM_Q, "grad_q_base")):
        a.flags = flag
        saved = getattr(a, field)
        setattr(a, field, _lib.View())
        assert L.vmo_fea_bwd(ctypes.byref(a), None) == 1
        assert b"SUM" in L.vmo_last_error()
        setattr(a, field, saved)


def test_fea_fwd_noalloc_rejects_oversized_splits_without_launching(L):
    """vmo_fea_fwd_noalloc holds the split-KV partials in a fixed library scratch: a call whose partials
    would not fit is rejected with VMO_ERR_WORKSPACE before any launch."""
    from vmonarch_amd import _lib
    a = _fwd_args(nq=4096, nk=65536, num_splits=16, heads=8)
    need = L.vmo_fea_fwd_workspace_size(ctypes.byref(a))
    assert need > _lib.FEA_FWD_SCRATCH_BYTES
    assert L.vmo_fea_fwd_noalloc(ctypes.byref(a), None) == 3
    assert b"scratch" in L.vmo_last_error()
    assert L.vmo_fea_fwd_noalloc(None, None) == 1


def test_fea_bwd_workspace_holds_ds_for_the_ds_route(L):
    """The dS route keeps dS^T (problems x nk x nq, both rounded up to 32, 16-bit) in the workspace.  It is
    the default for d = 128 with dv = 256 under the size cap and is taken for any d in {64, 128} with
    VMO_BWD_DS_DQ; with VMO_BWD_RECOMPUTE_DQ, for other head dims, for dv = d without the flag, or past the
    cap, only the small recompute-route workspace is asked for."""
    from vmonarch_amd import _lib
    a = _lib.FeaBwdArgs()
    a.dtype, a.batch, a.heads, a.frames, a.nq, a.nk, a.d, a.dv = 0, 1, 3, 7, 1557, 1000, 128, 256
    with_ds = L.vmo_fea_bwd_workspace_size(ctypes.byref(a))
    a.flags = _lib.BWD_RECOMPUTE_DQ
    without = L.vmo_fea_bwd_workspace_size(ctypes.byref(a))
    assert with_ds - without == 21 * 1024 * 1568 * 2
    a.flags, a.dv = 0, 128                        # dv = d: the recompute route unless asked for
    assert L.vmo_fea_bwd_workspace_size(ctypes.byref(a)) == without
    a.flags = _lib.BWD_DS_DQ
    assert L.vmo_fea_bwd_workspace_size(ctypes.byref(a)) == with_ds
    a.flags, a.d, a.dv = _lib.BWD_DS_DQ, 256, 256   # no dS route for d = 256
    big_d = L.vmo_fea_bwd_workspace_size(ctypes.byref(a))
    a.flags = _lib.BWD_RECOMPUTE_DQ
    assert big_d == L.vmo_fea_bwd_workspace_size(ctypes.byref(a))
    a.flags, a.d, a.dv, a.heads, a.nq, a.nk = 0, 128, 256, 24, 16384, 16384   # 12.9 GB of dS^T: past the cap
    capped = L.vmo_fea_bwd_workspace_size(ctypes.byref(a))
    a.flags = _lib.BWD_RECOMPUTE_DQ
    assert capped == L.vmo_fea_bwd_workspace_size(ctypes.byref(a))


@pytest.mark.parametrize("heads, n", [(8, 16384), (1, 8192), (2, 4100)])
def test_fea_bwd_long_standalone_backward_stays_on_the_recompute_route(L, heads, n):
    """A standalone flash_entropy_attention backward at d = 128, dv = 256 with long sequences -- (1, 8, 16384)
    would need exactly 4 GiB of dS^T, (1, 1, 8192) 128 MiB -- takes the recompute route (O(nq) workspace) by
    default: the dS route is the default only for the short frame problems it was measured on (nq, nk <= 4096),
    as VMonarch's R-step passes them (cfg4: 252 problems of 1560 x 1560, 1.24 GB)."""
    from vmonarch_amd import _lib
    a = _lib.FeaBwdArgs()
    a.dtype, a.batch, a.heads, a.frames, a.nq, a.nk, a.d, a.dv = 0, 1, heads, 1, n, n, 128, 256
    default = L.vmo_fea_bwd_workspace_size(ctypes.byref(a))
    a.flags = _lib.BWD_RECOMPUTE_DQ
    assert default == L.vmo_fea_bwd_workspace_size(ctypes.byref(a))
    assert default < 64 << 20
    a.flags = _lib.BWD_DS_DQ   # still available on request
    assert L.vmo_fea_bwd_workspace_size(ctypes.byref(a)) - default == heads * ((n + 31) // 32) ** 2 * 2048
    # the cfg4 R-step geometry keeps the dS route
    a.flags, a.heads, a.frames, a.nq, a.nk = 0, 12, 21, 1560, 1560
    with_ds = L.vmo_fea_bwd_workspace_size(ctypes.byref(a))
    a.flags = _lib.BWD_RECOMPUTE_DQ
    assert with_ds - L.vmo_fea_bwd_workspace_size(ctypes.byref(a)) == 252 * 49 * 49 * 2048


def test_fea_fwd_qk_fp8_workspace_and_rejections(L):
    """vmo_fea_fwd_args.qk_fp8: the workspace grows by the fp8 keys (problems x nk x d bytes, from a 256-byte
    boundary) and one float per 64-key tile; values that are not k, d = 64, or a value other than 0 / 1 are
    rejected before any launch."""
    from vmonarch_amd import _lib
    a = _fwd_args(frames=3, nk=1000, heads=2)
    a.w0 = a.k   # values k (the R-step variants)
    a.ent = _addr()
    base = L.vmo_fea_fwd_workspace_size(ctypes.byref(a))
    a.qk_fp8 = 1
    assert L.vmo_fea_fwd_workspace_size(ctypes.byref(a)) - base == (6 * 1000 * 128 + 255) // 256 * 256 + 6 * 16 * 4
    a.qk_fp8 = 2
    a.workspace, a.workspace_bytes = _addr(1 << 22), 1 << 22
    assert L.vmo_fea_fwd(ctypes.byref(a), None) == 1
    a.qk_fp8 = 1
    a.w0 = _lib.View(_addr(1 << 20), 128, 128 * 128, 128)   # values that are not k
    assert L.vmo_fea_fwd(ctypes.byref(a), None) == 2
    assert b"qk_fp8" in L.vmo_last_error()
