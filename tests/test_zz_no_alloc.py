"""vmo_fea_fwd_noalloc (the allocation-free forward: split-KV partials in the library's static device
scratch) against vmo_fea_fwd with a caller workspace, both called through the C ABI: bit for bit the same
o and LSE, on two calls in a row -- the second smaller, so stale partials of the first would show -- plus
a call without splits (entropy output, no scratch used) and the size limit."""
import ctypes

import pytest
import torch

from conftest import hip_library_loaded, randn_lp

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _args(q, k, v, o, lse, ent, splits, sm_scale):
    from vmonarch_amd import _lib
    a = _lib.FeaFwdArgs()
    a.dtype = _lib.DTYPES[q.dtype]
    a.batch, a.heads, a.frames = q.shape[0], q.shape[1], 1
    a.nq, a.nk = q.shape[2], k.shape[2]
    a.d, a.dw0, a.dw1 = q.shape[3], v.shape[3], 0
    a.q, a.k, a.w0, a.o = _lib.view(q), _lib.view(k), _lib.view(v), _lib.view(o)
    a.w1 = _lib.View(0, 0, 0, 0)
    a.lse = lse.data_ptr()
    a.ent = ent.data_ptr() if ent is not None else None
    a.stat_stride_b, a.stat_stride_h = lse.stride(0), lse.stride(1)
    a.sm_scale = sm_scale
    a.num_splits = splits
    return a


def _run_both(q, k, v, splits, with_ent=False):
    from vmonarch_amd import _lib
    L = _lib.lib()
    B, H, nq, _ = q.shape
    stream = _lib.stream_of(q)
    outs = []
    for noalloc in (False, True):
        o = torch.full((B, H, nq, v.shape[-1]), 7.0, device=DEV, dtype=q.dtype)
        lse = torch.full((B, H, nq), 7.0, device=DEV)
        ent = torch.full((B, H, nq), 7.0, device=DEV) if with_ent else None
        a = _args(q, k, v, o, lse, ent, splits, q.shape[-1] ** -0.5)
        if noalloc:
            a.workspace, a.workspace_bytes = None, 0
            rc = L.vmo_fea_fwd_noalloc(ctypes.byref(a), stream)
        else:
            nbytes = L.vmo_fea_fwd_workspace_size(ctypes.byref(a))
            ws = torch.empty(max(nbytes, 1), device=DEV, dtype=torch.uint8)
            a.workspace, a.workspace_bytes = ws.data_ptr(), nbytes
            rc = L.vmo_fea_fwd(ctypes.byref(a), stream)
        _lib.check(rc, "vmo_fea_fwd_noalloc" if noalloc else "vmo_fea_fwd")
        torch.cuda.synchronize()
        outs.append((o, lse, ent))
    return outs


def test_noalloc_forward_matches_the_workspace_entry_point():
    g = torch.Generator().manual_seed(77)
    # two split-KV calls in a row, the second smaller, then one without splits (entropy output)
    for nq, nk, splits in ((300, 6000, 8), (100, 1500, 3)):
        q, k, v = randn_lp(g, 1, 3, nq, 128), randn_lp(g, 1, 3, nk, 128), randn_lp(g, 1, 3, nk, 128)
        print(f"noalloc forward nq={nq} nk={nk} splits={splits}", flush=True)
        (o_ref, lse_ref, _), (o, lse, _) = _run_both(q.to(DEV), k.to(DEV), v.to(DEV), splits)
        assert torch.equal(o, o_ref) and torch.equal(lse, lse_ref)
        assert torch.isfinite(o.float()).all()
    q, k, v = (randn_lp(g, 2, 2, 200, 64) for _ in range(3))
    print("noalloc forward without splits (entropy)", flush=True)
    (o_ref, lse_ref, e_ref), (o, lse, e) = _run_both(q.to(DEV), k.to(DEV), v.to(DEV), 1, with_ent=True)
    assert torch.equal(o, o_ref) and torch.equal(lse, lse_ref) and torch.equal(e, e_ref)
    assert hip_library_loaded()


def test_noalloc_forward_rejects_calls_beyond_its_scratch():
    from vmonarch_amd import _lib
    L = _lib.lib()
    q = torch.zeros(1, 8, 4096, 128, device=DEV, dtype=torch.bfloat16)
    kv = torch.zeros(1, 8, 65536, 128, device=DEV, dtype=torch.bfloat16)
    o = torch.zeros_like(q)
    lse = torch.zeros(1, 8, 4096, device=DEV)
    a = _args(q, kv, kv, o, lse, None, 16, 0.1)
    assert L.vmo_fea_fwd_workspace_size(ctypes.byref(a)) > _lib.FEA_FWD_SCRATCH_BYTES
    assert L.vmo_fea_fwd_noalloc(ctypes.byref(a), _lib.stream_of(q)) == 3
    assert b"scratch" in L.vmo_last_error()


def test_noalloc_forward_replays_from_a_hip_graph():
    """vmo_fea_fwd_noalloc with split-KV captured in a torch.cuda.CUDAGraph (after one uncaptured call, which
    looks up the scratch address on this device): every replay -- with eager work and a sentinel fill of the
    outputs between replays -- gives o and LSE bit for bit equal to an eager vmo_fea_fwd with a caller
    workspace.  The forward records no memset node (its partials are written in full before the merge reads
    them), so nothing in the graph depends on state a replay leaves behind."""
    from vmonarch_amd import _lib
    L = _lib.lib()
    g = torch.Generator().manual_seed(78)
    nq, nk, splits = 300, 6000, 8
    q, k, v = (randn_lp(g, 1, 3, n, 128).to(DEV) for n in (nq, nk, nk))
    (o_ref, lse_ref, _), _ = _run_both(q, k, v, splits)   # eager reference; also the uncaptured set-up call
    o = torch.empty_like(o_ref)
    lse = torch.empty_like(lse_ref)
    a = _args(q, k, v, o, lse, None, splits, 128 ** -0.5)
    a.workspace, a.workspace_bytes = None, 0
    graph = torch.cuda.CUDAGraph()
    print("noalloc forward: capture", flush=True)
    with torch.cuda.graph(graph):
        _lib.check(L.vmo_fea_fwd_noalloc(ctypes.byref(a), _lib.stream_of(q)), "vmo_fea_fwd_noalloc (captured)")
    for rep in range(3):
        o.fill_(7.0)
        lse.fill_(7.0)
        # eager work between replays that also uses the scratch: a smaller split-KV call
        q2, k2, v2 = (randn_lp(g, 1, 2, n, 128).to(DEV) for n in (100, 1500, 1500))
        _run_both(q2, k2, v2, 3)
        print(f"noalloc forward: replay {rep}", flush=True)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(o, o_ref) and torch.equal(lse, lse_ref), f"replay {rep}"
    del graph
