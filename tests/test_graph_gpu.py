"""The all-HIP VMonarch forward and the flash-entropy forward captured in a HIP graph (torch.cuda.CUDAGraph over
the library's launches on the capturing stream; the recompute's second stream joins the capture through its
fork / join events) and replayed: every replay bit for bit the eager result, with eager work and new input
values between the replays."""
import pytest
import torch

from conftest import hip_library_loaded, randn_lp

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _warm(fn):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()


@pytest.mark.parametrize("m, b, D, rt, dtype", [(4, 256, 64, 256, torch.bfloat16), (21, 120, 128, 120, torch.bfloat16),
                                                (8, 100, 32, 100, torch.bfloat16), (21, 120, 128, 60, torch.float16)])
def test_vmonarch_forward_replays_from_a_graph(m, b, D, rt, dtype):
    from vmonarch_amd import vmonarch_attention
    g = torch.Generator().manual_seed(31 + m + D)
    q, k, v = (randn_lp(g, 1, 2, m * b, D, scale=0.5, dtype=dtype).to(DEV) for _ in range(3))
    inputs = [[randn_lp(g, 1, 2, m * b, D, scale=0.5, dtype=dtype).to(DEV) for _ in range(3)] for _ in range(3)]
    run = lambda: vmonarch_attention(q, k, v, m, b, 2, recompute_tokens=rt)   # noqa: E731
    print(f"graph vmonarch m={m} b={b} D={D} rt={rt} {dtype}", flush=True)
    with torch.no_grad():
        _warm(run)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            z = run()
        for i, (q2, k2, v2) in enumerate(inputs):
            for dst, src in ((q, q2), (k, k2), (v, v2)):
                dst.copy_(src)
            ref = run()                                # eager, on the new inputs
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(z, ref), f"replay {i}"
            _ = run() * 2                              # eager work between replays
    assert hip_library_loaded()


def test_flash_entropy_forward_replays_from_a_graph():
    from vmonarch_amd import flash_entropy_attention
    g = torch.Generator().manual_seed(41)
    q, k, v = (randn_lp(g, 2, 3, 1000, 128).to(DEV) for _ in range(3))
    run = lambda: flash_entropy_attention(q, k, v)   # noqa: E731
    with torch.no_grad():
        o_ref, e_ref = run()
        _warm(run)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            o, e = run()
        for i in range(3):
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(o, o_ref) and torch.equal(e, e_ref), f"replay {i}"
            _ = run()
