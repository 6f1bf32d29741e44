"""Write the golden fixtures under tests/golden/ from the reference's own Python code.

Run in the build container only (it needs /root/reference; the GPU box never runs it):
    python tests/golden/make_golden.py [fea] [vmonarch] [lowp]      (default: all three sets)

Importing the reference writes nothing under /root/reference (no bytecode caches).

What it imports from the reference, and why (nothing else pins these):
  * video_monarch_attention/vmonarch.py:29-69  ``vmonarch_attention`` -- the general m>1, b>1,
    num_iters>=2 glue (einsum index conventions, sign of the entropy bias, col_mass clamp).
  * tests/test_vmonarch.py:12-15  ``entropy_attention_ref`` -- the fp32 FEA oracle, used as the
    R-step exactly as tests/test_vmonarch.py:55-61 does (monkeypatched ``_row_block_attention``).
Both run on the CPU in fp32 (the Triton kernels are never launched).
  * the same ``vmonarch_attention`` run on bf16 tensors (CPU), with the R-step seam returning the
    fp32 oracle's output cast to bf16 as a bf16 kernel stores it: the rounding points of the
    reference's own bf16 path (vmonarch.py:47-67), which nothing but a run of that code pins.

Inputs are drawn from a seeded generator and rounded to bf16 (stored as their uint16 bit
patterns), so the GPU parity tests can feed the very same values to the bf16 HIP path; the
reference outputs are float32.  Each fixture is an .npz
holding inputs, parameters and the reference outputs.
"""
import sys

sys.dont_write_bytecode = True   # importing the reference must not write caches under /root/reference

import importlib.util  # noqa: E402
import os  # noqa: E402

import numpy as np  # noqa: E402
import torch  # noqa: E402

REF = "/root/reference"
HERE = os.path.dirname(os.path.abspath(__file__))


def _load_reference():
    sys.path.insert(0, REF)
    import video_monarch_attention.vmonarch as vm  # noqa: E402  (reference package)
    spec = importlib.util.spec_from_file_location("ref_test_vmonarch", os.path.join(REF, "tests", "test_vmonarch.py"))
    t = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(t)
    return vm, t.entropy_attention_ref


def _bf16_randn(g, *shape, scale=1.0):
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16).float()


def _bits(t):
    """bf16-exact float32 tensor -> its bf16 bit pattern as uint16 (half the bytes of float32)."""
    return t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def main(sets):
    vm, entropy_attention_ref = _load_reference()

    def row_block_attention_ref(x, k, w):  # tests/test_vmonarch.py:55-57
        out, ent = entropy_attention_ref(x, k, w, 1.0)
        return out, -ent.detach()

    vm._row_block_attention = row_block_attention_ref
    written = []

    # FlashEntropyAttention forward: (B, H, N, D, Dv) -- N=200 exercises the reference's padding path
    for (B, H, N, D, Dv) in [] if "fea" not in sets else [(1, 2, 200, 64, 64), (1, 1, 128, 128, 256), (2, 1, 77, 64, 128)]:
        g = torch.Generator().manual_seed(1000 + N + D + Dv)
        q, k, v = _bf16_randn(g, B, H, N, D), _bf16_randn(g, B, H, N, D), _bf16_randn(g, B, H, N, Dv)
        o, e = entropy_attention_ref(q, k, v, D ** -0.5)
        name = f"fea_B{B}H{H}N{N}D{D}Dv{Dv}.npz"
        np.savez_compressed(os.path.join(HERE, name), q=_bits(q), k=_bits(k), v=_bits(v),
                            sm_scale=np.float64(D ** -0.5), o=o.numpy(), e=e.numpy())
        written.append(name)

    # VMonarch forward: (m, b, D, num_iters, recompute_tokens)
    cases = [(4, 64, 32, 1, 0), (4, 64, 32, 2, 64), (4, 64, 32, 3, 0), (8, 100, 32, 2, 100),
             (3, 40, 64, 2, 0), (3, 40, 64, 3, 40), (16, 16, 32, 2, 16), (21, 12, 64, 2, 12),
             (4, 48, 128, 2, 48), (5, 36, 128, 3, 0), (6, 20, 64, 1, 20)]
    for (m, b, D, iters, rt) in cases if "vmonarch" in sets else []:
        g = torch.Generator().manual_seed(7 * m + b + D + iters + rt)
        B, H, N = 1, 2, m * b
        q, k, v = (_bf16_randn(g, B, H, N, D) for _ in range(3))
        z = vm.vmonarch_attention(q, k, v, m, b, iters, recompute_tokens=rt)
        name = f"vmonarch_m{m}b{b}D{D}it{iters}rt{rt}.npz"
        np.savez_compressed(os.path.join(HERE, name), q=_bits(q), k=_bits(k), v=_bits(v),
                            num_blocks=np.int64(m), block_size=np.int64(b), num_iters=np.int64(iters),
                            recompute_tokens=np.int64(rt), z=z.numpy())
        written.append(name)

    # VMonarch forward on bf16 tensors, the reference's rounding points around an exact R-step:
    # (m, b, D, num_iters, recompute_tokens, input scale); scaled inputs make every rounding visible
    def row_block_attention_lowp(x, k, w):
        out, ent = entropy_attention_ref(x.float(), k.float(), w.float(), 1.0)
        return out.to(x.dtype), -ent.detach()

    vm._row_block_attention = row_block_attention_lowp
    lowp = [(4, 64, 64, 2, 64, 3.0), (8, 40, 32, 3, 0, 1.0), (3, 50, 128, 2, 50, 2.0)]
    for (m, b, D, iters, rt, sc) in lowp if "lowp" in sets else []:
        g = torch.Generator().manual_seed(11 * m + b + D + iters + rt)
        B, H, N = 1, 2, m * b
        q, k = (_bf16_randn(g, B, H, N, D, scale=sc) for _ in range(2))
        v = _bf16_randn(g, B, H, N, D)
        z = vm.vmonarch_attention(*(t.to(torch.bfloat16) for t in (q, k, v)), m, b, iters, recompute_tokens=rt)
        assert z.dtype == torch.bfloat16
        name = f"lowp_vmonarch_m{m}b{b}D{D}it{iters}rt{rt}x{sc:g}.npz"
        np.savez_compressed(os.path.join(HERE, name), q=_bits(q), k=_bits(k), v=_bits(v),
                            num_blocks=np.int64(m), block_size=np.int64(b), num_iters=np.int64(iters),
                            recompute_tokens=np.int64(rt), z=_bits(z.float()))
        written.append(name)
    for n in written:
        print(n, os.path.getsize(os.path.join(HERE, n)), "bytes")


if __name__ == "__main__":
    main(set(sys.argv[1:]) or {"fea", "vmonarch", "lowp"})
