"""Write the golden fixtures under tests/golden/ from the reference's own Python code.

Run in the build container only (it needs /root/reference; the GPU box never runs it):
    python tests/golden/make_golden.py

What it imports from the reference, and why (nothing else pins these):
  * video_monarch_attention/vmonarch.py:29-69  ``vmonarch_attention`` -- the general m>1, b>1,
    num_iters>=2 glue (einsum index conventions, sign of the entropy bias, col_mass clamp).
  * tests/test_vmonarch.py:12-15  ``entropy_attention_ref`` -- the fp32 FEA oracle, used as the
    R-step exactly as tests/test_vmonarch.py:55-61 does (monkeypatched ``_row_block_attention``).
Both run on the CPU in fp32 (the Triton kernels are never launched).

Inputs are drawn from a seeded generator and rounded to bf16 (stored as their uint16 bit
patterns), so the GPU parity tests can feed the very same values to the bf16 HIP path; the
reference outputs are float32.  Each fixture is an .npz
holding inputs, parameters and the reference outputs.
"""
import importlib.util
import os
import sys

import numpy as np
import torch

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


def main():
    vm, entropy_attention_ref = _load_reference()

    def row_block_attention_ref(x, k, w):  # tests/test_vmonarch.py:55-57
        out, ent = entropy_attention_ref(x, k, w, 1.0)
        return out, -ent.detach()

    vm._row_block_attention = row_block_attention_ref
    written = []

    # FlashEntropyAttention forward: (B, H, N, D, Dv) -- N=200 exercises the reference's padding path
    for (B, H, N, D, Dv) in [(1, 2, 200, 64, 64), (1, 1, 128, 128, 256), (2, 1, 77, 64, 128)]:
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
    for (m, b, D, iters, rt) in cases:
        g = torch.Generator().manual_seed(7 * m + b + D + iters + rt)
        B, H, N = 1, 2, m * b
        q, k, v = (_bf16_randn(g, B, H, N, D) for _ in range(3))
        z = vm.vmonarch_attention(q, k, v, m, b, iters, recompute_tokens=rt)
        name = f"vmonarch_m{m}b{b}D{D}it{iters}rt{rt}.npz"
        np.savez_compressed(os.path.join(HERE, name), q=_bits(q), k=_bits(k), v=_bits(v),
                            num_blocks=np.int64(m), block_size=np.int64(b), num_iters=np.int64(iters),
                            recompute_tokens=np.int64(rt), z=z.numpy())
        written.append(name)
    for n in written:
        print(n, os.path.getsize(os.path.join(HERE, n)), "bytes")


if __name__ == "__main__":
    main()
