"""CPU oracle for the VMonarch attention hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``
may import this package, and only as the checker (or the timed CPU baseline).  The product
package ``vmonarch_amd`` never imports it; it runs on the HIP extension or raises.

Contents
  fea.entropy_attention        forward of FlashEntropyAttention (o, e)
  fea.entropy_attention_grad   analytic backward (dq, dk, dv) incl. the entropy term
  vmonarch.vmonarch_attention  alternating-minimisation glue (R-step, L-step, recompute)
  vmonarch.lstep_grad          backward of one L-step (entropy bias detached)
  vmonarch.vmonarch_attention_grad  backward of the whole glue (dq, dk, dv)
  vmonarch.vmonarch_attention_lowp  the glue with the reference's bf16 roundings (how far the
                                    reference's own bf16 path lands from the fp32 one)

Every function cites the reference file:line it restates.  Arithmetic is numpy float64 by
default (float32 for the CPU baseline timing).  How each function is pinned:
  entropy_attention       brute-force pure-Python loops, closed forms (uniform keys -> ln n,
                          two keys -> binary entropy, one dominant logit -> 0), golden
                          vectors written from the reference's own oracle
                          (tests/test_vmonarch.py:12-15)
  entropy_attention_grad  central finite differences of entropy_attention in float64
  vmonarch_attention      golden vectors written by the reference's own vmonarch_attention
                          (video_monarch_attention/vmonarch.py:29-69) with its R-step
                          swapped to the fp32 oracle as in tests/test_vmonarch.py:55-61, plus
                          the m=1 / b=1 / rt=N reductions to exact attention.
  vmonarch_attention_lowp golden vectors written by the reference's own vmonarch_attention run on
                          bf16 tensors (CPU) around an exact R-step; with the rounding switched
                          off it is vmonarch_attention.
  lstep_grad,             central finite differences (random directions, float64) of
  vmonarch_attention_grad lstep / vmonarch_attention with the entropy biases frozen at the
                          base point, as the reference's detach (vmonarch.py:26) makes them;
                          with and without the col_mass clamp active, 1-3 iterations, rt 0 and b.
"""
from .fea import entropy_attention, entropy_attention_grad, exact_attention, kernel_rounding_attention  # noqa: F401
from .vmonarch import (vmonarch_attention, row_block_attention, lstep, lstep_grad,  # noqa: F401
                       vmonarch_attention_grad, vmonarch_attention_lowp, round_bf16)
