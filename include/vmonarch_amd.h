/*
 * vmonarch_amd -- C ABI of the MI355X (gfx950) VMonarch attention hot path.
 *
 * The reference (EricLina/VMonarch) has no C/C++ API: its device code is Triton JIT kernels
 * launched from Python.  Each entry point below replaces one launch site of the reference's
 * Python, keeping the argument meaning; the Python package `vmonarch_amd` (and the alias
 * package `video_monarch_attention`) binds them with ctypes and keeps the reference's Python
 * API unchanged.
 *
 * Conventions
 *   - Every call is asynchronous on the given HIP stream (a hipStream_t passed as void*,
 *     NULL = the default stream) and never allocates device memory: scratch comes from the
 *     caller's `workspace`.
 *   - Return 0 (VMO_OK) on success, a VMO_ERR_* code otherwise; vmo_last_error() then holds a
 *     message for the calling thread.  Argument errors are detected before any launch.
 *   - Tensors are (batch, heads, tokens, features) views with element strides for the first
 *     three dims and contiguous features (feature stride 1), 16-byte aligned rows.
 *   - Element type is bf16 or fp16 (VMO_DTYPE_*); statistics (lse, entropy) are fp32.
 */
#ifndef VMONARCH_AMD_H
#define VMONARCH_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VMO_ABI_VERSION 13

enum {
  VMO_OK = 0,
  VMO_ERR_INVALID = 1,     /* bad shape / stride / pointer / alignment */
  VMO_ERR_UNSUPPORTED = 2, /* valid request this build has no kernel for (e.g. head dim 48) */
  VMO_ERR_WORKSPACE = 3,   /* workspace missing or too small */
  VMO_ERR_LAUNCH = 4       /* HIP reported an error at launch */
};

enum { VMO_DTYPE_BF16 = 0, VMO_DTYPE_F16 = 1 };

/* A strided 4-d view (batch, heads, tokens, features); strides in elements. */
typedef struct vmo_view {
  void* data;
  int64_t stride_b, stride_h, stride_n;
} vmo_view;

/*
 * FlashEntropyAttention forward.
 *
 * Replaces the `_attn_fwd` launch of _FlashEntropyAttention.forward
 * (video_monarch_attention/kernel.py:318-358, kernel :104-151, inner loop :32-67).
 *
 * Problems: batch * heads * frames independent attentions.  Frame f of (b, h) uses query rows
 * [f*nq, (f+1)*nq) of q / o / lse / ent and key rows [f*nk, (f+1)*nk) of k / w0 / w1, so
 * frames = m turns one (B, H, m*b, D) tensor into the reference's R-step batch
 * (vmonarch.py:25 flattens (B, H, m, b, .) to (B, H*m, b, .)) without a copy.
 *
 *   o[:, :, i, 0:dw0]        = sum_j P_ij w0_j
 *   o[:, :, i, dw0:dw0+dw1]  = sum_j P_ij w1_j          (dw1 = 0: no second value tensor)
 *   P = softmax_j(sm_scale * q_i . k_j) over the nk keys of the problem (non-causal)
 *   ent[i] = -sum_j P_ij ln P_ij (nats)    lse[i] = log2(sum_j 2^(sm_scale*log2(e)*q_i.k_j))
 * Two value tensors replace the reference's torch.cat([k, v], -1) (vmonarch.py:50); when w0
 * aliases k (same data and strides, dw0 == d) the K tile is staged once and used twice.
 * ent / lse may be NULL.  num_splits > 1 splits the keys of each problem into num_splits
 * ranges (split-KV, for problems with few query tiles such as the recompute of
 * vmonarch.py:66-68); it needs ent == NULL and a workspace of
 * vmo_fea_fwd_workspace_size() bytes.  Supported (d, dw0): with entropy output and one split, d in {64, 128}
 * with dw0 in {64, 128, 256}, (256, 256), d = 16 or 32 with dw0 in {d, 32, 64, 128, 256}, (64, 32), (128, 32);
 * without entropy, one split or several, (16, 16), (32, 32), (64, 64), (64, 128), (128, 64), (128, 128).  Values
 * that start with k (w0 aliasing k, entropy, one split): d = dw0 in {16, 32, 64, 128} with dw1 in {0, d}, and
 * dw1 = 128 at d = 64, dw1 = 64 at d = 128.  16-wide q / k or values are read as they are (no padded copy is
 * expected from the caller).  sm_scale >= 0.
 */
typedef struct vmo_fea_fwd_args {
  int32_t dtype;
  int32_t batch, heads, frames;
  int32_t nq, nk;
  int32_t d, dw0, dw1;
  vmo_view q, k, w0, w1, o;
  float* lse;                      /* optional: (batch, heads, frames*nq), token stride 1 */
  float* ent;                      /* optional: same layout as lse */
  int64_t stat_stride_b, stat_stride_h;
  float sm_scale;
  int32_t num_splits;              /* 1 = no split */
  void* workspace;
  size_t workspace_bytes;
  /* 1: S = q k^T in fp8 (e4m3; no counterpart in the reference, which computes S in bf16 / fp16): q rows
   * scaled by their own max |q| / 448 in the kernel, k by one max |k| / 448 per 64-key tile in a pass before it (into the
   * workspace: vmo_fea_fwd_workspace_size() counts nk * d bytes per problem and the tile scales); P, the
   * value products, o, the entropy and lse as without it.  Built for the VMonarch R-steps (d = 128, w0 = k,
   * dw1 in {0, 128}, entropy, num_splits = 1); an approximation: each logit off by up to ~4% of its size
   * (e4m3's 3-bit mantissa), within the 16-bit tolerances for logits of std <= 0.25, an fp8 class
   * (6e-2 + 3e-2 |ref| for o, 5e-2 for e) at std 1.  Measured slower than 16-bit S on MI355X (the
   * R-steps are bound by their tile stream, which the fp8 K tile adds to); 0 is the default. */
  int32_t qk_fp8;
} vmo_fea_fwd_args;

/*
 * One L-step of the alternating minimisation (vmonarch.py:51-63), fused.
 *
 * For every (b, h) and grid column j of the (m, b) token grid (token n = i*block + j):
 *   logits[i,k] = scale * q[i,j] . out[k,j,0:d]                         (vmonarch.py:51, :55)
 *   attn[i,:]   = softmax_k(logits[i,k] + ent[k,j])                      (vmonarch.py:56)
 *   last == 0:  u[k,j]  = scale / max(sum_i attn[i,k], min_col_mass) * sum_i attn[i,k] q[i,j]
 *                                                                         (vmonarch.py:61-63)
 *   last == 1:  z[i,j]  = sum_k attn[i,k] out[k,j,d:d+dv]                (vmonarch.py:57-59)
 * ent is the R-step entropy (the reference subtracts neg_ent = -ent).  `res` receives u
 * (d features) or z (dv features).  With last == 1, tokens n < skip_tokens are not written
 * (the recompute of vmonarch.py:66-68 owns them).  Kernels by grid: one MFMA tile per grid column for
 * m <= 32 with d and dv in {64, 128}; multi-block MFMA kernels (one workgroup per column, 32 x 32 blocks)
 * for m <= 128 with d and dv in {32, 64, 128} or d = dv = 16; otherwise a general kernel that takes any m whose
 * per-column tiles fit the LDS and d, dv multiples of 8 up to 256.  Larger grids are rejected with
 * VMO_ERR_UNSUPPORTED before any launch.
 */
typedef struct vmo_lstep_args {
  int32_t dtype;
  int32_t batch, heads;
  int32_t num_blocks, block_size;  /* m, b */
  int32_t d, dv;
  int32_t last;
  int32_t skip_tokens;
  vmo_view q;                      /* (B, H, m*b, d) */
  vmo_view out;                    /* (B, H, m*b, d + dv*last): R-step output [P k | P v] */
  const float* ent;                /* (B, H, m*b) with token stride 1 */
  int64_t ent_stride_b, ent_stride_h;
  vmo_view res;                    /* u: (B, H, m*b, d)   or   z: (B, H, m*b, dv) */
  float scale;
  float min_col_mass;
} vmo_lstep_args;

/*
 * FlashEntropyAttention backward.
 *
 * Replaces the two launches of _FlashEntropyAttention.backward (kernel.py:360-381:
 * _attn_bwd_preprocess :154-162 and _attn_bwd :251-313).  For the loss L with upstream grads
 * grad_o = dL/do and grad_ent = dL/dent, writes grad_q, grad_k, grad_v (same dtype as q):
 *   dS = P (dP - delta) + grad_ent P (-ent - ln P),  dP = grad_o v^T,  delta = rowsum(o * grad_o)
 *   grad_q = sm_scale dS k,  grad_k = sm_scale dS^T q,  grad_v = P^T grad_o
 * with P rebuilt from `lse` (log2 units, as written by vmo_fea_fwd).  nq queries attend to nk
 * keys per (batch, head) (nq != nk allowed).  Supported: d in {64, 128} with dv in {64, 128, 256},
 * d = dv = 256, d = 16 or 32 with dv in {d, 32, 64, 128, 256}, (64, 32) and (128, 32) (16-wide rows read as
 * they are).  Needs vmo_fea_bwd_workspace_size() bytes of workspace.
 */
/* vmo_fea_bwd_args.flags: the marked gradient is float32 and the kernels add into it (+=, ACCUM) or
 * overwrite it (=, F32); without either bit it has the inputs' dtype.  ACCUM and F32 of the same
 * gradient together are rejected.
 * VMO_BWD_FOLD_K: the values are k, or [k | v1] (v is k: same address and strides), as in the
 * VMonarch R-steps (vmonarch.py:50, where autograd sums k's two gradients).  grad_k then receives
 * k's whole gradient, key role plus value role, and grad_v only v1's (dv1 columns; with values k
 * alone grad_v is not written and may be null).  Built for (d, dv) = (16, 16), (32, 32), (64, 64), (128, 128)
 * and, with v1, (16, 32), (32, 64), (64, 128), (128, 256); other shapes, or values that do not start with k,
 * are rejected. */
enum {
  VMO_BWD_ACCUM_Q = 1, VMO_BWD_ACCUM_K = 2, VMO_BWD_ACCUM_V = 4,
  VMO_BWD_F32_Q = 8, VMO_BWD_F32_K = 16, VMO_BWD_F32_V = 32,
  VMO_BWD_FOLD_K = 64,
  /* grad_k (grad_v) in the inputs' dtype = grad_k_base (grad_v_base, an fp32 view of the same shape)
   * + this call's gradient: the last of several calls that sum one gradient writes it once, in the
   * caller's dtype, instead of adding into fp32 and converting afterwards.  Not with ACCUM / F32 of
   * the same gradient. */
  VMO_BWD_SUM_K = 128, VMO_BWD_SUM_V = 256,
  /* Route for grad_q, results within rounding of each other.  Recompute route: a dq pass recomputes S
   * and dP.  dS route: the dkdv pass stores dS^T (16-bit, nk and nq rounded up to 32, per problem) in
   * the workspace and grad_q = sm_scale dS k is a GEMM over it -- no second S and dP, 4 bytes of HBM
   * traffic per query-key pair instead.  Its workspace is 2 bytes per query-key pair (the recompute
   * route needs O(nq)), so by default it is taken only for d = 128 with dv = 256 (where the recompute
   * is dearest) on short problems -- nq and nk at most 4096, the VMonarch R-step's frames -- while dS^T
   * of all problems stays within 2 GiB; a long standalone backward stays on the recompute route.
   * VMO_BWD_RECOMPUTE_DQ never takes it, VMO_BWD_DS_DQ takes it at any size for d in {64, 128} (not
   * both).  vmo_fea_bwd_workspace_size() includes the dS^T bytes when the route is taken. */
  VMO_BWD_RECOMPUTE_DQ = 512, VMO_BWD_DS_DQ = 1024,
  /* grad_q in the inputs' dtype = grad_q_base (fp32, shaped like grad_q) + this call's gradient, as
   * VMO_BWD_SUM_K / _V.  Not with ACCUM_Q / F32_Q. */
  VMO_BWD_SUM_Q = 2048
};

typedef struct vmo_fea_bwd_args {
  int32_t dtype;
  int32_t batch, heads;
  int32_t nq, nk;
  int32_t d, dv;
  vmo_view q, k, v, o, grad_o;
  vmo_view grad_q, grad_k, grad_v;
  const float* lse;                /* (batch, heads, nq), token stride 1 */
  const float* ent;                /* same layout as lse */
  const float* grad_ent;           /* (batch, heads, nq), token stride 1 */
  int64_t stat_stride_b, stat_stride_h;
  int64_t grad_ent_stride_b, grad_ent_stride_h;
  float sm_scale;
  void* workspace;
  size_t workspace_bytes;
  int32_t flags;                   /* VMO_BWD_ACCUM_* | VMO_BWD_F32_* | VMO_BWD_FOLD_K | VMO_BWD_SUM_* |
                                      VMO_BWD_RECOMPUTE_DQ | VMO_BWD_DS_DQ | VMO_BWD_SUM_Q */
  /* Values given in two parts: with dv1 > 0 the value tensor is [v | v1], v holding columns
   * [0, dv - dv1) and v1 (same strides as v) the last dv1 (VMonarch's last R-step, values [k | v],
   * vmonarch.py:50, without the concatenated copy).  Built for dv1 = dv / 2 with (d, dv) = (64, 128)
   * and (128, 256), and when v is k also (16, 32) and (32, 64).  grad_v stays one (.., dv) tensor. */
  vmo_view v1;
  int32_t dv1;
  vmo_view grad_k_base, grad_v_base;   /* fp32, read with VMO_BWD_SUM_K / VMO_BWD_SUM_V */
  /* frames (0 or 1: one): batch * heads * frames problems, as vmo_fea_fwd_args.frames -- frame f of
   * (b, h) uses query rows [f*nq, (f+1)*nq) of q / o / grad_o / grad_q / lse / ent / grad_ent and key
   * rows [f*nk, (f+1)*nk) of k / v / v1 / grad_k / grad_v and the bases, so the R-steps' backward reads
   * a (B, H, m*b, .) tensor in any memory order (a DiT block's (B, N, H, D)) without a copy. */
  int32_t frames;
  vmo_view grad_q_base;                /* fp32, read with VMO_BWD_SUM_Q */
  /* Optional: delta = rowsum(o * grad_o) per query row, fp32 with the strides below and token stride 1
   * (vmo_lstep_bwd_args.delta writes it); null: formed here from o and grad_o. */
  const float* delta;
  int64_t delta_stride_b, delta_stride_h;
} vmo_fea_bwd_args;

/*
 * Backward of one L-step (the gradient autograd takes through vmonarch.py:51-63, with the entropy
 * bias detached as vmonarch.py:26 does), fused per grid column j.  With attn as in
 * vmo_lstep_args, y = out[..., d:] and g = grad_res (dL/dz when last, dL/du otherwise):
 *   last == 1:  d attn[i,k] = g[i,j] . y[k,j];  grad_out[k,j,d:] = sum_i attn[i,k] g[i,j]
 *               (tokens n < skip_tokens carry no gradient: the recompute overwrote them)
 *   last == 0:  c_k = sum_i attn[i,k], cm_k = max(c_k, min_col_mass), f_k = scale / cm_k,
 *               v_k = sum_i attn[i,k] q[i,j];  dv_k = f_k g[k,j];
 *               d attn[i,k] = dv_k . q[i,j] - [c_k >= min_col_mass] (g[k,j] . v_k) f_k / cm_k;
 *               grad_q[i,j] += sum_k attn[i,k] dv_k
 *   both:       dlogit = attn (d attn - sum_k attn d attn);
 *               grad_q[i,j] += scale sum_k dlogit[i,k] out[k,j,:d];
 *               grad_out[k,j,:d] = scale sum_i dlogit[i,k] q[i,j]
 * grad_q is float32 and accumulated into (+=); grad_out (the dtype of q) is written.  Replaces
 * the autograd graph of the reference's L-step (batched einsum/softmax/clamp backward); there is
 * no launch site of its own in the reference.  Supported grids and head dims: as vmo_lstep_args (one-tile
 * kernels for m <= 32 at d, dv in {64, 128}; multi-block MFMA kernels for m <= 128 at d, dv in {32, 64, 128} or
 * d = dv = 16;
 * the general kernel, which keeps one more m x m matrix and the gradient rows in LDS, beyond).
 */
typedef struct vmo_lstep_bwd_args {
  int32_t dtype;
  int32_t batch, heads;
  int32_t num_blocks, block_size;  /* m, b */
  int32_t d, dv;
  int32_t last;
  int32_t skip_tokens;
  vmo_view q;                      /* (B, H, m*b, d) */
  vmo_view out;                    /* (B, H, m*b, d + dv*last): R-step output */
  const float* ent;                /* (B, H, m*b) with token stride 1 */
  int64_t ent_stride_b, ent_stride_h;
  vmo_view grad_res;               /* dL/dz (B, H, m*b, dv)   or   dL/du (B, H, m*b, d) */
  vmo_view grad_q;                 /* float32 (B, H, m*b, d), accumulated into (or overwritten) */
  vmo_view grad_out;               /* (B, H, m*b, d + dv*last), written */
  float scale;
  float min_col_mass;
  int32_t flags;                   /* VMO_LSTEP_BWD_OVERWRITE_Q: grad_q = dL/dq instead of += */
  /* Optional (null: not written): delta[token] = sum_f out[token][f] * grad_out[token][f] in fp32 over the
   * 16-bit values as stored, (B, H, m*b) with token stride 1 -- the per-row sum the flash-entropy backward of
   * the R-step that produced `out` needs (vmo_fea_bwd_args.delta), formed here from rows this kernel holds
   * anyway.  Built for the one-tile kernels (m <= 32, d and dv in {64, 128}); other shapes reject it. */
  float* delta;
  int64_t delta_stride_b, delta_stride_h;
} vmo_lstep_bwd_args;
enum { VMO_LSTEP_BWD_OVERWRITE_Q = 1 };

/* ABI version of the loaded library (VMO_ABI_VERSION at build time). */
int vmo_abi_version(void);

/* Message of the calling thread's last failed call ("" if none). */
const char* vmo_last_error(void);

/* Bytes of workspace vmo_fea_fwd needs for these arguments (0 when num_splits <= 1). */
size_t vmo_fea_fwd_workspace_size(const vmo_fea_fwd_args* args);

/* FlashEntropyAttention forward; see vmo_fea_fwd_args. */
int vmo_fea_fwd(const vmo_fea_fwd_args* args, void* stream);

/*
 * Allocation-free variant of vmo_fea_fwd.  No counterpart in the reference: it is for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  Same arguments and results as vmo_fea_fwd, except that `workspace` /
 * `workspace_bytes` are ignored: the split-KV partials (and with qk_fp8 the fp8 keys) go to a library-owned
 * static device array of VMO_FEA_FWD_SCRATCH_BYTES on each GPU (held until the process ends).  A call whose
 * workspace needs more (vmo_fea_fwd_workspace_size() > VMO_FEA_FWD_SCRATCH_BYTES) is rejected with
 * VMO_ERR_WORKSPACE before any launch; calls with num_splits <= 1 and qk_fp8 = 0 use no scratch.  The call allocates nothing and calls no
 * allocating routine.  All calls on one GPU share its scratch: calls that overlap in time on one GPU
 * (different streams without ordering, or several host threads) race; order them on one stream.
 * Set-up: the first call on a device looks up the scratch's device address (hipGetSymbolAddress, which
 * may load the library's code object and its scratch on that device).  Make that first call outside any
 * graph capture -- one uncaptured call per device (any arguments, e.g. an empty problem) -- and every
 * later call, captured or not, launches its kernels only.
 */
#define VMO_FEA_FWD_SCRATCH_BYTES (32u << 20)
int vmo_fea_fwd_noalloc(const vmo_fea_fwd_args* args, void* stream);

/* Bytes of workspace vmo_fea_bwd needs for these arguments. */
size_t vmo_fea_bwd_workspace_size(const vmo_fea_bwd_args* args);

/* FlashEntropyAttention backward; see vmo_fea_bwd_args. */
int vmo_fea_bwd(const vmo_fea_bwd_args* args, void* stream);

/* Fused L-step; see vmo_lstep_args. */
int vmo_lstep_fwd(const vmo_lstep_args* args, void* stream);

/* Backward of the fused L-step; see vmo_lstep_bwd_args. */
int vmo_lstep_bwd(const vmo_lstep_bwd_args* args, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* VMONARCH_AMD_H */
