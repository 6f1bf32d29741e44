// FlashEntropyAttention backward for gfx950.
//
// Reference: video_monarch_attention/kernel.py:154-313 (_attn_bwd_preprocess, _attn_bwd_dkdv,
// _attn_bwd_dq, _attn_bwd) launched from _FlashEntropyAttention.backward (kernel.py:360-381).
// Gradient of a natural-units logit S_ij = sm_scale q_i . k_j (kernel.py:165-167):
//   dS = P (dP - delta) + dE P (-E - ln P),  delta_i = sum_d o_id dO_id,  dP = dO V^T
// rewritten per query row as  dS = P (dP + alpha_i + beta_i x),  x = log2 P = s c - lse,
//   alpha_i = -delta_i - dE_i E_i,   beta_i = -dE_i ln 2
// so the inner loops need three per-row scalars (lse, alpha, beta).  Then
//   dQ = sm_scale dS K,  dK = sm_scale dS^T Q,  dV = P^T dO.
//
// Two kernels on the caller's stream:
//  * fea_bwd_dq: one workgroup = 128 queries (32 per wave), loop over 64-key stages exactly like
//    the forward (S^T = K Q^T and dP^T = V dO^T with Q / dO held as B operands in registers, one
//    query per lane); dQ^T += K^T dS^T reads K^T from the same LDS tile by ds_read_tr16_b64.  Its
//    prologue forms delta from o and dO in registers and writes alpha / beta for the second kernel.
//  * fea_bwd_dkdv: one workgroup = 128 keys (32 per wave, K / V rows held as B operands), loop over
//    32-query stages: S = Q K^T and dP = dO V^T (one key per lane), then dV^T += dO^T P and
//    dK^T += Q^T dS with dO^T / Q^T read transposed from the staged tiles.
// Values may come in two parts [v | v1] (VMonarch's [k | v] without a concatenated copy), and when
// they are k itself or start with it the K operands double as dP's V operands for those columns.
// Gradients are written in the inputs' dtype or into fp32 buffers (added to or overwritten).
// P and dS enter the MFMAs as bf16 / fp16 (the reference's dK / dQ dots run in fp32 = tf32 on its
// hardware; gfx950 has no xf32 MFMA -- parity is checked at the stated gradient tolerance).
#include <type_traits>

#include "vmo_common.h"
#include "vmo_host.h"

namespace vmo {

constexpr int kBwdWaves = 4;
constexpr int kDqBM = 128;     // queries per dq workgroup
constexpr int kDqBN = 64;      // keys per dq stage
constexpr int kKvBN = 128;     // keys per dkdv workgroup
constexpr int kKvBM = 32;      // queries per dkdv stage
constexpr int kBwdPrefetch = 2;   // LDS operand reads kept in flight ahead of the MFMA that uses them
// ... in the dq kernel: none for 64 / 64, which then fits three waves per SIMD (168 registers)
template <int D, int DV>
constexpr int dq_prefetch() { return D + DV <= 128 ? 0 : kBwdPrefetch; }

struct BwdParams {
  const void* q;
  const void* k;
  const void* v;
  const void* v1;   // second value part ([v | v1], same strides as v), or null
  int v0_is_k;      // the values are k itself, or with v1 start with it (same address and strides)
  const void* o;
  const void* dO;
  void* dq;
  void* dk;
  void* dv;
  const float* lse;
  const float* ent;
  const float* dent;
  float* alpha;     // workspace (problems, nq)
  float* beta;
  float* dq_part;   // workspace (dq_splits, problems, nq, D): split-KV partial dQ, when dq_splits > 1
  int64_t q_sb, q_sh, q_sn, k_sb, k_sh, k_sn, v_sb, v_sh, v_sn, o_sb, o_sh, o_sn, do_sb, do_sh, do_sn;
  int64_t dq_sb, dq_sh, dq_sn, dk_sb, dk_sh, dk_sn, dv_sb, dv_sh, dv_sn;
  int64_t st_sb, st_sh, de_sb, de_sh;
  int heads, frames, nq, nk, problems;   // problems = batch * heads * frames
  int dq_tiles, kv_tiles;
  int dq_total, kv_total;
  int dq_splits, keys_per_split;   // dq workgroups per query tile, each over one key range
  int accum;                       // VMO_BWD_ACCUM_* / VMO_BWD_F32_* bits: that gradient is fp32, added to / stored
  int fold_k;                      // (values k or [k | v1]) k's value-role gradient goes into dk; dv holds v1's
  const void* dk_base;             // VMO_BWD_SUM_K / _V: fp32 rows added to dk / dv before their dtype store
  const void* dv_base;
  void* ds;                        // dS route: dS^T of every problem in 32 x 32 blocks (the inputs' dtype),
  int ds_kblocks, ds_qblocks;      // (problems, ceil(nk / 32), ceil(nq / 32), 32 keys, 32 queries)
  int64_t dkb_sb, dkb_sh, dkb_sn, dvb_sb, dvb_sh, dvb_sn;
  const void* dq_base;             // VMO_BWD_SUM_Q: fp32 rows added to dq before its dtype store
  int64_t dqb_sb, dqb_sh, dqb_sn;
  const float* delta;              // optional rowsum(o * dO) per query (else formed from o and dO)
  int64_t dl_sb, dl_sh;
  float c;          // sm_scale * log2(e)
  float sm_scale;
  float ds_scale;   // factor of the dq GEMM over a stored dS^T: sm_scale, or 1 when the stored dS carries it
};

// Copy rows row0 .. row0 + ROWS - 1 (clamped to nrows - 1) of a row-major (token, W) tensor into an
// LDS tile with the 64-bank chunk swizzle swz_rows<2 W>, by the 4 waves together.  The copies are
// asynchronous (dma16_async); the caller orders them with tile_sync<>.
template <class T, int W, int ROWS>
__device__ __forceinline__ void stage_rows_n(const T* __restrict__ base, int64_t sn, int row0, int nrows,
                                             uint32_t dst, int wave, int lane) {
  constexpr int CH = W / 8;
  constexpr int RPI = 64 / CH;
  constexpr int NI = ROWS / RPI;          // wave instructions for the whole tile
  static_assert(CH >= 8 && NI % kBwdWaves == 0, "tile shape");
#pragma unroll
  for (int i = 0; i < NI / kBwdWaves; ++i) {
    const int inst = i * kBwdWaves + wave;
    const int r = inst * RPI + lane / CH;
    const int lc = (lane % CH) ^ swz_rows<W * 2>(r);
    int gr = row0 + r;
    gr = gr < nrows ? gr : nrows - 1;
    dma16_async(base + (int64_t)gr * sn + lc * 8, dst + inst * 1024);
  }
}

// The same copy of a tile whose rows are [a | b]: columns [0, W/2) from a, [W/2, W) from b (same
// strides).  swz_rows only flips a chunk index within its 16-chunk group, so for W >= 256 each lane's
// source stays in the half of its destination; for W = 128 the half follows the swizzled chunk.
template <class T, int W, int ROWS>
__device__ __forceinline__ void stage_rows_n2(const T* __restrict__ a, const T* __restrict__ b, int64_t sn, int row0,
                                              int nrows, uint32_t dst, int wave, int lane) {
  constexpr int CH = W / 8;
  constexpr int RPI = 64 / CH;
  constexpr int NI = ROWS / RPI;
  static_assert(CH >= 8 && NI % kBwdWaves == 0, "tile shape");
#pragma unroll
  for (int i = 0; i < NI / kBwdWaves; ++i) {
    const int inst = i * kBwdWaves + wave;
    const int r = inst * RPI + lane / CH;
    const int lc = (lane % CH) ^ swz_rows<W * 2>(r);
    int gr = row0 + r;
    gr = gr < nrows ? gr : nrows - 1;
    const T* src = lc < CH / 2 ? a : b;
    dma16_async(src + (int64_t)gr * sn + (lc % (CH / 2)) * 8, dst + inst * 1024);
  }
}

// The same copy for the tiles staged inside the key / query loops: per-lane byte offsets computed
// once, a scalar row base per tile (a full tile costs scalar adds only; the clamped per-lane path is
// taken by a tile that runs past the end).  Row strides must stay below 2^27 elements (32-bit lane
// offsets over up to 7 rows).  SW < W (a 16-wide tensor in a 32-wide tile, tile_w): logical chunk c of a row
// holds the source row's chunk c % (SW / 8).
template <class T, int W, int ROWS, int SW = W>
struct BwdTileCopy {
  static constexpr int CH = W / 8;
  static constexpr int RPI = 64 / CH;
  static constexpr int TI = ROWS / RPI;   // copy instructions per tile: a narrow tile has fewer than the waves
  static constexpr int NI = (TI + kBwdWaves - 1) / kBwdWaves;   // ... and waves wave < TI copy it
  static constexpr int NV = (kBwdWaves * RPI) % 16 == 0 ? 1 : 2;   // distinct lane offsets (swizzle period 16)
  static_assert(CH >= 4 && TI >= 1 && RPI >= 2 && ROWS % RPI == 0 && (TI % kBwdWaves == 0 || TI < kBwdWaves),
                "tile shape");
  uint64_t ubase, rbytes;
  uint32_t voff[NV];
  int wave, lane;

  __device__ __forceinline__ BwdTileCopy(const T* b, int64_t sn, int w, int l) : wave(w), lane(l) {
    ubase = uniform64((uint64_t)(uintptr_t)b);
    rbytes = uniform64((uint64_t)sn * 2);
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int r = (v * kBwdWaves + w) * RPI + l / CH;
      voff[v] = (uint32_t)((int64_t)(l / CH) * sn * 2) + (uint32_t)((((l % CH) ^ swz_rows<W * 2>(r)) & (SW / 8 - 1)) * 16);
    }
  }
  __device__ __forceinline__ void issue(int row0, int nrows, uint32_t dst) const {
    uint64_t ub = ubase;
    asm volatile("" : "+s"(ub));   // recomputed per call: hoisted, the addresses would pin scalar registers
    if (TI < kBwdWaves && wave >= TI) return;   // (wave-uniform)
    if (row0 + ROWS <= nrows) {
      const uint64_t tb = ub + (uint64_t)(row0 + wave * RPI) * rbytes;
#pragma unroll
      for (int i = 0; i < NI; ++i)
        dma16_async_s(tb + (uint64_t)(i * kBwdWaves * RPI) * rbytes, voff[i % NV], dst + (i * kBwdWaves + wave) * 1024);
    } else {
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int inst = i * kBwdWaves + wave;
        const int r = inst * RPI + lane / CH;
        const int gr = min(row0 + r, nrows - 1);
        dma16_async((const void*)(uintptr_t)(ub + (uint64_t)gr * rbytes +
                                             (((lane % CH) ^ swz_rows<W * 2>(r)) & (SW / 8 - 1)) * 16),
                    dst + inst * 1024);
      }
    }
  }
};

// BwdTileCopy for a tile whose rows are [a | b] (as stage_rows_n2): each lane keeps the 64-bit
// address of its chunk in its instruction's first row, so a full tile costs one 64-bit add per copy.
template <class T, int W, int ROWS>
struct BwdTileCopy2 {
  static constexpr int CH = W / 8;
  static constexpr int RPI = 64 / CH;
  static constexpr int NI = ROWS / RPI / kBwdWaves;
  static constexpr int NV = (kBwdWaves * RPI) % 16 == 0 ? 1 : 2;
  static_assert(CH >= 8 && NI >= 1 && RPI >= 2, "tile shape");
  const T* a;
  const T* b;
  int64_t sn;
  uint64_t rbytes;
  uint64_t lbase[NV];
  int wave, lane;

  __device__ __forceinline__ BwdTileCopy2(const T* a_, const T* b_, int64_t sn_, int w, int l)
      : a(a_), b(b_), sn(sn_), wave(w), lane(l) {
    rbytes = uniform64((uint64_t)sn_ * 2);
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int r = (v * kBwdWaves + w) * RPI + l / CH;
      const int lc = (l % CH) ^ swz_rows<W * 2>(r);
      lbase[v] = (uint64_t)(uintptr_t)((lc < CH / 2 ? a_ : b_) + (int64_t)(l / CH) * sn_ + (lc % (CH / 2)) * 8);
    }
  }
  __device__ __forceinline__ void issue(int row0, int nrows, uint32_t dst) const {
    if (row0 + ROWS <= nrows) {
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const uint64_t roff = (uint64_t)(row0 + (i * kBwdWaves + wave) * RPI) * rbytes;
        dma16_async((const void*)(uintptr_t)(lbase[i % NV] + roff), dst + (i * kBwdWaves + wave) * 1024);
      }
    } else {
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int inst = i * kBwdWaves + wave;
        const int r = inst * RPI + lane / CH;
        const int lc = (lane % CH) ^ swz_rows<W * 2>(r);
        const int gr = min(row0 + r, nrows - 1);
        dma16_async((lc < CH / 2 ? a : b) + (int64_t)gr * sn + (lc % (CH / 2)) * 8, dst + inst * 1024);
      }
    }
  }
};

// Byte offset, within a 32-row block of a row-major LDS tile with RB-byte rows, of this lane's
// first ds_read_tr16_b64 for accumulator block a (rows trow and trow + 4 of the 4-row groups); the
// second read of the pair is 8 rows down at (offset ^ 32), since swz_rows(r + 8) = swz_rows(r) ^ 2.
template <int RB>
__device__ __forceinline__ int tr_offset(int trow, int tchunk, int tbyte, int a) {
  return trow * RB + (((4 * a + tchunk) ^ swz_rows<RB>(trow)) * 16 + tbyte);
}
template <class V8, int RB>
__device__ __forceinline__ V8 tr_pair(const VMO_LDS char* block16, int c0) {
  return lds_read_tr8<V8>(block16 + c0, block16 + 8 * RB + (c0 ^ 32));
}

// Waves per SIMD the register budget is sized for: wide value heads keep more accumulators live.
template <int D, int DV>
constexpr int bwd_waves_per_simd() { return D + DV > 320 ? 1 : 2; }

// The dkdv kernel for 256-wide values runs as two launches (PART 1: dK and dV[:, :128], with dP over
// all 256 value columns; PART 2: dV[:, 128:] from P alone): one launch holding dK and the whole dV
// needs ~290 accumulator and operand registers, and the compiler then moves every accumulator
// between AGPRs and VGPRs around each MFMA.  PART 0 is the single launch of the narrower variants,
// and of values [k | v1] at 128 / 256, whose V operand registers the K operand replaces (it then fits
// one wave per SIMD without moving accumulators).
template <int D, int DV, bool W0K>
constexpr int dkdv_parts() { return DV > 128 && !(W0K && D == 128 && DV == 256) ? 2 : 1; }
// PART 3: values [k | v1] with VMO_BWD_FOLD_K at 128 / 256, the first of two launches (PART 2 gives v1's
// gradient): dK and k's value-role gradient accumulate in one set of registers -- dK = sm_scale dS^T Q +
// P^T dO[:, :D] with dS entering the MFMA already times sm_scale -- so that the launch holds 64 accumulator
// registers instead of the 192 of PART 0 (dK and all 256 dV columns) and runs two waves per SIMD with K and
// V1 as register operands.
template <int DV, int PART>
constexpr int dkdv_do_width() { return PART == 2 ? DV / 2 : DV; }   // dO columns staged per stage
template <int DV, int PART>
constexpr int dkdv_dv_width() { return PART == 0 ? DV : PART == 3 ? 0 : DV / 2; }   // dV columns accumulated
// dkdv variants that read the V operand of dP = dO V^T from an LDS copy of the workgroup's 128 V rows
// instead of holding it in registers (128 / 128 and the 256-wide value variants would otherwise spill).
template <int D, int DV, int PART>
constexpr bool dkdv_v_in_lds() { return PART != 2 && PART != 3 && D + DV >= 256; }
// ... and of K for S = Q K^T, in the first part of the 128 / 256 variant
template <int D, int DV, int PART>
constexpr bool dkdv_k_in_lds() { return PART == 1 && D == 128 && DV == 256; }
// 256-wide q/k heads (K alone is 64 registers, dK 128) run one wave per SIMD in both parts
template <int D, int DV, int PART>
constexpr int dkdv_waves_per_simd() { return D >= 256 ? 1 : PART != 0 ? 2 : bwd_waves_per_simd<D, DV>(); }
// V columns the dkdv kernel holds per key: all DV, or when the values start with k itself (W0K) only
// the columns after k (none for values k) -- dP's k part takes the K operand that S = Q K^T reads anyway
template <int D, int DV, bool W0K>
constexpr int dkdv_v_width() { return W0K ? DV - D : DV; }
template <int D, int DV, int PART, bool W0K>
constexpr int dkdv_lds_bytes() {
  // (at least the four waves' epilogue patches: the narrow heads' stages are smaller)
  constexpr int ring = 2 * (kKvBM * (tile_w(D) + tile_w(dkdv_do_width<DV, PART>())) * 2 + 512) +
                       (dkdv_v_in_lds<D, DV, PART>() ? kKvBN * dkdv_v_width<D, DV, W0K>() * 2 : 0) +
                       (dkdv_k_in_lds<D, DV, PART>() ? kKvBN * D * 2 : 0);
  return ring > kBwdWaves * kEpiPatchBytes ? ring : kBwdWaves * kEpiPatchBytes;
}

// ------------------------------------------------------------------------------------------------
// Value columns the dq kernel stages per key: all DV, or when the values start with k itself (W0K:
// values k, or [k | v1]) only the columns after k -- dP's k part reuses the K fragments that
// S = K Q^T reads anyway (values k alone stage no V tile at all).
template <int D, int DV, bool W0K>
constexpr int dq_staged_dv() { return W0K ? DV - D : DV; }

// The dq kernels' epilogue: a wave's 32 rows of dQ (accumulated unscaled, times sm_scale here) as the fp32
// partial of its key split (summed by fea_bwd_dq_reduce), or into grad_q in the mode the flags ask for.
template <bool F16, int D>
__device__ __forceinline__ void store_dq(const BwdParams& p, const f32x16 (&acc)[tile_w(D) / 32], VMO_LDS float* patch,
                                         int prob, int split, int bb, int hh, int64_t qoff, int q0, int lane,
                                         float scale) {
  constexpr int NA = tile_w(D) / 32, CW = D < 32 ? 16 : 32;
  const int nrows = min(32, p.nq - q0);
  if (p.dq_splits > 1) {
    float* pr = p.dq_part + (((int64_t)split * p.problems + prob) * p.nq + q0) * D;
    store_acc_rows<F16, CW>(patch, acc, NA, scale, kGradStoreF32, (char*)pr, (int64_t)D * 4, nrows, lane);
  } else {
    const int mode = grad_mode(p.accum, VMO_BWD_ACCUM_Q, VMO_BWD_F32_Q, VMO_BWD_SUM_Q);
    const int64_t es = mode == kGradStore || mode == kGradSumStore ? 2 : 4;
    char* row0 = (char*)p.dq + (bb * p.dq_sb + hh * p.dq_sh + (qoff + q0) * p.dq_sn) * es;
    const char* src0 = mode == kGradSumStore
                           ? (const char*)p.dq_base + (bb * p.dqb_sb + hh * p.dqb_sh + (qoff + q0) * p.dqb_sn) * 4
                           : nullptr;
    store_acc_rows<F16, CW>(patch, acc, NA, scale, mode, row0, p.dq_sn * es, nrows, lane, 0, src0, p.dqb_sn * 4);
  }
}

template <bool F16, int D, int DV, bool V2, bool W0K>
__global__ __launch_bounds__(256, (bwd_waves_per_simd<D, DV>())) void fea_bwd_dq_kernel(BwdParams p) {
  using E = Elem<F16>;
  using T = typename E::T;
  using V8 = typename E::V8;
  using V4 = typename E::V4;
  static_assert(!W0K || (V2 ? DV == 2 * D : DV == D), "values k or [k | v1]");
  constexpr int DVL = dq_staged_dv<D, DV, W0K>();
  constexpr int DK = tile_w(D), DVLK = DVL ? tile_w(DVL) : 0;   // widths in LDS
  constexpr int K_BYTES = kDqBN * DK * 2;
  constexpr int STAGE = kDqBN * (DK + DVLK) * 2;
  constexpr int NA = DK / 32;
  extern __shared__ __attribute__((aligned(1024))) char smem_raw[];
  VMO_LDS char* smem = (VMO_LDS char*)smem_raw;

  const int L = xcd_remap(gridDim.x);
  if (L >= p.dq_total) return;
  // workgroup-uniform indices, moved to scalar registers (integer division runs on the vector unit)
  auto uni = [](int x) __attribute__((always_inline)) { return __builtin_amdgcn_readfirstlane(x); };
  const int qt = uni(L % p.dq_tiles), split = uni((L / p.dq_tiles) % p.dq_splits);
  const int prob = uni(L / p.dq_tiles / p.dq_splits);
  const int kbeg = split * p.keys_per_split;
  const int kend = min(p.nk, kbeg + p.keys_per_split);
  // problem (b, h, f): query rows [f nq, (f + 1) nq) and key rows [f nk, (f + 1) nk) of the (b, h) tensors
  const int fr = uni(prob % p.frames), bh = uni(prob / p.frames);
  const int hh = uni(bh % p.heads), bb = uni(bh / p.heads);
  const int64_t qoff = (int64_t)fr * p.nq, koff = (int64_t)fr * p.nk;
  const int tid = threadIdx.x, wave = uni(tid >> 6), lane = tid & 63, hl = lane >> 5, l32 = lane & 31;
  const int q0 = qt * kDqBM + wave * 32;
  const bool wave_live = q0 < p.nq;
  const int qrow = q0 + l32;
  const bool qvalid = qrow < p.nq;
  const int qr = qvalid ? qrow : 0;

  const T* kb = (const T*)p.k + bb * p.k_sb + hh * p.k_sh + koff * p.k_sn;
  const T* vb = (const T*)p.v + bb * p.v_sb + hh * p.v_sh + koff * p.v_sn;
  const T* v1b = (const T*)p.v1 + bb * p.v_sb + hh * p.v_sh + koff * p.v_sn;

  // Q^T and dO^T as B operands (one query per lane); delta = o . dO in fp32
  V8 qf[D / 16], dof[DV / 16];
  float delta = 0.f;
  {
    const T* qp = (const T*)p.q + bb * p.q_sb + hh * p.q_sh + (qoff + qr) * p.q_sn + hl * 8;
    const T* dp = (const T*)p.dO + bb * p.do_sb + hh * p.do_sh + (qoff + qr) * p.do_sn + hl * 8;
    const T* op = (const T*)p.o + bb * p.o_sb + hh * p.o_sh + (qoff + qr) * p.o_sn + hl * 8;
#pragma unroll
    for (int ds = 0; ds < D / 16; ++ds) {
      V8 x = *(const V8*)(qp + ds * 16);
      qf[ds] = qvalid ? x : V8{};
      asm volatile("" : "+v"(qf[ds]));   // loaded and waited for here, never re-loaded in the loop
    }
#pragma unroll
    for (int ds = 0; ds < DV / 16; ++ds) {
      V8 x = *(const V8*)(dp + ds * 16);
      dof[ds] = qvalid ? x : V8{};
      asm volatile("" : "+v"(dof[ds]));
      if (!p.delta) {   // o is read for delta alone
        V8 y = *(const V8*)(op + ds * 16);
#pragma unroll
        for (int e = 0; e < 8; ++e) delta = fmaf((float)x[e], (float)y[e], delta);
      }
    }
  }
  delta = p.delta ? p.delta[bb * p.dl_sb + hh * p.dl_sh + qoff + qr] : wave_sum32(delta);
  const int64_t si = bb * p.st_sb + hh * p.st_sh + qoff + qr;
  const float lse = p.lse[si];
  const float dE = p.dent[bb * p.de_sb + hh * p.de_sh + qoff + qr];
  float alpha = -delta - dE * p.ent[si];
  float beta = -dE * kLn2;
  float lse_r = lse;
  // the per-row scalars are waited for here: a wait inside the key loop would also wait for the copies
  asm volatile("" : "+v"(alpha), "+v"(beta), "+v"(lse_r));
  if (qvalid && hl == 0 && split == 0) {
    p.alpha[(int64_t)prob * p.nq + qrow] = alpha;
    p.beta[(int64_t)prob * p.nq + qrow] = beta;
  }

  const int n_tiles = (kend - kbeg + kDqBN - 1) / kDqBN;
  const uint32_t smem_u32 = (uint32_t)(uintptr_t)smem;
  const BwdTileCopy<T, DK, kDqBN, D> kcopy(kb, p.k_sn, wave, lane);
  const auto vcopy = [&]() __attribute__((always_inline)) {
    if constexpr (W0K && DVL == 0)
      return 0;   // values k: nothing beyond the K tile
    else if constexpr (W0K)
      return BwdTileCopy<T, DVLK, kDqBN, DVL>(v1b, p.v_sn, wave, lane);
    else if constexpr (V2)
      return BwdTileCopy2<T, DV, kDqBN>(vb, v1b, p.v_sn, wave, lane);
    else
      return BwdTileCopy<T, DVLK, kDqBN, DV>(vb, p.v_sn, wave, lane);
  }();
  auto issue = [&](int t) {
    const uint32_t st = smem_u32 + (uint32_t)((t & 1) * STAGE);
    kcopy.issue(kbeg + t * kDqBN, kend, st);
    if constexpr (DVL > 0) vcopy.issue(kbeg + t * kDqBN, kend, st + K_BYTES);
  };

  f32x16 acc[NA];
#pragma unroll
  for (int a = 0; a < NA; ++a) acc[a] = f32x16{};
  const float c = p.c;
  const int ksw = swz_rows<DK * 2>(l32), vsw = swz_rows<(DVL > 0 ? DVLK : DK) * 2>(l32);
  const int trow = 4 * hl + ((lane & 15) >> 2);
  const int tchunk = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
  const int tbyte = (lane & 1) * 8;

  // one 64-key stage; only a partial last stage masks its keys, and it is peeled out of the loop
  auto iteration = [&](int t, auto masked_tag) __attribute__((always_inline)) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    tile_sync<0>();   // stage t has landed for every wave, and stage t - 1's slot is free
    if (t + 1 < n_tiles) issue(t + 1);
    if (!wave_live) return;
    const VMO_LDS char* Ks = smem + (t & 1) * STAGE;
    const VMO_LDS char* Vs = Ks + K_BYTES;
    const int nvalid = kend - kbeg - t * kDqBN;
    f32x16 s[2] = {f32x16{}, f32x16{}}, dp[2] = {f32x16{}, f32x16{}};
    // S = K Q^T and dP = V dO^T for two 32-key blocks (with W0K the K fragments also give dP's k half)
    constexpr int NSQ = D / 16, NSD = D / 16 + DVL / 16, DO0 = (DV - DVL) / 16;
    prefetched_chain<2 * NSD, dq_prefetch<D, DV>()>(
        [&](int i) __attribute__((always_inline)) {
          const int kb2 = i / NSD, j = i % NSD;
          return j < NSQ ? lds_read8<V8>(Ks + (32 * kb2 + l32) * (DK * 2) + ((2 * j + hl) ^ ksw) * 16)
                         : lds_read8<V8>(Vs + (32 * kb2 + l32) * (DVLK * 2) + ((2 * (j - NSQ) + hl) ^ vsw) * 16);
        },
        [&](int i, const V8& x) __attribute__((always_inline)) {
          const int kb2 = i / NSD, j = i % NSD;
          if (j < NSQ) {
            s[kb2] = E::mfma(x, qf[j], s[kb2]);
            if constexpr (W0K) dp[kb2] = E::mfma(x, dof[j], dp[kb2]);
          } else {
            dp[kb2] = E::mfma(x, dof[DO0 + j - NSQ], dp[kb2]);
          }
        });
    if constexpr (dq_prefetch<D, DV>() > 0) {   // reads two steps ahead of their MFMAs, as in dkdv
      struct Chain {
        static constexpr int reads(int) { return 1; }
        static constexpr int mfmas(int i) { return W0K && i % NSD < NSQ ? 2 : 1; }
        static constexpr int ahead(int) { return 2; }
        static constexpr int lead() { return 0; }
      };
      pin_chain<Chain, 2 * NSD>();
    }
    V8 G[4];
#pragma unroll
    for (int kb2 = 0; kb2 < 2; ++kb2) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float x = fmaf(s[kb2][r], c, -lse_r);
        float g = fast_exp2(x) * (dp[kb2][r] + fmaf(beta, x, alpha));
        if (MASKED && 32 * kb2 + 8 * (r >> 2) + 4 * hl + (r & 3) >= nvalid) g = 0.f;
        G[2 * kb2 + (r >> 3)][r & 7] = to_elem<T>(g);
      }
    }
    // dQ^T[d][q] += K^T dS^T (transposed reads of the staged K tile)
    prefetched_chain<4 * NA, dq_prefetch<D, DV>()>(
        [&](int i) __attribute__((always_inline)) {
          return tr_pair<V8, DK * 2>(Ks + 16 * (i % 4) * (DK * 2), tr_offset<DK * 2>(trow, tchunk, tbyte, i / 4));
        },
        [&](int i, const V8& x) __attribute__((always_inline)) { acc[i / 4] = E::mfma(x, G[i % 4], acc[i / 4]); });
  };
  issue(0);
  const int n_full = (kend - kbeg) / kDqBN;   // stages with 64 valid keys
  for (int t = 0; t < n_full; ++t) iteration(t, std::false_type{});
  if (n_full < n_tiles) iteration(n_full, std::true_type{});
  __syncthreads();   // every wave is done with the stage ring, which the epilogue patches reuse
  if (!wave_live) return;
  store_dq<F16, D>(p, acc, (VMO_LDS float*)(smem + wave * kEpiPatchBytes), prob, split, bb, hh, qoff, q0, lane,
                   p.sm_scale);
}

// Sum the split-KV partials of dQ (fixed split order, so the result does not depend on timing) and
// write grad_q (with VMO_BWD_SUM_Q: plus its fp32 base row), or store / add them into an fp32 grad_q.
template <bool F16, int D>
__global__ __launch_bounds__(256) void fea_bwd_dq_reduce(BwdParams p) {
  using T = typename Elem<F16>::T;
  using V4 = typename Elem<F16>::V4;
  constexpr int TPR = D / 4;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t row = gid / TPR;
  const int c4 = (int)(gid % TPR);
  if (row >= (int64_t)p.problems * p.nq) return;
  const int prob = (int)(row / p.nq), qi = (int)(row % p.nq);
  f32x4 acc = f32x4{};
  for (int sp = 0; sp < p.dq_splits; ++sp)
    acc += *(const f32x4*)(p.dq_part + (((int64_t)sp * p.problems + prob) * p.nq + qi) * D + 4 * c4);
  const int fr = prob % p.frames, bh = prob / p.frames, hh = bh % p.heads, bb = bh / p.heads;
  const int64_t row_q = (int64_t)fr * p.nq + qi;
  const int mode = grad_mode(p.accum, VMO_BWD_ACCUM_Q, VMO_BWD_F32_Q, VMO_BWD_SUM_Q);
  if (mode == kGradAddF32 || mode == kGradStoreF32) {
    f32x4* ptr = (f32x4*)((float*)p.dq + bb * p.dq_sb + hh * p.dq_sh + row_q * p.dq_sn + 4 * c4);
    *ptr = mode == kGradAddF32 ? *ptr + acc : acc;
  } else {
    if (mode == kGradSumStore)   // the base plus the (unrounded) sum of the partials, rounded once
      acc += *(const f32x4*)((const float*)p.dq_base + bb * p.dqb_sb + hh * p.dqb_sh + row_q * p.dqb_sn + 4 * c4);
    V4 v;
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = to_elem<T>(acc[e]);
    *(V4*)((T*)p.dq + bb * p.dq_sb + hh * p.dq_sh + row_q * p.dq_sn + 4 * c4) = v;
  }
}

// ------------------------------------------------------------------------------------------------
// The dS route.  For short rows (VMonarch's frame blocks: 1560 keys) the dq kernel above spends most of
// its MFMAs recomputing S and dP; here the dkdv kernel, which forms dS anyway, stores it (dS^T, in the
// inputs' dtype -- the value both routes feed the dQ MFMAs), and dQ = sm_scale dS K becomes a GEMM that
// streams it back.  Three launches: fea_bwd_prep (the per-row scalars the dq kernel's prologue forms),
// fea_bwd_dkdv with DS, fea_bwd_dq_ds (+ fea_bwd_dq_reduce for key splits).

// delta = o . dO of every query row (fp32; or the given delta), then alpha = -delta - dE E and
// beta = -dE ln 2 into the workspace; DV / 8 lanes per row, 16 bytes each.
template <bool F16, int DV>
__global__ __launch_bounds__(256) void fea_bwd_prep_kernel(BwdParams p) {
  using T = typename Elem<F16>::T;
  using V8 = typename Elem<F16>::V8;
  constexpr int TPR = DV / 8;
  if (p.delta) {   // given (formed by the L-step backward that wrote dO): one lane per row
    const int64_t row = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (row >= (int64_t)p.problems * p.nq) return;
    const int prob = (int)(row / p.nq), qi = (int)(row % p.nq);
    const int fr = prob % p.frames, bh = prob / p.frames, hh = bh % p.heads, bb = bh / p.heads;
    const int64_t qrow = (int64_t)fr * p.nq + qi;
    const float dE = p.dent[bb * p.de_sb + hh * p.de_sh + qrow];
    p.alpha[row] = -p.delta[bb * p.dl_sb + hh * p.dl_sh + qrow] - dE * p.ent[bb * p.st_sb + hh * p.st_sh + qrow];
    p.beta[row] = -dE * kLn2;
    return;
  }
  static_assert(TPR >= 2 && TPR <= 64 && 64 % TPR == 0, "row lanes within one wave");
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t rows = (int64_t)p.problems * p.nq;
  const int64_t row = gid / TPR;
  const int part = (int)(gid % TPR);
  const int64_t rr = row < rows ? row : rows - 1;
  const int prob = (int)(rr / p.nq), qi = (int)(rr % p.nq);
  const int fr = prob % p.frames, bh = prob / p.frames, hh = bh % p.heads, bb = bh / p.heads;
  const int64_t qrow = (int64_t)fr * p.nq + qi;
  const V8 x = *(const V8*)((const T*)p.dO + bb * p.do_sb + hh * p.do_sh + qrow * p.do_sn + 8 * part);
  const V8 y = *(const V8*)((const T*)p.o + bb * p.o_sb + hh * p.o_sh + qrow * p.o_sn + 8 * part);
  float d = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) d = fmaf((float)x[e], (float)y[e], d);
#pragma unroll
  for (int m = TPR / 2; m >= 1; m >>= 1) d += __shfl_xor(d, m);
  if (row < rows && part == 0) {
    const int64_t si = bb * p.st_sb + hh * p.st_sh + qrow;
    const float dE = p.dent[bb * p.de_sb + hh * p.de_sh + qrow];
    p.alpha[row] = -d - dE * p.ent[si];
    p.beta[row] = -dE * kLn2;
  }
}

// dQ from the stored dS^T: one workgroup = 128 queries (32 per wave) of one problem and one key range,
// 64-key stages of K rows and of dS^T (keys x the tile's 128 query columns, gathered from the 32 x 32
// blocks) staged by global_load_lds; dQ^T += K^T dS^T with both operands read transposed
// (ds_read_tr16_b64), so both hold the same 4-key groups.
template <bool F16, int D>
__global__ __launch_bounds__(256, 2) void fea_bwd_dq_ds_kernel(BwdParams p) {
  using E = Elem<F16>;
  using T = typename E::T;
  using V8 = typename E::V8;
  constexpr int K_BYTES = kDqBN * D * 2;
  constexpr int SRB = kDqBM * 2;   // bytes of one staged dS^T row
  constexpr int STAGE = K_BYTES + kDqBN * SRB;
  constexpr int NA = D / 32;
  extern __shared__ __attribute__((aligned(1024))) char smem_raw[];
  VMO_LDS char* smem = (VMO_LDS char*)smem_raw;

  const int L = xcd_remap(gridDim.x);
  if (L >= p.dq_total) return;
  auto uni = [](int x) __attribute__((always_inline)) { return __builtin_amdgcn_readfirstlane(x); };
  const int qt = uni(L % p.dq_tiles), split = uni((L / p.dq_tiles) % p.dq_splits);
  const int prob = uni(L / p.dq_tiles / p.dq_splits);
  const int kbeg = split * p.keys_per_split;
  const int kend = min(p.nk, kbeg + p.keys_per_split);
  const int fr = uni(prob % p.frames), bh = uni(prob / p.frames);
  const int hh = uni(bh % p.heads), bb = uni(bh / p.heads);
  const int64_t qoff = (int64_t)fr * p.nq, koff = (int64_t)fr * p.nk;
  const int tid = threadIdx.x, wave = uni(tid >> 6), lane = tid & 63, hl = lane >> 5;
  const int q0 = qt * kDqBM + wave * 32;
  const bool wave_live = q0 < p.nq;

  const T* kb = (const T*)p.k + bb * p.k_sb + hh * p.k_sh + koff * p.k_sn;
  const int n_tiles = (kend - kbeg + kDqBN - 1) / kDqBN;
  const uint32_t smem_u32 = (uint32_t)(uintptr_t)smem;
  const BwdTileCopy<T, D, kDqBN> kcopy(kb, p.k_sn, wave, lane);
  // The dS^T tile of a stage, [64 keys][128 queries] in LDS with the swz_rows<256> chunk swizzle: wave
  // instruction i (of 4) fills rows 4 (4 i + wave) .. + 3, lane l row 4 (4 i + wave) + l / 16 at chunk
  // position l % 16, i.e. the 16 bytes of logical chunk lc = (l % 16) ^ swz(row): 8 queries of query
  // block 4 qt + lc / 4.  Blocks past the last (the last tile's columns past nq) are clamped to it: they
  // only feed dQ rows that are never written.  Per lane, the byte offset from the stage's first key block.
  const uint64_t s_prob = uniform64((uint64_t)(uintptr_t)p.ds + (uint64_t)prob * p.ds_kblocks * p.ds_qblocks * 2048);
  const int qbs = p.ds_qblocks;
  uint32_t s_off[4];
  int s_row[4], s_col[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    s_row[i] = 4 * (4 * i + wave) + lane / 16;
    const int lc = (lane % 16) ^ swz_rows<SRB>(s_row[i]);
    s_col[i] = min(qt * 4 + lc / 4, qbs - 1) * 2048 + (lc & 3) * 16;
    s_off[i] = (uint32_t)(((s_row[i] >> 5) * qbs) * 2048 + (s_row[i] & 31) * 64 + s_col[i]);
  }
  auto issue = [&](int t) {
    const uint32_t st = smem_u32 + (uint32_t)((t & 1) * STAGE);
    const int row0 = kbeg + t * kDqBN;
    kcopy.issue(row0, kend, st);
    if (row0 + kDqBN <= kend) {
      const uint64_t sbase = s_prob + (uint64_t)(row0 >> 5) * qbs * 2048;
#pragma unroll
      for (int i = 0; i < 4; ++i) dma16_async_s(sbase, s_off[i], st + K_BYTES + (4 * i + wave) * 1024);
    } else {   // the last, partial stage: keys past the range repeat its last key (masked below)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int gr = min(row0 + s_row[i], kend - 1);
        const uint64_t src = s_prob + ((uint64_t)(gr >> 5) * qbs) * 2048 + (gr & 31) * 64 + s_col[i];
        dma16_async((const void*)(uintptr_t)src, st + K_BYTES + (4 * i + wave) * 1024);
      }
    }
  };

  f32x16 acc[NA];
#pragma unroll
  for (int a = 0; a < NA; ++a) acc[a] = f32x16{};
  const int trow = 4 * hl + ((lane & 15) >> 2);
  const int tchunk = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
  const int tbyte = (lane & 1) * 8;
  const int s_tr = tr_offset<SRB>(trow, tchunk, tbyte, wave);   // the wave's 32 query columns

  auto iteration = [&](int t, auto masked_tag) __attribute__((always_inline)) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    tile_sync<0>();   // stage t has landed for every wave, and stage t - 1's slot is free
    if (t + 1 < n_tiles) issue(t + 1);
    if (!wave_live) return;
    const VMO_LDS char* Ks = smem + (t & 1) * STAGE;
    const VMO_LDS char* Ss = Ks + K_BYTES;
    // dS^T operands of the four 16-key chunks: element e of chunk c is key 16 c + 8 (e / 4) + 4 hl + e % 4
    V8 G[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) G[c] = tr_pair<V8, SRB>(Ss + 16 * c * SRB, s_tr);
    if constexpr (MASKED) {   // the staged rows past the key range repeat its last row
      const int nvalid = kend - kbeg - t * kDqBN;
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (16 * c + 8 * (e >> 2) + 4 * hl + (e & 3) >= nvalid) G[c][e] = to_elem<T>(0.f);
    }
    prefetched_chain<4 * NA, kBwdPrefetch>(
        [&](int i) __attribute__((always_inline)) {
          return tr_pair<V8, D * 2>(Ks + 16 * (i % 4) * (D * 2), tr_offset<D * 2>(trow, tchunk, tbyte, i / 4));
        },
        [&](int i, const V8& x) __attribute__((always_inline)) { acc[i / 4] = E::mfma(x, G[i % 4], acc[i / 4]); });
  };
  issue(0);
  const int n_full = (kend - kbeg) / kDqBN;
  for (int t = 0; t < n_full; ++t) iteration(t, std::false_type{});
  if (n_full < n_tiles) iteration(n_full, std::true_type{});
  __syncthreads();   // every wave is done with the stage ring, which the epilogue patches reuse
  if (!wave_live) return;
  store_dq<F16, D>(p, acc, (VMO_LDS float*)(smem + wave * kEpiPatchBytes), prob, split, bb, hh, qoff, q0, lane,
                   p.ds_scale);
}

// ------------------------------------------------------------------------------------------------
template <bool F16, int D, int DV, int PART, bool W0K, bool DS>
__global__ __launch_bounds__(256, (dkdv_waves_per_simd<D, DV, PART>())) void fea_bwd_dkdv_kernel(BwdParams p) {
  using E = Elem<F16>;
  using T = typename E::T;
  using V8 = typename E::V8;
  using V4 = typename E::V4;
  constexpr int DOW = dkdv_do_width<DV, PART>();
  constexpr int VOFF = PART == 2 ? DV / 2 : 0;  // first dV (and staged dO) column of this launch
  constexpr bool WANT_DK = PART != 2;           // dK, and with it dP and dS
  constexpr int DK = tile_w(D), DOWK = tile_w(DOW);   // widths in LDS
  constexpr int Q_BYTES = kKvBM * DK * 2;
  constexpr int DO_BYTES = kKvBM * DOWK * 2;
  constexpr int ST_BYTES = 512;                 // lse[32] | alpha[32] | beta[32] | spare
  constexpr int STAGE = Q_BYTES + DO_BYTES + ST_BYTES;
  constexpr int NK = DK / 32, NV = (dkdv_dv_width<DV, PART>() + 31) / 32;
  constexpr int CWK = D < 32 ? 16 : 32, CWV = DV < 32 ? 16 : 32;   // stored columns per dK / dV block
  constexpr bool V_LDS = dkdv_v_in_lds<D, DV, PART>();
  constexpr bool K_LDS = dkdv_k_in_lds<D, DV, PART>();
  constexpr int VW = dkdv_v_width<D, DV, W0K>();   // V columns held (LDS tile or registers)
  constexpr int V_TILE = V_LDS ? kKvBN * VW * 2 : 0;
  static_assert(!W0K || DV == 2 * D || DV == D, "values k or [k | v1]");
  static_assert(!DS || PART != 2, "the dS route stores dS from the launch that forms it");
  static_assert(PART != 3 || (W0K && DV == 2 * D), "the folded launch is for values [k | v1]");
  constexpr bool FOLD = PART == 3;   // k's value-role gradient in the dK accumulators
  extern __shared__ __attribute__((aligned(1024))) char smem_raw[];
  VMO_LDS char* smem = (VMO_LDS char*)smem_raw;

  const int L = xcd_remap(gridDim.x);
  if (L >= p.kv_total) return;
  auto uni = [](int x) __attribute__((always_inline)) { return __builtin_amdgcn_readfirstlane(x); };
  const int kt = uni(L % p.kv_tiles), prob = uni(L / p.kv_tiles);
  const int fr = uni(prob % p.frames), bh = uni(prob / p.frames);
  const int hh = uni(bh % p.heads), bb = uni(bh / p.heads);
  const int64_t qoff = (int64_t)fr * p.nq, koff = (int64_t)fr * p.nk;
  const int tid = threadIdx.x, wave = uni(tid >> 6), lane = tid & 63, hl = lane >> 5, l32 = lane & 31;
  const int k0 = kt * kKvBN + wave * 32;
  const bool wave_live = k0 < p.nk;
  const int krow = k0 + l32;
  const bool kvalid = krow < p.nk;
  const int kr = kvalid ? krow : p.nk - 1;

  // K^T and V^T as B operands (one key per lane); V^T from LDS in the V_LDS variants
  V8 kf[K_LDS ? 1 : D / 16], vf[(V_LDS || !WANT_DK || VW == 0) ? 1 : VW / 16];
  {
    const T* kp = (const T*)p.k + bb * p.k_sb + hh * p.k_sh + (koff + kr) * p.k_sn + hl * 8;
    const T* vp = (const T*)p.v + bb * p.v_sb + hh * p.v_sh + (koff + kr) * p.v_sn + hl * 8;
    const T* vp1 = p.v1 ? (const T*)p.v1 + bb * p.v_sb + hh * p.v_sh + (koff + kr) * p.v_sn + hl * 8 : vp;
#pragma unroll
    for (int ds = 0; ds < (K_LDS ? 0 : D / 16); ++ds) {
      kf[ds] = *(const V8*)(kp + ds * 16);
      // opaque to the optimiser: otherwise it re-loads K inside the loop under register pressure,
      // and those loads' waits would also wait for the tile copies in flight
      asm volatile("" : "+v"(kf[ds]));
    }
    if constexpr (!V_LDS && WANT_DK) {
#pragma unroll
      for (int ds = 0; ds < VW / 16; ++ds) {
        // columns 16 ds + 8 hl + 0..7 (of the v1 half with W0K): from the second value part when
        // there is one and ds >= DV / 32
        if constexpr (W0K)
          vf[ds] = *(const V8*)(vp1 + ds * 16);
        else
          vf[ds] = p.v1 && ds >= DV / 32 ? *(const V8*)(vp1 + (ds - DV / 32) * 16) : *(const V8*)(vp + ds * 16);
        asm volatile("" : "+v"(vf[ds]));   // as kf: waited for here, not inside the loop
      }
    }
  }
  const T* qb = (const T*)p.q + bb * p.q_sb + hh * p.q_sh + qoff * p.q_sn;
  const T* dob = (const T*)p.dO + bb * p.do_sb + hh * p.do_sh + qoff * p.do_sn;
  const float* lseb = p.lse + bb * p.st_sb + hh * p.st_sh + qoff;
  const float* alb = p.alpha + (int64_t)prob * p.nq;
  const float* beb = p.beta + (int64_t)prob * p.nq;

  const int n_tiles = (p.nq + kKvBM - 1) / kKvBM;
  const uint32_t smem_u32 = (uint32_t)(uintptr_t)smem;
  // dS route: the wave's row of 32 x 32 dS^T blocks (keys k0 .. k0 + 31, one block per query stage)
  const uint64_t ds_base =
      DS ? uniform64((uint64_t)(uintptr_t)p.ds + (((uint64_t)prob * p.ds_kblocks + (k0 >> 5)) * p.ds_qblocks) * 2048) : 0;
  const BwdTileCopy<T, DK, kKvBM, D> qcopy(qb, p.q_sn, wave, lane);
  const BwdTileCopy<T, DOWK, kKvBM, DOW> docopy(dob + VOFF, p.do_sn, wave, lane);
  auto issue = [&](int t) {
    const uint32_t st = smem_u32 + (uint32_t)((t & 1) * STAGE);
    const int row0 = t * kKvBM;
    qcopy.issue(row0, p.nq, st);
    docopy.issue(row0, p.nq, st + Q_BYTES);
    if (wave == 0) {   // per-query scalars: lanes 0-31 lse, 32-63 alpha; then beta
      int qi = row0 + l32;
      qi = qi < p.nq ? qi : p.nq - 1;
      const float* src = hl ? alb + qi : lseb + qi;
      dma4_async(src, st + Q_BYTES + DO_BYTES);
      dma4_async(beb + qi, st + Q_BYTES + DO_BYTES + 256);
    }
  };

  f32x16 dk[NK], dv[NV > 0 ? NV : 1];
#pragma unroll
  for (int a = 0; a < NK; ++a) dk[a] = f32x16{};
#pragma unroll
  for (int a = 0; a < NV; ++a) dv[a] = f32x16{};
  const float gs = FOLD ? p.sm_scale : 1.f;   // dS enters the dK MFMAs times this
  const float c = p.c;
  const int qsw = swz_rows<DK * 2>(l32), dsw = swz_rows<DOWK * 2>(l32), vsw = swz_rows<tile_w(VW > 0 ? VW : D) * 2>(l32);
  const int trow = 4 * hl + ((lane & 15) >> 2);
  const int tchunk = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
  const int tbyte = (lane & 1) * 8;

  const VMO_LDS char* vt_row = smem + 2 * STAGE + (wave * 32 + l32) * (VW * 2);
  const VMO_LDS char* kt_row = smem + 2 * STAGE + V_TILE + (wave * 32 + l32) * (D * 2);
  if constexpr (V_LDS && VW > 0) {   // this workgroup's 128 V rows, once (landed by the first tile_sync)
    const T* vb0 = (const T*)p.v + bb * p.v_sb + hh * p.v_sh + koff * p.v_sn;
    const T* vb1 = (const T*)p.v1 + bb * p.v_sb + hh * p.v_sh + koff * p.v_sn;
    if constexpr (W0K)
      stage_rows_n<T, VW, kKvBN>(vb1, p.v_sn, kt * kKvBN, p.nk, smem_u32 + 2 * STAGE, wave, lane);
    else if (p.v1)
      stage_rows_n2<T, DV, kKvBN>(vb0, vb1, p.v_sn, kt * kKvBN, p.nk, smem_u32 + 2 * STAGE, wave, lane);
    else
      stage_rows_n<T, DV, kKvBN>(vb0, p.v_sn, kt * kKvBN, p.nk, smem_u32 + 2 * STAGE, wave, lane);
  }
  if constexpr (K_LDS)   // and its 128 K rows
    stage_rows_n<T, D, kKvBN>((const T*)p.k + bb * p.k_sb + hh * p.k_sh + koff * p.k_sn, p.k_sn, kt * kKvBN, p.nk,
                              smem_u32 + 2 * STAGE + V_TILE, wave, lane);
  // one 32-query stage; only a partial last stage masks its queries, and it is peeled out of the loop
  // (both versions inside one loop body made the compiler spill the accumulators)
  auto iteration = [&](int t, auto masked_tag) __attribute__((always_inline)) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    tile_sync<0>();   // stage t has landed for every wave, and stage t - 1's slot is free
    if (t + 1 < n_tiles) issue(t + 1);
    if (!wave_live) return;
    const VMO_LDS char* Qs = smem + (t & 1) * STAGE;
    const VMO_LDS char* dOs = Qs + Q_BYTES;
    const VMO_LDS float* sts = (const VMO_LDS float*)(dOs + DO_BYTES);
    const int nvalid = p.nq - t * kKvBM;

    // S[q][key] = Q K^T and dP[q][key] = dO V^T: lane = key l32, queries 8(r/4) + 4 hl + r%4
    f32x16 s = f32x16{}, dp = f32x16{};
    if constexpr (WANT_DK) {   // dP starts from alpha: G = P (dP + alpha + beta x) then costs one fma less
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 av = *(const VMO_LDS f32x4*)(sts + 32 + 8 * g + 4 * hl);
#pragma unroll
        for (int e = 0; e < 4; ++e) dp[4 * g + e] = av[e];
      }
    }
    {
      const VMO_LDS char* qrow = Qs + l32 * (DK * 2);
      const VMO_LDS char* drow = dOs + l32 * (DOWK * 2);
      // with W0K the K operand of S also multiplies dO's first D columns (dP's k half), in the
      // same column order as a concatenated [k | v1] would
      constexpr bool KDP = W0K && WANT_DK;
      struct Ops { V8 a, b, c; };
      constexpr int NS = D / 16, NOP = NS + (WANT_DK ? VW / 16 : 0), DO0 = KDP ? NS : 0;
      prefetched_chain<NOP, kBwdPrefetch>(
          [&](int i) __attribute__((always_inline)) {
            Ops o;
            if (i < NS) {
              const int off = ((2 * i + hl) ^ qsw) * 16;
              o.a = lds_read8<V8>(qrow + off);
              o.b = K_LDS ? lds_read8<V8>(kt_row + off) : kf[K_LDS ? 0 : i];
              if constexpr (KDP) o.c = lds_read8<V8>(drow + ((2 * i + hl) ^ dsw) * 16);
            } else {
              const int j = i - NS;
              o.a = lds_read8<V8>(drow + ((2 * (DO0 + j) + hl) ^ dsw) * 16);
              o.b = V_LDS ? lds_read8<V8>(vt_row + ((2 * j + hl) ^ vsw) * 16) : vf[V_LDS ? 0 : j];
            }
            return o;
          },
          [&](int i, const Ops& o) __attribute__((always_inline)) {
            if (i < NS) {
              s = E::mfma(o.a, o.b, s);
              if constexpr (KDP) dp = E::mfma(o.c, o.b, dp);
            } else {
              dp = E::mfma(o.a, o.b, dp);
            }
          });
      // the operand reads run two steps ahead of their MFMAs (at the register limit the scheduler would
      // otherwise move each read next to its MFMA and wait for it there)
      struct Chain {
        static constexpr int reads(int i) { return i < NS ? 1 + (K_LDS ? 1 : 0) + (KDP ? 1 : 0) : 1 + (V_LDS ? 1 : 0); }
        static constexpr int mfmas(int i) { return i < NS && KDP ? 2 : 1; }
        static constexpr int ahead(int) { return 2; }
        static constexpr int lead() { return WANT_DK ? 4 : 0; }   // the alpha rows that dP starts from
      };
      pin_chain<Chain, NOP>();
    }
    V8 P[2], G[2];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const f32x4 lv = *(const VMO_LDS f32x4*)(sts + 8 * g + 4 * hl);
      const f32x4 bv = *(const VMO_LDS f32x4*)(sts + 64 + 8 * g + 4 * hl);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = 4 * g + e;
        const float x = fmaf(s[r], c, -lv[e]);
        float pv = fast_exp2(x);
        float gv = WANT_DK ? pv * fmaf(bv[e], x, dp[r]) : 0.f;   // dp holds dP + alpha
        if constexpr (FOLD) gv *= gs;
        if (MASKED && 8 * g + 4 * hl + e >= nvalid) { pv = 0.f; gv = 0.f; }
        P[r >> 3][r & 7] = to_elem<T>(pv);
        G[r >> 3][r & 7] = to_elem<T>(gv);
      }
    }

    if constexpr (DS) {
      // The stage's 32 x 32 block of dS^T (unscaled -- the dq GEMM applies sm_scale -- or with FOLD times
      // sm_scale already, and the dq GEMM then applies p.ds_scale = 1), row = key l32, 64 bytes of
      // 32 queries.  Lane (l32, hl) holds queries 8 g + 4 hl .. + 3 of G[g / 2]; two permlane32 swaps per
      // operand trade the halves so that the lower lanes hold whole 8-query chunks 0 and 2 and the upper
      // lanes chunks 1 and 3: two 16-byte stores per lane, each wave store inside one 2 KB block.  Issued before
      // the dV / dK MFMAs, which hide their latency from the next stage's wait for its copies.
      typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
      // a global (not flat) store: a flat one would also hold every later LDS wait (lgkmcnt) until it lands
      typedef __attribute__((address_space(1))) u32x4 global_u32x4;
      const uint64_t blk = ds_base + (uint64_t)t * 2048 + l32 * 64 + hl * 16;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        u32x4 w = __builtin_bit_cast(u32x4, G[j]);
        const auto s0 = __builtin_amdgcn_permlane32_swap(w[0], w[2], false, false);
        const auto s1 = __builtin_amdgcn_permlane32_swap(w[1], w[3], false, false);
        w = u32x4{s0[0], s1[0], s0[1], s1[1]};
        *(global_u32x4*)(blk + 32 * j) = w;
      }
    }
    // dV^T[dv][key] += dO^T P,  dK^T[d][key] += Q^T dS  (transposed reads of the staged tiles); with FOLD the
    // first 2 NK products are dO[:, :D]^T P into the dK accumulators
    constexpr int NPV = FOLD ? NK : NV;   // accumulator blocks that take dO^T P
    constexpr int NT = 2 * NPV + (WANT_DK ? 2 * NK : 0);
    prefetched_chain<NT, kBwdPrefetch>(
        [&](int i) __attribute__((always_inline)) {
          if (i < 2 * NPV)
            return tr_pair<V8, DOWK * 2>(dOs + 16 * (i % 2) * (DOWK * 2), tr_offset<DOWK * 2>(trow, tchunk, tbyte, i / 2));
          const int j = i - 2 * NPV;
          return tr_pair<V8, DK * 2>(Qs + 16 * (j % 2) * (DK * 2), tr_offset<DK * 2>(trow, tchunk, tbyte, j / 2));
        },
        [&](int i, const V8& x) __attribute__((always_inline)) {
          if (i < 2 * NPV) {
            if constexpr (FOLD) dk[i / 2] = E::mfma(x, P[i % 2], dk[i / 2]);
            else dv[i / 2] = E::mfma(x, P[i % 2], dv[i / 2]);
          } else if constexpr (WANT_DK) {
            const int j = i - 2 * NPV;
            dk[j / 2] = E::mfma(x, G[j % 2], dk[j / 2]);
          }
        });
  };
  issue(0);
  const int n_full = p.nq / kKvBM;   // stages with 32 valid queries
  for (int t = 0; t < n_full; ++t) iteration(t, std::false_type{});
  if (n_full < n_tiles) iteration(n_full, std::true_type{});
  __syncthreads();   // every wave is done with the stage ring, which the epilogue patches reuse
  if (!wave_live) return;
  VMO_LDS float* patch = (VMO_LDS float*)(smem + wave * kEpiPatchBytes);
  const int nrows = min(32, p.nk - k0);
  // write NACC accumulator blocks times f: stored in T, added to / stored into an fp32 gradient, or
  // stored in T as the sum with an fp32 base (src, same column offset)
  auto put = [&](auto cw_tag, void* base, int64_t sb, int64_t sh, int64_t sn, int col0, const f32x16* acc, int nacc,
                 float f, int mode, const void* src = nullptr, int64_t ssb = 0, int64_t ssh = 0, int64_t ssn = 0)
      __attribute__((always_inline)) {
    const int64_t es = mode == kGradStore || mode == kGradSumStore ? 2 : 4;
    char* row0 = (char*)base + (bb * sb + hh * sh + (koff + k0) * sn + col0) * es;
    const char* src0 = src ? (const char*)src + (bb * ssb + hh * ssh + (koff + k0) * ssn + col0) * 4 : nullptr;
    store_acc_rows<F16, decltype(cw_tag)::value>(patch, acc, nacc, f, mode, row0, sn * es, nrows, lane, 0, src0, ssn * 4);
  };
  const std::integral_constant<int, CWK> cwk{};
  const std::integral_constant<int, CWV> cwv{};
  const int mode_k = grad_mode(p.accum, VMO_BWD_ACCUM_K, VMO_BWD_F32_K, VMO_BWD_SUM_K);
  const int mode_v = grad_mode(p.accum, VMO_BWD_ACCUM_V, VMO_BWD_F32_V, VMO_BWD_SUM_V);
  if constexpr (FOLD) {   // dK in natural units already (dS times sm_scale); v1's gradient is PART 2's
    put(cwk, p.dk, p.dk_sb, p.dk_sh, p.dk_sn, 0, dk, NK, 1.0f, mode_k, p.dk_base, p.dkb_sb, p.dkb_sh, p.dkb_sn);
    return;
  }
  if constexpr (W0K && PART == 0) {
    if (p.fold_k) {
      // Value columns [0, D) are k itself: their gradient (dV blocks 0 .. NK-1, laid out like dK's,
      // features x keys) joins dK here instead of being stored and summed by the caller.  Multiply and
      // add rounded separately (no contraction into an fma) give the bits of that sum of two fp32 stores.
      auto fold = [](float key, float s, float val) __attribute__((always_inline)) {
#pragma clang fp contract(off)
        return key * s + val;
      };
#pragma unroll
      for (int b = 0; b < NK; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) dk[b][r] = fold(dk[b][r], p.sm_scale, dv[b][r]);
      put(cwk, p.dk, p.dk_sb, p.dk_sh, p.dk_sn, 0, dk, NK, 1.0f, mode_k, p.dk_base, p.dkb_sb, p.dkb_sh, p.dkb_sn);
      if constexpr (D < 32 && DV == 2 * D) {
        // 16-wide k: v1's gradient is rows 16-31 of the one dV block (its registers 8-15)
        f32x16 v1g = f32x16{};
#pragma unroll
        for (int r = 0; r < 8; ++r) v1g[r] = dv[0][8 + r];
        put(std::integral_constant<int, 16>{}, p.dv, p.dv_sb, p.dv_sh, p.dv_sn, 0, &v1g, 1, 1.0f, mode_v, p.dv_base,
            p.dvb_sb, p.dvb_sh, p.dvb_sn);
      } else if constexpr (NV > NK) {
        put(cwv, p.dv, p.dv_sb, p.dv_sh, p.dv_sn, 0, dv + NK, NV - NK, 1.0f, mode_v, p.dv_base, p.dvb_sb, p.dvb_sh,
            p.dvb_sn);
      }
      return;
    }
  }
  if constexpr (WANT_DK)
    put(cwk, p.dk, p.dk_sb, p.dk_sh, p.dk_sn, 0, dk, NK, p.sm_scale, mode_k, p.dk_base, p.dkb_sb, p.dkb_sh, p.dkb_sn);
  // (PART 2 after the folded PART 3: dv holds v1's gradient alone, from its column 0)
  const int vcol = PART == 2 && p.fold_k ? 0 : VOFF;
  put(cwv, p.dv, p.dv_sb, p.dv_sh, p.dv_sn, vcol, dv, NV, 1.0f, mode_v, p.dv_base, p.dvb_sb, p.dvb_sh, p.dvb_sn);
}

template <bool F16, int D, int DV, int PART, bool W0K, bool DS = false>
static int launch_dkdv(const BwdParams& p, hipStream_t s) {
  constexpr int LDS_KV = dkdv_lds_bytes<D, DV, PART, W0K>();
  static_assert(LDS_KV <= 160 * 1024 && LDS_KV >= kBwdWaves * kEpiPatchBytes, "dkdv LDS");
  auto kern = fea_bwd_dkdv_kernel<F16, D, DV, PART, W0K, DS>;
  if (LDS_KV > 65536) {
    static bool done = false;
    if (!done) {
      if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, LDS_KV) != hipSuccess)
        return set_error(VMO_ERR_LAUNCH, "fea_bwd_dkdv: cannot raise the LDS limit to %d bytes", LDS_KV);
      done = true;
    }
  }
  hipLaunchKernelGGL(kern, dim3(xcd_grid(p.kv_total)), dim3(256), LDS_KV, s, p);
  return launch_status("fea_bwd_dkdv");
}

// Head dims the dS route is built for (the host takes it only for these).
template <int D>
constexpr bool bwd_ds_built() { return D == 64 || D == 128; }

template <bool F16, int D, int DV, bool W0K>
static int launch_bwd_ds(const BwdParams& p, hipStream_t s) {
  const int64_t threads = (int64_t)p.problems * p.nq * (p.delta ? 1 : DV / 8);
  hipLaunchKernelGGL((fea_bwd_prep_kernel<F16, DV>), dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, p);
  int rc = launch_status("fea_bwd_prep");
  if (rc != VMO_OK) return rc;
  if constexpr (W0K && D == 128 && DV == 256) {
    if (p.fold_k) {   // folded dK with dS^T stored times sm_scale (p.ds_scale = 1), then v1's gradient
      rc = launch_dkdv<F16, D, DV, 3, true, true>(p, s);
      if (rc == VMO_OK) rc = launch_dkdv<F16, D, DV, 2, false>(p, s);
    } else {
      rc = launch_dkdv<F16, D, DV, 0, W0K, true>(p, s);
    }
  } else if constexpr (dkdv_parts<D, DV, W0K>() == 1) {
    rc = launch_dkdv<F16, D, DV, 0, W0K, true>(p, s);
  } else {
    rc = launch_dkdv<F16, D, DV, 1, W0K, true>(p, s);
    if (rc == VMO_OK) rc = launch_dkdv<F16, D, DV, 2, false>(p, s);
  }
  if (rc != VMO_OK) return rc;
  constexpr int LDS = 2 * kDqBN * (D + kDqBM) * 2;
  static_assert(LDS <= 65536 && LDS >= kBwdWaves * kEpiPatchBytes, "dq_ds LDS");
  hipLaunchKernelGGL((fea_bwd_dq_ds_kernel<F16, D>), dim3(xcd_grid(p.dq_total)), dim3(256), LDS, s, p);
  rc = launch_status("fea_bwd_dq_ds");
  if (rc != VMO_OK || p.dq_splits == 1) return rc;
  const int64_t rthreads = (int64_t)p.problems * p.nq * (D / 4);
  hipLaunchKernelGGL((fea_bwd_dq_reduce<F16, D>), dim3((unsigned)((rthreads + 255) / 256)), dim3(256), 0, s, p);
  return launch_status("fea_bwd_dq_reduce");
}

template <bool F16, int D, int DV, bool V2 = false, bool W0K = false>
static int launch_bwd(const BwdParams& p, hipStream_t s) {
  if (p.ds) {
    if constexpr (bwd_ds_built<D>()) return launch_bwd_ds<F16, D, DV, W0K>(p, s);
    return set_error(VMO_ERR_UNSUPPORTED, "fea_bwd: no dS route for d=%d", D);
  }
  constexpr int DVL = dq_staged_dv<D, DV, W0K>();
  constexpr int RING_DQ = 2 * kDqBN * (tile_w(D) + (DVL ? tile_w(DVL) : 0)) * 2;
  constexpr int LDS_DQ = RING_DQ > kBwdWaves * kEpiPatchBytes ? RING_DQ : kBwdWaves * kEpiPatchBytes;   // + patches
  static_assert(LDS_DQ <= 160 * 1024 && LDS_DQ >= kBwdWaves * kEpiPatchBytes, "bwd LDS");
  if (LDS_DQ > 65536) {
    static bool done = false;
    if (!done) {
      if (hipFuncSetAttribute((const void*)fea_bwd_dq_kernel<F16, D, DV, V2, W0K>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, LDS_DQ) != hipSuccess)
        return set_error(VMO_ERR_LAUNCH, "fea_bwd_dq: cannot raise the LDS limit to %d bytes", LDS_DQ);
      done = true;
    }
  }
  hipLaunchKernelGGL((fea_bwd_dq_kernel<F16, D, DV, V2, W0K>), dim3(xcd_grid(p.dq_total)), dim3(256), LDS_DQ, s, p);
  int rc = launch_status("fea_bwd_dq");
  if (rc != VMO_OK) return rc;
  if (p.dq_splits > 1) {
    const int64_t threads = (int64_t)p.problems * p.nq * (D / 4);
    hipLaunchKernelGGL((fea_bwd_dq_reduce<F16, D>), dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, p);
    rc = launch_status("fea_bwd_dq_reduce");
    if (rc != VMO_OK) return rc;
  }
  if constexpr (W0K && D == 128 && DV == 256) {
    if (p.fold_k) {
      rc = launch_dkdv<F16, D, DV, 3, true>(p, s);
      if (rc != VMO_OK) return rc;
      return launch_dkdv<F16, D, DV, 2, false>(p, s);
    }
    return launch_dkdv<F16, D, DV, 0, W0K>(p, s);
  } else if constexpr (dkdv_parts<D, DV, W0K>() == 1) {
    return launch_dkdv<F16, D, DV, 0, W0K>(p, s);
  } else {
    rc = launch_dkdv<F16, D, DV, 1, W0K>(p, s);
    if (rc != VMO_OK) return rc;
    return launch_dkdv<F16, D, DV, 2, false>(p, s);   // dV's second half from P alone: no V read
  }
}

template <bool F16>
static int dispatch_bwd(const BwdParams& p, int d, int dv, hipStream_t s) {
  if (p.v1 && p.v0_is_k) {   // values [k | v1]
    if (d == 16 && dv == 32) return launch_bwd<F16, 16, 32, true, true>(p, s);
    if (d == 32 && dv == 64) return launch_bwd<F16, 32, 64, true, true>(p, s);
    if (d == 64 && dv == 128) return launch_bwd<F16, 64, 128, true, true>(p, s);
    if (d == 128 && dv == 256) return launch_bwd<F16, 128, 256, true, true>(p, s);
  } else if (p.v0_is_k) {   // values k (VMonarch's R-steps before the last, vmonarch.py:50)
    if (d == 16 && dv == 16) return launch_bwd<F16, 16, 16, false, true>(p, s);
    if (d == 32 && dv == 32) return launch_bwd<F16, 32, 32, false, true>(p, s);
    if (d == 64 && dv == 64) return launch_bwd<F16, 64, 64, false, true>(p, s);
    if (d == 128 && dv == 128) return launch_bwd<F16, 128, 128, false, true>(p, s);
  }
  if (p.fold_k)
    return set_error(VMO_ERR_UNSUPPORTED, "fea_bwd: VMO_BWD_FOLD_K is built for values k with (d, dv) = (16, 16), (32, 32), "
                     "(64, 64), (128, 128) and values [k | v1] with (16, 32), (32, 64), (64, 128), (128, 256); got d=%d "
                     "dv=%d", d, dv);
  if (p.v1 && p.v0_is_k) {
    return set_error(VMO_ERR_UNSUPPORTED, "fea_bwd: no kernel for d=%d with values [k | v1] of %d", d, dv);
  } else if (p.v1) {   // values in two halves (the caller checked dv1 = dv / 2)
    if (d == 64 && dv == 128) return launch_bwd<F16, 64, 128, true>(p, s);
    if (d == 128 && dv == 256) return launch_bwd<F16, 128, 256, true>(p, s);
    return set_error(VMO_ERR_UNSUPPORTED, "fea_bwd: no kernel for d=%d with values in two parts of %d", d, dv / 2);
  }
  if (d == 16 && dv == 16) return launch_bwd<F16, 16, 16>(p, s);   // 16-wide heads: 32-wide tiles, rows twice
  if (d == 16 && dv == 32) return launch_bwd<F16, 16, 32>(p, s);
  if (d == 16 && dv == 64) return launch_bwd<F16, 16, 64>(p, s);
  if (d == 16 && dv == 128) return launch_bwd<F16, 16, 128>(p, s);
  if (d == 16 && dv == 256) return launch_bwd<F16, 16, 256>(p, s);
  if (d == 32 && dv == 32) return launch_bwd<F16, 32, 32>(p, s);
  if (d == 32 && dv == 64) return launch_bwd<F16, 32, 64>(p, s);
  if (d == 32 && dv == 128) return launch_bwd<F16, 32, 128>(p, s);
  if (d == 64 && dv == 32) return launch_bwd<F16, 64, 32>(p, s);
  if (d == 128 && dv == 32) return launch_bwd<F16, 128, 32>(p, s);
  if (d == 64 && dv == 64) return launch_bwd<F16, 64, 64>(p, s);
  if (d == 64 && dv == 128) return launch_bwd<F16, 64, 128>(p, s);
  if (d == 128 && dv == 64) return launch_bwd<F16, 128, 64>(p, s);
  if (d == 128 && dv == 128) return launch_bwd<F16, 128, 128>(p, s);
  if (d == 32 && dv == 256) return launch_bwd<F16, 32, 256>(p, s);
  if (d == 64 && dv == 256) return launch_bwd<F16, 64, 256>(p, s);
  if (d == 128 && dv == 256) return launch_bwd<F16, 128, 256>(p, s);
  if (d == 256 && dv == 256) return launch_bwd<F16, 256, 256>(p, s);
  return set_error(VMO_ERR_UNSUPPORTED, "fea_bwd: no kernel for d=%d dv=%d", d, dv);
}

}  // namespace vmo

namespace vmo {
// Key splits of the dq kernel: a problem with few query tiles and many keys (the exact recompute of
// VMonarch: 13 query tiles per head against 32760 keys) would otherwise leave most CUs idle.
static int bwd_dq_splits(int64_t problems, int nq, int nk) {
  const int64_t wgs = problems * ((nq + kDqBM - 1) / kDqBM);
  int splits = 1;
  while (wgs * splits < 1024 && splits < 16 && nk / (splits * 2) >= 1024) splits *= 2;
  return splits;
}
static int bwd_keys_per_split(int nk, int splits) {
  return ((nk + splits - 1) / splits + kDqBN - 1) / kDqBN * kDqBN;
}
static size_t bwd_stats_bytes(int64_t problems, int nq) { return ((size_t)2 * problems * nq * 4 + 255) / 256 * 256; }
// The dS route (dkdv stores dS^T, dQ is a GEMM over it) trades the dq kernel's recompute of S and dP --
// 2 (d + dv) flops per query-key pair -- for 4 bytes of HBM traffic per pair (dS^T written and read
// back).  Measured on the VMonarch cfg4 geometries (1560 x 1560 problems), it wins where the recompute
// is dearest -- d = 128 with dv = 256 (the last R-step, values [k | v]; its dq kernel runs one wave per
// SIMD): 1.78 against 1.95-2.0 ms -- and loses for dv = d (R-step 0: 1.27 against 1.07 ms; the recompute
// backward: 1.08 against 1.04 ms), where the dkdv kernel is already close to the HBM bandwidth it shares
// with the write stream.  Its workspace grows as nq x nk per problem (2 bytes per query-key pair), while the
// recompute route needs O(nq) memory, so it is taken by default only where it was measured to win: d = 128,
// dv = 256, short problems (nq and nk at most kBwdDsMaxLen, the VMonarch R-step's frames) and dS^T of all
// problems (32 x 32 blocks, keys and queries rounded up to 32) within kBwdDsMaxBytes.  A long standalone
// flash_entropy_attention backward (nq = nk = 16384 and more) stays on the recompute route whatever its
// dims.  VMO_BWD_DS_DQ asks for the dS route at any size with d in {64, 128}, VMO_BWD_RECOMPUTE_DQ never.
// Returns the workspace bytes it needs, 0 when not taken.
constexpr int64_t kBwdDsMaxBytes = 2ll << 30;
constexpr int kBwdDsMaxLen = 4096;
static size_t bwd_ds_bytes(const vmo_fea_bwd_args* a, int64_t problems) {
  if ((a->flags & VMO_BWD_RECOMPUTE_DQ) || (a->d != 64 && a->d != 128)) return 0;
  const int64_t total = problems * ((a->nk + 31) / 32) * ((a->nq + 31) / 32) * 2048;
  if (a->flags & VMO_BWD_DS_DQ) return (size_t)total;
  const bool short_problems = a->nq <= kBwdDsMaxLen && a->nk <= kBwdDsMaxLen;
  return a->d == 128 && a->dv == 256 && short_problems && total <= kBwdDsMaxBytes ? (size_t)total : 0;
}
}  // namespace vmo

extern "C" size_t vmo_fea_bwd_workspace_size(const vmo_fea_bwd_args* a) {
  using namespace vmo;
  if (!a || a->batch <= 0 || a->heads <= 0 || a->nq <= 0 || a->nk <= 0) return 256;
  const int64_t problems = (int64_t)a->batch * a->heads * (a->frames > 0 ? a->frames : 1);
  const int splits = bwd_dq_splits(problems, a->nq, a->nk);
  size_t bytes = bwd_stats_bytes(problems, a->nq) + 256;
  if (splits > 1) bytes += ((size_t)splits * problems * a->nq * (a->d > 0 ? a->d : 0) * 4 + 255) / 256 * 256;
  return bytes + bwd_ds_bytes(a, problems);
}

extern "C" int vmo_fea_bwd(const vmo_fea_bwd_args* a, void* stream) {
  using namespace vmo;
  clear_error();
  if (!a) return set_error(VMO_ERR_INVALID, "fea_bwd: null args");
  if (a->dtype != VMO_DTYPE_BF16 && a->dtype != VMO_DTYPE_F16) return set_error(VMO_ERR_INVALID, "fea_bwd: dtype");
  if (a->batch < 0 || a->heads < 0 || a->nq < 0 || a->nk < 0) return set_error(VMO_ERR_INVALID, "fea_bwd: sizes");
  if ((int64_t)a->batch * a->heads == 0 || (a->nq == 0 && a->nk == 0)) return VMO_OK;
  if (a->nq == 0 || a->nk == 0) return set_error(VMO_ERR_INVALID, "fea_bwd: nq and nk must both be > 0");
  // with VMO_BWD_FOLD_K and values k alone there is no grad_v to write
  const bool fold_k = (a->flags & VMO_BWD_FOLD_K) != 0, no_grad_v = fold_k && a->dv1 == 0;
  if (!view_ok(a->q) || !view_ok(a->k) || !view_ok(a->v) || !view_ok(a->o) || !view_ok(a->grad_o) ||
      !view_ok(a->grad_q) || !view_ok(a->grad_k) || (!no_grad_v && !view_ok(a->grad_v)))
    return set_error(VMO_ERR_INVALID, "fea_bwd: tensors need 16-byte aligned rows");
  if (!a->lse || !a->ent || !a->grad_ent) return set_error(VMO_ERR_INVALID, "fea_bwd: lse / ent / dent required");
  if (a->dv1 < 0 || a->dv1 >= a->dv) return set_error(VMO_ERR_INVALID, "fea_bwd: dv1 = %d with dv = %d", a->dv1, a->dv);
  if (a->dv1 > 0) {
    if (a->dv1 * 2 != a->dv) return set_error(VMO_ERR_UNSUPPORTED, "fea_bwd: value parts must be dv / 2 wide");
    if (!view_ok(a->v1) || a->v1.stride_b != a->v.stride_b || a->v1.stride_h != a->v.stride_h ||
        a->v1.stride_n != a->v.stride_n)
      return set_error(VMO_ERR_INVALID, "fea_bwd: v1 needs 16-byte aligned rows and the strides of v");
  }
  constexpr int kFlags = VMO_BWD_ACCUM_Q | VMO_BWD_ACCUM_K | VMO_BWD_ACCUM_V | VMO_BWD_F32_Q | VMO_BWD_F32_K |
                         VMO_BWD_F32_V | VMO_BWD_FOLD_K | VMO_BWD_SUM_K | VMO_BWD_SUM_V | VMO_BWD_RECOMPUTE_DQ |
                         VMO_BWD_DS_DQ | VMO_BWD_SUM_Q;
  const bool sum_k = (a->flags & VMO_BWD_SUM_K) != 0, sum_v = (a->flags & VMO_BWD_SUM_V) != 0;
  const bool sum_q = (a->flags & VMO_BWD_SUM_Q) != 0;
  if ((a->flags & ~kFlags) || ((a->flags >> 3) & a->flags & 7) ||
      (sum_k && (a->flags & (VMO_BWD_ACCUM_K | VMO_BWD_F32_K))) ||
      (sum_v && (a->flags & (VMO_BWD_ACCUM_V | VMO_BWD_F32_V))) || (sum_v && no_grad_v) ||
      (sum_q && (a->flags & (VMO_BWD_ACCUM_Q | VMO_BWD_F32_Q))) ||
      ((a->flags & VMO_BWD_RECOMPUTE_DQ) && (a->flags & VMO_BWD_DS_DQ)))
    return set_error(VMO_ERR_INVALID, "fea_bwd: unknown or conflicting flags 0x%x", (unsigned)a->flags);
  if ((sum_k && !view_ok(a->grad_k_base)) || (sum_v && !view_ok(a->grad_v_base)) ||
      (sum_q && !view_ok(a->grad_q_base)))
    return set_error(VMO_ERR_INVALID, "fea_bwd: VMO_BWD_SUM_Q / _K / _V need a grad_q_base / grad_k_base / "
                     "grad_v_base view (fp32, 16-byte aligned rows)");
  const bool v0_is_k = a->v.data == a->k.data && a->v.stride_b == a->k.stride_b && a->v.stride_h == a->k.stride_h &&
                       a->v.stride_n == a->k.stride_n && a->dv - a->dv1 == a->d;
  if (fold_k && !v0_is_k)
    return set_error(VMO_ERR_INVALID, "fea_bwd: VMO_BWD_FOLD_K needs values that start with k (v is k: same address "
                     "and strides, dv - dv1 = d)");
  // shapes with a fold kernel (dispatch_bwd): rejected here, before any pointer is looked at further
  const bool fold_dims = a->d == 16 || a->d == 32 || a->d == 64 || a->d == 128;
  if (fold_k && !(fold_dims && a->dv == (a->dv1 == 0 ? a->d : 2 * a->d)))
    return set_error(VMO_ERR_UNSUPPORTED, "fea_bwd: VMO_BWD_FOLD_K is built for values k with (d, dv) = (16, 16), "
                     "(32, 32), (64, 64), (128, 128) and values [k | v1] with (16, 32), (32, 64), (64, 128), (128, 256); "
                     "got d=%d dv=%d", a->d, a->dv);
  if (!(a->sm_scale >= 0.f)) return set_error(VMO_ERR_INVALID, "fea_bwd: sm_scale");
  // the tile copies address up to 7 rows from a lane with a 32-bit byte offset
  const int64_t kMaxRowStride = 1ll << 27;
  if (a->q.stride_n >= kMaxRowStride || a->k.stride_n >= kMaxRowStride || a->v.stride_n >= kMaxRowStride ||
      a->grad_o.stride_n >= kMaxRowStride)
    return set_error(VMO_ERR_UNSUPPORTED, "fea_bwd: q / k / v / grad_o row stride must be below 2^27 elements");
  const size_t ws = vmo_fea_bwd_workspace_size(a);
  if (!a->workspace || a->workspace_bytes < ws || !aligned16(a->workspace))
    return set_error(VMO_ERR_WORKSPACE, "fea_bwd: needs %zu workspace bytes", ws);
  const int frames = a->frames > 0 ? a->frames : 1;
  const int64_t problems = (int64_t)a->batch * a->heads * frames;
  const int64_t dq_tiles = (a->nq + kDqBM - 1) / kDqBM, kv_tiles = (a->nk + kKvBN - 1) / kKvBN;
  if (problems * dq_tiles > (1ll << 30) || problems * kv_tiles > (1ll << 30))
    return set_error(VMO_ERR_UNSUPPORTED, "fea_bwd: problem too large");
  BwdParams p{};
  p.q = a->q.data; p.k = a->k.data; p.v = a->v.data; p.o = a->o.data; p.dO = a->grad_o.data;
  p.v1 = a->dv1 > 0 ? a->v1.data : nullptr;
  p.v0_is_k = v0_is_k;
  p.fold_k = fold_k;
  if (sum_k) {
    p.dk_base = a->grad_k_base.data;
    p.dkb_sb = a->grad_k_base.stride_b; p.dkb_sh = a->grad_k_base.stride_h; p.dkb_sn = a->grad_k_base.stride_n;
  }
  p.delta = a->delta;
  p.dl_sb = a->delta_stride_b; p.dl_sh = a->delta_stride_h;
  if (sum_q) {
    p.dq_base = a->grad_q_base.data;
    p.dqb_sb = a->grad_q_base.stride_b; p.dqb_sh = a->grad_q_base.stride_h; p.dqb_sn = a->grad_q_base.stride_n;
  }
  if (sum_v) {
    p.dv_base = a->grad_v_base.data;
    p.dvb_sb = a->grad_v_base.stride_b; p.dvb_sh = a->grad_v_base.stride_h; p.dvb_sn = a->grad_v_base.stride_n;
  }
  p.dq = a->grad_q.data; p.dk = a->grad_k.data; p.dv = a->grad_v.data;
  p.lse = a->lse; p.ent = a->ent; p.dent = a->grad_ent;
  p.alpha = (float*)a->workspace;
  p.beta = p.alpha + problems * a->nq;
  p.dq_splits = bwd_dq_splits(problems, a->nq, a->nk);
  p.keys_per_split = bwd_keys_per_split(a->nk, p.dq_splits);
  p.dq_part = (float*)((char*)a->workspace + bwd_stats_bytes(problems, a->nq));
  if (bwd_ds_bytes(a, problems)) {   // after the stats and the dq partials
    size_t off = bwd_stats_bytes(problems, a->nq) + 256;
    if (p.dq_splits > 1) off += ((size_t)p.dq_splits * problems * a->nq * a->d * 4 + 255) / 256 * 256;
    p.ds = (char*)a->workspace + off;
    p.ds_kblocks = (a->nk + 31) / 32;
    p.ds_qblocks = (a->nq + 31) / 32;
  }
  p.accum = a->flags;
  p.q_sb = a->q.stride_b; p.q_sh = a->q.stride_h; p.q_sn = a->q.stride_n;
  p.k_sb = a->k.stride_b; p.k_sh = a->k.stride_h; p.k_sn = a->k.stride_n;
  p.v_sb = a->v.stride_b; p.v_sh = a->v.stride_h; p.v_sn = a->v.stride_n;
  p.o_sb = a->o.stride_b; p.o_sh = a->o.stride_h; p.o_sn = a->o.stride_n;
  p.do_sb = a->grad_o.stride_b; p.do_sh = a->grad_o.stride_h; p.do_sn = a->grad_o.stride_n;
  p.dq_sb = a->grad_q.stride_b; p.dq_sh = a->grad_q.stride_h; p.dq_sn = a->grad_q.stride_n;
  p.dk_sb = a->grad_k.stride_b; p.dk_sh = a->grad_k.stride_h; p.dk_sn = a->grad_k.stride_n;
  p.dv_sb = a->grad_v.stride_b; p.dv_sh = a->grad_v.stride_h; p.dv_sn = a->grad_v.stride_n;
  p.st_sb = a->stat_stride_b; p.st_sh = a->stat_stride_h;
  p.de_sb = a->grad_ent_stride_b; p.de_sh = a->grad_ent_stride_h;
  p.heads = a->heads; p.frames = frames; p.nq = a->nq; p.nk = a->nk; p.problems = (int)problems;
  p.dq_tiles = (int)dq_tiles; p.kv_tiles = (int)kv_tiles;
  p.dq_total = (int)(problems * dq_tiles * p.dq_splits); p.kv_total = (int)(problems * kv_tiles);
  p.c = a->sm_scale * kLog2e;
  p.sm_scale = a->sm_scale;
  // the folded launch for values [k | v1] at 128 / 256 stores dS^T times sm_scale
  p.ds_scale = fold_k && a->dv1 > 0 && a->d == 128 ? 1.0f : a->sm_scale;
  hipStream_t s = (hipStream_t)stream;
  if (a->dtype == VMO_DTYPE_F16) return dispatch_bwd<true>(p, a->d, a->dv, s);
  return dispatch_bwd<false>(p, a->d, a->dv, s);
}
