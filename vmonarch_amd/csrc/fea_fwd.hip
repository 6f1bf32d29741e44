// FlashEntropyAttention forward for gfx950.
//
// Reference: video_monarch_attention/kernel.py:32-67 (_attn_fwd_inner) and :104-151 (_attn_fwd),
// launched from _FlashEntropyAttention.forward (kernel.py:318-358).  Same mathematics (online
// softmax in the log2 domain plus the running h = sum_j p_j (s_j - m) that yields the row
// entropy), different machine mapping:
//
//  * one workgroup = 4 waves = 128 queries; each wave owns 32 queries for the whole key loop;
//  * S^T = K Q^T on v_mfma_f32_32x32x16 (K tile = A operand from LDS, Q = B operand held in
//    registers), so each lane owns ONE query row: the row max needs one permlane32 swap per
//    64-key stage and the row sum / entropy sums stay per-lane until the end;
//  * O^T += W^T P^T with the P accumulator reused in place as the B operand; the W^T operand is
//    read from the row-major LDS tile with ds_read_tr16_b64, whose 4-key groups match the
//    accumulator layout of S^T, so no transposed copy and no key permutation is needed;
//  * K / W tiles are staged by global_load_lds (no register round trip) through a 2- or 3-slot
//    LDS ring, with an XOR swizzle of 16-byte chunks against LDS bank conflicts; the copies are
//    issued from inline asm and ordered by explicit waits, so the prefetch overlaps the reads of
//    the current tile;
//  * when w0 aliases k (the VMonarch R-step values [k | v]) the K tile doubles as W0;
//  * no rescaling in the loop: the reference point m of p = 2^(s c - m) is the max of the first
//    32 keys and stays fixed; a row whose block sum leaves the safe range of the 16-bit type's P
//    operand sends its workgroup through an exact two-pass fallback.  The entropy identity
//    e = log2 l - h / l holds for any m;
//  * tail keys are masked in-kernel (no padding copies, unlike kernel.py:399-400);
//  * split-KV (num_splits > 1) writes normalised fp32 partials + lse, merged by fea_combine.
#include <mutex>
#include <type_traits>

#include "vmo_common.h"
#include "vmo_host.h"

namespace vmo {

constexpr int kFwdQB = 1;             // 32-query MFMA blocks per wave
// Waves per workgroup (a template parameter of the kernel): 4 (128 queries, two workgroups per CU)
// or 8 (256 queries, one workgroup per CU).  Both keep two waves per SIMD; 8 halves the K / W tile
// traffic per flop, at the price of coarser query tiles.
constexpr int kFwdWavesSmall = 4;
constexpr int kFwdWavesLarge = 8;
constexpr int kFwdBN = 64;            // keys per pipeline stage
constexpr float kMaskLogit = -1.0e30f;

struct FwdParams {
  const void* q;
  const void* k;
  const void* w0;
  const void* w1;
  void* o;
  float* lse;
  float* ent;
  float* part_o;
  float* part_lse;
  int64_t q_sb, q_sh, q_sn;
  int64_t k_sb, k_sh, k_sn;
  int64_t w0_sb, w0_sh, w0_sn;
  int64_t w1_sb, w1_sh, w1_sn;
  int64_t o_sb, o_sh, o_sn;
  int64_t st_sb, st_sh;
  int heads, frames, nq, nk;
  int problems, q_tiles, splits, keys_per_split;
  int total_wg;
  float scale_log2;
  // fp8 S (QK8 variants): k quantized per problem, rows [nk][128] in the operand order of fea_fp8_keys_kernel,
  // one scale per 64-key tile (k8_tiles per problem)
  void* k8;
  float* k8_scale;
  int k8_tiles;
};

// Bytes of one pipeline stage: the K tile, the value tiles the K tile does not double as, and with fp8 S
// the fp8 K tile (one byte per element).
template <int D, int DW0, int DW1, bool W0K, bool QK8>
constexpr int fwd_stage_bytes() {
  return kFwdBN * (tile_w(D) + (W0K ? 0 : tile_w(DW0)) + (DW1 ? tile_w(DW1) : 0)) * 2 + (QK8 ? kFwdBN * D : 0);
}

// fp8 (e4m3) operand layout of the fp8 S product: a 128-wide row as two 64-dim products; lane half hl of
// product m takes dims 16 ds + 8 hl + e (ds = 4 m .. 4 m + 3, e = 0 .. 7), which are those the lane holds
// of the 16-bit q row, as 32 consecutive bytes.  Byte position of dim d in the stored row:
__host__ __device__ constexpr int fp8_dim_pos(int d) { return 64 * (d / 64) + 32 * ((d / 8) % 2) + 8 * ((d / 16) % 4) + d % 8; }
constexpr float kFp8Max = 448.f;   // e4m3's largest finite value (the conversion does not saturate: beyond it is NaN)

// LDS ring slots per workgroup: prefetch two tiles ahead when three slots fit the workgroup's share
// of the CU's 160 KB (two 4-wave workgroups or one 8-wave workgroup per CU), else one ahead.
constexpr int fwd_slots(int stage_bytes, int waves) {
  return 3 * stage_bytes <= (waves == kFwdWavesLarge ? 160 : 80) * 1024 ? 3 : 2;
}

// Copies of kFwdBN-row tiles of a row-major (token, W) tensor into swizzled LDS tiles.  Wave
// instruction inst (= i * WAVES + wave) covers rows inst * RPI .. inst * RPI + RPI - 1 (1 KB);
// lane l copies chunk l % CH of row inst * RPI + l / CH to chunk (l % CH) ^ swz_rows(row).  The
// swizzle depends on the row modulo 16 only, which does not change with i when WAVES * RPI is a
// multiple of 16 (and alternates with i otherwise), so the lane's byte offset from its instruction's
// first row takes one or two values: a full tile costs scalar address arithmetic only.  A tile that runs
// past the end of the tensor (row >= nrows) re-reads the last row instead: finite data, masked out
// later.  Each wave issues NI copies per tile (vmcnt units).  SW < W (a 16-wide tensor in a 32-wide tile):
// logical chunk c of a row holds the source row's chunk c % (SW / 8).
template <class T, int W, int WAVES, int SW = W>
struct TileCopy {
  static constexpr int CH = W / 8;       // 16-byte chunks per row
  static constexpr int RPI = 64 / CH;    // rows per wave instruction
  static constexpr int NI = kFwdBN / RPI / WAVES;
  static constexpr int NV = (WAVES * RPI) % 16 == 0 ? 1 : 2;   // distinct lane offsets
  static_assert(CH >= 4 && NI >= 1 && RPI >= 2, "tile shape");
  uint64_t ubase;     // base as a scalar byte address
  uint64_t rbytes;    // bytes per row
  uint32_t voff[NV];
  int wave, lane;

  __device__ __forceinline__ TileCopy(const T* b, int64_t s, int w, int l) : wave(w), lane(l) {
    ubase = uniform64((uint64_t)(uintptr_t)b);
    rbytes = uniform64((uint64_t)s * 2);
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int r = (v * WAVES + w) * RPI + l / CH;   // the lane's row in instruction i = v
      voff[v] = (uint32_t)((int64_t)(l / CH) * s * 2) + (uint32_t)((((l % CH) ^ swz_rows<W * 2>(r)) & (SW / 8 - 1)) * 16);
    }
  }
  __device__ __forceinline__ void issue(int row0, int nrows, uint32_t dst) const {
    // row0 and nrows are uniform, but may arrive in vector registers (the variants that keep the
    // tile indices in vector registers): without readfirstlane the full-tile test becomes an exec
    // mask branch and the tile address a vector 64-bit multiply per copy.
    row0 = __builtin_amdgcn_readfirstlane(row0);
    nrows = __builtin_amdgcn_readfirstlane(nrows);
    // The per-instruction addresses are loop invariant up to row0; hoisted out of the key loop
    // they would pin dozens of scalar registers.  The empty asm hides where ub comes from, so they
    // are recomputed here (a few scalar adds per copy).
    uint64_t ub = ubase;
    asm volatile("" : "+s"(ub));
    if (row0 + kFwdBN <= nrows) {
      const uint64_t tb = ub + (uint64_t)(row0 + wave * RPI) * rbytes;
#pragma unroll
      for (int i = 0; i < NI; ++i)
        dma16_async_s(tb + (uint64_t)(i * WAVES * RPI) * rbytes, voff[i % NV], dst + (i * WAVES + wave) * 1024);
    } else {
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int inst = i * WAVES + wave;
        const int r = inst * RPI + lane / CH;
        const int gr = min(row0 + r, nrows - 1);
        dma16_async((const void*)(uintptr_t)(ub + (uint64_t)gr * rbytes +
                                             (((lane % CH) ^ swz_rows<W * 2>(r)) & (SW / 8 - 1)) * 16),
                    dst + inst * 1024);
      }
    }
  }
};

// Entropy modes: none; online h = sum p (s c - m) in fp32 (kernel.py:49-50), e = log2 l - h / l; or,
// when the first value block is k itself (the VMonarch R-step), from the P.K accumulator at the end:
//   e = LSE ln2 - sm_scale q . (sum_j p~_j k_j) / l~   (nats), with l~ = sum_j p~_j
// -- no per-element product in the loop.  p~ is p rounded to the 16-bit type (the MFMA operand), and
// this mode sums exactly those rounded weights into l (also used for o and the LSE), so the mean logit
// is a proper average under one distribution.  Normalising the rounded moment by the fp32 sum instead
// leaves an error of (mean logit) x (relative rounding of the dominant p), several times the 2e-2
// tolerance on rows with logits of std 4 to 8.
enum { kEntNone = 0, kEntOnline = 1, kEntFromPK = 2 };

// Workgroups per CU the register budget is sized for: a 256-wide value tensor (its accumulators alone are
// 128 registers), 256-wide q/k heads, and two narrower shapes that spilled inside the key loop at two
// workgroups per CU (64-wide q/k with 128-wide values and the online entropy; [k | v] with v narrower
// than k) run one 4-wave workgroup per CU.
template <int D, int DW0, int DW1, int ENT, int WAVES>
constexpr int fwd_min_blocks() {
  return (D >= 256 || DW0 >= 256 || (ENT == kEntOnline && tile_w(D) < DW0) || (DW1 > 0 && DW1 < D)) ? 1 : 8 / WAVES;
}

template <bool F16, int D, int DW0, int DW1, bool W0K, int ENT, bool SPLIT, int WAVES, bool QK8>
__global__ __launch_bounds__(64 * WAVES, (fwd_min_blocks<D, DW0, DW1, ENT, WAVES>())) void fea_fwd_kernel(FwdParams p) {
  using E = Elem<F16>;
  using T = typename E::T;
  using V8 = typename E::V8;
  using V4 = typename E::V4;
  using V2 = typename E::V2;
  constexpr int DK = tile_w(D), DW0K = tile_w(DW0), DW1K = DW1 ? tile_w(DW1) : 0;   // widths in LDS
  constexpr int K_BYTES = kFwdBN * DK * 2;
  constexpr int W0_BYTES = W0K ? 0 : kFwdBN * DW0K * 2;
  constexpr int W1_BYTES = kFwdBN * DW1K * 2;
  constexpr int K8_OFF = K_BYTES + W0_BYTES + W1_BYTES;   // the fp8 K tile (QK8)
  constexpr int STAGE = fwd_stage_bytes<D, DW0, DW1, W0K, QK8>();
  constexpr int NSLOT = fwd_slots(STAGE, WAVES);
  static_assert(!QK8 || D == 128, "fp8 S is built for 128-wide q / k");
  constexpr int kBM = 32 * kFwdQB * WAVES;   // queries per workgroup
  constexpr int NA0 = DW0K / 32;
  constexpr int NA1 = DW1K / 32;
  constexpr int NA = NA0 + NA1;
  constexpr int NDS = D / 16;   // 16-dim MFMA steps of S (one for a 16-wide head)
  constexpr int CW = DW0 < 32 ? 16 : 32;   // stored columns per accumulator block
  static_assert(DW1 == 0 || (DW1 < 32) == (DW0 < 32), "value parts of one width class");
  constexpr int QB = kFwdQB;
  // global_load_lds instructions one tile costs each wave (vmcnt units)
  constexpr int DMA_PER_TILE = STAGE / 1024 / WAVES;
  static_assert(STAGE % (1024 * WAVES) == 0, "whole copy instructions per wave");
  static_assert(!W0K || DW0 == D, "w0 aliases k");
  static_assert(ENT != kEntFromPK || W0K, "entropy from P.K needs w0 == k");

  extern __shared__ __attribute__((aligned(1024))) char smem_raw[];
  VMO_LDS char* smem = (VMO_LDS char*)smem_raw;
  const uint32_t smem_u32 = (uint32_t)(uintptr_t)smem;

  // XCD-aware block -> tile map: block b runs on XCD b % 8, so give each XCD a contiguous run of
  // logical tiles (all query tiles of a problem then share one L2 for their K / W traffic).
  const int per_xcd = gridDim.x >> 3;
  const int L = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
  if (L >= p.total_wg) return;
  // Integer division runs on the vector unit; readfirstlane brings the uniform results back to
  // scalar registers, so the per-tile address arithmetic stays scalar.  The variants with eight
  // accumulator blocks are short of registers: for them the extra scalar values cost more (their
  // spills land in the key loop) than the few vector instructions they save.
  struct Loc { int qt, split, prob, f, hh, bb; };
  struct Div { int q_tiles, splits, frames, heads; };
  auto locate = [&](int lx, const Div& dv, auto scalar_tag) __attribute__((always_inline)) {
    constexpr bool S = decltype(scalar_tag)::value;
    auto u = [](int v) __attribute__((always_inline)) { return S ? __builtin_amdgcn_readfirstlane(v) : v; };
    Loc r;
    r.qt = u(lx % dv.q_tiles);
    const int rest = lx / dv.q_tiles;
    r.split = u(rest % dv.splits);
    r.prob = u(rest / dv.splits);
    r.f = u(r.prob % dv.frames);
    const int bh = r.prob / dv.frames;
    r.hh = u(bh % dv.heads);
    r.bb = u(bh / dv.heads);
    return r;
  };
  const Loc loc = locate(L, Div{p.q_tiles, p.splits, p.frames, p.heads}, std::integral_constant<bool, (NA < 8)>{});
  const int qt = loc.qt, split = loc.split, f = loc.f, hh = loc.hh, bb = loc.bb;

  const T* qb = (const T*)p.q + bb * p.q_sb + hh * p.q_sh + (int64_t)f * p.nq * p.q_sn;
  const T* kb = (const T*)p.k + bb * p.k_sb + hh * p.k_sh + (int64_t)f * p.nk * p.k_sn;
  const T* w0b = (const T*)p.w0 + bb * p.w0_sb + hh * p.w0_sh + (int64_t)f * p.nk * p.w0_sn;
  const T* w1b = DW1 ? (const T*)p.w1 + bb * p.w1_sb + hh * p.w1_sh + (int64_t)f * p.nk * p.w1_sn : nullptr;
  const int64_t q_sn = p.q_sn;

  const int kbeg = split * p.keys_per_split;
  const int kend = min(p.nk, kbeg + p.keys_per_split);
  // uniform by construction; readfirstlane lets the compiler branch on them with scalar compares
  const int n_tiles = __builtin_amdgcn_readfirstlane((kend - kbeg + kFwdBN - 1) / kFwdBN);

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int hl = lane >> 5;
  const int l32 = lane & 31;
  // wave owns QB blocks of 32 queries: rows q0 + 32 j + l32
  const int q0 = qt * kBM + wave * 32 * QB;
  const bool wave_live = q0 < p.nq;
  int qrow[QB];
  bool qvalid[QB];
#pragma unroll
  for (int j = 0; j < QB; ++j) {
    qrow[j] = q0 + 32 * j + l32;
    qvalid[j] = qrow[j] < p.nq;
  }

  // Q^T as the B operand: lane (query l32, half hl) holds q[query][16 ds + 8 hl + 0..7].
  V8 qf[QB][NDS];
#pragma unroll
  for (int j = 0; j < QB; ++j) {
    const T* qp = qb + (int64_t)(qvalid[j] ? qrow[j] : 0) * q_sn + hl * 8;
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds) {
      V8 v = *(const V8*)(qp + ds * 16);
      qf[j][ds] = qvalid[j] ? v : V8{};
    }
  }

  const TileCopy<T, DK, WAVES, D> kcopy(kb, p.k_sn, wave, lane);
  const TileCopy<T, W0K ? 64 : DW0K, WAVES, W0K ? 64 : DW0> w0copy(w0b, p.w0_sn, wave, lane);
  const TileCopy<T, DW1 ? DW1K : 64, WAVES, DW1 ? DW1 : 64> w1copy(w1b, p.w1_sn, wave, lane);
  // fp8 K rows: 128 bytes, copied as 64 16-bit elements
  const TileCopy<T, 64, WAVES> k8copy(QK8 ? (const T*)((const char*)p.k8 + (int64_t)loc.prob * p.nk * D) : kb, 64,
                                      wave, lane);
  auto issue = [&](int t) __attribute__((always_inline)) {
    uint32_t sb = smem_u32;
    asm volatile("" : "+s"(sb));   // keep the LDS destinations from being hoisted (see TileCopy)
    const uint32_t st = sb + (uint32_t)((t % NSLOT) * STAGE);
    const int row0 = kbeg + t * kFwdBN;
    kcopy.issue(row0, p.nk, st);
    if constexpr (!W0K) w0copy.issue(row0, p.nk, st + K_BYTES);
    if constexpr (DW1 > 0) w1copy.issue(row0, p.nk, st + K_BYTES + W0_BYTES);
    if constexpr (QK8) k8copy.issue(row0, p.nk, st + K8_OFF);
  };

  const float c = p.scale_log2;
  // Reference point m of x = s c - m (log2 units): the max of the first 32 keys, then fixed.  p = 2^x
  // is exact in fp32 for any x below ~126 and its bf16 rounding is finite there, so in bf16 rows whose
  // logits later rise by up to 64 above that max need no rescaling at all; a lane's block sum beyond
  // 2^64 flags the row and the workgroup redoes its tile with the exact row max (two passes).  fp16
  // overflows above 65504 (2^16): there a block sum above 65504 -- which any p above 65504 implies --
  // takes the same exact path, so P never rounds to inf.
  constexpr float kSumLimit = F16 ? 65504.f : 1.8446744e19f;   // fp16 max / 2^64
  float m_run[QB], l_run[QB], h_run[QB];

  // x = s cf - m with cf = c -- or, with fp8 S, c times the row's q scale times the tile's k scale (both
  // positive, so maxima commute with the scaling).  fp8 S: each q row is quantized here, in registers, by
  // its own max |q| / 448 (the lane pair l, l + 32 holds one row).
  typedef int i32x8 __attribute__((ext_vector_type(8)));
  i32x8 qf8[QK8 ? QB : 1][2];
  float cq[QB], cf[QB];
#pragma unroll
  for (int j = 0; j < QB; ++j) {
    cq[j] = c;
    if constexpr (QK8) {
      float amax = 0.f;
#pragma unroll
      for (int ds = 0; ds < NDS; ++ds)
#pragma unroll
        for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf((float)qf[j][ds][e]));
      amax = wave_max32(amax);
      const float inv = amax > 0.f ? kFp8Max / amax : 1.f;
      cq[j] = c * (amax > 0.f ? amax / kFp8Max : 1.f);
#pragma unroll
      for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int w = 0; w < 8; ++w) {   // bytes 4 w .. 4 w + 3 of product m: dims 16 (4 m + w / 2) + 8 hl + 4 (w % 2) + 0..3
          const V8& v = qf[j][4 * m + w / 2];
          const int e0 = 4 * (w % 2);
          int word = __builtin_amdgcn_cvt_pk_fp8_f32((float)v[e0] * inv, (float)v[e0 + 1] * inv, 0, false);
          qf8[j][m][w] = __builtin_amdgcn_cvt_pk_fp8_f32((float)v[e0 + 2] * inv, (float)v[e0 + 3] * inv, word, true);
        }
    }
    cf[j] = cq[j];
  }
  const int k8_row0 = QK8 ? __builtin_amdgcn_readfirstlane(loc.prob * p.k8_tiles + kbeg / kFwdBN) : 0;
  auto tile_scale = [&](int t) __attribute__((always_inline)) {
    if constexpr (QK8) {
      const float sk = p.k8_scale[k8_row0 + t];
#pragma unroll
      for (int j = 0; j < QB; ++j) cf[j] = cq[j] * sk;
    }
  };
  f32x16 acc[QB][NA];
  bool overflow = false;

  // per-lane LDS offsets
  const int srow_sw = swz_rows<DK * 2>(l32);                      // S operand rows 32 kb + l32
  const int trow = 4 * hl + ((lane & 15) >> 2);                   // W^T rows 16 ks + trow (+8)
  const int tchunk = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);   // logical chunk within 32 cols
  const int tbyte = (lane & 1) * 8;

  // S^T block kb (32 keys) for every query block: K fragments are read once, used QB times.  The
  // reads run kPre fragments ahead of the MFMAs (pinned by sched_group_barrier) so the LDS latency
  // hides behind the previous MFMAs instead of stalling each one.
  constexpr int kPre = 2;
  const int srow_sw8 = swz_rows<128>(l32);   // fp8 K rows (128 bytes)
  auto qk_block = [&](const VMO_LDS char* Ks, int kb2, f32x16 (&x)[QB], auto sched_tag)
      __attribute__((always_inline)) {
    if constexpr (QK8) {
      // S^T = K8 Q8^T: two 32x32x64 fp8 products; lane (key l32, half hl) reads the 32 bytes of product m
      // as chunks 4 m + 2 hl and + 1 of its key's row
      const VMO_LDS char* arow8 = Ks + K8_OFF + (32 * kb2 + l32) * 128;
      i32x8 a8[2];
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const i32x4 lo = *(const VMO_LDS i32x4*)(arow8 + ((4 * m + 2 * hl) ^ srow_sw8) * 16);
        const i32x4 hi = *(const VMO_LDS i32x4*)(arow8 + ((4 * m + 2 * hl + 1) ^ srow_sw8) * 16);
        a8[m] = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      }
#pragma unroll
      for (int j = 0; j < QB; ++j) {
        x[j] = f32x16{};
#pragma unroll
        for (int m = 0; m < 2; ++m)
          x[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a8[m], qf8[j][m], x[j], 0, 0, 0, 0, 0, 0);
      }
      return;
    }
    const VMO_LDS char* arow = Ks + (32 * kb2 + l32) * (DK * 2);
    V8 a[NDS];
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds) a[ds] = lds_read8<V8>(arow + ((2 * ds + hl) ^ srow_sw) * 16);
#pragma unroll
    for (int j = 0; j < QB; ++j) x[j] = f32x16{};
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds)
#pragma unroll
      for (int j = 0; j < QB; ++j) x[j] = E::mfma(a[ds], qf[j][ds], x[j]);
    if constexpr (decltype(sched_tag)::value && NDS >= kPre) {
      constexpr int NV = int(decltype(sched_tag)::value) - 1;
      __builtin_amdgcn_sched_group_barrier(0x100, kPre, 0);
#pragma unroll
      for (int ds = 0; ds < NDS - kPre; ++ds) {
        __builtin_amdgcn_sched_group_barrier(0x008, QB, 0);
        if constexpr (NV > 0) __builtin_amdgcn_sched_group_barrier(0x402, NV, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
#pragma unroll
      for (int ds = 0; ds < kPre; ++ds) {
        __builtin_amdgcn_sched_group_barrier(0x008, QB, 0);
        if constexpr (NV > 0) __builtin_amdgcn_sched_group_barrier(0x402, NV, 0);
      }
    }
  };

  // masked keys of a block (key index kofs + 8(r/4) + 4 hl + r%4 >= nvalid) get x = kMaskLogit
  auto mask_block = [&](f32x16& x, int kofs, int nvalid) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < 16; ++r)
      if (kofs + 8 * (r >> 2) + 4 * hl + (r & 3) >= nvalid) x[r] = kMaskLogit;
  };

  // x = s c - m; p = 2^x, rounded and packed as two B operands.  The row sums add the fp32 p, as
  // kernel.py:51 does (and with plain adds: v_dot2c_f32_bf16, which would sum the rounded pairs in
  // one instruction, measured to stall behind a concurrent MFMA of another wave on the SIMD) -- or,
  // for the P.K entropy, the rounded p~ (the packed halves widened back: a shift or a mask each).
  auto softmax_block = [&](f32x16 (&x)[QB], V8 (&P)[QB][2], int kofs, int nvalid, auto masked_tag)
      __attribute__((always_inline)) {
    constexpr bool MASKED = decltype(masked_tag)::value;
#pragma unroll
    for (int j = 0; j < QB; ++j) {
#pragma unroll
      for (int r = 0; r < 16; ++r) x[j][r] = fmaf(x[j][r], cf[j], -m_run[j]);
      if constexpr (MASKED) mask_block(x[j], kofs, nvalid);
      // two partial sums per lane (pairs r % 4 == 0 and == 2), each started from its first term: an
      // accumulator started at 0 costs an add of +0 per block that the compiler cannot drop (-0 + 0 = +0)
      float ls0, ls1, hs0, hs1;
      uint32_t w[8];
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        const float p0 = fast_exp2(x[j][r]), p1 = fast_exp2(x[j][r + 1]);
        const V2 pk = E::pack2(p0, p1);
        w[r / 2] = __builtin_bit_cast(uint32_t, pk);
        float s2;
        if constexpr (ENT == kEntFromPK) {
          // the rounded pair widened back from the packed word itself (left to itself, the compiler
          // rounds each p a second time, one value per conversion)
          if constexpr (F16) s2 = (float)pk[0] + (float)pk[1];
          else s2 = __uint_as_float(w[r / 2] << 16) + __uint_as_float(w[r / 2] & 0xffff0000u);
        } else {
          s2 = p0 + p1;
        }
        const float h2 = ENT == kEntOnline ? fmaf(p1, x[j][r + 1], p0 * x[j][r]) : 0.f;
        if (r == 0) { ls0 = s2; hs0 = h2; }
        else if (r == 2) { ls1 = s2; hs1 = h2; }
        else if (r & 2) { ls1 += s2; hs1 += h2; }
        else { ls0 += s2; hs0 += h2; }
      }
      typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
      P[j][0] = __builtin_bit_cast(V8, u32x4{w[0], w[1], w[2], w[3]});
      P[j][1] = __builtin_bit_cast(V8, u32x4{w[4], w[5], w[6], w[7]});
      const float ls = ls0 + ls1;
      overflow |= !(ls <= kSumLimit);   // also catches inf / nan
      l_run[j] += ls;
      if constexpr (ENT == kEntOnline) h_run[j] += hs0 + hs1;
    }
  };

  // O^T += W^T P^T for the 16-key steps 2 kb, 2 kb + 1 of one value part; W^T fragments are read
  // once and used for every query block.  Transposed reads (two per operand) run two operands
  // ahead of the MFMAs.
  auto pv_part = [&](const VMO_LDS char* W, auto rb_tag, auto na_tag, int a0, int kb2, const V8 (&P)[QB][2],
                     auto sched_tag) __attribute__((always_inline)) {
    constexpr int RB = decltype(rb_tag)::value;
    constexpr int NAP = decltype(na_tag)::value;
    constexpr int NOP = 2 * NAP;   // operands (MFMA A fragments) of this part
    V8 wt[NOP];
    // rows 32 kb + 16 h2 + trow and 8 further down: swizzles f and f ^ 2
    const int tsw = swz_rows<RB>(trow);
#pragma unroll
    for (int a = 0; a < NAP; ++a) {
      // rows 32 kb + 16 h2 + trow and 8 further down: swizzles f and f ^ 2 (chunk bit 1)
      const int c0 = trow * RB + (((4 * a + tchunk) ^ tsw) * 16 + tbyte);
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        const VMO_LDS char* rp = W + (32 * kb2 + 16 * h2) * RB;
        wt[2 * a + h2] = lds_read_tr8<V8>(rp + c0, rp + 8 * RB + (c0 ^ 32));
      }
    }
#pragma unroll
    for (int a = 0; a < NAP; ++a)
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
        for (int j = 0; j < QB; ++j) acc[j][a0 + a] = E::mfma(wt[2 * a + h2], P[j][h2], acc[j][a0 + a]);
    if constexpr (decltype(sched_tag)::value) {
      constexpr int NV = int(decltype(sched_tag)::value) - 1;
      constexpr int kPreOps = 2;
      __builtin_amdgcn_sched_group_barrier(0x100, 2 * kPreOps, 0);
#pragma unroll
      for (int o = 0; o < NOP - kPreOps; ++o) {
        __builtin_amdgcn_sched_group_barrier(0x008, QB, 0);
        if constexpr (NV > 0) __builtin_amdgcn_sched_group_barrier(0x402, NV, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      }
#pragma unroll
      for (int o = 0; o < kPreOps; ++o) {
        __builtin_amdgcn_sched_group_barrier(0x008, QB, 0);
        if constexpr (NV > 0) __builtin_amdgcn_sched_group_barrier(0x402, NV, 0);
      }
    }
  };
  auto pv_block = [&](const VMO_LDS char* Ks, int kb2, const V8 (&P)[QB][2], auto sched_tag)
      __attribute__((always_inline)) {
    pv_part(W0K ? Ks : Ks + K_BYTES, std::integral_constant<int, DW0K * 2>{}, std::integral_constant<int, NA0>{}, 0,
            kb2, P, sched_tag);
    if constexpr (DW1 > 0)
      pv_part(Ks + K_BYTES + W0_BYTES, std::integral_constant<int, DW1K * 2>{}, std::integral_constant<int, NA1>{}, NA0,
              kb2, P, sched_tag);
  };

  // One 64-key stage, as two 32-key blocks in sequence: S(kb) -> softmax(kb) -> PV(kb), with one
  // block's logits and P live at a time: the partial last tile, and the 256-wide value tensors (more
  // than eight accumulator blocks), whose softmax only the second wave on the SIMD overlaps.
  auto stage = [&](const VMO_LDS char* Ks, int nvalid, auto masked_tag, auto hi_tag) __attribute__((always_inline)) {
    constexpr bool HI = decltype(hi_tag)::value;
#pragma unroll
    for (int kb2 = 0; kb2 < (HI ? 2 : 1); ++kb2) {
      f32x16 x[QB];
      V8 P[QB][2];
      qk_block(Ks, kb2, x, std::true_type{});
      softmax_block(x, P, 32 * kb2, nvalid, masked_tag);
      pv_block(Ks, kb2, P, std::true_type{});
    }
  };

  // A full 64-key stage with the two 32-key blocks software-pipelined inside the wave: the S MFMAs
  // of block 1 are independent of the softmax of block 0, and the P.V MFMAs of block 0 of the
  // softmax of block 1, so the scheduler can interleave each pair (sched_barrier keeps the three
  // regions apart).  Needs one more S and P block live: up to eight accumulator blocks.  With more
  // than four ([k | v] values, 128 accumulator registers) the compiler, left to itself, hoists the
  // overlapped regions' operand reads and spills; pinned instead, each MFMA of S block 1 is followed
  // by 9 softmax instructions of block 0 and each of P.V block 0 by 5 of block 1 (about 72 vector
  // instructions per softmax block), with the operand reads two ahead: no spills, and R-step 1
  // ~1% faster than the sequential stage (the interleave counts 5/3 and 14/8 and three reads
  // ahead measured the same).
  constexpr bool kPipe = NA <= 8;
  constexpr bool kPipeSched = NA > 4;
  constexpr int kSchQk = 9, kSchPv = 5;
  auto stage_pipe = [&](const VMO_LDS char* Ks) __attribute__((always_inline)) {
    f32x16 x0[QB], x1[QB];
    V8 P0[QB][2], P1[QB][2];
    qk_block(Ks, 0, x0, std::true_type{});
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (kPipeSched) qk_block(Ks, 1, x1, std::integral_constant<int, 1 + kSchQk>{});
    else qk_block(Ks, 1, x1, std::false_type{});
    softmax_block(x0, P0, 0, kFwdBN, std::false_type{});
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (kPipeSched) pv_block(Ks, 0, P0, std::integral_constant<int, 1 + kSchPv>{});
    else pv_block(Ks, 0, P0, std::false_type{});
    softmax_block(x1, P1, 32, kFwdBN, std::false_type{});
    __builtin_amdgcn_sched_barrier(0);
    pv_block(Ks, 1, P1, std::true_type{});
  };

  // max over the valid keys of S^T block kb of a stage (whole row after the swap), in units of x (times
  // cf: the tile's factor)
  auto block_max = [&](const VMO_LDS char* Ks, int kb2, int nvalid, float (&mx)[QB]) __attribute__((always_inline)) {
    f32x16 x[QB];
    qk_block(Ks, kb2, x, std::true_type{});
#pragma unroll
    for (int j = 0; j < QB; ++j) {
      mask_block(x[j], 32 * kb2, nvalid);
      float v = x[j][0];
#pragma unroll
      for (int r = 1; r < 16; ++r) v = fmaxf(v, x[j][r]);
      mx[j] = fmaxf(mx[j], wave_max32(v) * cf[j]);
    }
  };

  auto reset = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < QB; ++j) {
      l_run[j] = 0.f;   // per-lane partial sum of p
      h_run[j] = 0.f;   // per-lane partial sum of p x (online entropy mode)
#pragma unroll
      for (int a = 0; a < NA; ++a) acc[j][a] = f32x16{};
    }
  };

  // Tiles t = 0 .. n_tiles-1 flow through an NSLOT-slot LDS ring; prime() issues tiles 0 ..
  // NSLOT-2.  At the top of tile t this wave's copies of tile t have landed -- only those of tile
  // t+1 may still be in flight (three slots) -- and after the barrier every wave's copies have,
  // and the slot of tile t-1 is free for tile t + NSLOT - 1.  Only the last tile can be partial, so
  // it is peeled: the steady-state body is one straight path and the accumulators stay in place
  // across iterations.  Waves without queries still take part in every barrier and tile copy.
  constexpr int kSteadyPending = NSLOT == 3 ? DMA_PER_TILE : 0;
  auto slot = [&](int t) __attribute__((always_inline)) { return (const VMO_LDS char*)smem + (t % NSLOT) * STAGE; };
  auto prime = [&]() __attribute__((always_inline)) {
    issue(0);
    if (NSLOT == 3 && n_tiles > 1) issue(1);
  };
  auto for_tiles = [&](auto&& steady_body, auto&& last_body) __attribute__((always_inline)) {
    int t = 0;
    for (; t < n_tiles - 1; ++t) {
      tile_sync<kSteadyPending>();
      if (t + NSLOT - 1 < n_tiles) issue(t + NSLOT - 1);
      steady_body(t);
    }
    tile_sync<0>();
    last_body(t);
  };
  auto key_loop = [&]() __attribute__((always_inline)) {
    if (wave_live) {
      // Full tiles in groups of NSLOT: tile t + S sits in ring slot S, a compile-time offset that
      // folds into the LDS reads' immediate field (no per-read address arithmetic in the loop).
      auto full_tile = [&](int t, auto slot_tag) __attribute__((always_inline)) {
        constexpr int S = decltype(slot_tag)::value;
        tile_sync<kSteadyPending>();
        if (t + NSLOT - 1 < n_tiles) issue(t + NSLOT - 1);
        tile_scale(t);
        if constexpr (kPipe)
          stage_pipe((const VMO_LDS char*)smem + S * STAGE);
        else
          stage((const VMO_LDS char*)smem + S * STAGE, kFwdBN, std::false_type{}, std::true_type{});
      };
      int t = 0;
      for (; t + NSLOT < n_tiles; t += NSLOT) {
        full_tile(t, std::integral_constant<int, 0>{});
        full_tile(t + 1, std::integral_constant<int, 1>{});
        if constexpr (NSLOT == 3) full_tile(t + 2, std::integral_constant<int, 2>{});
      }
      for (; t < n_tiles - 1; ++t) {   // fewer than NSLOT full tiles left
        tile_sync<kSteadyPending>();
        if (t + NSLOT - 1 < n_tiles) issue(t + NSLOT - 1);
        tile_scale(t);
        stage(slot(t), kFwdBN, std::false_type{}, std::true_type{});
      }
      tile_sync<0>();
      tile_scale(t);
      const int nvalid = kend - (kbeg + t * kFwdBN);   // 1 .. 64
      if (nvalid == kFwdBN)
        stage(slot(t), nvalid, std::false_type{}, std::true_type{});
      else if (nvalid > 32)
        stage(slot(t), nvalid, std::true_type{}, std::true_type{});
      else
        stage(slot(t), nvalid, std::true_type{}, std::false_type{});
    } else {
      for_tiles([](int) {}, [](int) {});
    }
  };

  // m from the first 32 keys of the range (tile 0 stays in slot 0 for the loop)
  prime();
  if constexpr (NSLOT == 3) {
    if (n_tiles > 1) tile_sync<DMA_PER_TILE>(); else tile_sync<0>();
  } else {
    tile_sync<0>();
  }
  {
    float mx[QB];
#pragma unroll
    for (int j = 0; j < QB; ++j) mx[j] = kMaskLogit;
    tile_scale(0);
    if (wave_live) block_max(slot(0), 0, kend - kbeg, mx);
#pragma unroll
    for (int j = 0; j < QB; ++j) m_run[j] = mx[j];
  }
  reset();
  key_loop();

  // Workgroup OR of the overflow flags through one word per wave in a ring slot that no wave reads and no
  // copy fills any more (that of tile n_tiles - NSLOT, or one never used): __syncthreads_or takes a static
  // LDS word, which the compiler pads to the ring's 1024-byte alignment -- 1 KB that costs the widest
  // variants their second workgroup per CU.  The second barrier keeps every word until all waves have read
  // them (a wave past it may refill the ring or write its epilogue patch).
  auto workgroup_any = [&](bool flag) __attribute__((always_inline)) {
    VMO_LDS int* words = (VMO_LDS int*)(smem + (n_tiles % NSLOT) * STAGE);
    const bool wave_any = __builtin_amdgcn_ballot_w64(flag) != 0;
    if (lane == 0) words[wave] = wave_any ? 1 : 0;
    __syncthreads();
    int any = 0;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) any |= words[w];
    __syncthreads();
    return any != 0;
  };
  if (workgroup_any(overflow)) {
    // exact two-pass fallback for this workgroup: the true row max, then the loop again
    float mx[QB];
#pragma unroll
    for (int j = 0; j < QB; ++j) mx[j] = kMaskLogit;
    auto max_tile = [&](int t) __attribute__((always_inline)) {
      if (!wave_live) return;
      const int nvalid = kend - (kbeg + t * kFwdBN);
      tile_scale(t);
      block_max(slot(t), 0, nvalid, mx);
      if (nvalid > 32) block_max(slot(t), 1, nvalid, mx);
    };
    prime();
    for_tiles(max_tile, max_tile);
#pragma unroll
    for (int j = 0; j < QB; ++j) m_run[j] = mx[j];
    reset();
    tile_sync<0>();   // every wave is done with the last max-pass tile before the ring is reused
    prime();
    key_loop();
    __syncthreads();   // the fallback's ring reads are done before the epilogue patches reuse it
  }

  // the stage ring is free (every wave passed the barrier above): each wave's 4 KB patch for the
  // row-segment stores of o
  // (the launch allocates at least the patches: the narrow heads' rings are smaller)
  VMO_LDS float* patch = (VMO_LDS float*)(smem + wave * kEpiPatchBytes);
  if (!wave_live) return;

  // sum_j p~_j q . k_j (the P.K entropy) from the B-operand q registers (rows past the end hold zeros): the
  // accumulator's lane (row l32, half hl) holds dims 32 a + 8 g + 4 hl + 0..3 and qf[ds] dims 16 ds + 8 hl +
  // 0..7, so one permlane32 swap of dwords (0, 2) and one of (1, 3) per ds hand every lane dims 16 ds + 4 hl
  // + 0..3 (g = 2 (ds % 2)) and 16 ds + 8 + 4 hl + 0..3 (g + 1) of its row.  (Re-reading q in the
  // accumulator's layout instead cost the launch a second pass over q, 100 MB at cfg4.)
  float pkdot[QB];
#pragma unroll
  for (int j = 0; j < QB; ++j) {
    pkdot[j] = 0.f;
    if constexpr (ENT == kEntFromPK) {
      typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
      float d = 0.f;
#pragma unroll
      for (int ds = 0; ds < NDS; ++ds) {
        const u32x4 w = __builtin_bit_cast(u32x4, qf[j][ds]);
        const auto s0 = __builtin_amdgcn_permlane32_swap(w[0], w[2], false, false);
        const auto s1 = __builtin_amdgcn_permlane32_swap(w[1], w[3], false, false);
        const uint32_t xy[4] = {s0[0], s1[0], s0[1], s1[1]};
        const int r0 = 8 * (ds & 1);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const V2 x = __builtin_bit_cast(V2, xy[u]);
          d = fmaf((float)x[0], acc[j][ds >> 1][r0 + 2 * u], d);
          d = fmaf((float)x[1], acc[j][ds >> 1][r0 + 2 * u + 1], d);
        }
      }
      pkdot[j] = wave_sum32(d);
    }
  }

  // The epilogue derives its indices and row bases again, from an opaque copy of the block's logical
  // index (scalar registers are free by now): kept from the prologue, the 64-bit bases sat in vector
  // registers across the whole key loop, and the tightest variants spilled them to scratch.
  // The divisors are opaque copies too: the division's reciprocal (a vector value) would otherwise be kept
  // from the prologue, and the [k | v] variant spilled it across the loop.
  int l_epi = __builtin_amdgcn_readfirstlane(L);
  Div d_epi{p.q_tiles, p.splits, p.frames, p.heads};
  asm volatile("" : "+s"(l_epi), "+s"(d_epi.q_tiles), "+s"(d_epi.splits), "+s"(d_epi.frames), "+s"(d_epi.heads));
  const Loc le = locate(l_epi, d_epi, std::true_type{});
  T* const ob = (T*)p.o + le.bb * p.o_sb + le.hh * p.o_sh + (int64_t)le.f * p.nq * p.o_sn;
  const int64_t o_sn = p.o_sn;
  const int64_t st0 = le.bb * p.st_sb + le.hh * p.st_sh + (int64_t)le.f * p.nq;
  const int64_t part0 = (int64_t)(le.split * p.problems + le.prob) * p.nq;
  const int q0_e = le.qt * kBM + wave * 32 * QB;

#pragma unroll
  for (int j = 0; j < QB; ++j) {
    // ---- finalise: combine the two half-waves' partial sums
    const float l_tot = wave_sum32(l_run[j]);
    const float inv_l = 1.0f / l_tot;
    const float log2l = fast_log2(l_tot);
    const float lse = m_run[j] + log2l;
    const int qb0 = q0_e + 32 * j, nrows = min(32, p.nq - qb0);
    const int qr = qb0 + l32;
    const bool qv = qr < p.nq;
    if constexpr (SPLIT) {
      store_acc_rows<F16, CW>(patch, acc[j], NA, inv_l, kGradStoreF32, (char*)(p.part_o + (part0 + qb0) * (int64_t)(DW0 + DW1)),
                          (int64_t)(DW0 + DW1) * 4, nrows, lane);
      if (qv && hl == 0) p.part_lse[part0 + qr] = lse;
    } else {
      float ent = 0.f;
      if constexpr (ENT == kEntOnline) {
        // h = sum_j p_j x_j with p_j = 2^x_j: entropy (bits) = log2 l - h / l
        ent = (log2l - wave_sum32(h_run[j]) * inv_l) * kLn2;
      } else if constexpr (ENT == kEntFromPK) {
        // sum_j P~_j s_j = q . (sum_j p~_j k_j) / l~
        ent = lse * kLn2 - (c * kLn2) * pkdot[j] * inv_l;
      }
      store_acc_rows<F16, CW>(patch, acc[j], NA, inv_l, kGradStore, (char*)(ob + (int64_t)qb0 * o_sn), o_sn * 2, nrows, lane);
      if (qv) {
        const int64_t si = st0 + qr;
        if (ENT != kEntNone && hl == 0 && p.ent) p.ent[si] = ent;
        if (hl == 0 && p.lse) p.lse[si] = lse;
      }
    }
  }
}

// Merge split-KV partials: o = sum_s 2^(lse_s - M) o_s / sum_s 2^(lse_s - M).
template <bool F16, int DWT>
__global__ __launch_bounds__(256) void fea_combine_kernel(FwdParams p) {
  using E = Elem<F16>;
  using T = typename E::T;
  using V4 = typename E::V4;
  constexpr int TPR = DWT / 4;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t row = gid / TPR;
  const int c4 = (int)(gid % TPR);
  if (row >= (int64_t)p.problems * p.nq) return;
  const int prob = (int)(row / p.nq);
  const int qi = (int)(row % p.nq);
  float M = -INFINITY;
  for (int s = 0; s < p.splits; ++s) M = fmaxf(M, p.part_lse[(int64_t)(s * p.problems + prob) * p.nq + qi]);
  float wsum = 0.f;
  f32x4 accv = f32x4{};
  for (int s = 0; s < p.splits; ++s) {
    const int64_t r = (int64_t)(s * p.problems + prob) * p.nq + qi;
    const float w = fast_exp2(p.part_lse[r] - M);
    wsum += w;
    accv += w * *(const f32x4*)(p.part_o + r * DWT + 4 * c4);
  }
  const float inv = 1.0f / wsum;
  const int f = prob % p.frames, bh = prob / p.frames, hh = bh % p.heads, bb = bh / p.heads;
  T* orow = (T*)p.o + bb * p.o_sb + hh * p.o_sh + ((int64_t)f * p.nq + qi) * p.o_sn;
  V4 v;
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = to_elem<T>(accv[e] * inv);
  *(V4*)(orow + 4 * c4) = v;
  if (c4 == 0 && p.lse) p.lse[bb * p.st_sb + hh * p.st_sh + (int64_t)f * p.nq + qi] = M + fast_log2(wsum);
}

// fp8 keys for the fp8-S variants: each 64-key tile of a problem (b, h, f) scaled by its own max |k| / 448
// (one scale per tile keeps the per-element work of the key loop at one multiply per tile and lane), its
// 128-dim rows stored in the operand order fp8_dim_pos.  One workgroup per tile, four 16-byte chunks per
// thread.
template <bool F16>
__global__ __launch_bounds__(256) void fea_fp8_keys_kernel(FwdParams p) {
  using T = typename Elem<F16>::T;
  using V8 = typename Elem<F16>::V8;
  const int tile = blockIdx.x, prob = tile / p.k8_tiles, t = tile % p.k8_tiles;
  const int f = prob % p.frames, bh = prob / p.frames, hh = bh % p.heads, bb = bh / p.heads;
  const T* kb = (const T*)p.k + bb * p.k_sb + hh * p.k_sh + ((int64_t)f * p.nk + (int64_t)t * kFwdBN) * p.k_sn;
  const int rows = min(kFwdBN, p.nk - t * kFwdBN);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  V8 v[4];
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {   // chunk tid + 256 i: row / 16, dims 8 (chunk % 16) .. + 7
    const int id = tid + 256 * i, r = id >> 4, ch = id & 15;
    v[i] = r < rows ? *(const V8*)(kb + (int64_t)r * p.k_sn + 8 * ch) : V8{};
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf((float)v[i][e]));
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) amax = fmaxf(amax, __shfl_xor(amax, m));
  __shared__ float wmax[4];
  if (lane == 0) wmax[wave] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
  const float inv = amax > 0.f ? kFp8Max / amax : 1.f;
  if (tid == 0) p.k8_scale[tile] = amax > 0.f ? amax / kFp8Max : 1.f;
  char* out = (char*)p.k8 + ((int64_t)prob * p.nk + (int64_t)t * kFwdBN) * 128;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int id = tid + 256 * i, r = id >> 4, ch = id & 15;
    if (r >= rows) continue;
    const int w0 = __builtin_amdgcn_cvt_pk_fp8_f32((float)v[i][0] * inv, (float)v[i][1] * inv, 0, false);
    const int w1 = __builtin_amdgcn_cvt_pk_fp8_f32((float)v[i][4] * inv, (float)v[i][5] * inv, 0, false);
    uint2 b;
    b.x = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32((float)v[i][2] * inv, (float)v[i][3] * inv, w0, true);
    b.y = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32((float)v[i][6] * inv, (float)v[i][7] * inv, w1, true);
    *(uint2*)(out + r * 128 + fp8_dim_pos(8 * ch)) = b;
  }
}

template <bool F16, int D, int DW0, int DW1, bool W0K, int ENT, bool SPLIT, int WAVES, bool QK8 = false>
static int launch_fwd(FwdParams p, hipStream_t stream) {
  constexpr int STAGE = fwd_stage_bytes<D, DW0, DW1, W0K, QK8>();
  constexpr int LDS = fwd_slots(STAGE, WAVES) * STAGE > WAVES * kEpiPatchBytes ? fwd_slots(STAGE, WAVES) * STAGE
                                                                              : WAVES * kEpiPatchBytes;
  constexpr int BM = 32 * kFwdQB * WAVES;
  p.q_tiles = (p.nq + BM - 1) / BM;
  p.total_wg = p.problems * p.splits * p.q_tiles;
  auto kern = fea_fwd_kernel<F16, D, DW0, DW1, W0K, ENT, SPLIT, WAVES, QK8>;
  if constexpr (QK8) {
    hipLaunchKernelGGL((fea_fp8_keys_kernel<F16>), dim3((unsigned)((int64_t)p.problems * p.k8_tiles)), dim3(256), 0, stream, p);
    const int rc = launch_status("fea_fp8_keys");
    if (rc != VMO_OK) return rc;
  }
  if (LDS > 65536) {
    static bool done = false;   // attribute is per function; idempotent, so a benign race
    if (!done) {
      if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, LDS) != hipSuccess)
        return set_error(VMO_ERR_LAUNCH, "fea_fwd: cannot raise the LDS limit to %d bytes", LDS);
      done = true;
    }
  }
  hipLaunchKernelGGL(kern, dim3(xcd_grid(p.total_wg)), dim3(64 * WAVES), LDS, stream, p);
  int rc = launch_status("fea_fwd");
  if (rc != VMO_OK || !SPLIT) return rc;
  constexpr int DWT = DW0 + DW1;
  const int64_t threads = (int64_t)p.problems * p.nq * (DWT / 4);
  hipLaunchKernelGGL((fea_combine_kernel<F16, DWT>), dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, p);
  return launch_status("fea_combine");
}

// Waves per workgroup for a variant.  Measured at cfg4 (b = 1560 queries per problem), the 8-wave
// workgroup was slower for every variant (coarser query tiles, one workgroup per CU), so all use 4.
constexpr int kFwdWavesFor(int, int, int, bool) { return kFwdWavesSmall; }

// Runtime -> template dispatch over the supported shapes.
template <bool F16>
static int dispatch_fwd(const FwdParams& p, int d, int dw0, int dw1, bool w0k, bool ent, bool split, bool qk8,
                        hipStream_t s) {
  if (qk8) {
    // fp8 S: the VMonarch R-step variants (values k or [k | v], d = 128), with the P.K entropy: e = LSE -
    // (exact q . sum p k) / l, the LSE from the fp8 logits, so e carries the fp8 error of the row's mean logit
    // (negligible on the soft rows the mode is for; up to ~2 nats on rows whose logits reach ~80).  The online
    // entropy (sum p x over the fp8 logits themselves) spills 64-93 dwords in these values-k variants.
    if (d == 128 && dw0 == 128 && w0k && ent && !split) {
      if (dw1 == 0) return launch_fwd<F16, 128, 128, 0, true, kEntFromPK, false, kFwdWavesSmall, true>(p, s);
      if (dw1 == 128) return launch_fwd<F16, 128, 128, 128, true, kEntFromPK, false, kFwdWavesSmall, true>(p, s);
    }
    return set_error(VMO_ERR_UNSUPPORTED, "fea_fwd: qk_fp8 is built for the VMonarch R-steps (d = 128, values k or "
                     "[k | v1] with dw1 = 128, entropy, one split); got d=%d dw0=%d dw1=%d w0_is_k=%d entropy=%d "
                     "split=%d", d, dw0, dw1, (int)w0k, (int)ent, (int)split);
  }
#define VMO_FWD(D_, DW0_, DW1_, W0K_, ENT_, SPLIT_)                                                  \
  if (d == D_ && dw0 == DW0_ && dw1 == DW1_ && w0k == W0K_ && ent == (ENT_ != kEntNone) && split == SPLIT_) \
    return launch_fwd<F16, D_, DW0_, DW1_, W0K_, ENT_, SPLIT_, kFwdWavesFor(D_, DW0_, DW1_, SPLIT_)>(p, s);
  // standalone flash_entropy_attention (kernel.py:384-402): online entropy
  VMO_FWD(16, 16, 0, false, kEntOnline, false)
  VMO_FWD(16, 32, 0, false, kEntOnline, false)
  VMO_FWD(16, 64, 0, false, kEntOnline, false)
  VMO_FWD(16, 128, 0, false, kEntOnline, false)
  VMO_FWD(16, 256, 0, false, kEntOnline, false)
  VMO_FWD(32, 32, 0, false, kEntOnline, false)
  VMO_FWD(32, 64, 0, false, kEntOnline, false)
  VMO_FWD(32, 128, 0, false, kEntOnline, false)
  VMO_FWD(64, 32, 0, false, kEntOnline, false)
  VMO_FWD(128, 32, 0, false, kEntOnline, false)
  VMO_FWD(32, 32, 0, false, kEntNone, false)
  VMO_FWD(64, 64, 0, false, kEntOnline, false)
  VMO_FWD(64, 128, 0, false, kEntOnline, false)
  VMO_FWD(32, 256, 0, false, kEntOnline, false)
  VMO_FWD(64, 256, 0, false, kEntOnline, false)
  VMO_FWD(128, 64, 0, false, kEntOnline, false)
  VMO_FWD(128, 128, 0, false, kEntOnline, false)
  VMO_FWD(128, 256, 0, false, kEntOnline, false)
  VMO_FWD(256, 256, 0, false, kEntOnline, false)
  // VMonarch R-step (vmonarch.py:50): values k, or [k | v]; entropy from the P.K accumulator
  VMO_FWD(16, 16, 0, true, kEntFromPK, false)
  VMO_FWD(16, 16, 16, true, kEntFromPK, false)
  VMO_FWD(32, 32, 0, true, kEntFromPK, false)
  VMO_FWD(32, 32, 32, true, kEntFromPK, false)
  VMO_FWD(64, 64, 0, true, kEntFromPK, false)
  VMO_FWD(64, 64, 64, true, kEntFromPK, false)
  VMO_FWD(64, 64, 128, true, kEntFromPK, false)
  VMO_FWD(128, 128, 0, true, kEntFromPK, false)
  VMO_FWD(128, 128, 64, true, kEntFromPK, false)
  VMO_FWD(128, 128, 128, true, kEntFromPK, false)
  // exact recompute (vmonarch.py:66-68): no entropy, optionally split-KV
  VMO_FWD(16, 16, 0, false, kEntNone, false)
  VMO_FWD(64, 64, 0, false, kEntNone, false)
  VMO_FWD(64, 128, 0, false, kEntNone, false)
  VMO_FWD(128, 64, 0, false, kEntNone, false)
  VMO_FWD(128, 128, 0, false, kEntNone, false)
  VMO_FWD(16, 16, 0, false, kEntNone, true)
  VMO_FWD(32, 32, 0, false, kEntNone, true)
  VMO_FWD(64, 64, 0, false, kEntNone, true)
  VMO_FWD(64, 128, 0, false, kEntNone, true)
  VMO_FWD(128, 64, 0, false, kEntNone, true)
  VMO_FWD(128, 128, 0, false, kEntNone, true)
#undef VMO_FWD
  return set_error(VMO_ERR_UNSUPPORTED, "fea_fwd: no kernel for d=%d dw0=%d dw1=%d w0_is_k=%d entropy=%d split=%d", d,
                   dw0, dw1, (int)w0k, (int)ent, (int)split);
}

static int64_t split_layout(const vmo_fea_fwd_args* a, int* splits_out, int* kps_out);
// Workspace: the split-KV partials, then with qk_fp8 the fp8 keys (problems x nk x d bytes) and their
// per-tile scales.  *k8_off: where the fp8 keys start.
static int64_t fwd_workspace(const vmo_fea_fwd_args* a, int* splits, int* kps, int64_t* k8_off) {
  const int64_t part = (split_layout(a, splits, kps) + 255) / 256 * 256;
  *k8_off = part;
  if (!a->qk_fp8) return part;
  const int64_t problems = (int64_t)a->batch * a->heads * a->frames;
  const int64_t k8 = (problems * a->nk * a->d + 255) / 256 * 256;
  return part + k8 + problems * ((a->nk + kFwdBN - 1) / kFwdBN) * 4;
}

static int64_t split_layout(const vmo_fea_fwd_args* a, int* splits_out, int* kps_out) {
  const int tiles = (a->nk + kFwdBN - 1) / kFwdBN;
  int want = a->num_splits < 1 ? 1 : a->num_splits;
  if (want > tiles) want = tiles;
  const int tps = (tiles + want - 1) / want;
  const int splits = (tiles + tps - 1) / tps;   // every split non-empty
  *splits_out = splits;
  *kps_out = tps * kFwdBN;
  if (splits <= 1) return 0;
  const int64_t rows = (int64_t)a->batch * a->heads * a->frames * a->nq;
  return (int64_t)splits * rows * (a->dw0 + a->dw1) * 4 + (int64_t)splits * rows * 4 + 256;
}

}  // namespace vmo

extern "C" size_t vmo_fea_fwd_workspace_size(const vmo_fea_fwd_args* a) {
  if (!a || a->nk <= 0 || a->batch <= 0 || a->heads <= 0 || a->frames <= 0) return 0;
  int s, kps;
  int64_t k8_off;
  return (size_t)vmo::fwd_workspace(a, &s, &kps, &k8_off);
}

namespace vmo {

// The forward behind both entry points: `workspace` / `workspace_bytes` hold the split-KV partials (the
// caller's for vmo_fea_fwd, the library's static scratch for vmo_fea_fwd_noalloc).
static int fea_fwd_impl(const vmo_fea_fwd_args* a, void* workspace, size_t workspace_bytes, void* stream) {
  if (!a) return set_error(VMO_ERR_INVALID, "fea_fwd: null args");
  if (a->dtype != VMO_DTYPE_BF16 && a->dtype != VMO_DTYPE_F16)
    return set_error(VMO_ERR_INVALID, "fea_fwd: dtype %d", a->dtype);
  if (a->batch < 0 || a->heads < 0 || a->frames < 0 || a->nq < 0 || a->nk < 0)
    return set_error(VMO_ERR_INVALID, "fea_fwd: negative size");
  if ((int64_t)a->batch * a->heads * a->frames * a->nq == 0) return VMO_OK;
  if (a->nk == 0) return set_error(VMO_ERR_INVALID, "fea_fwd: no keys");
  if (!(a->sm_scale >= 0.f) || a->sm_scale > 3.0e38f)
    return set_error(VMO_ERR_INVALID, "fea_fwd: sm_scale must be finite and >= 0");
  if (!view_ok(a->q) || !view_ok(a->k) || !view_ok(a->w0) || !view_ok(a->o) || (a->dw1 > 0 && !view_ok(a->w1)))
    return set_error(VMO_ERR_INVALID, "fea_fwd: tensors need 16-byte aligned rows (strides multiple of 8 elements)");
  // tile copies address up to 8 rows from a lane with a 32-bit byte offset
  const int64_t kMaxRowStride = 1ll << 27;
  if (a->k.stride_n >= kMaxRowStride || a->w0.stride_n >= kMaxRowStride ||
      (a->dw1 > 0 && a->w1.stride_n >= kMaxRowStride))
    return set_error(VMO_ERR_UNSUPPORTED, "fea_fwd: key / value row stride must be below 2^27 elements");
  const bool w0k = a->w0.data == a->k.data && a->w0.stride_b == a->k.stride_b && a->w0.stride_h == a->k.stride_h &&
                   a->w0.stride_n == a->k.stride_n && a->dw0 == a->d;
  if (a->dw1 > 0 && !w0k) return set_error(VMO_ERR_UNSUPPORTED, "fea_fwd: a second value tensor needs w0 == k");
  int splits, kps;
  int64_t k8_off;
  const int64_t ws = fwd_workspace(a, &splits, &kps, &k8_off);
  const bool ent = a->ent != nullptr;
  if (splits > 1 && ent) return set_error(VMO_ERR_UNSUPPORTED, "fea_fwd: split-KV with entropy output");
  if (a->qk_fp8 != 0 && a->qk_fp8 != 1) return set_error(VMO_ERR_INVALID, "fea_fwd: qk_fp8 is 0 or 1");
  if (ws > 0 && (workspace == nullptr || workspace_bytes < (size_t)ws || !aligned16(workspace)))
    return set_error(VMO_ERR_WORKSPACE, "fea_fwd: needs %lld workspace bytes, has %llu", (long long)ws,
                     (unsigned long long)(workspace ? workspace_bytes : 0));
  const int64_t q_tiles = (a->nq + 32 * kFwdQB * kFwdWavesSmall - 1) / (32 * kFwdQB * kFwdWavesSmall);
  const int64_t problems = (int64_t)a->batch * a->heads * a->frames;
  const int64_t total = problems * splits * q_tiles;   // the most workgroups any variant launches
  if (total > (1ll << 30) || (int64_t)a->frames * a->nq > (1ll << 30) || (int64_t)a->frames * a->nk > (1ll << 30))
    return set_error(VMO_ERR_UNSUPPORTED, "fea_fwd: problem too large");

  FwdParams p{};
  p.q = a->q.data; p.k = a->k.data; p.w0 = a->w0.data; p.w1 = a->w1.data; p.o = a->o.data;
  p.lse = a->lse; p.ent = a->ent;
  if (splits > 1) {
    const int64_t rows = problems * a->nq;
    p.part_o = (float*)workspace;
    p.part_lse = (float*)((char*)workspace + (int64_t)splits * rows * (a->dw0 + a->dw1) * 4);
  }
  p.q_sb = a->q.stride_b; p.q_sh = a->q.stride_h; p.q_sn = a->q.stride_n;
  p.k_sb = a->k.stride_b; p.k_sh = a->k.stride_h; p.k_sn = a->k.stride_n;
  p.w0_sb = a->w0.stride_b; p.w0_sh = a->w0.stride_h; p.w0_sn = a->w0.stride_n;
  p.w1_sb = a->w1.stride_b; p.w1_sh = a->w1.stride_h; p.w1_sn = a->w1.stride_n;
  p.o_sb = a->o.stride_b; p.o_sh = a->o.stride_h; p.o_sn = a->o.stride_n;
  p.st_sb = a->stat_stride_b; p.st_sh = a->stat_stride_h;
  p.heads = a->heads; p.frames = a->frames; p.nq = a->nq; p.nk = a->nk;
  p.problems = (int)problems; p.q_tiles = (int)q_tiles; p.splits = splits; p.keys_per_split = kps;
  p.total_wg = (int)total;
  p.scale_log2 = a->sm_scale * kLog2e;
  if (a->qk_fp8) {
    p.k8 = (char*)workspace + k8_off;
    p.k8_tiles = (a->nk + kFwdBN - 1) / kFwdBN;
    p.k8_scale = (float*)((char*)p.k8 + (problems * a->nk * a->d + 255) / 256 * 256);
  }
  hipStream_t s = (hipStream_t)stream;
  const bool qk8 = a->qk_fp8 != 0;
  if (a->dtype == VMO_DTYPE_F16) return dispatch_fwd<true>(p, a->d, a->dw0, a->dw1, w0k, ent, splits > 1, qk8, s);
  return dispatch_fwd<false>(p, a->d, a->dw0, a->dw1, w0k, ent, splits > 1, qk8, s);
}

// Scratch of the allocation-free entry point: split-KV partials (fp32 o and lse of every split), fully
// written by the split kernels before the merge reads them, and with qk_fp8 the fp8 keys and their scales,
// fully written by fea_fp8_keys_kernel before the forward reads them, so nothing needs clearing between calls.
// Each GPU the library runs on holds its own copy, at its own address, until the process ends.
static __device__ __align__(256) char scratch[VMO_FEA_FWD_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
static void* g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mutex;

// Device address of `scratch` on the current device, looked up once per device (in host code the
// array's name is only a stand-in for the symbol, not a device address).
static int scratch_on_current_device(void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return set_error(VMO_ERR_LAUNCH, "fea_fwd_noalloc: no current HIP device (or device id >= %d)", kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr)
      return set_error(VMO_ERR_LAUNCH, "fea_fwd_noalloc: scratch address on device %d: %s", dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return VMO_OK;
}

}  // namespace vmo

extern "C" int vmo_fea_fwd(const vmo_fea_fwd_args* a, void* stream) {
  vmo::clear_error();
  return vmo::fea_fwd_impl(a, a ? a->workspace : nullptr, a ? a->workspace_bytes : 0, stream);
}

extern "C" int vmo_fea_fwd_noalloc(const vmo_fea_fwd_args* a, void* stream) {
  using namespace vmo;
  clear_error();
  if (!a) return set_error(VMO_ERR_INVALID, "fea_fwd_noalloc: null args");
  if (vmo_fea_fwd_workspace_size(a) > VMO_FEA_FWD_SCRATCH_BYTES)
    return set_error(VMO_ERR_WORKSPACE, "fea_fwd_noalloc: the workspace (split-KV partials, fp8 keys) needs %llu bytes, "
                     "the library scratch holds %llu (use fewer splits, or 16-bit S)", (unsigned long long)vmo_fea_fwd_workspace_size(a),
                     (unsigned long long)VMO_FEA_FWD_SCRATCH_BYTES);
  void* ws = nullptr;
  const int rc = scratch_on_current_device(&ws);
  if (rc != VMO_OK) return rc;
  return fea_fwd_impl(a, ws, VMO_FEA_FWD_SCRATCH_BYTES, stream);
}
