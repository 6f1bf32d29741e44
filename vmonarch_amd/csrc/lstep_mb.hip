// Multi-block fused L-step for gfx950: grids of more than 32 frames (and head dims 16 / 32 / 64 / 128 at
// any frame count up to kMbMaxFrames), on MFMA.
//
// Reference: video_monarch_attention/vmonarch.py:51-63 -- per grid column j (the same spatial position in
// all m frames) an m x m attention over the frames:
//   attn[i, k] = softmax_k(scale q_i . kr_k + ent_k),  kr = out[..., :D]
//   last:      z_i = sum_k attn[i, k] y_k,  y = out[..., D:]
//   otherwise: u_k = scale / max(sum_i attn[i, k], min_col_mass) * sum_i attn[i, k] q_i
// (the one-tile kernels in lstep.hip take m <= 32 in a single 32 x 32 MFMA tile per column).
//
// Here one 4-wave workgroup owns a column: its q, kr (and y) rows -- tokens i b + j, i < m -- are staged
// whole into swizzled LDS tiles of M = 32 * MB rows (MB = ceil(m / 32) <= kMbMaxBlocks; rows past m are
// finite data whose weights are exact zeros), and the m x m products run on v_mfma_f32_32x32x16 in 32 x 32
// blocks (two-block grids run kernel instantiations, TWO, whose passes split over all four waves):
//   * last: wave w owns query block w.  S^T blocks (keys x queries: one query row per lane) for every key
//     block, softmax over all of them in registers (max, sum, normalise: the attention is rounded to the
//     16-bit type only once normalised, as the reference's attn.to(y.dtype)), then z^T += Y^T P^T with the
//     S^T accumulators as the B operand and Y^T read by ds_read_tr16_b64, whose 4-row groups match the
//     accumulator's (no key permutation);
//   * otherwise two passes: (1) wave w computes the log-sum-exp of its query block's rows (S^T blocks as
//     above) into LDS; (2) wave w owns key block w: L blocks (queries x keys: one key per lane) = Q Kr^T for
//     every query block, attn = exp2(L c + ent_k - lse_i) exactly normalised, the column mass as an in-lane
//     sum of the fp32 attn, and u^T += Q^T attn with Q^T by transposed reads.
// Rounding points as the one-tile kernels: logits in fp32 from the 16-bit q and kr, attn rounded to the
// 16-bit type where it multiplies q or y, the column mass from the fp32 attn, u / z rounded once when stored.
// Results leave through per-wave LDS patches as whole row segments (store_acc_rows).
#include <atomic>

#include "vmo_common.h"
#include "vmo_host.h"
#include "lstep_params.h"

namespace vmo {

constexpr int kMbWaves = 4;
constexpr int kMbMaxBlocks = 4;                  // one 32-row block per wave
constexpr int kMbMaxFrames = 32 * kMbMaxBlocks;  // m <= 128

// Byte offsets of a column's LDS arrays: 16-bit row tiles (q, kr, and y for the last step; the backward's
// upstream gradient), M-float vectors (entropy bias, row LSE; the backward's row sums rs_i, column factors f_k
// and dc_k).  The forward's row-store patches (kEpiPatchBytes per wave) reuse the start of the allocation
// once every wave has passed the barrier that ends the compute; the backward, which stores between its
// passes, has patches of its own -- half-size ones (16 rows at a time) for the last step up to 64 frames, whose
// four tiles at head dim 128 then leave room for two workgroups per CU (73.3 instead of 81.3 KB); beyond that one
// workgroup fits either way, and the whole patches store faster.
__host__ __device__ constexpr int mb_bwd_patch_rows(bool last, int M) { return last && M <= 64 ? 16 : 32; }
struct MbLayout {
  int q, k, y, g, e, lse, part, rs, f, dc, patch, total;
};
// A staged tile holds M = 32 ceil(m / 32) rows, those past m zeros (finite data whose weights are exact zeros).
// A compact tile (CT: the two-block last-step kernels up to kMbCompactMaxFrames, where it lets one more column
// share the CU) holds the m rows, the rows by which the last copy instruction overhangs them (copies of row
// m - 1; one instruction covers 1024 / rb rows of rb bytes) and one zero row, at which every operand read of a
// row past m is pointed.  The other kernels keep whole blocks: their reads take each block's rows at immediate
// offsets from one per-lane address, where the compact tile needs a clamped address per block (a build with
// compact tiles everywhere ran up to 14% slower on the grids it gave no extra column).
__host__ __device__ constexpr int mb_zero_row(int m, int rb) { return (m + 1024 / rb - 1) / (1024 / rb) * (1024 / rb); }
__host__ __device__ constexpr int mb_tile_bytes(int m, int rb, bool compact) {
  return compact ? (mb_zero_row(m, rb) + 1) * rb : (m + 31) / 32 * 32 * rb;
}
// Compact tiles are built for the two-block last step at head dims 128 / 128 and taken up to 40 frames: there its
// four tiles (three in the forward) shrink enough for one more column per CU (the backward 3 instead of 2, the
// forward 4 instead of 3); beyond that, or with narrower tiles, the per-row clamp costs without a column to gain.
constexpr int kMbCompactMaxFrames = 40;
constexpr bool mb_compact_built(int d, int dv, bool last) { return last && d == 128 && dv == 128; }
template <int RB, bool CT>
__device__ __forceinline__ int mb_phys_row(int r, int m) {
  if constexpr (CT) return r < m ? r : mb_zero_row(m, RB);
  else return r;
}

__host__ __device__ inline MbLayout mb_layout(int m, int d, int dv, bool last, bool bwd, bool compact) {
  MbLayout L;
  const int M = 32 * ((m + 31) / 32);
  int off = 0;
  auto take = [&](int bytes) { const int o = off; off += (bytes + 255) / 256 * 256; return o; };
  L.q = take(mb_tile_bytes(m, d * 2, compact));
  L.k = take(mb_tile_bytes(m, d * 2, compact));
  L.y = last ? take(mb_tile_bytes(m, dv * 2, compact)) : 0;
  L.g = bwd ? take(mb_tile_bytes(m, (last ? dv : d) * 2, compact)) : 0;
  L.e = take(M * 4);
  L.lse = take(M * 4);
  L.part = take(4 * M * 4);   // two blocks' partial row / column vectors (the two-block passes)
  L.rs = bwd ? take(M * 4) : 0;
  L.f = bwd ? take(M * 4) : 0;
  L.dc = bwd ? take(M * 4) : 0;
  L.patch = bwd ? take(kMbWaves * mb_bwd_patch_rows(last, M) * 32 * 4) : 0;
  L.total = off > kMbWaves * kEpiPatchBytes ? off : kMbWaves * kEpiPatchBytes;
  return L;
}

// Stage the m rows of W 16-bit values (row r: src + r rs) into a tile whose chunk c of row r sits at chunk
// c ^ swz_rows(r): wave instruction inst covers rows inst RPI .. + RPI - 1, lane l lands at byte 16 l of its
// 1 KB and so loads global chunk (l % CH) ^ swz_rows(row).  Only instructions that hold a row below m copy
// (their rows past m repeat row m - 1); the rows after them are zeroed up to M (a compact tile: the one zero
// row, mb_zero_row).  SW < W: a 16-wide tensor in a 32-wide tile (tile_w), each row's two chunks stored twice.
template <class T, int W, int SW = W, bool CT = false>
__device__ __forceinline__ void mb_stage(const T* src, int64_t rs, int m, VMO_LDS char* dst, int wave, int lane) {
  constexpr int RB = W * 2, CH = RB / 16, RPI = 64 / CH;
  const int c = lane % CH;
  const int ninst = (m + RPI - 1) / RPI;
  for (int inst = wave; inst < ninst; inst += kMbWaves) {
    const int r = inst * RPI + lane / CH;
    const int rr = r < m ? r : m - 1;
    g2l_16(src + (int64_t)rr * rs + ((c ^ swz_rows<RB>(r)) & (SW / 8 - 1)) * 8, dst + inst * 1024);
  }
  const int end = CT ? ninst * 1024 + RB : (m + 31) / 32 * 32 * RB;
  for (int o = ninst * 1024 + (64 * wave + lane) * 16; o < end; o += 64 * kMbWaves * 16)
    *(VMO_LDS i32x4*)(dst + o) = i32x4{0, 0, 0, 0};
}

// Row-read MFMA operand: lane (row l32 of 32-row block blk of the tile, half hl) gets elements 16 ds + 8 hl .. + 7
// (zeros for a row past m).
template <class V8, int RB, bool CT = false>
__device__ __forceinline__ V8 mb_row8(const VMO_LDS char* tile, int blk, int m, int l32, int hl, int ds) {
  if constexpr (CT) {
    const int r = mb_phys_row<RB, CT>(32 * blk + l32, m);
    return lds_read8<V8>(tile + r * RB + ((2 * ds + hl) ^ swz_rows<RB>(r)) * 16);
  } else {   // (swz_rows depends on the row mod 16 alone)
    return lds_read8<V8>(tile + 32 * blk * RB + l32 * RB + ((2 * ds + hl) ^ swz_rows<RB>(l32)) * 16);
  }
}

// Transposed MFMA A operand for the 32 columns 32 a .. 32 a + 31 of a row-major tile, K step h2 (16 rows) of
// its 32-row block blk: the rows are taken in the S^T / L accumulator's order (rows 4 hl + 0..3 and
// 8 + 4 hl + 0..3 of the step), so that accumulator rows 8 h2 .. 8 h2 + 7, rounded, are the B operand.  Each
// lane reads 8 bytes of one row; a row past m is read from the zero row.
template <class V8, int RB, bool CT = false>
__device__ __forceinline__ V8 mb_tr8(const VMO_LDS char* tile, int blk, int m, int lane, int a, int h2) {
  const int hl = lane >> 5;
  const int trow = 4 * hl + ((lane & 15) >> 2);
  const int tchunk = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
  const int tbyte = (lane & 1) * 8;
  if constexpr (CT) {
    const int r0 = mb_phys_row<RB, CT>(32 * blk + 16 * h2 + trow, m);
    const int r1 = mb_phys_row<RB, CT>(32 * blk + 16 * h2 + trow + 8, m);
    return lds_read_tr8<V8>(tile + r0 * RB + ((4 * a + tchunk) ^ swz_rows<RB>(r0)) * 16 + tbyte,
                            tile + r1 * RB + ((4 * a + tchunk) ^ swz_rows<RB>(r1)) * 16 + tbyte);
  } else {   // row 8 further on: the swizzle's chunk bit 1 flips
    const int c0 = trow * RB + (((4 * a + tchunk) ^ swz_rows<RB>(trow)) * 16 + tbyte);
    const VMO_LDS char* rp = tile + (32 * blk + 16 * h2) * RB;
    return lds_read_tr8<V8>(rp + c0, rp + 8 * RB + (c0 ^ 32));
  }
}

// Accumulator rows 8 h2 .. 8 h2 + 7 of x, times f, rounded to the 16-bit type: a B operand.
template <class T, class V8>
__device__ __forceinline__ V8 mb_pack(const f32x16& x, int h2, float f) {
  V8 v;
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = to_elem<T>(x[8 * h2 + e] * f);
  return v;
}

template <bool F16, int D, int DV, bool LAST, bool TWO, bool CT>
__global__ __launch_bounds__(64 * kMbWaves, TWO && !LAST ? 4 : 2) void lstep_mb_kernel(LParams p) {
  using E = Elem<F16>;
  using T = typename E::T;
  using V8 = typename E::V8;
  constexpr int DK = tile_w(D), DVK = tile_w(DV);   // widths in LDS
  static_assert(!CT || (LAST && TWO), "compact tiles: the two-block last-step kernels");
  constexpr int NDS = D / 16;
  constexpr int NACC = (LAST ? DVK : DK) / 32;
  constexpr int CW = (LAST ? DV : D) < 32 ? 16 : 32;   // stored columns per accumulator block
  constexpr int RBD = DK * 2, RBY = DVK * 2;
  extern __shared__ __attribute__((aligned(1024))) char smem_raw[];
  VMO_LDS char* sm = (VMO_LDS char*)smem_raw;

  const int m = p.m, MB = (m + 31) / 32, M = 32 * MB;
  const MbLayout Lo = mb_layout(m, DK, DVK, LAST, false, CT);
  VMO_LDS char* q_t = sm + Lo.q;
  VMO_LDS char* k_t = sm + Lo.k;
  VMO_LDS char* y_t = sm + Lo.y;
  VMO_LDS float* e_t = (VMO_LDS float*)(sm + Lo.e);
  VMO_LDS float* lse_t = (VMO_LDS float*)(sm + Lo.lse);
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int hl = lane >> 5, l32 = lane & 31;

  const int col = blockIdx.x, bh = col / p.bs, j = col % p.bs, hh = bh % p.heads, bb = bh / p.heads;
  const int64_t q_rs = (int64_t)p.bs * p.q_sn, o_rs = (int64_t)p.bs * p.out_sn, r_rs = (int64_t)p.bs * p.res_sn;
  const T* qcol = (const T*)p.q + bb * p.q_sb + hh * p.q_sh + (int64_t)j * p.q_sn;
  const T* ocol = (const T*)p.out + bb * p.out_sb + hh * p.out_sh + (int64_t)j * p.out_sn;
  T* rcol = (T*)p.res + bb * p.res_sb + hh * p.res_sh + (int64_t)j * p.res_sn;

  mb_stage<T, DK, D, CT>(qcol, q_rs, m, q_t, wave, lane);
  mb_stage<T, DK, D, CT>(ocol, o_rs, m, k_t, wave, lane);
  if constexpr (LAST) mb_stage<T, DVK, DV, CT>(ocol + D, o_rs, m, y_t, wave, lane);
  const float* ep = p.ent + bb * p.ent_sb + hh * p.ent_sh + j;
  for (int k = tid; k < M; k += 64 * kMbWaves) e_t[k] = k < m ? ep[(int64_t)k * p.bs] * kLog2e : -1.0e30f;
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  const float c = p.logit_scale_log2;
  // S^T blocks of query block ib against every key block, biased and in log2 units (keys past m at -1e30):
  // x[kb][r] for key 32 kb + 8 (r / 4) + 4 hl + r % 4 and query 32 ib + l32; returns the row max.
  auto s_blocks = [&](int ib, f32x16 (&x)[kMbMaxBlocks]) __attribute__((always_inline)) {
    V8 qb[NDS];
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds) qb[ds] = mb_row8<V8, RBD, CT>(q_t, ib, m, l32, hl, ds);
    float mx = -3.0e38f;
#pragma unroll
    for (int kb = 0; kb < kMbMaxBlocks; ++kb) {
      if (kb >= MB) break;
      x[kb] = f32x16{};
#pragma unroll
      for (int ds = 0; ds < NDS; ++ds) x[kb] = E::mfma(mb_row8<V8, RBD, CT>(k_t, kb, m, l32, hl, ds), qb[ds], x[kb]);
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 ev = *(const VMO_LDS f32x4*)(e_t + 32 * kb + 8 * g + 4 * hl);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          x[kb][4 * g + e] = fmaf(x[kb][4 * g + e], c, ev[e]);
          mx = fmaxf(mx, x[kb][4 * g + e]);
        }
      }
    }
    return wave_max32(mx);
  };

  // Two 32-frame blocks (33-64 frames) with an even number of output blocks: all four waves compute (with one
  // wave per block, waves 2 and 3 -- and so two of the CU's four SIMDs -- would idle through the passes, which
  // then took half of the launch at 33 frames).  The LSE pass splits the keys (wave w: query block w & 1 against
  // key block w >> 1; partial row max and sum through LDS), the product pass the output columns (wave w: row
  // block w & 1, column half w >> 1; both halves recompute the block's attention, the products' MFMAs are split).
  constexpr int NH = NACC / 2;
  if constexpr (TWO) {
    const int rb = wave & 1, half = wave >> 1;
    f32x16 acch[NH > 0 ? NH : 1];
#pragma unroll
    for (int a = 0; a < NH; ++a) acch[a] = f32x16{};
    float fsc = 1.f;
    if constexpr (LAST) {
      f32x16 x[kMbMaxBlocks];
      const float mx = s_blocks(rb, x);
      float sum = 0.f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          x[kb][r] = fast_exp2(x[kb][r] - mx);
          sum += x[kb][r];
        }
      const float inv = 1.0f / wave_sum32(sum);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const V8 P0 = mb_pack<T, V8>(x[kb], 0, inv), P1 = mb_pack<T, V8>(x[kb], 1, inv);
#pragma unroll
        for (int a = 0; a < NH; ++a) {
          acch[a] = E::mfma(mb_tr8<V8, RBY, CT>(y_t, kb, m, lane, half * NH + a, 0), P0, acch[a]);
          acch[a] = E::mfma(mb_tr8<V8, RBY, CT>(y_t, kb, m, lane, half * NH + a, 1), P1, acch[a]);
        }
      }
    } else {
      VMO_LDS float* pmax = (VMO_LDS float*)(sm + Lo.part);   // [key block][M]
      VMO_LDS float* psum = pmax + 2 * M;
      // The LSE pass takes key block rb against query block half: the kr rows it reads are the product pass's
      // B operand (same lanes and dims), and its q rows that pass's A operand for query block half, so both stay
      // in registers and the product pass reads one query block's rows from LDS instead of both and kr.
      V8 kr_op[NDS], q_op[NDS];
#pragma unroll
      for (int ds = 0; ds < NDS; ++ds) {
        kr_op[ds] = mb_row8<V8, RBD, CT>(k_t, rb, m, l32, hl, ds);
        q_op[ds] = mb_row8<V8, RBD, CT>(q_t, half, m, l32, hl, ds);
      }
      {   // S^T block (keys of block rb, queries of block half): partial max and sum per query row
        f32x16 x = f32x16{};
#pragma unroll
        for (int ds = 0; ds < NDS; ++ds) x = E::mfma(kr_op[ds], q_op[ds], x);
        float mx = -3.0e38f;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 ev = *(const VMO_LDS f32x4*)(e_t + 32 * rb + 8 * g + 4 * hl);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            x[4 * g + e] = fmaf(x[4 * g + e], c, ev[e]);
            mx = fmaxf(mx, x[4 * g + e]);
          }
        }
        mx = wave_max32(mx);
        float sum = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) sum += fast_exp2(x[r] - mx);
        sum = wave_sum32(sum);
        if (hl == 0) {
          pmax[rb * M + 32 * half + l32] = mx;
          psum[rb * M + 32 * half + l32] = sum;
        }
      }
      __syncthreads();
      if (tid < M) {   // LSE of query row tid from the two key blocks' partials; rows past m get +1e30
        const float m0 = pmax[tid], m1 = pmax[M + tid], mm = fmaxf(m0, m1);
        const float l = psum[tid] * fast_exp2(m0 - mm) + psum[M + tid] * fast_exp2(m1 - mm);
        lse_t[tid] = tid < m ? mm + fast_log2(l) : 1.0e30f;
      }
      __syncthreads();
      // u^T columns of half `half` for key block rb: one key per lane; query block half first (rows in registers)
      const float ek = e_t[32 * rb + l32];
      float cm = 0.f;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int ib = t == 0 ? half : 1 - half;
        f32x16 x = f32x16{};
#pragma unroll
        for (int ds = 0; ds < NDS; ++ds)
          x = E::mfma(t == 0 ? q_op[ds] : mb_row8<V8, RBD, CT>(q_t, ib, m, l32, hl, ds), kr_op[ds], x);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 lv = *(const VMO_LDS f32x4*)(lse_t + 32 * ib + 8 * g + 4 * hl);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float a = fast_exp2(fmaf(x[4 * g + e], c, ek - lv[e]));
            x[4 * g + e] = a;
            cm += a;
          }
        }
        const V8 P0 = mb_pack<T, V8>(x, 0, 1.f), P1 = mb_pack<T, V8>(x, 1, 1.f);
#pragma unroll
        for (int a = 0; a < NH; ++a) {
          acch[a] = E::mfma(mb_tr8<V8, RBD, CT>(q_t, ib, m, lane, half * NH + a, 0), P0, acch[a]);
          acch[a] = E::mfma(mb_tr8<V8, RBD, CT>(q_t, ib, m, lane, half * NH + a, 1), P1, acch[a]);
        }
      }
      fsc = p.scale / fmaxf(wave_sum32(cm), p.min_col_mass);
    }
    __syncthreads();   // every wave is done with the tiles: the patches reuse them
    VMO_LDS float* patch = (VMO_LDS float*)(sm + wave * kEpiPatchBytes);
    const int nrows = min(32, m - 32 * rb);
    T* const rows = rcol + 32 * rb * r_rs + half * NH * 32;
    if constexpr (LAST) {
      const int ibeg = p.skip > j ? (p.skip - j + p.bs - 1) / p.bs : 0;
      store_acc_rows<F16, CW>(patch, acch, NH, 1.f, kGradStore, (char*)rows, r_rs * 2, nrows, lane, max(0, ibeg - 32 * rb));
    } else {
      store_acc_rows<F16, CW>(patch, acch, NH, fsc, kGradStore, (char*)rows, r_rs * 2, nrows, lane);
    }
    return;
  } else {
    f32x16 acc[NACC];
#pragma unroll
    for (int a = 0; a < NACC; ++a) acc[a] = f32x16{};
    const int blk = wave;            // this wave's query block (last) or key block (otherwise)
    const bool busy = blk < MB;
    float fscale = 1.f;

    if constexpr (LAST) {
      if (busy) {
        f32x16 x[kMbMaxBlocks];
        const float mx = s_blocks(blk, x);
        float sum = 0.f;
#pragma unroll
        for (int kb = 0; kb < kMbMaxBlocks; ++kb) {
          if (kb >= MB) break;
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            x[kb][r] = fast_exp2(x[kb][r] - mx);
            sum += x[kb][r];
          }
        }
        const float inv = 1.0f / wave_sum32(sum);
        // z^T[dv][i] = sum_k y^T[dv][k] attn^T[k][i]
#pragma unroll
        for (int kb = 0; kb < kMbMaxBlocks; ++kb) {
          if (kb >= MB) break;
          const V8 P0 = mb_pack<T, V8>(x[kb], 0, inv), P1 = mb_pack<T, V8>(x[kb], 1, inv);
#pragma unroll
          for (int a = 0; a < NACC; ++a) {
            acc[a] = E::mfma(mb_tr8<V8, RBY, CT>(y_t, kb, m, lane, a, 0), P0, acc[a]);
            acc[a] = E::mfma(mb_tr8<V8, RBY, CT>(y_t, kb, m, lane, a, 1), P1, acc[a]);
          }
        }
      }
    } else {
      // pass 1: row log-sum-exp (log2 units) of every query row; rows past m get +1e30 (zero attention)
      if (busy) {
        f32x16 x[kMbMaxBlocks];
        const float mx = s_blocks(blk, x);
        float sum = 0.f;
#pragma unroll
        for (int kb = 0; kb < kMbMaxBlocks; ++kb) {
          if (kb >= MB) break;
#pragma unroll
          for (int r = 0; r < 16; ++r) sum += fast_exp2(x[kb][r] - mx);
        }
        const float lse = mx + fast_log2(wave_sum32(sum));
        if (hl == 0) lse_t[32 * blk + l32] = 32 * blk + l32 < m ? lse : 1.0e30f;
      }
      __syncthreads();
      // pass 2: key block blk; one key per lane
      if (busy) {
        V8 kb_op[NDS];
#pragma unroll
        for (int ds = 0; ds < NDS; ++ds) kb_op[ds] = mb_row8<V8, RBD, CT>(k_t, blk, m, l32, hl, ds);
        const float ek = e_t[32 * blk + l32];
        float cm = 0.f;
#pragma unroll
        for (int ib = 0; ib < kMbMaxBlocks; ++ib) {
          if (ib >= MB) break;
          // L[i][k] = q_i . kr_k: A = q rows (lane = query row), B = kr rows (lane = key)
          f32x16 x = f32x16{};
#pragma unroll
          for (int ds = 0; ds < NDS; ++ds) x = E::mfma(mb_row8<V8, RBD, CT>(q_t, ib, m, l32, hl, ds), kb_op[ds], x);
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const f32x4 lv = *(const VMO_LDS f32x4*)(lse_t + 32 * ib + 8 * g + 4 * hl);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float a = fast_exp2(fmaf(x[4 * g + e], c, ek - lv[e]));
              x[4 * g + e] = a;
              cm += a;
            }
          }
          // u^T[d][k] += sum_i q^T[d][i] attn[i][k]
          const V8 P0 = mb_pack<T, V8>(x, 0, 1.f), P1 = mb_pack<T, V8>(x, 1, 1.f);
#pragma unroll
          for (int a = 0; a < NACC; ++a) {
            acc[a] = E::mfma(mb_tr8<V8, RBD, CT>(q_t, ib, m, lane, a, 0), P0, acc[a]);
            acc[a] = E::mfma(mb_tr8<V8, RBD, CT>(q_t, ib, m, lane, a, 1), P1, acc[a]);
          }
        }
        fscale = p.scale / fmaxf(wave_sum32(cm), p.min_col_mass);
      }
    }

    __syncthreads();   // every wave is done with the tiles: the patches reuse them
    if (!busy) return;
    VMO_LDS float* patch = (VMO_LDS float*)(sm + wave * kEpiPatchBytes);
    const int nrows = min(32, m - 32 * blk);
    T* const rows = rcol + 32 * blk * r_rs;
    if constexpr (LAST) {
      // z rows i from the first one the recompute does not overwrite (token i b + j >= skip)
      const int ibeg = p.skip > j ? (p.skip - j + p.bs - 1) / p.bs : 0;
      store_acc_rows<F16, CW>(patch, acc, NACC, 1.f, kGradStore, (char*)rows, r_rs * 2, nrows, lane, max(0, ibeg - 32 * blk));
    } else {
      store_acc_rows<F16, CW>(patch, acc, NACC, fscale, kGradStore, (char*)rows, r_rs * 2, nrows, lane);
    }
  }
}


// Backward of the multi-block L-step (the gradient autograd takes through vmonarch.py:51-63 with the entropy
// bias detached, vmonarch.py:26), one 4-wave workgroup per grid column as the forward, with g the upstream
// gradient rows (dz rows i when last, du rows k otherwise) staged beside q, kr (and y):
//   last:  da[i,k] = g_i . y_k,  rs_i = sum_k a da,  dl = scale a (da - rs_i)
//          pass A (wave = query block, one query row per lane): S^T and DA^T blocks -> lse_i, rs_i, then
//          dq^T += Kr^T dl^T;  pass B (wave = key block, one key per lane): L and DA blocks ->
//          dy^T += G^T a, dkr^T += Q^T dl
//   else:  c_k = sum_i a, gv_k = sum_i a (g_k . q_i), f_k = scale / max(c_k, mcm),
//          dc_k = -[c_k >= mcm] gv_k f_k / max(c_k, mcm),  da[i,k] = f_k (g_k . q_i) + dc_k
//          pass 0 (query blocks): lse_i;  pass 1 (key blocks): c_k, gv_k -> f_k, dc_k;
//          pass 2 (query blocks): rs_i, dq^T += Kr^T dl^T + G^T (a f)^T;  pass 3 (key blocks): dkr^T += Q^T dl
// Every m x m block is recomputed where an orientation needs it (the MFMAs are cheap next to the column's
// HBM traffic); the attention is exp2(logit - lse_i), exactly normalised.  MFMA operands a, dl and a f are
// rounded to the 16-bit type, the sums rs, c, gv kept in fp32 from the fp32 attention.  dq (fp32) is added
// to or overwritten, d out (the 16-bit type) written; rows past m carry zero attention and are not stored.
template <bool F16, int D, int DV, bool LAST, bool TWO, bool CT>
__global__ __launch_bounds__(64 * kMbWaves, 2) void lstep_mb_bwd_kernel(LBParams p) {
  using E = Elem<F16>;
  using T = typename E::T;
  using V8 = typename E::V8;
  constexpr int DK = tile_w(D), DVK = tile_w(DV);   // widths in LDS
  static_assert(!CT || (LAST && TWO), "compact tiles: the two-block last-step kernels");
  constexpr int NDS = D / 16, NDSV = DV / 16;
  constexpr int ND = DK / 32, NV = DVK / 32;
  constexpr int CWD = D < 32 ? 16 : 32, CWV = DV < 32 ? 16 : 32;   // stored columns per accumulator block
  constexpr int GW = LAST ? DV : D, GWK = tile_w(GW);
  constexpr int RBD = DK * 2, RBY = DVK * 2, RBG = GWK * 2;
  extern __shared__ __attribute__((aligned(1024))) char smem_raw[];
  VMO_LDS char* sm = (VMO_LDS char*)smem_raw;

  const int m = p.m, MB = (m + 31) / 32, M = 32 * MB;
  const MbLayout Lo = mb_layout(m, DK, DVK, LAST, true, CT);
  VMO_LDS char* q_t = sm + Lo.q;
  VMO_LDS char* k_t = sm + Lo.k;
  VMO_LDS char* y_t = sm + Lo.y;
  VMO_LDS char* g_t = sm + Lo.g;
  VMO_LDS float* e_t = (VMO_LDS float*)(sm + Lo.e);
  VMO_LDS float* lse_t = (VMO_LDS float*)(sm + Lo.lse);
  VMO_LDS float* rs_t = (VMO_LDS float*)(sm + Lo.rs);
  VMO_LDS float* f_t = (VMO_LDS float*)(sm + Lo.f);
  VMO_LDS float* dc_t = (VMO_LDS float*)(sm + Lo.dc);
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int hl = lane >> 5, l32 = lane & 31;
  const bool half_patch = mb_bwd_patch_rows(LAST, M) == 16;
  VMO_LDS float* patch = (VMO_LDS float*)(sm + Lo.patch + wave * mb_bwd_patch_rows(LAST, M) * 32 * 4);

  const int col = blockIdx.x, bh = col / p.bs, j = col % p.bs, hh = bh % p.heads, bb = bh / p.heads;
  const int64_t q_rs = (int64_t)p.bs * p.q_sn, o_rs = (int64_t)p.bs * p.out_sn, g_rs = (int64_t)p.bs * p.g_sn;
  const int64_t dq_rs = (int64_t)p.bs * p.dq_sn, do_rs = (int64_t)p.bs * p.do_sn;
  const T* qcol = (const T*)p.q + bb * p.q_sb + hh * p.q_sh + (int64_t)j * p.q_sn;
  const T* ocol = (const T*)p.out + bb * p.out_sb + hh * p.out_sh + (int64_t)j * p.out_sn;
  const T* gcol = (const T*)p.g + bb * p.g_sb + hh * p.g_sh + (int64_t)j * p.g_sn;
  float* dqcol = p.dq + bb * p.dq_sb + hh * p.dq_sh + (int64_t)j * p.dq_sn;
  T* dcol = (T*)p.dout + bb * p.do_sb + hh * p.do_sh + (int64_t)j * p.do_sn;

  mb_stage<T, DK, D, CT>(qcol, q_rs, m, q_t, wave, lane);
  mb_stage<T, DK, D, CT>(ocol, o_rs, m, k_t, wave, lane);
  if constexpr (LAST) mb_stage<T, DVK, DV, CT>(ocol + D, o_rs, m, y_t, wave, lane);
  mb_stage<T, GWK, GW, CT>(gcol, g_rs, m, g_t, wave, lane);
  const float* ep = p.ent + bb * p.ent_sb + hh * p.ent_sh + j;
  for (int k = tid; k < M; k += 64 * kMbWaves) e_t[k] = k < m ? ep[(int64_t)k * p.bs] * kLog2e : -1.0e30f;
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if constexpr (LAST) {   // z rows of tokens < skip are the recompute's: no gradient reaches the L-path
    constexpr int CH = RBG / 16;
    for (int idx = tid; idx < m * CH; idx += 64 * kMbWaves) {
      const int r = idx / CH;
      if ((int64_t)r * p.bs + j < p.skip) *(VMO_LDS i32x4*)(g_t + r * RBG + (idx % CH) * 16) = i32x4{0, 0, 0, 0};
    }
    __syncthreads();
  }

  const float c = p.logit_scale_log2;
  const int blk = wave;
  const bool busy = blk < MB;
  const int dq_mode = p.dq_overwrite ? kGradStoreF32 : kGradAddF32;

  // S^T block (keys kb x queries of qb, one query row per lane), biased, log2 units
  auto s_block = [&](int kb, const V8 (&qb)[NDS]) __attribute__((always_inline)) {
    f32x16 x = f32x16{};
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds) x = E::mfma(mb_row8<V8, RBD, CT>(k_t, kb, m, l32, hl, ds), qb[ds], x);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const f32x4 ev = *(const VMO_LDS f32x4*)(e_t + 32 * kb + 8 * g + 4 * hl);
#pragma unroll
      for (int e = 0; e < 4; ++e) x[4 * g + e] = fmaf(x[4 * g + e], c, ev[e]);
    }
    return x;
  };
  // L block (queries ib x keys of key block kb, one key per lane): attn = exp2(c q.kr + e_k - lse_i); the kr
  // operand rows are read at each use (the passes that call this hold two accumulator sets)
  auto attn_block = [&](int ib, int kb, float ek) __attribute__((always_inline)) {
    f32x16 x = f32x16{};
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds)
      x = E::mfma(mb_row8<V8, RBD, CT>(q_t, ib, m, l32, hl, ds), mb_row8<V8, RBD, CT>(k_t, kb, m, l32, hl, ds), x);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const f32x4 lv = *(const VMO_LDS f32x4*)(lse_t + 32 * ib + 8 * g + 4 * hl);
#pragma unroll
      for (int e = 0; e < 4; ++e) x[4 * g + e] = fast_exp2(fmaf(x[4 * g + e], c, ek - lv[e]));
    }
    return x;
  };
  // query block's row LSE from its S^T blocks (kept in x for the caller)
  auto row_lse = [&](const V8 (&qb)[NDS], f32x16 (&x)[kMbMaxBlocks]) __attribute__((always_inline)) {
    float mx = -3.0e38f;
#pragma unroll
    for (int kb = 0; kb < kMbMaxBlocks; ++kb) {
      if (kb >= MB) break;
      x[kb] = s_block(kb, qb);
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, x[kb][r]);
    }
    mx = wave_max32(mx);
    float sum = 0.f;
#pragma unroll
    for (int kb = 0; kb < kMbMaxBlocks; ++kb) {
      if (kb >= MB) break;
#pragma unroll
      for (int r = 0; r < 16; ++r) sum += fast_exp2(x[kb][r] - mx);
    }
    return mx + fast_log2(wave_sum32(sum));
  };
  auto load_rows = [&](V8 (&op)[NDS], const VMO_LDS char* tile, int b) __attribute__((always_inline)) {
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds) op[ds] = mb_row8<V8, RBD, CT>(tile, b, m, l32, hl, ds);
  };
  const bool row_ok = 32 * blk + l32 < m;   // this lane's query row (query-block passes) or key (key-block passes)
  const int nrows = busy ? min(32, m - 32 * blk) : 0;
  // row stores through the patch: whole (32 rows) or half (16 rows at a time)
  auto store_rows = [&](auto cw_tag, const f32x16* acc, int nacc, int mode, char* row0, int64_t stride, int nr)
      __attribute__((always_inline)) {
    constexpr int CWS = decltype(cw_tag)::value;
    if (half_patch) store_acc_rows<F16, CWS, 16>(patch, acc, nacc, 1.f, mode, row0, stride, nr, lane);
    else store_acc_rows<F16, CWS, 32>(patch, acc, nacc, 1.f, mode, row0, stride, nr, lane);
  };
  // The two-block kernels (TWO) give each wave a (query block ib, key block kb) pair.  pair_lse: the row LSE of
  // the query rows from the S^T blocks of the pairs (each wave's x), as the partial max and sum of each key
  // block combined through `part` (rows past m get +1e30: their attention is exactly zero).  pair_row_sum: a
  // per-query-row sum over the two key blocks, each wave's partial v for its pair (every lane gets the total).
  VMO_LDS float* part = (VMO_LDS float*)(sm + Lo.part);   // [block][M] x two vectors
  auto pair_lse = [&](const f32x16& x, int ib, int kb) __attribute__((always_inline)) {
    float mx = -3.0e38f;
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, x[r]);
    mx = wave_max32(mx);
    float sum = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) sum += fast_exp2(x[r] - mx);
    sum = wave_sum32(sum);
    if (hl == 0) {
      part[kb * M + 32 * ib + l32] = mx;
      part[2 * M + kb * M + 32 * ib + l32] = sum;
    }
    __syncthreads();
    if (tid < M) {
      const float m0 = part[tid], m1 = part[M + tid], mm = fmaxf(m0, m1);
      const float l = part[2 * M + tid] * fast_exp2(m0 - mm) + part[3 * M + tid] * fast_exp2(m1 - mm);
      lse_t[tid] = tid < m ? mm + fast_log2(l) : 1.0e30f;
    }
    __syncthreads();
  };
  auto pair_row_sum = [&](float v, int ib, int kb) __attribute__((always_inline)) {
    if (hl == 0) part[kb * M + 32 * ib + l32] = v;
    __syncthreads();
    return part[32 * ib + l32] + part[M + 32 * ib + l32];
  };

  if constexpr (LAST) {
    if constexpr (TWO) {
      // Two blocks on four waves, as the non-last step's passes below: (query block, key block) pairs, the row
      // sums combined through `part`, the products split by output columns over operands exchanged in `xch`
      // (the row-store patches: 16-row ones up to 64 frames, room for two operands per wave and lane).
      constexpr int NH = ND / 2, NVH = NV / 2;
      VMO_LDS V8* xch = (VMO_LDS V8*)(sm + Lo.patch);
      const int ib = wave >> 1, kb = wave & 1;   // pass A: query block ib against key block kb
      const int kq = wave >> 1, iq = wave & 1;   // pass B: key block kq against query block iq
      // ---- pass A: row LSE from two partials, rs_i from two partials, then dq (query block ib, column half kb)
      {
        V8 qb[NDS];
        load_rows(qb, q_t, ib);
        f32x16 x = s_block(kb, qb);
        pair_lse(x, ib, kb);
        const float lse = lse_t[32 * ib + l32];
#pragma unroll
        for (int r = 0; r < 16; ++r) x[r] = fast_exp2(x[r] - lse);   // attn^T[k][i]
        f32x16 d = f32x16{};   // DA^T[k][i] = y_k . g_i
#pragma unroll
        for (int ds = 0; ds < NDSV; ++ds)
          d = E::mfma(mb_row8<V8, RBY, CT>(y_t, kb, m, l32, hl, ds), mb_row8<V8, RBY, CT>(g_t, ib, m, l32, hl, ds), d);
        float rs = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) rs = fmaf(x[r], d[r], rs);
        rs = pair_row_sum(wave_sum32(rs), ib, kb);
        if (kb == 0 && hl == 0) rs_t[32 * ib + l32] = 32 * ib + l32 < m ? rs : 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) d[r] = p.scale * x[r] * (d[r] - rs);   // dl^T
        VMO_LDS V8* mine = xch + wave * 2 * 64 + lane;
        mine[0] = mb_pack<T, V8>(d, 0, 1.f);
        mine[64] = mb_pack<T, V8>(d, 1, 1.f);
        __syncthreads();
        f32x16 accq[NH];
#pragma unroll
        for (int a = 0; a < NH; ++a) accq[a] = f32x16{};
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2) {
          const VMO_LDS V8* src = xch + (2 * ib + k2) * 2 * 64 + lane;
          const V8 P0 = src[0], P1 = src[64];
#pragma unroll
          for (int a = 0; a < NH; ++a) {
            accq[a] = E::mfma(mb_tr8<V8, RBD, CT>(k_t, k2, m, lane, kb * NH + a, 0), P0, accq[a]);
            accq[a] = E::mfma(mb_tr8<V8, RBD, CT>(k_t, k2, m, lane, kb * NH + a, 1), P1, accq[a]);
          }
        }
        __syncthreads();   // every wave is done with xch: the patches may reuse it
        store_rows(std::integral_constant<int, CWD>{}, accq, NH, dq_mode, (char*)(dqcol + 32 * ib * dq_rs + 32 * kb * NH),
                   dq_rs * 4, min(32, m - 32 * ib));
      }
      __syncthreads();   // the patches are free again for xch, and rs_t is complete
      // ---- pass B: dy and dkr (key block kq, column half iq) over the two query blocks
      {
        const f32x16 at = attn_block(iq, kq, e_t[32 * kq + l32]);
        f32x16 dl = f32x16{};   // DA[i][k] = g_i . y_k
#pragma unroll
        for (int ds = 0; ds < NDSV; ++ds)
          dl = E::mfma(mb_row8<V8, RBY, CT>(g_t, iq, m, l32, hl, ds), mb_row8<V8, RBY, CT>(y_t, kq, m, l32, hl, ds), dl);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 rv = *(const VMO_LDS f32x4*)(rs_t + 32 * iq + 8 * g + 4 * hl);
#pragma unroll
          for (int e = 0; e < 4; ++e) dl[4 * g + e] = p.scale * at[4 * g + e] * (dl[4 * g + e] - rv[e]);
        }
        VMO_LDS V8* mine = xch + wave * 2 * 64 + lane;
        mine[0] = mb_pack<T, V8>(at, 0, 1.f);   // the attention block first: dy^T += G^T a
        mine[64] = mb_pack<T, V8>(at, 1, 1.f);
        __syncthreads();
        f32x16 accy[NVH];
#pragma unroll
        for (int a = 0; a < NVH; ++a) accy[a] = f32x16{};
#pragma unroll
        for (int i2 = 0; i2 < 2; ++i2) {
          const VMO_LDS V8* src = xch + (2 * kq + i2) * 2 * 64 + lane;
          const V8 A0 = src[0], A1 = src[64];
#pragma unroll
          for (int a = 0; a < NVH; ++a) {
            accy[a] = E::mfma(mb_tr8<V8, RBY, CT>(g_t, i2, m, lane, iq * NVH + a, 0), A0, accy[a]);
            accy[a] = E::mfma(mb_tr8<V8, RBY, CT>(g_t, i2, m, lane, iq * NVH + a, 1), A1, accy[a]);
          }
        }
        __syncthreads();
        mine[0] = mb_pack<T, V8>(dl, 0, 1.f);   // then dl: dkr^T += Q^T dl
        mine[64] = mb_pack<T, V8>(dl, 1, 1.f);
        __syncthreads();
        f32x16 acck[NH];
#pragma unroll
        for (int a = 0; a < NH; ++a) acck[a] = f32x16{};
#pragma unroll
        for (int i2 = 0; i2 < 2; ++i2) {
          const VMO_LDS V8* src = xch + (2 * kq + i2) * 2 * 64 + lane;
          const V8 P0 = src[0], P1 = src[64];
#pragma unroll
          for (int a = 0; a < NH; ++a) {
            acck[a] = E::mfma(mb_tr8<V8, RBD, CT>(q_t, i2, m, lane, iq * NH + a, 0), P0, acck[a]);
            acck[a] = E::mfma(mb_tr8<V8, RBD, CT>(q_t, i2, m, lane, iq * NH + a, 1), P1, acck[a]);
          }
        }
        __syncthreads();
        const int nr = min(32, m - 32 * kq);
        store_rows(std::integral_constant<int, CWV>{}, accy, NVH, kGradStore,
                   (char*)(dcol + 32 * kq * do_rs + D + 32 * iq * NVH), do_rs * 2, nr);
        store_rows(std::integral_constant<int, CWD>{}, acck, NH, kGradStore, (char*)(dcol + 32 * kq * do_rs + 32 * iq * NH),
                   do_rs * 2, nr);
      }
      return;
    }
    // ---- pass A: one query row per lane
    if (busy) {
      V8 qb[NDS];
      load_rows(qb, q_t, blk);
      f32x16 x[kMbMaxBlocks];
      const float lse = row_lse(qb, x);
      auto da_block = [&](int kb) __attribute__((always_inline)) {   // DA^T[k][i] = y_k . g_i (g rows read at each use)
        f32x16 d = f32x16{};
#pragma unroll
        for (int ds = 0; ds < NDSV; ++ds)
          d = E::mfma(mb_row8<V8, RBY, CT>(y_t, kb, m, l32, hl, ds), mb_row8<V8, RBY, CT>(g_t, blk, m, l32, hl, ds),
                      d);
        return d;
      };
      float rs = 0.f;
#pragma unroll
      for (int kb = 0; kb < kMbMaxBlocks; ++kb) {
        if (kb >= MB) break;
        const f32x16 d = da_block(kb);
#pragma unroll
        for (int r = 0; r < 16; ++r) rs = fmaf(fast_exp2(x[kb][r] - lse), d[r], rs);
      }
      rs = wave_sum32(rs);
      if (hl == 0) {
        lse_t[32 * blk + l32] = row_ok ? lse : 1.0e30f;
        rs_t[32 * blk + l32] = row_ok ? rs : 0.f;
      }
      f32x16 accq[ND];
#pragma unroll
      for (int a = 0; a < ND; ++a) accq[a] = f32x16{};
#pragma unroll
      for (int kb = 0; kb < kMbMaxBlocks; ++kb) {
        if (kb >= MB) break;
        f32x16 dl = da_block(kb);
#pragma unroll
        for (int r = 0; r < 16; ++r) dl[r] = p.scale * fast_exp2(x[kb][r] - lse) * (dl[r] - rs);
        const V8 P0 = mb_pack<T, V8>(dl, 0, 1.f), P1 = mb_pack<T, V8>(dl, 1, 1.f);
#pragma unroll
        for (int a = 0; a < ND; ++a) {
          accq[a] = E::mfma(mb_tr8<V8, RBD, CT>(k_t, kb, m, lane, a, 0), P0, accq[a]);
          accq[a] = E::mfma(mb_tr8<V8, RBD, CT>(k_t, kb, m, lane, a, 1), P1, accq[a]);
        }
      }
      store_rows(std::integral_constant<int, CWD>{}, accq, ND, dq_mode, (char*)(dqcol + 32 * blk * dq_rs), dq_rs * 4, nrows);
    }
    __syncthreads();
    // ---- pass B: one key per lane, as two sweeps over the query blocks (dy, then dkr: holding both accumulator
    // sets at once spills at 128 / 128, and recomputing the attention block is cheap next to the HBM traffic)
    if (busy) {
      const float ek = e_t[32 * blk + l32];
      f32x16 accy[NV];
#pragma unroll
      for (int a = 0; a < NV; ++a) accy[a] = f32x16{};
#pragma unroll
      for (int ib = 0; ib < kMbMaxBlocks; ++ib) {
        if (ib >= MB) break;
        const f32x16 at = attn_block(ib, blk, ek);
        // dy^T[dv][k] += sum_i g^T[dv][i] a[i][k]
        const V8 A0 = mb_pack<T, V8>(at, 0, 1.f), A1 = mb_pack<T, V8>(at, 1, 1.f);
#pragma unroll
        for (int a = 0; a < NV; ++a) {
          accy[a] = E::mfma(mb_tr8<V8, RBY, CT>(g_t, ib, m, lane, a, 0), A0, accy[a]);
          accy[a] = E::mfma(mb_tr8<V8, RBY, CT>(g_t, ib, m, lane, a, 1), A1, accy[a]);
        }
      }
      store_rows(std::integral_constant<int, CWV>{}, accy, NV, kGradStore, (char*)(dcol + 32 * blk * do_rs + D),
                 do_rs * 2, nrows);
      f32x16 acck[ND];
#pragma unroll
      for (int a = 0; a < ND; ++a) acck[a] = f32x16{};
#pragma unroll
      for (int ib = 0; ib < kMbMaxBlocks; ++ib) {
        if (ib >= MB) break;
        const f32x16 at = attn_block(ib, blk, ek);
        // DA[i][k] = g_i . y_k, dl = scale a (da - rs_i)
        f32x16 dl = f32x16{};
#pragma unroll
        for (int ds = 0; ds < NDSV; ++ds)
          dl = E::mfma(mb_row8<V8, RBY, CT>(g_t, ib, m, l32, hl, ds), mb_row8<V8, RBY, CT>(y_t, blk, m, l32, hl, ds),
                       dl);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 rv = *(const VMO_LDS f32x4*)(rs_t + 32 * ib + 8 * g + 4 * hl);
#pragma unroll
          for (int e = 0; e < 4; ++e) dl[4 * g + e] = p.scale * at[4 * g + e] * (dl[4 * g + e] - rv[e]);
        }
        const V8 P0 = mb_pack<T, V8>(dl, 0, 1.f), P1 = mb_pack<T, V8>(dl, 1, 1.f);
#pragma unroll
        for (int a = 0; a < ND; ++a) {
          acck[a] = E::mfma(mb_tr8<V8, RBD, CT>(q_t, ib, m, lane, a, 0), P0, acck[a]);
          acck[a] = E::mfma(mb_tr8<V8, RBD, CT>(q_t, ib, m, lane, a, 1), P1, acck[a]);
        }
      }
      store_rows(std::integral_constant<int, CWD>{}, acck, ND, kGradStore, (char*)(dcol + 32 * blk * do_rs), do_rs * 2,
                 nrows);
    }
  } else {
    if constexpr (TWO) {
      // Two blocks on four waves: each pass takes one (query block, key block) pair per wave instead of one block
      // per wave (which left two waves idle).  The per-row / per-column sums over the pair's two blocks are
      // combined through `part`; the dq and dkr products are split by output columns (half NH of the ND
      // blocks per wave), each wave reading the 16-bit B operands that its block pair's waves wrote to `xch`
      // (the row-store patch region, free until the stores).  Each accumulator takes its products in the same
      // order as the one-block-per-wave passes.
      constexpr int NH = ND / 2;
      VMO_LDS V8* xch = (VMO_LDS V8*)(sm + Lo.patch);         // [wave][operand][lane]
      const int ib = wave >> 1, kb = wave & 1;   // passes 0 and 2: query block ib against key block kb
      const int kq = wave >> 1, iq = wave & 1;   // passes 1 and 3: key block kq against query block iq
      const bool ib_ok = 32 * ib + l32 < m;
      V8 qb[NDS];
      load_rows(qb, q_t, ib);
      // ---- pass 0: row LSE from the two key blocks' partial max / sum
      pair_lse(s_block(kb, qb), ib, kb);
      // ---- pass 1: column mass c_k and gv_k from the two query blocks' partials -> f_k, dc_k
      {
        V8 gop[NDS];
        load_rows(gop, g_t, kq);
        const f32x16 at = attn_block(iq, kq, e_t[32 * kq + l32]);
        f32x16 gq = f32x16{};   // GQ[i][k] = q_i . g_k
#pragma unroll
        for (int ds = 0; ds < NDS; ++ds) gq = E::mfma(mb_row8<V8, RBD, CT>(q_t, iq, m, l32, hl, ds), gop[ds], gq);
        float cs = 0.f, gv = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          cs += at[r];
          gv = fmaf(at[r], gq[r], gv);
        }
        cs = wave_sum32(cs);
        gv = wave_sum32(gv);
        if (hl == 0) {
          part[iq * M + 32 * kq + l32] = cs;
          part[2 * M + iq * M + 32 * kq + l32] = gv;
        }
      }
      __syncthreads();
      if (tid < M) {
        const float cs = part[tid] + part[M + tid], gv = part[2 * M + tid] + part[3 * M + tid];
        const float cm = fmaxf(cs, p.min_col_mass), f = p.scale / cm;
        f_t[tid] = f;
        dc_t[tid] = (tid < m && cs >= p.min_col_mass) ? -gv * f / cm : 0.f;
      }
      __syncthreads();
      // ---- pass 2: rs_i from the two key blocks' partials, then dq (query block ib, column half kb)
      {
        f32x16 x = s_block(kb, qb);
        const float lse = lse_t[32 * ib + l32];
#pragma unroll
        for (int r = 0; r < 16; ++r) x[r] = fast_exp2(x[r] - lse);   // attn^T[k][i]
        f32x16 d = f32x16{};   // da^T[k][i] = f_k (g_k . q_i) + dc_k
#pragma unroll
        for (int ds = 0; ds < NDS; ++ds) d = E::mfma(mb_row8<V8, RBD, CT>(g_t, kb, m, l32, hl, ds), qb[ds], d);
        f32x4 fv[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          fv[g] = *(const VMO_LDS f32x4*)(f_t + 32 * kb + 8 * g + 4 * hl);
          const f32x4 cv = *(const VMO_LDS f32x4*)(dc_t + 32 * kb + 8 * g + 4 * hl);
#pragma unroll
          for (int e = 0; e < 4; ++e) d[4 * g + e] = fmaf(fv[g][e], d[4 * g + e], cv[e]);
        }
        float rs = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) rs = fmaf(x[r], d[r], rs);
        rs = pair_row_sum(wave_sum32(rs), ib, kb);
        if (kb == 0 && hl == 0) rs_t[32 * ib + l32] = ib_ok ? rs : 0.f;
        f32x16 dl, af;
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int r = 4 * g + e;
            af[r] = x[r] * fv[g][e];
            dl[r] = p.scale * x[r] * (d[r] - rs);
          }
        VMO_LDS V8* mine = xch + wave * 4 * 64 + lane;
        mine[0] = mb_pack<T, V8>(dl, 0, 1.f);
        mine[64] = mb_pack<T, V8>(dl, 1, 1.f);
        mine[128] = mb_pack<T, V8>(af, 0, 1.f);
        mine[192] = mb_pack<T, V8>(af, 1, 1.f);
        __syncthreads();
        f32x16 accq[NH];
#pragma unroll
        for (int a = 0; a < NH; ++a) accq[a] = f32x16{};
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2) {
          const VMO_LDS V8* src = xch + (2 * ib + k2) * 4 * 64 + lane;
          const V8 P0 = src[0], P1 = src[64], F0 = src[128], F1 = src[192];
#pragma unroll
          for (int a = 0; a < NH; ++a) {
            const int ca = kb * NH + a;   // this wave's column half
            accq[a] = E::mfma(mb_tr8<V8, RBD, CT>(k_t, k2, m, lane, ca, 0), P0, accq[a]);
            accq[a] = E::mfma(mb_tr8<V8, RBD, CT>(k_t, k2, m, lane, ca, 1), P1, accq[a]);
            accq[a] = E::mfma(mb_tr8<V8, RBD, CT>(g_t, k2, m, lane, ca, 0), F0, accq[a]);
            accq[a] = E::mfma(mb_tr8<V8, RBD, CT>(g_t, k2, m, lane, ca, 1), F1, accq[a]);
          }
        }
        __syncthreads();   // every wave is done with xch: the patches may reuse it
        store_rows(std::integral_constant<int, CWD>{}, accq, NH, dq_mode, (char*)(dqcol + 32 * ib * dq_rs + 32 * kb * NH),
                   dq_rs * 4, min(32, m - 32 * ib));
      }
      __syncthreads();   // the patches are free again for xch, and rs_t is complete
      // ---- pass 3: dkr (key block kq, column half iq) over the two query blocks
      {
        V8 gop[NDS];
        load_rows(gop, g_t, kq);
        const float fk = f_t[32 * kq + l32], dck = dc_t[32 * kq + l32];
        const f32x16 at = attn_block(iq, kq, e_t[32 * kq + l32]);
        f32x16 dl = f32x16{};
#pragma unroll
        for (int ds = 0; ds < NDS; ++ds) dl = E::mfma(mb_row8<V8, RBD, CT>(q_t, iq, m, l32, hl, ds), gop[ds], dl);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 rv = *(const VMO_LDS f32x4*)(rs_t + 32 * iq + 8 * g + 4 * hl);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int r = 4 * g + e;
            dl[r] = p.scale * at[r] * (fmaf(fk, dl[r], dck) - rv[e]);
          }
        }
        VMO_LDS V8* mine = xch + wave * 2 * 64 + lane;
        mine[0] = mb_pack<T, V8>(dl, 0, 1.f);
        mine[64] = mb_pack<T, V8>(dl, 1, 1.f);
        __syncthreads();
        f32x16 acck[NH];
#pragma unroll
        for (int a = 0; a < NH; ++a) acck[a] = f32x16{};
#pragma unroll
        for (int i2 = 0; i2 < 2; ++i2) {
          const VMO_LDS V8* src = xch + (2 * kq + i2) * 2 * 64 + lane;
          const V8 P0 = src[0], P1 = src[64];
#pragma unroll
          for (int a = 0; a < NH; ++a) {
            const int ca = iq * NH + a;
            acck[a] = E::mfma(mb_tr8<V8, RBD, CT>(q_t, i2, m, lane, ca, 0), P0, acck[a]);
            acck[a] = E::mfma(mb_tr8<V8, RBD, CT>(q_t, i2, m, lane, ca, 1), P1, acck[a]);
          }
        }
        __syncthreads();
        store_rows(std::integral_constant<int, CWD>{}, acck, NH, kGradStore, (char*)(dcol + 32 * kq * do_rs + 32 * iq * NH),
                   do_rs * 2, min(32, m - 32 * kq));
      }
      return;
    }
    // ---- pass 0: row LSE (query blocks)
    if (busy) {
      V8 qb[NDS];
      load_rows(qb, q_t, blk);
      f32x16 x[kMbMaxBlocks];
      const float lse = row_lse(qb, x);
      if (hl == 0) lse_t[32 * blk + l32] = row_ok ? lse : 1.0e30f;
    }
    __syncthreads();
    // ---- pass 1: column mass c_k and gv_k = sum_i a (g_k . q_i) (key blocks) -> f_k, dc_k
    if (busy) {
      V8 gop[NDS];
      load_rows(gop, g_t, blk);
      const float ek = e_t[32 * blk + l32];
      float cs = 0.f, gv = 0.f;
#pragma unroll
      for (int ib = 0; ib < kMbMaxBlocks; ++ib) {
        if (ib >= MB) break;
        const f32x16 at = attn_block(ib, blk, ek);
        f32x16 gq = f32x16{};   // GQ[i][k] = q_i . g_k
#pragma unroll
        for (int ds = 0; ds < NDS; ++ds) gq = E::mfma(mb_row8<V8, RBD, CT>(q_t, ib, m, l32, hl, ds), gop[ds], gq);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          cs += at[r];
          gv = fmaf(at[r], gq[r], gv);
        }
      }
      cs = wave_sum32(cs);
      gv = wave_sum32(gv);
      const float cm = fmaxf(cs, p.min_col_mass), f = p.scale / cm;
      if (hl == 0) {
        f_t[32 * blk + l32] = f;
        dc_t[32 * blk + l32] = (row_ok && cs >= p.min_col_mass) ? -gv * f / cm : 0.f;
      }
    }
    __syncthreads();
    // ---- pass 2: rs_i and dq (query blocks)
    if (busy) {
      V8 qb[NDS];
      load_rows(qb, q_t, blk);
      f32x16 x[kMbMaxBlocks];
      const float lse = lse_t[32 * blk + l32];
#pragma unroll
      for (int kb = 0; kb < kMbMaxBlocks; ++kb) {
        if (kb >= MB) break;
        x[kb] = s_block(kb, qb);
#pragma unroll
        for (int r = 0; r < 16; ++r) x[kb][r] = fast_exp2(x[kb][r] - lse);   // attn^T[k][i]
      }
      // da^T[k][i] = f_k (g_k . q_i) + dc_k
      auto da_block = [&](int kb) __attribute__((always_inline)) {
        f32x16 d = f32x16{};
#pragma unroll
        for (int ds = 0; ds < NDS; ++ds) d = E::mfma(mb_row8<V8, RBD, CT>(g_t, kb, m, l32, hl, ds), qb[ds], d);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 fv = *(const VMO_LDS f32x4*)(f_t + 32 * kb + 8 * g + 4 * hl);
          const f32x4 cv = *(const VMO_LDS f32x4*)(dc_t + 32 * kb + 8 * g + 4 * hl);
#pragma unroll
          for (int e = 0; e < 4; ++e) d[4 * g + e] = fmaf(fv[e], d[4 * g + e], cv[e]);
        }
        return d;
      };
      float rs = 0.f;
#pragma unroll
      for (int kb = 0; kb < kMbMaxBlocks; ++kb) {
        if (kb >= MB) break;
        const f32x16 d = da_block(kb);
#pragma unroll
        for (int r = 0; r < 16; ++r) rs = fmaf(x[kb][r], d[r], rs);
      }
      rs = wave_sum32(rs);
      if (hl == 0) rs_t[32 * blk + l32] = row_ok ? rs : 0.f;
      f32x16 accq[ND];
#pragma unroll
      for (int a = 0; a < ND; ++a) accq[a] = f32x16{};
#pragma unroll
      for (int kb = 0; kb < kMbMaxBlocks; ++kb) {
        if (kb >= MB) break;
        f32x16 dl = da_block(kb), af;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 fv = *(const VMO_LDS f32x4*)(f_t + 32 * kb + 8 * g + 4 * hl);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int r = 4 * g + e;
            af[r] = x[kb][r] * fv[e];
            dl[r] = p.scale * x[kb][r] * (dl[r] - rs);
          }
        }
        const V8 P0 = mb_pack<T, V8>(dl, 0, 1.f), P1 = mb_pack<T, V8>(dl, 1, 1.f);
        const V8 F0 = mb_pack<T, V8>(af, 0, 1.f), F1 = mb_pack<T, V8>(af, 1, 1.f);
#pragma unroll
        for (int a = 0; a < ND; ++a) {
          accq[a] = E::mfma(mb_tr8<V8, RBD, CT>(k_t, kb, m, lane, a, 0), P0, accq[a]);
          accq[a] = E::mfma(mb_tr8<V8, RBD, CT>(k_t, kb, m, lane, a, 1), P1, accq[a]);
          accq[a] = E::mfma(mb_tr8<V8, RBD, CT>(g_t, kb, m, lane, a, 0), F0, accq[a]);
          accq[a] = E::mfma(mb_tr8<V8, RBD, CT>(g_t, kb, m, lane, a, 1), F1, accq[a]);
        }
      }
      store_acc_rows<F16, CWD>(patch, accq, ND, 1.f, dq_mode, (char*)(dqcol + 32 * blk * dq_rs), dq_rs * 4, nrows, lane);
    }
    __syncthreads();
    // ---- pass 3: dkr (key blocks)
    if (busy) {
      V8 gop[NDS];
      load_rows(gop, g_t, blk);
      const float ek = e_t[32 * blk + l32];
      const float fk = f_t[32 * blk + l32], dck = dc_t[32 * blk + l32];
      f32x16 acck[ND];
#pragma unroll
      for (int a = 0; a < ND; ++a) acck[a] = f32x16{};
#pragma unroll
      for (int ib = 0; ib < kMbMaxBlocks; ++ib) {
        if (ib >= MB) break;
        const f32x16 at = attn_block(ib, blk, ek);
        f32x16 dl = f32x16{};
#pragma unroll
        for (int ds = 0; ds < NDS; ++ds) dl = E::mfma(mb_row8<V8, RBD, CT>(q_t, ib, m, l32, hl, ds), gop[ds], dl);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 rv = *(const VMO_LDS f32x4*)(rs_t + 32 * ib + 8 * g + 4 * hl);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int r = 4 * g + e;
            dl[r] = p.scale * at[r] * (fmaf(fk, dl[r], dck) - rv[e]);
          }
        }
        const V8 P0 = mb_pack<T, V8>(dl, 0, 1.f), P1 = mb_pack<T, V8>(dl, 1, 1.f);
#pragma unroll
        for (int a = 0; a < ND; ++a) {
          acck[a] = E::mfma(mb_tr8<V8, RBD, CT>(q_t, ib, m, lane, a, 0), P0, acck[a]);
          acck[a] = E::mfma(mb_tr8<V8, RBD, CT>(q_t, ib, m, lane, a, 1), P1, acck[a]);
        }
      }
      store_acc_rows<F16, CWD>(patch, acck, ND, 1.f, kGradStore, (char*)(dcol + 32 * blk * do_rs), do_rs * 2, nrows, lane);
    }
  }
}

// Head-dim pairs the multi-block kernels are built for: 32 / 64 / 128 in any pair, and 16 with 16 (the
// reference's VMonarch runs d = dv).
static bool mb_dims(int d, int dv, bool last) {
  const auto ok = [](int x) { return x == 32 || x == 64 || x == 128; };
  if (d == 16) return !last || dv == 16;
  return ok(d) && (!last || ok(dv));
}

int mb_lstep_check(int m, int d, int dv, bool last, bool bwd) {
  if (!mb_dims(d, dv, last) || m < 1 || m > kMbMaxFrames) return 0;
  return mb_layout(m, tile_w(d), last ? tile_w(dv) : 0, last, bwd, false).total <= 160 * 1024;
}

template <bool F16, int D, int DV, bool LAST, bool TWO, bool CT>
static int launch_mb_k(const LParams& p, hipStream_t s) {
  int lds = mb_layout(p.m, tile_w(D), tile_w(DV), LAST, false, CT).total;
  // The two-block non-last kernel is built for four columns per CU (33-48 frames: their chain of passes is
  // the bound, and a fourth column in flight hides more of it); past 48 frames the column's bytes dominate,
  // and its LDS request is raised to hold the CU at three (measured faster there).
  if constexpr (TWO && !LAST)
    if (p.m > 48) lds = lds > 160 * 1024 / 4 + 256 ? lds : 160 * 1024 / 4 + 256;
  auto kern = lstep_mb_kernel<F16, D, DV, LAST, TWO, CT>;
  static std::atomic<int> lds_limit{65536};   // this kernel's dynamic-LDS limit as raised so far
  if (lds > lds_limit.load(std::memory_order_relaxed)) {   // (idempotent: a race only repeats the call)
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds) != hipSuccess)
      return set_error(VMO_ERR_LAUNCH, "lstep_mb: cannot raise the LDS limit to %d bytes", lds);
    lds_limit.store(lds, std::memory_order_relaxed);
  }
  hipLaunchKernelGGL(kern, dim3(p.cols_total), dim3(64 * kMbWaves), lds, s, p);
  return launch_status("lstep_mb");
}
// Two 32-frame blocks with an even number of output blocks run the instantiation whose passes split over all
// four waves (TWO).
template <bool F16, int D, int DV, bool LAST>
static int launch_mb(const LParams& p, hipStream_t s) {
  constexpr bool TWO_OK = (tile_w(LAST ? DV : D) / 32) % 2 == 0;
  if constexpr (TWO_OK) {
    if ((p.m + 31) / 32 == 2) {
      if constexpr (mb_compact_built(D, DV, LAST))
        if (p.m <= kMbCompactMaxFrames) return launch_mb_k<F16, D, DV, LAST, true, true>(p, s);
      return launch_mb_k<F16, D, DV, LAST, true, false>(p, s);
    }
  }
  return launch_mb_k<F16, D, DV, LAST, false, false>(p, s);
}

template <bool F16>
static int dispatch_mb(const LParams& p, int d, int dv, bool last, hipStream_t s) {
#define VMO_MB(D_, DV_)                                                                   \
  if (d == D_ && dv == DV_ && last) return launch_mb<F16, D_, DV_, true>(p, s);
#define VMO_MB_U(D_) \
  if (d == D_ && !last) return launch_mb<F16, D_, D_, false>(p, s);
  VMO_MB_U(16) VMO_MB_U(32) VMO_MB_U(64) VMO_MB_U(128)
  VMO_MB(16, 16) VMO_MB(32, 32) VMO_MB(32, 64) VMO_MB(32, 128)
  VMO_MB(64, 32) VMO_MB(64, 64) VMO_MB(64, 128)
  VMO_MB(128, 32) VMO_MB(128, 64) VMO_MB(128, 128)
#undef VMO_MB
#undef VMO_MB_U
  return set_error(VMO_ERR_UNSUPPORTED, "lstep_mb: no kernel for d=%d dv=%d last=%d", d, dv, (int)last);
}

int mb_lstep_fwd(const LParams& p, bool f16, int d, int dv, bool last, hipStream_t s) {
  return f16 ? dispatch_mb<true>(p, d, dv, last, s) : dispatch_mb<false>(p, d, dv, last, s);
}

template <bool F16, int D, int DV, bool LAST, bool TWO, bool CT>
static int launch_mb_bwd_k(const LBParams& p, hipStream_t s) {
  const int lds = mb_layout(p.m, tile_w(D), tile_w(DV), LAST, true, CT).total;
  auto kern = lstep_mb_bwd_kernel<F16, D, DV, LAST, TWO, CT>;
  static std::atomic<int> lds_limit{65536};   // as in launch_mb, per kernel
  if (lds > lds_limit.load(std::memory_order_relaxed)) {
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds) != hipSuccess)
      return set_error(VMO_ERR_LAUNCH, "lstep_mb_bwd: cannot raise the LDS limit to %d bytes", lds);
    lds_limit.store(lds, std::memory_order_relaxed);
  }
  hipLaunchKernelGGL(kern, dim3(p.cols_total), dim3(64 * kMbWaves), lds, s, p);
  return launch_status("lstep_mb_bwd");
}

// Grids of two row blocks (33-64 frames) take the kernel whose passes split the block pairs over all four waves,
// where the accumulator blocks split evenly (32-wide heads and 16-wide tiles have one block); larger grids keep
// one block per wave.
template <bool F16, int D, int DV, bool LAST>
static int launch_mb_bwd(const LBParams& p, hipStream_t s) {
  constexpr bool TWO_OK = (tile_w(D) / 32) % 2 == 0 && (!LAST || (tile_w(DV) / 32) % 2 == 0);
  if constexpr (TWO_OK) {
    if ((p.m + 31) / 32 == 2) {
      if constexpr (mb_compact_built(D, DV, LAST))
        if (p.m <= kMbCompactMaxFrames) return launch_mb_bwd_k<F16, D, DV, LAST, true, true>(p, s);
      return launch_mb_bwd_k<F16, D, DV, LAST, true, false>(p, s);
    }
  }
  return launch_mb_bwd_k<F16, D, DV, LAST, false, false>(p, s);
}

template <bool F16>
static int dispatch_mb_bwd(const LBParams& p, int d, int dv, bool last, hipStream_t s) {
#define VMO_MB(D_, DV_)                                                                   \
  if (d == D_ && dv == DV_ && last) return launch_mb_bwd<F16, D_, DV_, true>(p, s);
#define VMO_MB_U(D_) \
  if (d == D_ && !last) return launch_mb_bwd<F16, D_, D_, false>(p, s);
  VMO_MB_U(16) VMO_MB_U(32) VMO_MB_U(64) VMO_MB_U(128)
  VMO_MB(16, 16) VMO_MB(32, 32) VMO_MB(32, 64) VMO_MB(32, 128)
  VMO_MB(64, 32) VMO_MB(64, 64) VMO_MB(64, 128)
  VMO_MB(128, 32) VMO_MB(128, 64) VMO_MB(128, 128)
#undef VMO_MB
#undef VMO_MB_U
  return set_error(VMO_ERR_UNSUPPORTED, "lstep_mb_bwd: no kernel for d=%d dv=%d last=%d", d, dv, (int)last);
}

int mb_lstep_bwd(const LBParams& p, bool f16, int d, int dv, bool last, hipStream_t s) {
  return f16 ? dispatch_mb_bwd<true>(p, d, dv, last, s) : dispatch_mb_bwd<false>(p, d, dv, last, s);
}

}  // namespace vmo
