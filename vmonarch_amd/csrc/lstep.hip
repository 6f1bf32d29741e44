// Fused L-step of the VMonarch alternating minimisation for gfx950.
//
// Reference: video_monarch_attention/vmonarch.py:51-63 -- per grid column j (the same spatial
// position in all m frames) a tiny m x m attention:
//   kr      = out[..., :D] * scale                                   (vmonarch.py:51)
//   logits  = einsum("bhijd,bhkjd->bhjik", q, kr)                    (vmonarch.py:55)
//   attn    = softmax_k(logits - neg_ent[k, j])                      (vmonarch.py:56)
//   last:     z = einsum("bhjik,bhkjd->bhijd", attn, out[..., D:])   (vmonarch.py:57-59)
//   else:     col_mass = clamp_min(sum_i attn, min_col_mass)         (vmonarch.py:61)
//             u = einsum("bhjik,bhijd->bhkjd", attn, q) * scale / col_mass   (vmonarch.py:62-63)
// The reference runs this as cuBLAS batched m x m GEMMs plus permutes and a softmax over an fp32
// (B, H, b, m, m) tensor.  Here one wave owns one column end to end (m <= 32 padded to one
// 32 x 32 MFMA tile), so q, out and ent are read once and u / z written once: the kernel is an
// HBM stream.  Layouts as in the flash-entropy kernel: logits are computed transposed
// (L^T = kr q^T) so the softmax over k is in-lane; z = attn y reuses the logits accumulator as
// the B operand with y^T read by ds_read_tr16_b64; for u the attention matrix goes through LDS
// once to switch to one-lane-per-k, where the column mass is an in-lane sum.  The result rows
// (tokens i b + j, b rows apart) leave through a dead LDS tile as whole row segments
// (store_acc_rows).  The backward of the step (lstep_bwd_kernel, below) follows the same layout.
#include <type_traits>

#include "vmo_common.h"
#include "vmo_host.h"
#include "lstep_params.h"

namespace vmo {

constexpr int kLWaves = 4;   // columns per workgroup
constexpr int kAttStride = 36;   // floats per row of the LDS attention tile (bank-conflict pad)



template <int D, int DV, bool LAST>
struct LLds {
  static constexpr int QT = LAST ? 0 : 32 * D * 2;
  static constexpr int YT = LAST ? 32 * DV * 2 : 0;
  static constexpr int AT = LAST ? 0 : 32 * kAttStride * 4;
  static constexpr int ET = 32 * 4;
  static constexpr int PER_WAVE = QT + YT + AT + ET;
};

// Stage 32 rows (row i = token i*bs + j, clamped to i < m) of width W into a swizzled tile.
template <class T, int W, int ROWS = 32>
__device__ __forceinline__ void stage_col_rows(const T* __restrict__ colbase, int64_t row_stride, int m,
                                               VMO_LDS char* dst, int lane) {
  constexpr int CH = W / 8;
  constexpr int RPI = 64 / CH;
  constexpr int NI = ROWS / RPI;
  static_assert(ROWS % RPI == 0, "whole copy instructions");
#pragma unroll
  for (int inst = 0; inst < NI; ++inst) {
    const int r = inst * RPI + lane / CH;
    const int lc = (lane % CH) ^ swz(r);
    const int rr = r < m ? r : m - 1;
    g2l_16(colbase + (int64_t)rr * row_stride + lc * 8, dst + inst * 1024);
  }
}

template <bool F16, int D, int DV, bool LAST>
__global__ __launch_bounds__(256) void lstep_kernel(LParams p) {
  using E = Elem<F16>;
  using T = typename E::T;
  using V8 = typename E::V8;
  using V4 = typename E::V4;
  using LL = LLds<D, DV, LAST>;
  constexpr int NACC = (LAST ? DV : D) / 32;

  extern __shared__ __attribute__((aligned(1024))) char smem_raw[];
  // the wave's column and its decoded indices are wave-uniform: held in scalar registers, so that the integer
  // divisions and the 64-bit address arithmetic run on the scalar unit instead of once per lane
  auto uni = [](int x) __attribute__((always_inline)) { return __builtin_amdgcn_readfirstlane(x); };
  const int tid = threadIdx.x, wave = uni(tid >> 6), lane = tid & 63, hl = lane >> 5, l32 = lane & 31;
  const bool live = blockIdx.x * kLWaves + wave < p.cols_total;   // tail waves compute, never store
  const int col = live ? blockIdx.x * kLWaves + wave : p.cols_total - 1;
  VMO_LDS char* wl = (VMO_LDS char*)smem_raw + wave * LL::PER_WAVE;
  VMO_LDS char* q_t = wl;
  VMO_LDS char* y_t = wl + LL::QT;
  VMO_LDS float* att = (VMO_LDS float*)(wl + LL::QT + LL::YT);
  VMO_LDS float* e_t = (VMO_LDS float*)(wl + LL::QT + LL::YT + LL::AT);

  const int bh = uni(col / p.bs), j = uni(col % p.bs);
  const int hh = uni(bh % p.heads), bb = uni(bh / p.heads);
  const int m = p.m;
  const int64_t q_rs = (int64_t)p.bs * p.q_sn;       // stride between grid rows i, i+1 of column j
  const int64_t o_rs = (int64_t)p.bs * p.out_sn;
  const T* qcol = (const T*)p.q + bb * p.q_sb + hh * p.q_sh + (int64_t)j * p.q_sn;
  const T* ocol = (const T*)p.out + bb * p.out_sb + hh * p.out_sh + (int64_t)j * p.out_sn;

  // ---- loads: LDS tiles by DMA, MFMA A operand kr (rows k) straight into registers
  if constexpr (!LAST) stage_col_rows<T, D>(qcol, q_rs, m, q_t, lane);
  if constexpr (LAST) stage_col_rows<T, DV>(ocol + D, o_rs, m, y_t, lane);
  const int rk = l32 < m ? l32 : m - 1;
  V8 krf[D / 16];
  {
    const T* kp = ocol + (int64_t)rk * o_rs + hl * 8;
#pragma unroll
    for (int ds = 0; ds < D / 16; ++ds) krf[ds] = *(const V8*)(kp + ds * 16);
  }
  V8 qf[LAST ? D / 16 : 1];
  if constexpr (LAST) {
    const T* qp = qcol + (int64_t)rk * q_rs + hl * 8;
#pragma unroll
    for (int ds = 0; ds < D / 16; ++ds) qf[ds] = *(const V8*)(qp + ds * 16);
  }
  if (hl == 0) {
    const float* ep = p.ent + bb * p.ent_sb + hh * p.ent_sh + j;
    e_t[l32] = l32 < m ? ep[(int64_t)l32 * p.bs] * kLog2e : -1.0e30f;
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  // ---- L^T[k][i] = kr_k . q_i  (lane: query row i = l32, keys k = 8(r/4) + 4 hl + r%4)
  f32x16 s = f32x16{};
  if constexpr (LAST) {
#pragma unroll
    for (int ds = 0; ds < D / 16; ++ds) s = E::mfma(krf[ds], qf[ds], s);
  } else {
    const VMO_LDS char* qrow = q_t + l32 * (D * 2);
    const int sw = swz(l32);
#pragma unroll
    for (int ds = 0; ds < D / 16; ++ds)
      s = E::mfma(krf[ds], lds_read8<V8>(qrow + ((2 * ds + hl) ^ sw) * 16), s);
  }

  // ---- attn[i][k] = softmax_k(scale * L + ent[k]) in the log2 domain
  float mx = -3.0e38f;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const f32x4 ev = *(const VMO_LDS f32x4*)(e_t + 8 * g + 4 * hl);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int r = 4 * g + e;
      s[r] = fmaf(s[r], p.logit_scale_log2, ev[e]);
      mx = fmaxf(mx, s[r]);
    }
  }
  mx = wave_max32(mx);
  float sum = 0.f;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    s[r] = fast_exp2(s[r] - mx);
    sum += s[r];
  }
  const float inv = 1.0f / wave_sum32(sum);
#pragma unroll
  for (int r = 0; r < 16; ++r) s[r] *= inv;

  f32x16 acc[NACC];
#pragma unroll
  for (int a = 0; a < NACC; ++a) acc[a] = f32x16{};
  const int tchunk = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
  const int tbyte = (lane & 1) * 8;
  const int tj = (lane & 15) >> 2;

  if constexpr (LAST) {
    // z^T[dv][i] = sum_k y^T[dv][k] attn^T[k][i]: attn stays in registers as the B operand
    V8 P[2];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      P[0][e] = to_elem<T>(s[e]);
      P[1][e] = to_elem<T>(s[8 + e]);
    }
    const int trow = 4 * hl + tj;
    const int tsw = swz(trow);
#pragma unroll
    for (int a = 0; a < NACC; ++a) {
      const int coff = ((4 * a + tchunk) ^ tsw) * 16 + tbyte;
#pragma unroll
      for (int ss = 0; ss < 2; ++ss) {
        const VMO_LDS char* r0 = y_t + (16 * ss + trow) * (DV * 2) + coff;
        acc[a] = E::mfma(lds_read_tr8<V8>(r0, r0 + 8 * DV * 2), P[ss], acc[a]);
      }
    }
    // z rows i (tokens i b + j) from the first one the recompute does not overwrite (token >= skip),
    // through the y tile (dead now) as the row-store patch
    if (live) {
      const int ibeg = p.skip > j ? (p.skip - j + p.bs - 1) / p.bs : 0;
      T* z0 = (T*)p.res + bb * p.res_sb + hh * p.res_sh + (int64_t)j * p.res_sn;
      store_acc_rows<F16>((VMO_LDS float*)y_t, acc, NACC, 1.f, kGradStore, (char*)z0, (int64_t)p.bs * p.res_sn * 2,
                          m, lane, ibeg);
    }
  } else {
    // attn -> LDS as [k][i] (rows i >= m zeroed so they drop out of the sums over i)
    const bool ivalid = l32 < m;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int k = 8 * (r >> 2) + 4 * hl + (r & 3);
      att[k * kAttStride + l32] = ivalid ? s[r] : 0.f;
    }
    // one lane per k: B operand attn[i][k] for i = 16 is + 8 hl + 0..7, and the column mass
    V8 Bu[2];
    float cs = 0.f;
#pragma unroll
    for (int is = 0; is < 2; ++is) {
      const VMO_LDS float* ap = att + l32 * kAttStride + 16 * is + 8 * hl;
      const f32x4 x0 = *(const VMO_LDS f32x4*)ap;
      const f32x4 x1 = *(const VMO_LDS f32x4*)(ap + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        Bu[is][e] = to_elem<T>(x0[e]);
        Bu[is][4 + e] = to_elem<T>(x1[e]);
        cs += x0[e] + x1[e];
      }
    }
    cs = wave_sum32(cs);
    // u^T[d][k] = sum_i q^T[d][i] attn[i][k]; q^T from the row-major q tile by transposed reads
#pragma unroll
    for (int a = 0; a < NACC; ++a) {
#pragma unroll
      for (int is = 0; is < 2; ++is) {
        const int row0 = 16 * is + 8 * hl + tj;           // t = 0 rows; t = 1 adds 4
        const VMO_LDS char* r0 = q_t + row0 * (D * 2) + ((4 * a + tchunk) ^ (2 * tj)) * 16 + tbyte;
        const VMO_LDS char* r1 = q_t + (row0 + 4) * (D * 2) + ((4 * a + tchunk) ^ (2 * tj + 1)) * 16 + tbyte;
        acc[a] = E::mfma(lds_read_tr8<V8>(r0, r1), Bu[is], acc[a]);
      }
    }
    // u rows k (tokens k b + j) scaled by scale / col_mass, through the q tile (dead now) as the patch
    if (live) {
      const float f = p.scale / fmaxf(cs, p.min_col_mass);
      T* u0 = (T*)p.res + bb * p.res_sb + hh * p.res_sh + (int64_t)j * p.res_sn;
      store_acc_rows<F16>((VMO_LDS float*)q_t, acc, NACC, f, kGradStore, (char*)u0, (int64_t)p.bs * p.res_sn * 2, m,
                          lane);
    }
  }
}

template <bool F16, int D, int DV, bool LAST>
static int launch_lstep(const LParams& p, hipStream_t s) {
  constexpr int LDS = LLds<D, DV, LAST>::PER_WAVE * kLWaves;
  static_assert(LDS <= 65536, "lstep LDS");
  const int wgs = (p.cols_total + kLWaves - 1) / kLWaves;
  hipLaunchKernelGGL((lstep_kernel<F16, D, DV, LAST>), dim3(wgs), dim3(64 * kLWaves), LDS, s, p);
  return launch_status("lstep");
}

template <bool F16>
static int dispatch_lstep(const LParams& p, int d, int dv, bool last, hipStream_t s) {
#define VMO_L(D_, DV_, LAST_) \
  if (d == D_ && (!LAST_ || dv == DV_) && last == LAST_) return launch_lstep<F16, D_, DV_, LAST_>(p, s);
  VMO_L(64, 64, false)
  VMO_L(128, 128, false)
  VMO_L(64, 64, true)
  VMO_L(64, 128, true)
  VMO_L(128, 64, true)
  VMO_L(128, 128, true)
#undef VMO_L
  return set_error(VMO_ERR_UNSUPPORTED, "lstep: no kernel for d=%d dv=%d last=%d", d, dv, (int)last);
}

// ---------------------------------------------------------------------------------------------
// Backward of the fused L-step: the gradient that autograd takes through vmonarch.py:51-63 (the
// entropy bias is detached, vmonarch.py:26).  Per grid column, with a = attn, y = out[..., D:]
// and g the upstream gradient (dz when last, du otherwise):
//   last:  da[i,k] = g_i . y_k                        dy_k = sum_i a[i,k] g_i
//   else:  v_k = sum_i a[i,k] q_i,  c_k = sum_i a[i,k],  f_k = scale / max(c_k, min_col_mass)
//          dv_k = f_k g_k,  dc_k = -(g_k . v_k) f_k / max(c_k, mcm)  where c_k >= mcm, else 0
//          da[i,k] = dv_k . q_i + dc_k,  dq_i += sum_k a[i,k] dv_k
//   both:  dL[i,k] = scale a[i,k] (da[i,k] - sum_k' a[i,k'] da[i,k'])     (softmax backward)
//          dq_i += sum_k dL[i,k] kr_k,   dkr_k = sum_i dL[i,k] q_i       (kr = out[..., :D])
// One wave per column as in the forward, with the same operand layouts: every m x m matrix lives
// transposed in the accumulator layout (one query row i per lane), and goes through an LDS tile
// [k][i] wherever a product needs one lane per k.  dq is accumulated (read-modify-write) into an
// fp32 buffer, since every L-step and the R-step chain add to it; d out is written.
// Columns (waves) per workgroup: one, so that the LDS a wave needs (29 KB at 128 / 128) is the whole
// allocation unit and five waves share a CU (two per workgroup fitted four).  The register budget is
// sized for two waves per SIMD: left free, the compiler took 316 registers at 128 / 128 (one wave per
// SIMD, four per CU); within 256 it needs 176-224 and spills none.
constexpr int kLBWaves = 1;



// ROWS: rows held per tile, 32 or (for m <= 24) 24.  The MFMAs take 32 rows of a tile; with 24 tile rows
// their reads of rows 24..31 land in the first 8 rows of the next tile (q -> kr -> dz / dv, all 16-bit, so
// finite) or, past the last, in a zeroed pad, and those rows only ever meet zero factors (attention rows
// and columns past m).  The row-store patches (fp32 / 16-bit words, kEpiPatchBytes) therefore go where no
// later read lands: see the ALIAS-marked stores.  Built for the 128-wide tiles (6 KB, each holding a patch),
// where the smaller tiles let six waves share a CU instead of five.
template <int D, int DV, bool LAST, int ROWS>
struct LBLds {
  static constexpr int QT = ROWS * D * 2;                 // q rows i
  static constexpr int KT = ROWS * D * 2;                 // kr rows k
  static constexpr int GT = LAST ? ROWS * DV * 2 : 0;     // dz rows i
  static constexpr int VT = LAST ? 0 : ROWS * D * 2;      // dv rows k
  static constexpr int PT = (32 - ROWS) * (LAST ? DV : D) * 2;   // zeroed pad after the last tile
  static constexpr int AT = 32 * kAttStride * 4;          // an m x m matrix as [k][i]
  static constexpr int ET = 32 * 4;
  static constexpr int CT = 32 * 4;
  static constexpr int PER_WAVE = QT + KT + GT + VT + PT + AT + ET + CT;   // y is read into registers
  // the aliased first 8 rows of a tile, and a patch in the rest of the dz tile
  static constexpr int ALIAS = (32 - ROWS) * D * 2;
  static_assert(ROWS == 32 || (ROWS == 24 && D == 128 && (!LAST || DV == 128)), "tile rows");
  static_assert(QT >= kEpiPatchBytes && (LAST ? GT - ALIAS >= kEpiPatchBytes : VT >= kEpiPatchBytes), "patch room");
};
template <int D, int DV, bool LAST>
constexpr bool lbwd_rows24() { return D == 128 && (!LAST || DV == 128); }

template <bool F16, int D, int DV, bool LAST, int ROWS>
__global__ __launch_bounds__(64 * kLBWaves, 2) void lstep_bwd_kernel(LBParams p) {
  using E = Elem<F16>;
  using T = typename E::T;
  using V8 = typename E::V8;
  using V4 = typename E::V4;
  using LL = LBLds<D, DV, LAST, ROWS>;
  constexpr int ND = D / 32;
  constexpr int NV = DV / 32;

  extern __shared__ __attribute__((aligned(1024))) char smem_raw[];
  auto uni = [](int x) __attribute__((always_inline)) { return __builtin_amdgcn_readfirstlane(x); };
  const int tid = threadIdx.x, wave = uni(tid >> 6), lane = tid & 63, hl = lane >> 5, l32 = lane & 31;
  const bool live = blockIdx.x * kLBWaves + wave < p.cols_total;   // tail waves compute, never store
  const int col = live ? blockIdx.x * kLBWaves + wave : p.cols_total - 1;   // (wave-uniform, as lstep_kernel)
  VMO_LDS char* q_t = (VMO_LDS char*)smem_raw + wave * LL::PER_WAVE;
  VMO_LDS char* k_t = q_t + LL::QT;
  VMO_LDS char* g_t = k_t + LL::KT;
  VMO_LDS char* v_t = g_t + LL::GT;
  VMO_LDS char* pad = v_t + LL::VT;
  VMO_LDS float* att = (VMO_LDS float*)(pad + LL::PT);
  VMO_LDS float* e_t = att + 32 * kAttStride;
  VMO_LDS float* c_t = e_t + 32;

  const int bh = uni(col / p.bs), j = uni(col % p.bs);
  const int hh = uni(bh % p.heads), bb = uni(bh / p.heads);
  const int m = p.m;
  const int64_t q_rs = (int64_t)p.bs * p.q_sn;
  const int64_t o_rs = (int64_t)p.bs * p.out_sn;
  const int64_t g_rs = (int64_t)p.bs * p.g_sn;
  const T* qcol = (const T*)p.q + bb * p.q_sb + hh * p.q_sh + (int64_t)j * p.q_sn;
  const T* ocol = (const T*)p.out + bb * p.out_sb + hh * p.out_sh + (int64_t)j * p.out_sn;
  const T* gcol = (const T*)p.g + bb * p.g_sb + hh * p.g_sh + (int64_t)j * p.g_sn;

  stage_col_rows<T, D, ROWS>(qcol, q_rs, m, q_t, lane);
  stage_col_rows<T, D, ROWS>(ocol, o_rs, m, k_t, lane);
  if constexpr (LAST)
    stage_col_rows<T, DV, ROWS>(gcol, g_rs, m, g_t, lane);
  else   // du rows k, into the dv tile: each lane turns its du values into dv in place
    stage_col_rows<T, D, ROWS>(gcol, g_rs, m, v_t, lane);
  for (int o = lane * 16; o < LL::PT; o += 64 * 16) *(VMO_LDS i32x4*)(pad + o) = i32x4{0, 0, 0, 0};
  const int rk = l32 < m ? l32 : m - 1;
  V8 krf[D / 16], yf[LAST ? DV / 16 : 1];   // kr and y rows k (lane = k) as MFMA operands
  {
    const T* kp = ocol + (int64_t)rk * o_rs + hl * 8;
#pragma unroll
    for (int ds = 0; ds < D / 16; ++ds) krf[ds] = *(const V8*)(kp + ds * 16);
    if constexpr (LAST) {
#pragma unroll
      for (int ds = 0; ds < DV / 16; ++ds) yf[ds] = *(const V8*)(kp + D + ds * 16);
    }
  }
  if (hl == 0) {
    const float* ep = p.ent + bb * p.ent_sb + hh * p.ent_sh + j;
    e_t[l32] = l32 < m ? ep[(int64_t)l32 * p.bs] * kLog2e : -1.0e30f;
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  // Non-last steps add to dq (the last one overwrites it): its fp32 rows are loaded now, in the layout of
  // the final store (lane: rows rr0 + 8 i, 4 columns at 32 a + 4 c), so that the read's latency hides
  // behind the whole column's work instead of stalling that store.  (The last step keeps the generic
  // store: these 64 registers would spill its operands.)
  float* const dq0 = p.dq + bb * p.dq_sb + hh * p.dq_sh + (int64_t)j * p.dq_sn;
  const int64_t dq_rs = (int64_t)p.bs * p.dq_sn;
  constexpr int DQ_RG = ROWS / 8;   // row groups that can hold rows < m
  f32x4 dq_pre[LAST ? 1 : ND][DQ_RG];
  if constexpr (!LAST) {
    const bool dq_add = !p.dq_overwrite;
#pragma unroll
    for (int a = 0; a < ND; ++a)
#pragma unroll
      for (int i = 0; i < DQ_RG; ++i) {
        const int rr = (lane >> 3) + 8 * i;
        dq_pre[a][i] = (dq_add && live && rr < m) ? *(const f32x4*)(dq0 + rr * dq_rs + 32 * a + 4 * (lane & 7))
                                                 : f32x4{0.f, 0.f, 0.f, 0.f};
      }
  }
  if constexpr (LAST) {
    // z rows of tokens < skip are overwritten by the recompute: no gradient reaches the L-path
    constexpr int CH = DV / 8;
    for (int idx = lane; idx < ROWS * CH; idx += 64) {
      const int r = idx / CH;
      if (r * p.bs + j < p.skip) *(VMO_LDS i32x4*)(g_t + r * (DV * 2) + (idx % CH) * 16) = i32x4{0, 0, 0, 0};
    }
    __syncthreads();
  }

  // ---- attn^T[k][i] (lane: query row i = l32, keys k = 8(r/4) + 4 hl + r%4), as lstep_kernel
  const VMO_LDS char* qrow = q_t + l32 * (D * 2);
  const int sw = swz(l32);
  f32x16 s = f32x16{};
#pragma unroll
  for (int ds = 0; ds < D / 16; ++ds) s = E::mfma(krf[ds], lds_read8<V8>(qrow + ((2 * ds + hl) ^ sw) * 16), s);
  float mx = -3.0e38f;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const f32x4 ev = *(const VMO_LDS f32x4*)(e_t + 8 * g + 4 * hl);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int r = 4 * g + e;
      s[r] = fmaf(s[r], p.logit_scale_log2, ev[e]);
      mx = fmaxf(mx, s[r]);
    }
  }
  mx = wave_max32(mx);
  float sum = 0.f;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    s[r] = fast_exp2(s[r] - mx);
    sum += s[r];
  }
  const float inv = 1.0f / wave_sum32(sum);
#pragma unroll
  for (int r = 0; r < 16; ++r) s[r] *= inv;

  const bool ivalid = l32 < m;
  const int tchunk = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
  const int tbyte = (lane & 1) * 8;
  const int tj = (lane & 15) >> 2;
  const int trow = 4 * hl + tj;
  const int tsw = swz(trow);
  const int k = l32;   // the lane's key in the one-lane-per-k products
  const bool kvalid = k < m;
  const int ksw = swz(k);

  // m x m matrix (accumulator layout, rows k) -> att[k][i]; rows i >= m written as zero
  auto to_att = [&](const f32x16& x) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < 16; ++r) att[(8 * (r >> 2) + 4 * hl + (r & 3)) * kAttStride + l32] = ivalid ? x[r] : 0.f;
  };
  // B operand x[i][k] for i = 16 is + 8 hl + 0..7, from att row k (one lane per k)
  auto att_rows = [&](V8 (&B)[2], float* colsum) __attribute__((always_inline)) {
    float cs = 0.f;
#pragma unroll
    for (int is = 0; is < 2; ++is) {
      const VMO_LDS float* ap = att + k * kAttStride + 16 * is + 8 * hl;
      const f32x4 x0 = *(const VMO_LDS f32x4*)ap;
      const f32x4 x1 = *(const VMO_LDS f32x4*)(ap + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        B[is][e] = to_elem<T>(x0[e]);
        B[is][4 + e] = to_elem<T>(x1[e]);
        cs += x0[e] + x1[e];
      }
    }
    if (colsum) *colsum = wave_sum32(cs);
  };
  // acc^T[w][k] += sum_i tile^T[w][i] B[i][k] for a row-major [i][w] LDS tile (transposed reads)
  auto mma_rows_t = [&](f32x16* acc, const VMO_LDS char* tile, auto width_tag, const V8 (&B)[2])
      __attribute__((always_inline)) {
    constexpr int W = decltype(width_tag)::value;
#pragma unroll
    for (int a = 0; a < W / 32; ++a)
#pragma unroll
      for (int is = 0; is < 2; ++is) {
        const int row0 = 16 * is + 8 * hl + tj;
        const VMO_LDS char* r0 = tile + row0 * (W * 2) + ((4 * a + tchunk) ^ (2 * tj)) * 16 + tbyte;
        const VMO_LDS char* r1 = tile + (row0 + 4) * (W * 2) + ((4 * a + tchunk) ^ (2 * tj + 1)) * 16 + tbyte;
        acc[a] = E::mfma(lds_read_tr8<V8>(r0, r1), B[is], acc[a]);
      }
  };
  // acc^T[w][i] += sum_k tile^T[w][k] x^T[k][i] for a row-major [k][w] LDS tile and x in the
  // accumulator layout (its 4-key groups are the transposed reads' row groups)
  auto mma_acc_t = [&](f32x16* acc, const VMO_LDS char* tile, const f32x16& x) __attribute__((always_inline)) {
    V8 P[2];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      P[0][e] = to_elem<T>(x[e]);
      P[1][e] = to_elem<T>(x[8 + e]);
    }
#pragma unroll
    for (int a = 0; a < D / 32; ++a) {
      const int coff = ((4 * a + tchunk) ^ tsw) * 16 + tbyte;
#pragma unroll
      for (int ss = 0; ss < 2; ++ss) {
        const VMO_LDS char* r0 = tile + (16 * ss + trow) * (D * 2) + coff;
        acc[a] = E::mfma(lds_read_tr8<V8>(r0, r0 + 8 * D * 2), P[ss], acc[a]);
      }
    }
  };
  T* const dcol = (T*)p.dout + bb * p.do_sb + hh * p.do_sh + (int64_t)j * p.do_sn;
  const int64_t do_rs = (int64_t)p.bs * p.do_sn;

  // delta_k = sum_f out[k][f] d out[k][f] (p.delta): d out's accumulator blocks (lane (k, hl): features 32 a +
  // 8 g + 4 hl + 0..3), rounded as they are stored, against out's row k held as MFMA operands (features
  // 16 ds + 8 hl + 0..7).  Two permlane32 swaps per operand trade the middle 4-feature groups between the
  // halves, so that lane (k, hl) holds features 16 ds + 4 hl + 0..3 (X) and 16 ds + 8 + 4 hl + 0..3 (Y):
  // groups g = 2 (ds % 2) and 2 (ds % 2) + 1 of block ds / 2.
  auto row_dot = [&](const V8* rowf, const f32x16* acc, auto nblocks_tag) __attribute__((always_inline)) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    using V2 = typename E::V2;
    float d = 0.f;
#pragma unroll
    for (int ds = 0; ds < 2 * decltype(nblocks_tag)::value; ++ds) {
      const u32x4 w = __builtin_bit_cast(u32x4, rowf[ds]);
      const auto s0 = __builtin_amdgcn_permlane32_swap(w[0], w[2], false, false);
      const auto s1 = __builtin_amdgcn_permlane32_swap(w[1], w[3], false, false);
      const uint32_t xy[4] = {s0[0], s1[0], s0[1], s1[1]};   // X: accumulator rows r0 .. r0+3, Y: r0+4 .. r0+7
      const int r0 = 8 * (ds & 1);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const V2 x = __builtin_bit_cast(V2, xy[u]);
        d = fmaf((float)to_elem<T>(acc[ds >> 1][r0 + 2 * u]), (float)x[0], d);
        d = fmaf((float)to_elem<T>(acc[ds >> 1][r0 + 2 * u + 1]), (float)x[1], d);
      }
    }
    return d;
  };
  float dlt = 0.f;

  // ---- d attn^T[k][i]
  f32x16 da = f32x16{};
  if constexpr (LAST) {
    const VMO_LDS char* grow = g_t + l32 * (DV * 2);
#pragma unroll
    for (int ds = 0; ds < DV / 16; ++ds) {
      const int off = ((2 * ds + hl) ^ sw) * 16;
      da = E::mfma(yf[ds], lds_read8<V8>(grow + off), da);
    }
    // dy_k = sum_i a[i,k] dz_i -> d out[k, D:]
    to_att(s);
    __syncthreads();
    V8 Bu[2];
    att_rows(Bu, nullptr);
    f32x16 accy[NV];
#pragma unroll
    for (int a = 0; a < NV; ++a) accy[a] = f32x16{};
    mma_rows_t(accy, g_t, std::integral_constant<int, DV>{}, Bu);
    if (p.delta) dlt = row_dot(yf, accy, std::integral_constant<int, NV>{});
    // the dz tile is dead now: it takes the row-store patch (whole row segments per store), past its first
    // rows, which the kr tile's reads of rows ROWS.. still land in (ALIAS)
    if (live)
      store_acc_rows<F16>((VMO_LDS float*)(g_t + LL::ALIAS), accy, NV, 1.f, kGradStore, (char*)(dcol + D), do_rs * 2,
                          m, lane);
  } else {
    to_att(s);
    __syncthreads();
    V8 Bu[2];
    float cs;
    att_rows(Bu, &cs);
    f32x16 accv[ND];   // v^T[d][k] = sum_i q^T[d][i] a[i][k]
#pragma unroll
    for (int a = 0; a < ND; ++a) accv[a] = f32x16{};
    mma_rows_t(accv, q_t, std::integral_constant<int, D>{}, Bu);
    const float cm = fmaxf(cs, p.min_col_mass);
    const float f = p.scale / cm;
    float df = 0.f;
#pragma unroll
    for (int a = 0; a < ND; ++a)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        VMO_LDS V4* dvp = (VMO_LDS V4*)(v_t + k * (D * 2) + ((4 * a + g) ^ ksw) * 16 + hl * 8);
        const V4 d4 = *dvp;   // du[k][32 a + 8 g + 4 hl + 0..3], staged by stage_col_rows' swizzle
        V4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float du = kvalid ? (float)d4[e] : 0.f;
          df = fmaf(du, accv[a][4 * g + e], df);
          w[e] = to_elem<T>(du * f);
        }
        *dvp = w;   // rows k >= ROWS: the pad, which stays zero (du = 0 there)
      }
    df = wave_sum32(df);
    if (hl == 0) c_t[k] = (kvalid && cs >= p.min_col_mass) ? -df * f / cm : 0.f;
    __syncthreads();
    const VMO_LDS char* vrow = v_t + l32 * (D * 2);
#pragma unroll
    for (int ds = 0; ds < D / 16; ++ds) {
      const int off = ((2 * ds + hl) ^ sw) * 16;
      da = E::mfma(lds_read8<V8>(vrow + off), lds_read8<V8>(qrow + off), da);
    }
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const f32x4 cv = *(const VMO_LDS f32x4*)(c_t + 8 * g + 4 * hl);
#pragma unroll
      for (int e = 0; e < 4; ++e) da[4 * g + e] += cv[e];
    }
  }

  // ---- softmax backward: dL = scale a (da - sum_k a da)
  float rs = 0.f;
#pragma unroll
  for (int r = 0; r < 16; ++r) rs = fmaf(s[r], da[r], rs);
  rs = wave_sum32(rs);
  f32x16 dl;
#pragma unroll
  for (int r = 0; r < 16; ++r) dl[r] = ivalid ? p.scale * s[r] * (da[r] - rs) : 0.f;

  // ---- dq_i += sum_k dL[i,k] kr_k (+ sum_k a[i,k] dv_k): fp32 read-modify-write (or store)
  {
    f32x16 accq[ND];
#pragma unroll
    for (int a = 0; a < ND; ++a) accq[a] = f32x16{};
    mma_acc_t(accq, k_t, dl);
    if constexpr (!LAST) mma_acc_t(accq, v_t, s);
    // the dz (dv) tile is dead now and takes the row-store patch: not the kr tile, whose first rows the q
    // tile's reads of rows ROWS.. still land in (ALIAS)
    if (LAST && live) {
      store_acc_rows<F16>((VMO_LDS float*)g_t, accq, ND, 1.f, p.dq_overwrite ? kGradStoreF32 : kGradAddF32,
                          (char*)dq0, dq_rs * 4, m, lane);
    } else if (live) {   // dq_pre holds the rows added to
      VMO_LDS float* patch = (VMO_LDS float*)v_t;
      const int rr0 = lane >> 3, c = lane & 7;
#pragma unroll
      for (int a = 0; a < ND; ++a) {
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {   // row l32, 16-byte chunk 2 jj + hl, swizzled by row
          f32x4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = accq[a][4 * jj + e];
          *(VMO_LDS f32x4*)(patch + l32 * 32 + ((2 * jj + hl) ^ (l32 & 7)) * 4) = v;
        }
#pragma unroll
        for (int i = 0; i < DQ_RG; ++i) {   // rows rr0 + 8 i, chunk c: 8 lanes per row
          const int rr = rr0 + 8 * i;
          const f32x4 v = *(const VMO_LDS f32x4*)(patch + rr * 32 + (c ^ (rr & 7)) * 4);
          if (rr < m) *(f32x4*)(dq0 + rr * dq_rs + 32 * a + 4 * c) = v + dq_pre[LAST ? 0 : a][i];
        }
      }
    }
  }

  // ---- dkr_k = sum_i dL[i,k] q_i -> d out[k, :D]
  __syncthreads();   // every lane's reads of att are done
  to_att(dl);
  __syncthreads();
  {
    V8 Bd[2];
    att_rows(Bd, nullptr);
    f32x16 acck[ND];
#pragma unroll
    for (int a = 0; a < ND; ++a) acck[a] = f32x16{};
    mma_rows_t(acck, q_t, std::integral_constant<int, D>{}, Bd);
    if (p.delta) {
      dlt = wave_sum32(dlt + row_dot(krf, acck, std::integral_constant<int, ND>{}));
      if (live && kvalid && hl == 0) p.delta[bb * p.dl_sb + hh * p.dl_sh + (int64_t)k * p.bs + j] = dlt;
    }
    if (live)   // the q tile is dead now: it takes the row-store patch
      store_acc_rows<F16>((VMO_LDS float*)q_t, acck, ND, 1.f, kGradStore, (char*)dcol, do_rs * 2, m, lane);
  }
}

template <bool F16, int D, int DV, bool LAST, int ROWS>
static int launch_lstep_bwd(const LBParams& p, hipStream_t s) {
  constexpr int LDS = LBLds<D, DV, LAST, ROWS>::PER_WAVE * kLBWaves;
  static_assert(LDS <= 160 * 1024, "lstep_bwd LDS");
  auto kern = lstep_bwd_kernel<F16, D, DV, LAST, ROWS>;
  if (LDS > 65536) {
    static bool done = false;   // attribute is per function; idempotent, so a benign race
    if (!done) {
      if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, LDS) != hipSuccess)
        return set_error(VMO_ERR_LAUNCH, "lstep_bwd: cannot raise the LDS limit to %d bytes", LDS);
      done = true;
    }
  }
  const int wgs = (p.cols_total + kLBWaves - 1) / kLBWaves;
  hipLaunchKernelGGL(kern, dim3(wgs), dim3(64 * kLBWaves), LDS, s, p);
  return launch_status("lstep_bwd");
}

template <bool F16>
static int dispatch_lstep_bwd(const LBParams& p, int d, int dv, bool last, hipStream_t s) {
#define VMO_LB(D_, DV_, LAST_)                                        \
  if (d == D_ && (!LAST_ || dv == DV_) && last == LAST_)              \
    return p.m <= 24 && lbwd_rows24<D_, DV_, LAST_>()                 \
               ? launch_lstep_bwd<F16, D_, DV_, LAST_, lbwd_rows24<D_, DV_, LAST_>() ? 24 : 32>(p, s) \
               : launch_lstep_bwd<F16, D_, DV_, LAST_, 32>(p, s);
  VMO_LB(64, 64, false)
  VMO_LB(128, 128, false)
  VMO_LB(64, 64, true)
  VMO_LB(64, 128, true)
  VMO_LB(128, 64, true)
  VMO_LB(128, 128, true)
#undef VMO_LB
  return set_error(VMO_ERR_UNSUPPORTED, "lstep_bwd: no kernel for d=%d dv=%d last=%d", d, dv, (int)last);
}

// Head dims the one-tile kernels are built for (with m <= 32).
static bool one_tile_built(int d, int dv, bool last) {
  return (d == 64 || d == 128) && (!last || dv == 64 || dv == 128);
}

// ---------------------------------------------------------------------------------------------
// General L-step, forward and backward, for the grids the one-tile kernels above do not cover:
// more than 32 frames (m > 32: HunyuanVideo's 129 frames give 33 latent frames) or head dims other
// than 64 / 128.  Same mathematics and the same rounding points as the one-tile kernels (logits in
// fp32 from the 16-bit q and kr, attn rounded to the 16-bit type where it multiplies q or y, the
// column mass from the fp32 attn; u / z / d out rounded once when stored), but one 256-thread
// workgroup per grid column with the column's rows staged in LDS and the m x m products on the
// vector unit in fp32: a column is small (m x D values), so the L2-resident rows are read once and
// every product is an LDS sweep.  LDS rows are padded by 16 bytes, so that the 16 rows a wave reads
// at one feature offset fall on 16 distinct bank groups.  Supported: any m whose tiles fit the CU's
// 160 KB (m <= 64 for every head dim up to 128), d and dv multiples of 8 up to 256.
constexpr int kLWThreads = 256;

struct LWLayout {   // byte offsets of the per-column LDS arrays
  int ldq, ldy, ldm;                 // row strides: 16-bit rows (elements), fp32 m x m matrices (floats)
  int q, k, g, y, a, b, vec, total;  // q rows, kr rows, upstream gradient rows, y rows, two m x m, vectors
};

__host__ __device__ inline LWLayout lw_layout(int m, int d, int dv, bool last, bool bwd) {
  LWLayout L;
  L.ldq = d + 8;
  L.ldy = dv + 8;
  L.ldm = m + 1;
  int off = 0;
  auto take = [&](int bytes) { const int o = off; off += (bytes + 15) / 16 * 16; return o; };
  L.q = take(m * L.ldq * 2);
  L.k = take(m * L.ldq * 2);
  L.g = bwd ? take(m * (last ? L.ldy : L.ldq) * 2) : 0;
  L.y = last ? take(m * L.ldy * 2) : 0;
  L.a = take(m * L.ldm * 4);
  L.b = bwd ? take(m * L.ldm * 4) : 0;
  L.vec = take(4 * m * 4);
  L.total = off;
  return L;
}

// rows r < m of F 16-bit values (F % 8 == 0), global row stride rs (elements) -> LDS stride ld
template <class T>
__device__ __forceinline__ void lw_stage(VMO_LDS T* dst, int ld, const T* src, int64_t rs, int m, int F, int tid) {
  const int ch = F / 8;
  for (int idx = tid; idx < m * ch; idx += kLWThreads) {
    const int r = idx / ch, c = idx % ch;
    *(VMO_LDS i32x4*)(dst + r * ld + 8 * c) = *(const i32x4*)(src + r * rs + 8 * c);
  }
}

template <class V8>
__device__ __forceinline__ float lw_dot8(const V8& a, const V8& b, float acc) {
#pragma unroll
  for (int e = 0; e < 8; ++e) acc = fmaf((float)a[e], (float)b[e], acc);
  return acc;
}

// out[r * ldo + s] = sum_f A[r][f] B[s][f] over F features, r, s < m (rows r: 64 per pass, 4 threads
// each; a thread takes s = s0 + 4 u, u < 16: its A row chunk is read once per 16 products)
template <bool F16>
__device__ __forceinline__ void lw_dots(VMO_LDS float* out, int ldo, const VMO_LDS typename Elem<F16>::T* A, int lda,
                                        const VMO_LDS typename Elem<F16>::T* B, int ldb, int m, int F, int tid) {
  using V8 = typename Elem<F16>::V8;
  for (int r0 = 0; r0 < m; r0 += 64) {
    const int r = r0 + (tid >> 2);
    if (r >= m) continue;
    for (int s0 = tid & 3; s0 < m; s0 += 64) {
      float acc[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) acc[u] = 0.f;
      for (int f = 0; f < F; f += 8) {
        const V8 a = *(const VMO_LDS V8*)(A + r * lda + f);
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          const int s = min(s0 + 4 * u, m - 1);
          const V8 b = *(const VMO_LDS V8*)(B + s * ldb + f);
          acc[u] = lw_dot8(a, b, acc[u]);
        }
      }
#pragma unroll
      for (int u = 0; u < 16; ++u)
        if (s0 + 4 * u < m) out[r * ldo + s0 + 4 * u] = acc[u];
    }
  }
}

// For every output row r < m and 8-column group fb < F / 8 (4 threads per row, 64 rows per pass):
// acc[e] = sum_s w(r, s) X[s][8 fb + e] (+ the same for a second weight / row set), then emit(r, fb, acc).
template <bool F16, class W, class Emit>
__device__ __forceinline__ void lw_mix(W w, const VMO_LDS typename Elem<F16>::T* X, int ldx, int m, int F, int tid,
                                       Emit emit) {
  using V8 = typename Elem<F16>::V8;
  for (int r0 = 0; r0 < m; r0 += 64) {
    const int r = r0 + (tid >> 2);
    if (r >= m) continue;
    for (int fb = tid & 3; fb < F / 8; fb += 4) {
      float acc[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = 0.f;
      for (int s = 0; s < m; ++s) {
        const float ws = w(r, s);
        const V8 x = *(const VMO_LDS V8*)(X + s * ldx + 8 * fb);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = fmaf(ws, (float)x[e], acc[e]);
      }
      emit(r, fb, acc);
    }
  }
}

template <bool F16>
__device__ __forceinline__ void lw_store8(typename Elem<F16>::T* dst, const float (&x)[8], float f) {
  using V8 = typename Elem<F16>::V8;
  V8 v;
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = to_elem<typename Elem<F16>::T>(x[e] * f);
  *(V8*)dst = v;
}

// attn[i][k] = softmax_k(logit[i][k] * scale * log2 e + ent[k] log2 e) in place, one thread per row i
__device__ __forceinline__ void lw_softmax_rows(VMO_LDS float* A, int ldm, const VMO_LDS float* ev, int m, float c,
                                                int tid) {
  for (int i = tid; i < m; i += kLWThreads) {
    VMO_LDS float* row = A + i * ldm;
    float mx = -3.0e38f;
    for (int k = 0; k < m; ++k) {
      const float x = fmaf(row[k], c, ev[k]);
      row[k] = x;
      mx = fmaxf(mx, x);
    }
    float sum = 0.f;
    for (int k = 0; k < m; ++k) {
      const float e = fast_exp2(row[k] - mx);
      row[k] = e;
      sum += e;
    }
    const float inv = 1.0f / sum;
    for (int k = 0; k < m; ++k) row[k] *= inv;
  }
}

template <bool F16, bool LAST>
__global__ __launch_bounds__(kLWThreads) void lstep_wide_kernel(LParams p) {
  using T = typename Elem<F16>::T;
  extern __shared__ __attribute__((aligned(16))) char smem_raw[];
  VMO_LDS char* sm = (VMO_LDS char*)smem_raw;
  const int m = p.m, D = p.d, DV = p.dv, tid = threadIdx.x;
  const LWLayout L = lw_layout(m, D, DV, LAST, false);
  VMO_LDS T* qs = (VMO_LDS T*)(sm + L.q);
  VMO_LDS T* ks = (VMO_LDS T*)(sm + L.k);
  VMO_LDS T* ys = (VMO_LDS T*)(sm + L.y);
  VMO_LDS float* A = (VMO_LDS float*)(sm + L.a);
  VMO_LDS float* ev = (VMO_LDS float*)(sm + L.vec);
  VMO_LDS float* fk = ev + m;

  const int col = blockIdx.x, bh = col / p.bs, j = col % p.bs, hh = bh % p.heads, bb = bh / p.heads;
  const T* qcol = (const T*)p.q + bb * p.q_sb + hh * p.q_sh + (int64_t)j * p.q_sn;
  const T* ocol = (const T*)p.out + bb * p.out_sb + hh * p.out_sh + (int64_t)j * p.out_sn;
  lw_stage<T>(qs, L.ldq, qcol, (int64_t)p.bs * p.q_sn, m, D, tid);
  lw_stage<T>(ks, L.ldq, ocol, (int64_t)p.bs * p.out_sn, m, D, tid);
  if constexpr (LAST) lw_stage<T>(ys, L.ldy, ocol + D, (int64_t)p.bs * p.out_sn, m, DV, tid);
  const float* ep = p.ent + bb * p.ent_sb + hh * p.ent_sh + j;
  for (int k = tid; k < m; k += kLWThreads) ev[k] = ep[(int64_t)k * p.bs] * kLog2e;
  __syncthreads();
  lw_dots<F16>(A, L.ldm, qs, L.ldq, ks, L.ldq, m, D, tid);   // q_i . kr_k
  __syncthreads();
  lw_softmax_rows(A, L.ldm, ev, m, p.logit_scale_log2, tid);
  __syncthreads();
  T* rcol = (T*)p.res + bb * p.res_sb + hh * p.res_sh + (int64_t)j * p.res_sn;
  const int64_t rrs = (int64_t)p.bs * p.res_sn;
  auto rounded = [](float x) { return (float)to_elem<T>(x); };   // attn as the 16-bit operand
  if constexpr (LAST) {
    // z_i = sum_k attn[i][k] y_k, rows whose token the recompute owns left alone
    lw_mix<F16>([&](int i, int k) { return rounded(A[i * L.ldm + k]); }, ys, L.ldy, m, DV, tid,
                [&](int i, int fb, const float (&acc)[8]) {
                  if ((int64_t)i * p.bs + j >= p.skip) lw_store8<F16>(rcol + i * rrs + 8 * fb, acc, 1.f);
                });
  } else {
    // u_k = scale / max(sum_i attn[i][k], min_col_mass) * sum_i attn[i][k] q_i
    for (int k = tid; k < m; k += kLWThreads) {
      float c = 0.f;
      for (int i = 0; i < m; ++i) c += A[i * L.ldm + k];
      fk[k] = p.scale / fmaxf(c, p.min_col_mass);
    }
    __syncthreads();
    lw_mix<F16>([&](int k, int i) { return rounded(A[i * L.ldm + k]); }, qs, L.ldq, m, D, tid,
                [&](int k, int fb, const float (&acc)[8]) { lw_store8<F16>(rcol + k * rrs + 8 * fb, acc, fk[k]); });
  }
}

// Backward of the general L-step (same mathematics as lstep_bwd_kernel, fp32 products).  With
// G[k][i] = g_k . q_i (non-last), the column-mass terms need no v_k = sum_i a[i,k] q_i of their own:
// g_k . v_k = sum_i a[i,k] G[k][i] and dv_k . q_i = f_k G[k][i].
template <bool F16, bool LAST>
__global__ __launch_bounds__(kLWThreads) void lstep_wide_bwd_kernel(LBParams p) {
  using T = typename Elem<F16>::T;
  extern __shared__ __attribute__((aligned(16))) char smem_raw[];
  VMO_LDS char* sm = (VMO_LDS char*)smem_raw;
  const int m = p.m, D = p.d, DV = p.dv, tid = threadIdx.x;
  const LWLayout L = lw_layout(m, D, DV, LAST, true);
  VMO_LDS T* qs = (VMO_LDS T*)(sm + L.q);
  VMO_LDS T* ks = (VMO_LDS T*)(sm + L.k);
  VMO_LDS T* gs = (VMO_LDS T*)(sm + L.g);
  VMO_LDS T* ys = (VMO_LDS T*)(sm + L.y);
  VMO_LDS float* A = (VMO_LDS float*)(sm + L.a);   // attn[i][k]
  VMO_LDS float* Bm = (VMO_LDS float*)(sm + L.b);  // d attn[i][k], then dL[i][k]
  VMO_LDS float* ev = (VMO_LDS float*)(sm + L.vec);
  VMO_LDS float* fk = ev + m;    // f_k = scale / cm_k (non-last)
  VMO_LDS float* dck = fk + m;   // dc_k (non-last)
  VMO_LDS float* rsi = dck + m;  // sum_k a[i,k] da[i,k]
  const int gw = LAST ? DV : D, ldg = LAST ? L.ldy : L.ldq;

  const int col = blockIdx.x, bh = col / p.bs, j = col % p.bs, hh = bh % p.heads, bb = bh / p.heads;
  const T* qcol = (const T*)p.q + bb * p.q_sb + hh * p.q_sh + (int64_t)j * p.q_sn;
  const T* ocol = (const T*)p.out + bb * p.out_sb + hh * p.out_sh + (int64_t)j * p.out_sn;
  const T* gcol = (const T*)p.g + bb * p.g_sb + hh * p.g_sh + (int64_t)j * p.g_sn;
  lw_stage<T>(qs, L.ldq, qcol, (int64_t)p.bs * p.q_sn, m, D, tid);
  lw_stage<T>(ks, L.ldq, ocol, (int64_t)p.bs * p.out_sn, m, D, tid);
  lw_stage<T>(gs, ldg, gcol, (int64_t)p.bs * p.g_sn, m, gw, tid);
  if constexpr (LAST) lw_stage<T>(ys, L.ldy, ocol + D, (int64_t)p.bs * p.out_sn, m, DV, tid);
  const float* ep = p.ent + bb * p.ent_sb + hh * p.ent_sh + j;
  for (int k = tid; k < m; k += kLWThreads) ev[k] = ep[(int64_t)k * p.bs] * kLog2e;
  __syncthreads();
  if constexpr (LAST) {   // z rows of tokens < skip are the recompute's: no gradient reaches the L-path
    for (int idx = tid; idx < m * (DV / 8); idx += kLWThreads) {
      const int r = idx / (DV / 8);
      if ((int64_t)r * p.bs + j < p.skip) *(VMO_LDS i32x4*)(gs + r * ldg + 8 * (idx % (DV / 8))) = i32x4{0, 0, 0, 0};
    }
    __syncthreads();
  }
  lw_dots<F16>(A, L.ldm, qs, L.ldq, ks, L.ldq, m, D, tid);
  if constexpr (LAST)
    lw_dots<F16>(Bm, L.ldm, gs, ldg, ys, L.ldy, m, DV, tid);   // d attn[i][k] = g_i . y_k
  else
    lw_dots<F16>(Bm, L.ldm, gs, ldg, qs, L.ldq, m, D, tid);    // G[k][i] = g_k . q_i (rows k)
  __syncthreads();
  lw_softmax_rows(A, L.ldm, ev, m, p.logit_scale_log2, tid);
  __syncthreads();
  T* dcol = (T*)p.dout + bb * p.do_sb + hh * p.do_sh + (int64_t)j * p.do_sn;
  const int64_t drs = (int64_t)p.bs * p.do_sn;
  if constexpr (LAST) {
    // dy_k = sum_i a[i,k] g_i -> d out[k, D:]
    lw_mix<F16>([&](int k, int i) { return A[i * L.ldm + k]; }, gs, ldg, m, DV, tid,
                [&](int k, int fb, const float (&acc)[8]) { lw_store8<F16>(dcol + k * drs + D + 8 * fb, acc, 1.f); });
  } else {
    for (int k = tid; k < m; k += kLWThreads) {
      float c = 0.f, df = 0.f;
      for (int i = 0; i < m; ++i) {
        const float a = A[i * L.ldm + k];
        c += a;
        df = fmaf(a, Bm[k * L.ldm + i], df);   // g_k . v_k
      }
      const float cm = fmaxf(c, p.min_col_mass), f = p.scale / cm;
      fk[k] = f;
      dck[k] = c >= p.min_col_mass ? -df * f / cm : 0.f;
    }
    __syncthreads();
  }
  // softmax backward, row i: rs_i = sum_k a[i,k] da[i,k]; dL[i,k] = scale a[i,k] (da[i,k] - rs_i)
  // (non-last: da[i,k] = f_k G[k][i] + dc_k, read from the rows-k matrix)
  auto da_of = [&](int i, int k) {
    return LAST ? Bm[i * L.ldm + k] : fmaf(fk[k], Bm[k * L.ldm + i], dck[k]);
  };
  for (int i = tid; i < m; i += kLWThreads) {
    float rs = 0.f;
    for (int k = 0; k < m; ++k) rs = fmaf(A[i * L.ldm + k], da_of(i, k), rs);
    rsi[i] = rs;
  }
  __syncthreads();
  // dL in place of da: LAST rows i are each written by their own thread after their reads; the
  // non-last matrix is indexed [k][i], so every thread computes its dL row into registers first
  if constexpr (LAST) {
    for (int i = tid; i < m; i += kLWThreads)
      for (int k = 0; k < m; ++k) Bm[i * L.ldm + k] = p.scale * A[i * L.ldm + k] * (Bm[i * L.ldm + k] - rsi[i]);
    __syncthreads();
  } else {
    // dL[i][k] overwrites G[k][i]: each (k, i) entry is read and written by the same thread only
    for (int idx = tid; idx < m * m; idx += kLWThreads) {
      const int k = idx / m, i = idx % m;
      const float g = Bm[k * L.ldm + i];
      Bm[k * L.ldm + i] = p.scale * A[i * L.ldm + k] * (fmaf(fk[k], g, dck[k]) - rsi[i]);
    }
    __syncthreads();
  }
  // dL[i][k] accessor over the layout in use
  auto dl_of = [&](int i, int k) { return LAST ? Bm[i * L.ldm + k] : Bm[k * L.ldm + i]; };
  // dq_i (+)= sum_k dL[i,k] kr_k (+ sum_k a[i,k] f_k g_k, non-last)
  float* dqcol = p.dq + bb * p.dq_sb + hh * p.dq_sh + (int64_t)j * p.dq_sn;
  const int64_t dqrs = (int64_t)p.bs * p.dq_sn;
  lw_mix<F16>(dl_of, ks, L.ldq, m, D, tid, [&](int i, int fb, const float (&acc)[8]) {
    float tot[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) tot[e] = acc[e];
    if constexpr (!LAST) {
      using V8 = typename Elem<F16>::V8;
      for (int k = 0; k < m; ++k) {
        const float w = A[i * L.ldm + k] * fk[k];
        const V8 x = *(const VMO_LDS V8*)(gs + k * ldg + 8 * fb);
#pragma unroll
        for (int e = 0; e < 8; ++e) tot[e] = fmaf(w, (float)x[e], tot[e]);
      }
    }
    f32x4* dst = (f32x4*)(dqcol + i * dqrs + 8 * fb);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const f32x4 v = f32x4{tot[4 * h], tot[4 * h + 1], tot[4 * h + 2], tot[4 * h + 3]};
      dst[h] = p.dq_overwrite ? v : dst[h] + v;
    }
  });
  // d kr_k = sum_i dL[i,k] q_i -> d out[k, :D]
  lw_mix<F16>([&](int k, int i) { return dl_of(i, k); }, qs, L.ldq, m, D, tid,
              [&](int k, int fb, const float (&acc)[8]) { lw_store8<F16>(dcol + k * drs + 8 * fb, acc, 1.f); });
}

constexpr int kLWMaxLds = 160 * 1024;

template <class P>
static int lw_launch(void (*kern)(P), int lds, int cols, hipStream_t s, const char* what, const P& params) {
  if (lds > 65536 && hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds) != hipSuccess)
    return set_error(VMO_ERR_LAUNCH, "%s: cannot raise the LDS limit to %d bytes", what, lds);
  hipLaunchKernelGGL(kern, dim3(cols), dim3(kLWThreads), lds, s, params);
  return launch_status(what);
}

// The general kernels take any m whose per-column tiles fit the LDS and head dims that are multiples of 8
// up to 256; VMO_OK when they can run it, else the error to report.
static int lw_check(int m, int d, int dv, bool last, bool bwd, const char* what) {
  if (d % 8 != 0 || d > 256 || (last && (dv % 8 != 0 || dv > 256 || dv <= 0)))
    return set_error(VMO_ERR_UNSUPPORTED, "%s: head dims must be multiples of 8 up to 256 (d=%d dv=%d)", what, d, dv);
  const int lds = lw_layout(m, d, dv, last, bwd).total;
  if (lds > kLWMaxLds)
    return set_error(VMO_ERR_UNSUPPORTED, "%s: %d frames with d=%d dv=%d need %d bytes of LDS per grid column (max %d)",
                     what, m, d, dv, lds, kLWMaxLds);
  return VMO_OK;
}

}  // namespace vmo

extern "C" int vmo_lstep_fwd(const vmo_lstep_args* a, void* stream) {
  using namespace vmo;
  clear_error();
  if (!a) return set_error(VMO_ERR_INVALID, "lstep: null args");
  if (a->dtype != VMO_DTYPE_BF16 && a->dtype != VMO_DTYPE_F16) return set_error(VMO_ERR_INVALID, "lstep: dtype");
  if (a->batch < 0 || a->heads < 0 || a->num_blocks < 1 || a->block_size < 1)
    return set_error(VMO_ERR_INVALID, "lstep: bad sizes");
  if ((int64_t)a->batch * a->heads == 0) return VMO_OK;
  if (!view_ok(a->q) || !view_ok(a->out) || !view_ok(a->res) || a->ent == nullptr)
    return set_error(VMO_ERR_INVALID, "lstep: tensors need 16-byte aligned rows");
  if (a->d <= 0 || (a->d % 8) != 0) return set_error(VMO_ERR_INVALID, "lstep: d");
  const bool one_tile = a->num_blocks <= 32 && one_tile_built(a->d, a->dv, a->last != 0);
  const bool multi_block = !one_tile && mb_lstep_check(a->num_blocks, a->d, a->dv, a->last != 0, false);
  if (!one_tile && !multi_block) {
    const int rc = lw_check(a->num_blocks, a->d, a->dv, a->last != 0, false, "lstep");
    if (rc != VMO_OK) return rc;
  }
  const int64_t cols = (int64_t)a->batch * a->heads * a->block_size;
  if (cols > (1ll << 30) || (int64_t)a->num_blocks * a->block_size > (1ll << 30))
    return set_error(VMO_ERR_UNSUPPORTED, "lstep: problem too large");
  LParams p{};
  p.q = a->q.data; p.out = a->out.data; p.ent = a->ent; p.res = a->res.data;
  p.q_sb = a->q.stride_b; p.q_sh = a->q.stride_h; p.q_sn = a->q.stride_n;
  p.out_sb = a->out.stride_b; p.out_sh = a->out.stride_h; p.out_sn = a->out.stride_n;
  p.ent_sb = a->ent_stride_b; p.ent_sh = a->ent_stride_h;
  p.res_sb = a->res.stride_b; p.res_sh = a->res.stride_h; p.res_sn = a->res.stride_n;
  p.heads = a->heads; p.m = a->num_blocks; p.bs = a->block_size; p.skip = a->last ? a->skip_tokens : 0;
  p.cols_total = (int)cols;
  p.d = a->d;
  p.dv = a->last ? a->dv : 0;
  p.logit_scale_log2 = a->scale * kLog2e;
  p.scale = a->scale;
  p.min_col_mass = a->min_col_mass;
  hipStream_t s = (hipStream_t)stream;
  if (multi_block) return mb_lstep_fwd(p, a->dtype == VMO_DTYPE_F16, a->d, a->dv, a->last != 0, s);
  if (!one_tile) {
    const int lds = lw_layout(p.m, p.d, p.dv, a->last != 0, false).total;
    if (a->dtype == VMO_DTYPE_F16)
      return a->last ? lw_launch(lstep_wide_kernel<true, true>, lds, p.cols_total, s, "lstep_wide", p)
                     : lw_launch(lstep_wide_kernel<true, false>, lds, p.cols_total, s, "lstep_wide", p);
    return a->last ? lw_launch(lstep_wide_kernel<false, true>, lds, p.cols_total, s, "lstep_wide", p)
                   : lw_launch(lstep_wide_kernel<false, false>, lds, p.cols_total, s, "lstep_wide", p);
  }
  if (a->dtype == VMO_DTYPE_F16) return dispatch_lstep<true>(p, a->d, a->dv, a->last != 0, s);
  return dispatch_lstep<false>(p, a->d, a->dv, a->last != 0, s);
}


extern "C" int vmo_lstep_bwd(const vmo_lstep_bwd_args* a, void* stream) {
  using namespace vmo;
  clear_error();
  if (!a) return set_error(VMO_ERR_INVALID, "lstep_bwd: null args");
  if (a->dtype != VMO_DTYPE_BF16 && a->dtype != VMO_DTYPE_F16) return set_error(VMO_ERR_INVALID, "lstep_bwd: dtype");
  if (a->batch < 0 || a->heads < 0 || a->num_blocks < 1 || a->block_size < 1)
    return set_error(VMO_ERR_INVALID, "lstep_bwd: bad sizes");
  if ((int64_t)a->batch * a->heads == 0) return VMO_OK;
  if (a->d <= 0 || (a->d % 8) != 0) return set_error(VMO_ERR_INVALID, "lstep_bwd: d");
  const bool one_tile = a->num_blocks <= 32 && one_tile_built(a->d, a->dv, a->last != 0);
  const bool multi_block = !one_tile && mb_lstep_check(a->num_blocks, a->d, a->dv, a->last != 0, true);
  if (!one_tile && !multi_block) {
    const int rc = lw_check(a->num_blocks, a->d, a->dv, a->last != 0, true, "lstep_bwd");
    if (rc != VMO_OK) return rc;
  }
  if (!view_ok(a->q) || !view_ok(a->out) || !view_ok(a->grad_res) || !view_ok(a->grad_out) || a->ent == nullptr ||
      a->grad_q.data == nullptr || ((uintptr_t)a->grad_q.data & 15) != 0 || (a->grad_q.stride_n & 3) != 0 ||
      (a->grad_q.stride_h & 3) != 0 || (a->grad_q.stride_b & 3) != 0)
    return set_error(VMO_ERR_INVALID, "lstep_bwd: tensors need 16-byte aligned rows");
  const int64_t cols = (int64_t)a->batch * a->heads * a->block_size;
  if (cols > (1ll << 30) || (int64_t)a->num_blocks * a->block_size > (1ll << 30))
    return set_error(VMO_ERR_UNSUPPORTED, "lstep_bwd: problem too large");
  if (a->flags & ~VMO_LSTEP_BWD_OVERWRITE_Q) return set_error(VMO_ERR_INVALID, "lstep_bwd: unknown flags 0x%x", (unsigned)a->flags);
  if (a->delta && !one_tile)
    return set_error(VMO_ERR_UNSUPPORTED, "lstep_bwd: delta is built for the one-tile kernels (m <= 32, d and dv in "
                     "{64, 128}); got m=%d d=%d dv=%d", a->num_blocks, a->d, a->dv);
  LBParams p{};
  p.delta = a->delta;
  p.dl_sb = a->delta_stride_b; p.dl_sh = a->delta_stride_h;
  p.dq_overwrite = (a->flags & VMO_LSTEP_BWD_OVERWRITE_Q) != 0;
  p.q = a->q.data; p.out = a->out.data; p.ent = a->ent; p.g = a->grad_res.data;
  p.dq = (float*)a->grad_q.data; p.dout = a->grad_out.data;
  p.q_sb = a->q.stride_b; p.q_sh = a->q.stride_h; p.q_sn = a->q.stride_n;
  p.out_sb = a->out.stride_b; p.out_sh = a->out.stride_h; p.out_sn = a->out.stride_n;
  p.ent_sb = a->ent_stride_b; p.ent_sh = a->ent_stride_h;
  p.g_sb = a->grad_res.stride_b; p.g_sh = a->grad_res.stride_h; p.g_sn = a->grad_res.stride_n;
  p.dq_sb = a->grad_q.stride_b; p.dq_sh = a->grad_q.stride_h; p.dq_sn = a->grad_q.stride_n;
  p.do_sb = a->grad_out.stride_b; p.do_sh = a->grad_out.stride_h; p.do_sn = a->grad_out.stride_n;
  p.heads = a->heads; p.m = a->num_blocks; p.bs = a->block_size; p.skip = a->last ? a->skip_tokens : 0;
  p.cols_total = (int)cols;
  p.d = a->d;
  p.dv = a->last ? a->dv : 0;
  p.logit_scale_log2 = a->scale * kLog2e;
  p.scale = a->scale;
  p.min_col_mass = a->min_col_mass;
  hipStream_t s = (hipStream_t)stream;
  if (multi_block) return mb_lstep_bwd(p, a->dtype == VMO_DTYPE_F16, a->d, a->dv, a->last != 0, s);
  if (!one_tile) {
    const int lds = lw_layout(p.m, p.d, p.dv, a->last != 0, true).total;
    if (a->dtype == VMO_DTYPE_F16)
      return a->last ? lw_launch(lstep_wide_bwd_kernel<true, true>, lds, p.cols_total, s, "lstep_wide_bwd", p)
                     : lw_launch(lstep_wide_bwd_kernel<true, false>, lds, p.cols_total, s, "lstep_wide_bwd", p);
    return a->last ? lw_launch(lstep_wide_bwd_kernel<false, true>, lds, p.cols_total, s, "lstep_wide_bwd", p)
                   : lw_launch(lstep_wide_bwd_kernel<false, false>, lds, p.cols_total, s, "lstep_wide_bwd", p);
  }
  if (a->dtype == VMO_DTYPE_F16) return dispatch_lstep_bwd<true>(p, a->d, a->dv, a->last != 0, s);
  return dispatch_lstep_bwd<false>(p, a->d, a->dv, a->last != 0, s);
}
