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

namespace vmo {

constexpr int kLWaves = 4;   // columns per workgroup
constexpr int kAttStride = 36;   // floats per row of the LDS attention tile (bank-conflict pad)

struct LParams {
  const void* q;
  const void* out;
  const float* ent;
  void* res;
  int64_t q_sb, q_sh, q_sn;
  int64_t out_sb, out_sh, out_sn;
  int64_t ent_sb, ent_sh;
  int64_t res_sb, res_sh, res_sn;
  int heads, m, bs, skip;
  int cols_total;
  float logit_scale_log2;   // scale * log2(e)
  float scale;
  float min_col_mass;
};

template <int D, int DV, bool LAST>
struct LLds {
  static constexpr int QT = LAST ? 0 : 32 * D * 2;
  static constexpr int YT = LAST ? 32 * DV * 2 : 0;
  static constexpr int AT = LAST ? 0 : 32 * kAttStride * 4;
  static constexpr int ET = 32 * 4;
  static constexpr int PER_WAVE = QT + YT + AT + ET;
};

// Stage 32 rows (row i = token i*bs + j, clamped to i < m) of width W into a swizzled tile.
template <class T, int W>
__device__ __forceinline__ void stage_col_rows(const T* __restrict__ colbase, int64_t row_stride, int m,
                                               VMO_LDS char* dst, int lane) {
  constexpr int CH = W / 8;
  constexpr int RPI = 64 / CH;
  constexpr int NI = 32 / RPI;
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
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, hl = lane >> 5, l32 = lane & 31;
  const bool live = blockIdx.x * kLWaves + wave < p.cols_total;   // tail waves compute, never store
  const int col = live ? blockIdx.x * kLWaves + wave : p.cols_total - 1;
  VMO_LDS char* wl = (VMO_LDS char*)smem_raw + wave * LL::PER_WAVE;
  VMO_LDS char* q_t = wl;
  VMO_LDS char* y_t = wl + LL::QT;
  VMO_LDS float* att = (VMO_LDS float*)(wl + LL::QT + LL::YT);
  VMO_LDS float* e_t = (VMO_LDS float*)(wl + LL::QT + LL::YT + LL::AT);

  const int bh = col / p.bs, j = col % p.bs;
  const int hh = bh % p.heads, bb = bh / p.heads;
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
// allocation unit and five waves share a CU (two per workgroup fitted four).
constexpr int kLBWaves = 1;

struct LBParams {
  const void* q;
  const void* out;
  const float* ent;
  const void* g;
  float* dq;
  int dq_overwrite;   // dq = dL/dq instead of +=
  void* dout;
  int64_t q_sb, q_sh, q_sn;
  int64_t out_sb, out_sh, out_sn;
  int64_t ent_sb, ent_sh;
  int64_t g_sb, g_sh, g_sn;
  int64_t dq_sb, dq_sh, dq_sn;
  int64_t do_sb, do_sh, do_sn;
  int heads, m, bs, skip;
  int cols_total;
  float logit_scale_log2;
  float scale;
  float min_col_mass;
};

template <int D, int DV, bool LAST>
struct LBLds {
  static constexpr int QT = 32 * D * 2;               // q rows i
  static constexpr int KT = 32 * D * 2;               // kr rows k
  static constexpr int GT = LAST ? 32 * DV * 2 : 0;   // dz rows i
  static constexpr int VT = LAST ? 0 : 32 * D * 2;    // dv rows k
  static constexpr int AT = 32 * kAttStride * 4;      // an m x m matrix as [k][i]
  static constexpr int ET = 32 * 4;
  static constexpr int CT = 32 * 4;
  static constexpr int PER_WAVE = QT + KT + GT + VT + AT + ET + CT;   // y is read into registers
};

template <bool F16, int D, int DV, bool LAST>
__global__ __launch_bounds__(64 * kLBWaves) void lstep_bwd_kernel(LBParams p) {
  using E = Elem<F16>;
  using T = typename E::T;
  using V8 = typename E::V8;
  using V4 = typename E::V4;
  using LL = LBLds<D, DV, LAST>;
  constexpr int ND = D / 32;
  constexpr int NV = DV / 32;

  extern __shared__ __attribute__((aligned(1024))) char smem_raw[];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, hl = lane >> 5, l32 = lane & 31;
  const bool live = blockIdx.x * kLBWaves + wave < p.cols_total;   // tail waves compute, never store
  const int col = live ? blockIdx.x * kLBWaves + wave : p.cols_total - 1;
  VMO_LDS char* q_t = (VMO_LDS char*)smem_raw + wave * LL::PER_WAVE;
  VMO_LDS char* k_t = q_t + LL::QT;
  VMO_LDS char* g_t = k_t + LL::KT;
  VMO_LDS char* v_t = g_t + LL::GT;
  VMO_LDS float* att = (VMO_LDS float*)(v_t + LL::VT);
  VMO_LDS float* e_t = att + 32 * kAttStride;
  VMO_LDS float* c_t = e_t + 32;

  const int bh = col / p.bs, j = col % p.bs;
  const int hh = bh % p.heads, bb = bh / p.heads;
  const int m = p.m;
  const int64_t q_rs = (int64_t)p.bs * p.q_sn;
  const int64_t o_rs = (int64_t)p.bs * p.out_sn;
  const int64_t g_rs = (int64_t)p.bs * p.g_sn;
  const T* qcol = (const T*)p.q + bb * p.q_sb + hh * p.q_sh + (int64_t)j * p.q_sn;
  const T* ocol = (const T*)p.out + bb * p.out_sb + hh * p.out_sh + (int64_t)j * p.out_sn;
  const T* gcol = (const T*)p.g + bb * p.g_sb + hh * p.g_sh + (int64_t)j * p.g_sn;

  stage_col_rows<T, D>(qcol, q_rs, m, q_t, lane);
  stage_col_rows<T, D>(ocol, o_rs, m, k_t, lane);
  if constexpr (LAST)
    stage_col_rows<T, DV>(gcol, g_rs, m, g_t, lane);
  else   // du rows k, into the dv tile: each lane turns its du values into dv in place
    stage_col_rows<T, D>(gcol, g_rs, m, v_t, lane);
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
  if constexpr (LAST) {
    // z rows of tokens < skip are overwritten by the recompute: no gradient reaches the L-path
    constexpr int CH = DV / 8;
    for (int idx = lane; idx < 32 * CH; idx += 64) {
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
    // the dz tile is dead now: it takes the row-store patch (whole row segments per store)
    if (live)
      store_acc_rows<F16>((VMO_LDS float*)g_t, accy, NV, 1.f, kGradStore, (char*)(dcol + D), do_rs * 2, m, lane);
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
        *dvp = w;
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
    if (live) {   // kr (and dv) tiles dead now: the kr tile takes the row-store patch
      float* dq0 = p.dq + bb * p.dq_sb + hh * p.dq_sh + (int64_t)j * p.dq_sn;
      store_acc_rows<F16>((VMO_LDS float*)k_t, accq, ND, 1.f, p.dq_overwrite ? kGradStoreF32 : kGradAddF32,
                          (char*)dq0, (int64_t)p.bs * p.dq_sn * 4, m, lane);
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
    if (live)   // the q tile is dead now: it takes the row-store patch
      store_acc_rows<F16>((VMO_LDS float*)q_t, acck, ND, 1.f, kGradStore, (char*)dcol, do_rs * 2, m, lane);
  }
}

template <bool F16, int D, int DV, bool LAST>
static int launch_lstep_bwd(const LBParams& p, hipStream_t s) {
  constexpr int LDS = LBLds<D, DV, LAST>::PER_WAVE * kLBWaves;
  static_assert(LDS <= 160 * 1024, "lstep_bwd LDS");
  auto kern = lstep_bwd_kernel<F16, D, DV, LAST>;
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
#define VMO_LB(D_, DV_, LAST_) \
  if (d == D_ && (!LAST_ || dv == DV_) && last == LAST_) return launch_lstep_bwd<F16, D_, DV_, LAST_>(p, s);
  VMO_LB(64, 64, false)
  VMO_LB(128, 128, false)
  VMO_LB(64, 64, true)
  VMO_LB(64, 128, true)
  VMO_LB(128, 64, true)
  VMO_LB(128, 128, true)
#undef VMO_LB
  return set_error(VMO_ERR_UNSUPPORTED, "lstep_bwd: no kernel for d=%d dv=%d last=%d", d, dv, (int)last);
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
  if (a->num_blocks > 32) return set_error(VMO_ERR_UNSUPPORTED, "lstep: num_blocks %d > 32", a->num_blocks);
  if (!view_ok(a->q) || !view_ok(a->out) || !view_ok(a->res) || a->ent == nullptr)
    return set_error(VMO_ERR_INVALID, "lstep: tensors need 16-byte aligned rows");
  if ((a->d % 8) != 0) return set_error(VMO_ERR_INVALID, "lstep: d");
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
  p.logit_scale_log2 = a->scale * kLog2e;
  p.scale = a->scale;
  p.min_col_mass = a->min_col_mass;
  hipStream_t s = (hipStream_t)stream;
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
  if (a->num_blocks > 32) return set_error(VMO_ERR_UNSUPPORTED, "lstep_bwd: num_blocks %d > 32", a->num_blocks);
  if (!view_ok(a->q) || !view_ok(a->out) || !view_ok(a->grad_res) || !view_ok(a->grad_out) || a->ent == nullptr ||
      a->grad_q.data == nullptr || ((uintptr_t)a->grad_q.data & 15) != 0 || (a->grad_q.stride_n & 3) != 0 ||
      (a->grad_q.stride_h & 3) != 0 || (a->grad_q.stride_b & 3) != 0)
    return set_error(VMO_ERR_INVALID, "lstep_bwd: tensors need 16-byte aligned rows");
  const int64_t cols = (int64_t)a->batch * a->heads * a->block_size;
  if (cols > (1ll << 30) || (int64_t)a->num_blocks * a->block_size > (1ll << 30))
    return set_error(VMO_ERR_UNSUPPORTED, "lstep_bwd: problem too large");
  if (a->flags & ~VMO_LSTEP_BWD_OVERWRITE_Q) return set_error(VMO_ERR_INVALID, "lstep_bwd: unknown flags 0x%x", (unsigned)a->flags);
  LBParams p{};
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
  p.logit_scale_log2 = a->scale * kLog2e;
  p.scale = a->scale;
  p.min_col_mass = a->min_col_mass;
  hipStream_t s = (hipStream_t)stream;
  if (a->dtype == VMO_DTYPE_F16) return dispatch_lstep_bwd<true>(p, a->d, a->dv, a->last != 0, s);
  return dispatch_lstep_bwd<false>(p, a->d, a->dv, a->last != 0, s);
}
