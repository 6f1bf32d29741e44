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
//  * K / W tiles are staged by global_load_lds (no register round trip), double-buffered, with
//    an XOR swizzle of 16-byte chunks against LDS bank conflicts;
//  * when w0 aliases k (the VMonarch R-step values [k | v]) the K tile doubles as W0;
//  * lazy rescaling: the running max only moves when a stage max exceeds it by > kTau (log2
//    units), so the O rescale is rare; the entropy identity e = log2 l - h / l holds for any
//    reference point;
//  * tail keys are masked in-kernel (no padding copies, unlike kernel.py:399-400);
//  * split-KV (num_splits > 1) writes normalised fp32 partials + lse, merged by fea_combine.
#include <type_traits>

#include "vmo_common.h"
#include "vmo_host.h"

namespace vmo {

constexpr int kFwdBM = 128;           // queries per workgroup
constexpr int kFwdBN = 64;            // keys per pipeline stage
constexpr int kFwdWaves = 4;
constexpr float kTau = 8.0f;          // lazy-rescale threshold, log2 units (p <= 2^8)
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
};

// Stage kFwdBN rows of a row-major (token, W) tensor into a swizzled LDS tile.  Rows past the end
// of the tensor (>= nrows) re-read the last row: they are finite and masked out later.
template <class T, int W>
__device__ __forceinline__ void stage_rows(const T* __restrict__ base, int64_t sn, int row0, int nrows,
                                           VMO_LDS char* dst, int wave, int lane) {
  constexpr int CH = W / 8;           // 16-byte chunks per row
  constexpr int RPI = 64 / CH;        // rows per wave instruction (1 KB)
  constexpr int NI = kFwdBN / RPI / kFwdWaves;
  static_assert(CH >= 8 && NI >= 1, "tile shape");
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int inst = i * kFwdWaves + wave;
    const int r = inst * RPI + lane / CH;
    const int lc = (lane % CH) ^ swz(r);
    int gr = row0 + r;
    gr = gr < nrows ? gr : nrows - 1;
    g2l_16(base + (int64_t)gr * sn + lc * 8, dst + inst * 1024);
  }
}

template <bool F16, int D, int DW0, int DW1, bool W0K, bool ENT, bool SPLIT>
__global__ __launch_bounds__(256, 2) void fea_fwd_kernel(FwdParams p) {
  using E = Elem<F16>;
  using T = typename E::T;
  using V8 = typename E::V8;
  using V4 = typename E::V4;
  constexpr int K_BYTES = kFwdBN * D * 2;
  constexpr int W0_BYTES = W0K ? 0 : kFwdBN * DW0 * 2;
  constexpr int W1_BYTES = kFwdBN * DW1 * 2;
  constexpr int STAGE = K_BYTES + W0_BYTES + W1_BYTES;
  constexpr int NA0 = DW0 / 32;
  constexpr int NA1 = DW1 / 32;
  constexpr int NA = NA0 + NA1;
  static_assert(!W0K || DW0 == D, "w0 aliases k");

  extern __shared__ __attribute__((aligned(1024))) char smem_raw[];
  VMO_LDS char* smem = (VMO_LDS char*)smem_raw;

  // XCD-aware block -> tile map: block b runs on XCD b % 8, so give each XCD a contiguous run of
  // logical tiles (all query tiles of a problem then share one L2 for their K / W traffic).
  const int per_xcd = gridDim.x >> 3;
  const int L = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
  if (L >= p.total_wg) return;
  const int qt = L % p.q_tiles;
  const int rest = L / p.q_tiles;
  const int split = rest % p.splits;
  const int prob = rest / p.splits;
  const int f = prob % p.frames;
  const int bh = prob / p.frames;
  const int hh = bh % p.heads;
  const int bb = bh / p.heads;

  const T* qb = (const T*)p.q + bb * p.q_sb + hh * p.q_sh + (int64_t)f * p.nq * p.q_sn;
  const T* kb = (const T*)p.k + bb * p.k_sb + hh * p.k_sh + (int64_t)f * p.nk * p.k_sn;
  const T* w0b = (const T*)p.w0 + bb * p.w0_sb + hh * p.w0_sh + (int64_t)f * p.nk * p.w0_sn;
  const T* w1b = DW1 ? (const T*)p.w1 + bb * p.w1_sb + hh * p.w1_sh + (int64_t)f * p.nk * p.w1_sn : nullptr;

  const int kbeg = split * p.keys_per_split;
  const int kend = min(p.nk, kbeg + p.keys_per_split);
  const int n_tiles = (kend - kbeg + kFwdBN - 1) / kFwdBN;

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int hl = lane >> 5;
  const int l32 = lane & 31;
  const int q0 = qt * kFwdBM + wave * 32;
  const bool wave_live = q0 < p.nq;
  const int qrow = q0 + l32;
  const bool qvalid = qrow < p.nq;

  // Q^T as the B operand: lane (query l32, half hl) holds q[query][16 ds + 8 hl + 0..7].
  V8 qf[D / 16];
  {
    const T* qp = qb + (int64_t)(qvalid ? qrow : 0) * p.q_sn + hl * 8;
#pragma unroll
    for (int ds = 0; ds < D / 16; ++ds) {
      V8 v = *(const V8*)(qp + ds * 16);
      qf[ds] = qvalid ? v : V8{};
    }
  }

  auto issue = [&](int t) {
    VMO_LDS char* st = smem + (t & 1) * STAGE;
    const int row0 = kbeg + t * kFwdBN;
    stage_rows<T, D>(kb, p.k_sn, row0, p.nk, st, wave, lane);
    if constexpr (!W0K) stage_rows<T, DW0>(w0b, p.w0_sn, row0, p.nk, st + K_BYTES, wave, lane);
    if constexpr (DW1 > 0) stage_rows<T, DW1>(w1b, p.w1_sn, row0, p.nk, st + K_BYTES + W0_BYTES, wave, lane);
  };

  const float c = p.scale_log2;
  float m_run = kMaskLogit;
  float l_run = 0.f;
  float h_run = 0.f;
  f32x16 acc[NA];
#pragma unroll
  for (int a = 0; a < NA; ++a) acc[a] = f32x16{};

  // per-lane LDS offsets
  const int srow_sw = swz(l32);                                   // S operand rows 32 kb + l32
  const int trow = 4 * hl + ((lane & 15) >> 2);                   // W^T rows 16 ks + trow (+8)
  const int tsw = swz(trow);
  const int tchunk = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);   // logical chunk within 32 cols
  const int tbyte = (lane & 1) * 8;

  issue(0);
  for (int t = 0; t < n_tiles; ++t) {
    __builtin_amdgcn_s_waitcnt(0);    // this wave's part of stage t has landed
    __syncthreads();                  // ... and everybody else's; stage t-1 is free again
    if (t + 1 < n_tiles) issue(t + 1);
    if (!wave_live) continue;

    const VMO_LDS char* Ks = smem + (t & 1) * STAGE;
    const int nvalid = kend - (kbeg + t * kFwdBN);   // valid keys in this stage (may exceed 64)
    const bool hi_live = nvalid > 32;

    // ---- S^T = K Q^T : s0 keys 0..31, s1 keys 32..63 of the stage
    f32x16 s0 = f32x16{}, s1 = f32x16{};
    {
      const VMO_LDS char* arow = Ks + l32 * (D * 2);
      if (hi_live) {
#pragma unroll
        for (int ds = 0; ds < D / 16; ++ds) {
          const int off = ((2 * ds + hl) ^ srow_sw) * 16;
          s0 = E::mfma(lds_read8<V8>(arow + off), qf[ds], s0);
          s1 = E::mfma(lds_read8<V8>(arow + 32 * D * 2 + off), qf[ds], s1);
        }
      } else {
#pragma unroll
        for (int ds = 0; ds < D / 16; ++ds) {
          const int off = ((2 * ds + hl) ^ srow_sw) * 16;
          s0 = E::mfma(lds_read8<V8>(arow + off), qf[ds], s0);
        }
      }
    }

    // ---- row max (raw logits); masked keys can not win while one key is valid
    const bool masked = nvalid < kFwdBN;
    if (masked) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = 8 * (r >> 2) + 4 * hl + (r & 3);
        if (key >= nvalid) s0[r] = kMaskLogit;
        if (key + 32 >= nvalid) s1[r] = kMaskLogit;
      }
    }
    float mx = s0[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s0[r]);
    if (hi_live) {
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s1[r]);
    }
    mx = wave_max32(mx) * c;

    if (t == 0) {
      m_run = mx;
    } else if (__builtin_amdgcn_ballot_w64(mx > m_run + kTau) != 0) {
      const float m_new = fmaxf(m_run, mx);
      const float alpha = fast_exp2(m_run - m_new);
      if constexpr (ENT) h_run = alpha * (h_run + (m_run - m_new) * l_run);
      l_run *= alpha;
#pragma unroll
      for (int a = 0; a < NA; ++a) acc[a] *= alpha;
      m_run = m_new;
    }

    // ---- p = 2^(s c - m), per-lane partial sums of p and p * (s c - m); P becomes the
    // B operand of O^T += W^T P^T.  Masked keys get p = 0 exactly (also when c == 0).
    float lsum = 0.f, hsum = 0.f;
    auto softmax_block = [&](f32x16& s, int kofs) {
      if (masked) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kofs + 8 * (r >> 2) + 4 * hl + (r & 3);
          float x = fmaf(s[r], c, -m_run);
          float pv = fast_exp2(x);
          if (key >= nvalid) { pv = 0.f; x = 0.f; }
          lsum += pv;
          if constexpr (ENT) hsum = fmaf(pv, x, hsum);
          s[r] = pv;
        }
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float x = fmaf(s[r], c, -m_run);
          const float pv = fast_exp2(x);
          lsum += pv;
          if constexpr (ENT) hsum = fmaf(pv, x, hsum);
          s[r] = pv;
        }
      }
    };
    softmax_block(s0, 0);
    if (hi_live) softmax_block(s1, 32);
    l_run += lsum;
    if constexpr (ENT) h_run += hsum;

    V8 P[4];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      P[0][e] = to_elem<T>(s0[e]);
      P[1][e] = to_elem<T>(s0[8 + e]);
      P[2][e] = to_elem<T>(s1[e]);
      P[3][e] = to_elem<T>(s1[8 + e]);
    }

    // ---- O^T += W^T P^T
    auto pv_part = [&](const VMO_LDS char* W, auto rb_tag, auto na_tag, int a0) {
      constexpr int RB = decltype(rb_tag)::value;
      constexpr int NAP = decltype(na_tag)::value;
#pragma unroll
      for (int a = 0; a < NAP; ++a) {
        const int coff = ((4 * a + tchunk) ^ tsw) * 16 + tbyte;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          if (ks >= 2 && !hi_live) break;
          const VMO_LDS char* r0 = W + (16 * ks + trow) * RB + coff;
          acc[a0 + a] = E::mfma(lds_read_tr8<V8>(r0, r0 + 8 * RB), P[ks], acc[a0 + a]);
        }
      }
    };
    pv_part(W0K ? Ks : Ks + K_BYTES, std::integral_constant<int, DW0 * 2>{}, std::integral_constant<int, NA0>{}, 0);
    if constexpr (DW1 > 0)
      pv_part(Ks + K_BYTES + W0_BYTES, std::integral_constant<int, DW1 * 2>{}, std::integral_constant<int, NA1>{}, NA0);
  }

  if (!wave_live) return;

  // ---- finalise: combine the two half-waves' partial sums
  const float l_tot = wave_sum32(l_run);
  const float inv_l = 1.0f / l_tot;
  const float log2l = fast_log2(l_tot);
  const float lse = m_run + log2l;

  if constexpr (SPLIT) {
    if (qvalid) {
      float* orow = p.part_o + ((int64_t)(split * p.problems + prob) * p.nq + qrow) * (int64_t)(DW0 + DW1);
#pragma unroll
      for (int a = 0; a < NA; ++a)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          f32x4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = acc[a][4 * j + e] * inv_l;
          *(f32x4*)(orow + 32 * a + 8 * j + 4 * hl) = v;
        }
      if (hl == 0) p.part_lse[(int64_t)(split * p.problems + prob) * p.nq + qrow] = lse;
    }
  } else {
    if (qvalid) {
      T* orow = (T*)p.o + bb * p.o_sb + hh * p.o_sh + ((int64_t)f * p.nq + qrow) * p.o_sn;
#pragma unroll
      for (int a = 0; a < NA; ++a)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          V4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = to_elem<T>(acc[a][4 * j + e] * inv_l);
          *(V4*)(orow + 32 * a + 8 * j + 4 * hl) = v;
        }
      const int64_t si = bb * p.st_sb + hh * p.st_sh + (int64_t)f * p.nq + qrow;
      if constexpr (ENT) {
        // h = sum_j p_j x_j with p_j = 2^x_j, x_j = s_j c - m: entropy (bits) = log2 l - h / l
        const float h_tot = wave_sum32(h_run);
        if (hl == 0 && p.ent) p.ent[si] = (log2l - h_tot * inv_l) * kLn2;
      }
      if (hl == 0 && p.lse) p.lse[si] = lse;
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

template <bool F16, int D, int DW0, int DW1, bool W0K, bool ENT, bool SPLIT>
static int launch_fwd(const FwdParams& p, hipStream_t stream) {
  constexpr int STAGE = kFwdBN * (D + (W0K ? 0 : DW0) + DW1) * 2;
  constexpr int LDS = 2 * STAGE;
  auto kern = fea_fwd_kernel<F16, D, DW0, DW1, W0K, ENT, SPLIT>;
  if (LDS > 65536) {
    static bool done = false;   // attribute is per function; idempotent, so a benign race
    if (!done) {
      if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, LDS) != hipSuccess)
        return set_error(VMO_ERR_LAUNCH, "fea_fwd: cannot raise the LDS limit to %d bytes", LDS);
      done = true;
    }
  }
  hipLaunchKernelGGL(kern, dim3(xcd_grid(p.total_wg)), dim3(256), LDS, stream, p);
  int rc = launch_status("fea_fwd");
  if (rc != VMO_OK || !SPLIT) return rc;
  constexpr int DWT = DW0 + DW1;
  const int64_t threads = (int64_t)p.problems * p.nq * (DWT / 4);
  hipLaunchKernelGGL((fea_combine_kernel<F16, DWT>), dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, p);
  return launch_status("fea_combine");
}

// Runtime -> template dispatch over the supported shapes.
template <bool F16>
static int dispatch_fwd(const FwdParams& p, int d, int dw0, int dw1, bool w0k, bool ent, bool split, hipStream_t s) {
#define VMO_FWD(D_, DW0_, DW1_, W0K_, ENT_, SPLIT_)                                                  \
  if (d == D_ && dw0 == DW0_ && dw1 == DW1_ && w0k == W0K_ && ent == ENT_ && split == SPLIT_)          \
    return launch_fwd<F16, D_, DW0_, DW1_, W0K_, ENT_, SPLIT_>(p, s);
  // standalone flash_entropy_attention (kernel.py:384-402): entropy on
  VMO_FWD(64, 64, 0, false, true, false)
  VMO_FWD(64, 128, 0, false, true, false)
  VMO_FWD(64, 256, 0, false, true, false)
  VMO_FWD(128, 64, 0, false, true, false)
  VMO_FWD(128, 128, 0, false, true, false)
  VMO_FWD(128, 256, 0, false, true, false)
  // VMonarch R-step (vmonarch.py:50): values k, or [k | v]
  VMO_FWD(64, 64, 0, true, true, false)
  VMO_FWD(64, 64, 64, true, true, false)
  VMO_FWD(64, 64, 128, true, true, false)
  VMO_FWD(128, 128, 0, true, true, false)
  VMO_FWD(128, 128, 64, true, true, false)
  VMO_FWD(128, 128, 128, true, true, false)
  // exact recompute (vmonarch.py:66-68): no entropy, optionally split-KV
  VMO_FWD(64, 64, 0, false, false, false)
  VMO_FWD(64, 128, 0, false, false, false)
  VMO_FWD(128, 64, 0, false, false, false)
  VMO_FWD(128, 128, 0, false, false, false)
  VMO_FWD(64, 64, 0, false, false, true)
  VMO_FWD(64, 128, 0, false, false, true)
  VMO_FWD(128, 64, 0, false, false, true)
  VMO_FWD(128, 128, 0, false, false, true)
#undef VMO_FWD
  return set_error(VMO_ERR_UNSUPPORTED, "fea_fwd: no kernel for d=%d dw0=%d dw1=%d w0_is_k=%d entropy=%d split=%d", d,
                   dw0, dw1, (int)w0k, (int)ent, (int)split);
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
  if (!a || a->nk <= 0) return 0;
  int s, kps;
  return (size_t)vmo::split_layout(a, &s, &kps);
}

extern "C" int vmo_fea_fwd(const vmo_fea_fwd_args* a, void* stream) {
  using namespace vmo;
  clear_error();
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
  const bool w0k = a->w0.data == a->k.data && a->w0.stride_b == a->k.stride_b && a->w0.stride_h == a->k.stride_h &&
                   a->w0.stride_n == a->k.stride_n && a->dw0 == a->d;
  if (a->dw1 > 0 && !w0k) return set_error(VMO_ERR_UNSUPPORTED, "fea_fwd: a second value tensor needs w0 == k");
  int splits, kps;
  const int64_t ws = split_layout(a, &splits, &kps);
  const bool ent = a->ent != nullptr;
  if (splits > 1 && ent) return set_error(VMO_ERR_UNSUPPORTED, "fea_fwd: split-KV with entropy output");
  if (splits > 1 && (a->workspace == nullptr || a->workspace_bytes < (size_t)ws || !aligned16(a->workspace)))
    return set_error(VMO_ERR_WORKSPACE, "fea_fwd: needs %lld workspace bytes", (long long)ws);
  const int64_t q_tiles = (a->nq + kFwdBM - 1) / kFwdBM;
  const int64_t problems = (int64_t)a->batch * a->heads * a->frames;
  const int64_t total = problems * splits * q_tiles;
  if (total > (1ll << 30) || (int64_t)a->frames * a->nq > (1ll << 30) || (int64_t)a->frames * a->nk > (1ll << 30))
    return set_error(VMO_ERR_UNSUPPORTED, "fea_fwd: problem too large");

  FwdParams p{};
  p.q = a->q.data; p.k = a->k.data; p.w0 = a->w0.data; p.w1 = a->w1.data; p.o = a->o.data;
  p.lse = a->lse; p.ent = a->ent;
  if (splits > 1) {
    const int64_t rows = problems * a->nq;
    p.part_o = (float*)a->workspace;
    p.part_lse = (float*)((char*)a->workspace + (int64_t)splits * rows * (a->dw0 + a->dw1) * 4);
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
  hipStream_t s = (hipStream_t)stream;
  if (a->dtype == VMO_DTYPE_F16) return dispatch_fwd<true>(p, a->d, a->dw0, a->dw1, w0k, ent, splits > 1, s);
  return dispatch_fwd<false>(p, a->d, a->dw0, a->dw1, w0k, ent, splits > 1, s);
}
