// Launch parameters of the L-step kernels (forward and backward), shared by the one-tile, multi-block and
// general kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vmo {

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
  int d, dv;                // head dims (the one-tile kernels take them as template parameters)
  float logit_scale_log2;   // scale * log2(e)
  float scale;
  float min_col_mass;
};

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
  int d, dv;
  float logit_scale_log2;
  float scale;
  float min_col_mass;
  float* delta;       // optional: sum_f out * d out per token (one-tile kernels)
  int64_t dl_sb, dl_sh;
};

// Multi-block kernels (lstep_mb.hip): grids of up to 128 frames with head dims 32 / 64 / 128 on MFMA.
// mb_lstep_check: whether they take (m, d, dv) (forward or backward); mb_lstep_fwd / mb_lstep_bwd launch.
int mb_lstep_check(int m, int d, int dv, bool last, bool bwd);
int mb_lstep_fwd(const LParams& p, bool f16, int d, int dv, bool last, hipStream_t s);
int mb_lstep_bwd(const LBParams& p, bool f16, int d, int dv, bool last, hipStream_t s);

}  // namespace vmo
