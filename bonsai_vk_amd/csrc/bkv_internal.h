// bkv_internal.h - kernel argument blocks and launchers shared by the API layer and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/bkv.h"

namespace bkv {

constexpr int kMaxChunk = 512;   // keys per decode partition held in LDS

}  // namespace bkv

#include "bkv_common.h"

namespace bkv {

struct AppendArgs {
  LayerView L;
  int nkv;
  uint32_t pos;
  const float *k, *v;            // [n_tok][nkv][hd]
};

struct QkArgs {
  LayerView L;
  int nkv;
  uint32_t nfill;
  int chunk, nch_qk;
  int64_t ld;                    // score row stride (floats)
  float scale;
  const float *q;                // [nh][hd]
  float *score;                  // [nh][ld]
  float2 *stats;                 // [nh][nch_qk]
  AppendArgs ap;                 // fused append of position ap.pos (decode_step)
};

struct PvArgs {
  LayerView L;
  int nkv, nh;
  uint32_t nfill;
  int chunk, nch_pv, nch_qk;
  int64_t ld;
  float scale;
  const float *score;
  const float2 *stats;
  float *part;                   // [nch_pv][nh][hd]
};

struct RedArgs {
  int nh, nch_pv;
  const float *part;
  const float *gate;
  float *out, *out_gated;
};

// decode partition plan for nfill keys
struct DecodePlan {
  int ch_qk, nch_qk, ch_pv, nch_pv;
  int64_t ld;
  size_t off_score, off_stats, off_part, total;
};

DecodePlan plan_decode(int nh, int nkv, int64_t nfill);

hipError_t launch_append(const AppendArgs &a, int kf, int vf, int n_tok, hipStream_t st);
hipError_t launch_decode(const QkArgs &qa, const PvArgs &pa, const RedArgs &ra, int kf, int vf,
                         bool fuse, hipStream_t st);

}  // namespace bkv
