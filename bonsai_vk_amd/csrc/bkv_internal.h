// bkv_internal.h - kernel argument blocks, workspace plan and launchers shared by the API layer and
// the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/bkv.h"
#include "bkv_common.h"

namespace bkv {

// ------------------------------------------------------------------ decode geometry
constexpr int kE2Chunk = 1024;     // keys per workgroup of the probability kernel
constexpr int kMaxSpecial = 64;    // exactly-added steps recorded per probability chunk
constexpr int kPvMaxChunk = 512;   // keys per PV partition held in LDS
constexpr int kCounterStride = 64; // u32 words between per-head arrival counters (own 256 B line)

// one probability chunk's contribution to the exact serial softmax sum
struct ChunkRec {
  long long tot;      // sum of the non-special increments, units of 2^-40
  int nsp;            // specials recorded (> kMaxSpecial: overflow)
  int blast;          // binade of the chunk's last step, kNoBinade if that step is special
};
// one step the walker adds in fp32 exactly as the serial loop does
struct Special {
  long long ipre;     // increments of the chunk's non-special steps before it, units of 2^-40
  float e;            // the term added
  int meta;           // bits 0..15: position in chunk; bits 16..23: binade+128 of the step
                      // just before it (0 = that step is special, 255 = it is the previous
                      // chunk's last step)
};
constexpr int kNoBinade = -1000;

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
  int nch;                       // QK partitions
  int64_t ld;                    // row stride of score / e (floats)
  float scale;
  const float *q;                // [nh][hd] fp32, head rows qs floats apart
  int qs;
  float *score;                  // [nh][ld]
  float2 *stats;                 // [nh][nch] (partition max of s*scale, sum exp(s*scale - max))
  unsigned *counters;            // [nh] arrivals of the probability kernel (zeroed here)
  AppendArgs ap;                 // fused append of position ap.pos (decode_step)
};

struct EArgs {
  int nh;
  uint32_t nfill;
  int nch_qk, qk_chunk, nch;     // QK partitions (stats), probability chunks
  int64_t ld;
  float scale;
  const float *score;
  const float2 *stats;
  float *e;                      // [nh][ld] exp(s*scale - max), correctly rounded
  ChunkRec *rec;                 // [nh][nch]
  Special *spec;                 // [nh][nch][kMaxSpecial]
  unsigned *counters;            // [nh]
  float *sum;                    // [nh] the exact serial sum
  unsigned *status;              // [nh] 1 when the walker fell back to the serial loop
  unsigned long long *dbg;       // [nh][8] phase timestamps of the walker (experiment builds)
};

struct PvArgs {
  LayerView L;
  int nkv, nh;
  uint32_t nfill;
  int chunk, nch;
  int64_t ld;
  const float *e;
  const float *sum;
  float *part;                   // [nch][nh][hd]
};

struct RedArgs {
  int nh, nch;
  const float *part;
  const float *gate;             // head rows gs floats apart
  int gs;
  float *out, *out_gated;
};

constexpr size_t kSyncBytes = 256 * 1024;  // counters / flags at the start of every workspace


// ------------------------------------------------------------------ the resident decode kernel
// One 512-thread workgroup per CU, G workgroups per KV group, every workgroup resident; a
// workgroup holds up to kResMaxPass*512 keys (scores and e in registers); with q8_0 V and at most
// 512 + kResTail keys it keeps its V rows in LDS, streamed in behind the exact-sum walk.
constexpr int kResNT = 512;
constexpr int kResMaxPass = 4;
constexpr int kResPgMax = 64;                  // block-table entries a paged workgroup copies into LDS
constexpr int kResTail = 16;                   // keys past kResNT a q8_0-V workgroup may hold
constexpr int kResMaxGroupWgs = 64;           // workgroups per KV group at most (walk scratch)
constexpr int kResGroupLines = 9;              // generation + 2 parities x 4 phase counters
constexpr size_t kResSyncOffset = 200 * 1024;  // inside the sync area, clear of the other paths
constexpr size_t kResTagOffset = 144 * 1024;   // tagged statistics, then tagged records (48 KiB)

struct ResArgs {
  LayerView L;
  int nkv, nh;
  uint32_t nfill;
  float scale;
  int G, kpw;                    // workgroups per KV group, keys per workgroup
  int64_t ld;
  const float *q;                // [nh][hd], head rows qs floats apart
  AppendArgs ap;                 // decode_step: the token to append first (ap.k null: none)
  const float *gate;             // head rows gs floats apart
  int qs, gs;
  float *out, *out_gated;
  unsigned long long *tstats;    // [nh][kResMaxGroupWgs] tagged (max, sum exp) per workgroup
  unsigned long long *trec;      // [nh][kResMaxGroupWgs][2] tagged chunk records
  Special *spec;                 // [nh][G][kMaxSpecial]
  float *e;                      // [nh][ld]: written when keep_e (diagnostics) or on the fallback
  int keep_e;
  float *sum;                    // [nh]
  unsigned *status;              // [nh]
  unsigned long long *part;      // [nkv][G][kGqa][hd] {float bits, call generation}
  unsigned *sync;                // the resident kernel's sync lines
  unsigned *ts;                  // phase timestamps (experiment builds), or null
  unsigned *tsw;                 // per-wave phase timestamps [workgroup][8 waves][8] (experiment builds)
};

// ------------------------------------------------------------------ chunked prefill (MFMA)
constexpr int kPfQ = 16;       // queries per workgroup (x 4 heads = 64 rows)
constexpr int kPfTile = 64;    // keys per tile
constexpr int kPfFill = 256;   // workgroups the split count aims for (one per CU)

struct PrefillArgs {
  LayerView L;
  int nkv, nh;
  uint32_t pos0;
  int n_q;
  float scale;
  int nqb, nsplit;               // query blocks, key splits per query block
  const float *q, *gate;         // [n_q][nh] rows, qs / gs floats apart
  int qs, gs;
  float *out, *out_gated;
  float2 *stats;                 // [nsplit][n_q][nh] (max, sum exp) of the split's keys
  float *part;                   // [nsplit][n_q][nh][hd] normalised partial outputs (nsplit > 1)
};

struct PrefillPlan {
  int nqb, nsplit;
  size_t off_stats, off_part, total;
};
PrefillPlan plan_prefill(int nh, int nkv, uint32_t pos0, int n_q, size_t base);
size_t prefill_workspace_bound(int nh, int nkv, size_t base);
hipError_t launch_prefill(const PrefillArgs &a, int kf, int vf, hipStream_t st);

// ------------------------------------------------------------------ exact chunked prefill
constexpr int kPxQ = 4;          // queries per workgroup (x 4 heads = 16 rows)
constexpr int kPxRows = kPxQ * kGqa;
constexpr int kPxTile = 256;     // keys per score / exp tile (one per lane of the workgroup)
constexpr int kPxSlice = 512;    // queries per launch (bounds the score scratch)
constexpr int kPvQ = 32;         // exact prefill, q8_0 V: queries per PV workgroup (4 kPvQ rows)
constexpr int kPvSplit = 4;      // ... and key ranges per query block (partials added in order)
constexpr int kPxMinQ = 16;      // shorter chunks run as decode rows

struct PrefillXArgs {
  LayerView L;
  int nkv, nh;
  uint32_t pos0;
  int q_base, n_q;               // this slice: queries q_base .. q_base + n_q - 1 of the chunk
  int chunk_q;                   // queries in the whole chunk (row stride of q / out)
  float scale;
  int nqb;
  int64_t ld;                    // keys per workgroup scratch region (multiple of kPxTile, one
                                 // tile past the last key)
  const float *q;                // [chunk_q][nh] rows of hd fp32, qs floats apart
  const float *gate;             // rows gs floats apart
  int qs, gs;
  float *out, *out_gated;
  float *sc;                     // [nkv * nqb][ld][kPxRows] scores, then exp (the slice's workgroups)
  float *sums;                   // q8_0 V: [nkv * nqb][kPxRows] the exact serial sums, for the PV kernel
  float *part;                   // q8_0 V: [kPvSplit][kPxSlice][nh][hd] the PV kernel's key-range partials
  unsigned *ts;                  // sweep timestamps (experiment builds), or null
};
hipError_t launch_prefill_exact(const PrefillXArgs &a, int kf, int vf, hipStream_t st);
size_t prefill_exact_workspace(int nh, int nkv, int64_t max_ctx, size_t base);

// ------------------------------------------------------------------ QK norm + rope + append
struct NormRopeArgs {
  LayerView L;
  int nkv, nh, nrot;
  uint32_t pos0;
  float eps, freq_base;
  const float *q_in, *k_in, *v_in;   // [n_tok][nh][hd], [n_tok][nkv][hd], [n_tok][nkv][hd]
  const float *qn_w, *kn_w;          // [hd] norm weights
  float *q_out;                      // [n_tok][nh][hd]
};
hipError_t launch_norm_rope_append(const NormRopeArgs &a, int kf, int vf, int n_tok, hipStream_t st);

#define BKV_FMT_SWITCH(KF, VF, ...)                                                    \
  do {                                                                                \
    if ((KF) == BKV_Q8_0 && (VF) == BKV_Q8_0) { constexpr int KF_ = 1, VF_ = 1; __VA_ARGS__; } \
    else if ((KF) == BKV_Q8_0) { constexpr int KF_ = 1, VF_ = 0; __VA_ARGS__; }       \
    else if ((VF) == BKV_Q8_0) { constexpr int KF_ = 0, VF_ = 1; __VA_ARGS__; }       \
    else { constexpr int KF_ = 0, VF_ = 0; __VA_ARGS__; }                             \
  } while (0)

// decode partition plan and workspace layout for nfill keys
struct DecodePlan {
  int qk_chunk, nch_qk, nch_e, pv_chunk, nch_pv;
  int64_t ld;
  size_t off_score, off_e, off_stats, off_rec, off_spec, off_cnt, off_sum, off_status, off_dbg, off_part,
      total;
  // resident path (rG == 0: not available for this nfill)
  int rG, rkpw;
  bool rvres, rstream;
  size_t r_spec, r_e, r_sum, r_status, r_part, r_total;
  size_t ts_off;                 // experiment builds: per-wave timestamps (the last 128 KiB)
};

DecodePlan plan_decode(int nh, int nkv, int kfmt, int vfmt, int64_t nfill, int page = 0);
int qk_keys_per_wg(int kfmt);

int resident_max_workgroups(int kf, int vf);
hipError_t launch_resident(const ResArgs &a, int kf, int vf, bool vres, hipStream_t st);
int stream_max_workgroups(bool paged);
hipError_t launch_stream(const ResArgs &a, int kf, hipStream_t st);
hipError_t launch_workspace_init(unsigned *sync, size_t nwords, hipStream_t st);
// records a HIP error for bkv_last_hip_error and maps it to BKV_EHIP (BKV_OK for hipSuccess)
int hip_fail(hipError_t e);
hipError_t launch_fill_words(unsigned *p, size_t nwords, unsigned value, hipStream_t st);
hipError_t launch_append(const AppendArgs &a, int kf, int vf, int n_tok, hipStream_t st);
hipError_t launch_decode(const QkArgs &qa, const EArgs &ea, const PvArgs &pa, const RedArgs &ra,
                         int kf, int vf, bool fuse, hipStream_t st);

}  // namespace bkv
