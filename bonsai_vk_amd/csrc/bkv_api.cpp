// bkv_api.cpp - the C ABI (include/bkv.h): descriptor validation, partition planning, workspace
// layout and kernel dispatch. No allocation, no host synchronisation, no exception crosses out.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "../../include/bkv.h"
#include "bkv_internal.h"

namespace bkv {

static thread_local char g_hip_err[256] = "";

int hip_fail(hipError_t e) {
  if (e == hipSuccess) return BKV_OK;
  std::snprintf(g_hip_err, sizeof g_hip_err, "%s: %s", hipGetErrorName(e), hipGetErrorString(e));
  return BKV_EHIP;
}

static inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
static inline int64_t next_pow2(int64_t x) {
  int64_t p = 1;
  while (p < x) p <<= 1;
  return p;
}
static inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }
// the fewest keys a resident or stream workgroup takes (short contexts use fewer workgroups; at 4K
// keys, config 2: 128 (33 workgroups per group) 149.7-150.8 us per token, 96 150.9-152.4, 112
// 150.9-153.6, 64 154.0-156.0, 80 159.1-164.0; more than 128 leaves the short plan)
constexpr int64_t kResMinKeysPerWg = 128;

// Partition sizes of the split path. QK: the LDS K tile of one workgroup (256 q8_0 / 128 fp16
// keys). Probability chunks: kE2Chunk keys. PV: enough workgroups to cover the chip (512 at nkv = 4)
// with 16..512 keys each. Every array is sized
// by a bound that grows monotonically with n, so a workspace sized for max_ctx fits every n <= max_ctx.
// BKV_DECODE forces a decode implementation where its plan fits: "split" (four launches),
// "resident" or "stream" (single launches). Without it, q8_0 K + V plans that fit the stream kernel
// take it, other single-launch plans the resident kernel, the rest the split path. Read on every
// call, so tests can switch it.
enum { kPathSplit = 0, kPathResident = 2, kPathStream = 3 };
static int forced_path() {
  const char *e = std::getenv("BKV_DECODE");
  if (!e) return -1;
  if (std::strcmp(e, "split") == 0) return kPathSplit;
  if (std::strcmp(e, "resident") == 0) return kPathResident;
  if (std::strcmp(e, "stream") == 0) return kPathStream;
  return -1;
}

// Chunked prefill: 16 queries x 4 heads per workgroup; when that gives fewer than kPfFill
// workgroups the key range of every query block is split so that the chip fills (never into more
// splits than the first query block has 64-key tiles).
static int prefill_splits(int nkv, int nqb, int64_t first_keys) {
  const int64_t want = std::max<int64_t>(1, cdiv(kPfFill, (int64_t)nkv * nqb));
  return (int)std::min<int64_t>(want, std::max<int64_t>(1, cdiv(first_keys, kPfTile)));
}

// BKV_PREFILL=mfma selects the matrix-core prefill (scores and sums in MFMA order: within
// tolerance of the serial reference on long rows, not bit-identical probabilities); the default
// is the exact path, one decode row per query.
static bool prefill_mfma_requested() {
  const char *e = std::getenv("BKV_PREFILL");
  return e && std::strcmp(e, "mfma") == 0;
}

// Prefill arrays start past every array a decode on the same workspace can use (the decode plan
// at the cache's full capacity): the resident decode polls its partials for generation tags, so no
// other path may leave bytes in that region.
PrefillPlan plan_prefill(int nh, int nkv, uint32_t pos0, int n_q, size_t base) {
  PrefillPlan p{};
  p.nqb = (int)cdiv(n_q, kPfQ);
  p.nsplit = prefill_splits(nkv, p.nqb, (int64_t)pos0 + std::min(n_q, kPfQ));
  const size_t rows = (size_t)n_q * nh;
  size_t o = base;
  p.off_stats = o;
  o = align256(o + (size_t)p.nsplit * rows * sizeof(float2));
  p.off_part = o;
  if (p.nsplit > 1) o = align256(o + (size_t)p.nsplit * rows * kHd * sizeof(float));
  p.total = o;
  return p;
}

// the exact prefill's workspace for chunks ending at or before max_ctx: per workgroup of one slice,
// the [keys][rows] score / exp scratch; then (q8_0 V) the slice's sums and the PV kernel's partials
static size_t prefill_exact_extra(int nh, int nkv) {
  const size_t wgs = (size_t)nkv * (kPxSlice / kPxQ);
  return align256(wgs * kPxRows * sizeof(float)) + align256((size_t)kPvSplit * kPxSlice * nh * kHd * sizeof(float));
}
size_t prefill_exact_workspace(int nh, int nkv, int64_t max_ctx, size_t base) {
  const int64_t ld = cdiv(max_ctx, kPxTile) * kPxTile + kPxTile;   // + the exp sweep's overhang
  const size_t wgs = (size_t)nkv * (kPxSlice / kPxQ);
  return base + align256(wgs * (size_t)ld * kPxRows * sizeof(float)) + prefill_exact_extra(nh, nkv);
}

// the largest plan_prefill(...).total over every chunk length and start position
size_t prefill_workspace_bound(int nh, int nkv, size_t base) {
  size_t worst = 0;
  for (int nqb = 1; nqb <= BKV_PREFILL_MAX_Q / kPfQ; ++nqb) {
    const int nsplit = (int)std::max<int64_t>(1, cdiv(kPfFill, (int64_t)nkv * nqb));
    const size_t rows = (size_t)nqb * kPfQ * nh;
    size_t o = align256(base + (size_t)nsplit * rows * sizeof(float2));
    if (nsplit > 1) o = align256(o + (size_t)nsplit * rows * kHd * sizeof(float));
    worst = std::max(worst, o);
  }
  return worst;
}

DecodePlan plan_decode(int nh, int nkv, int kfmt, int vfmt, int64_t n, int page) {
  DecodePlan p;
  p.qk_chunk = qk_keys_per_wg(kfmt);
  p.nch_qk = (int)cdiv(n, p.qk_chunk);
  p.nch_e = (int)cdiv(n, kE2Chunk);
  p.pv_chunk = (int)std::min<int64_t>(kPvMaxChunk, std::max<int64_t>(16, next_pow2(cdiv(n * nkv, 512))));
  p.nch_pv = (int)cdiv(n, p.pv_chunk);
  p.ld = cdiv(n, kE2Chunk) * kE2Chunk;
  const int64_t nq_bound = cdiv(n, 128);
  const int64_t np_bound = std::max<int64_t>(128, cdiv(n, kPvMaxChunk));
  // the single-launch kernels' tagged partials sit at a fixed offset that no other array of any
  // plan overlaps: a poll never sees bytes another path (or another context length) left there
  const size_t tagged_part = align256((size_t)nkv * kResMaxGroupWgs * kGqa * kHd * sizeof(unsigned long long));
  size_t o = kSyncBytes + tagged_part;
  p.off_score = o;  o += align256((size_t)nh * p.ld * sizeof(float));
  p.off_e = o;      o += align256((size_t)nh * p.ld * sizeof(float));
  p.off_stats = o;  o += align256((size_t)nh * nq_bound * sizeof(float2));
  p.off_rec = o;    o += align256((size_t)nh * p.nch_e * sizeof(ChunkRec));
  p.off_spec = o;   o += align256((size_t)nh * p.nch_e * kMaxSpecial * sizeof(Special));
  p.off_cnt = o;    o += align256((size_t)nh * kCounterStride * sizeof(unsigned));
  p.off_sum = o;    o += align256((size_t)nh * sizeof(float));
  p.off_status = o; o += align256((size_t)nh * sizeof(unsigned));
  p.off_dbg = o;    o += align256((size_t)nh * 8 * sizeof(unsigned long long));
  p.off_part = o;   o += align256((size_t)np_bound * nh * kHd * sizeof(float));
  size_t total = o;
  // the resident path: one workgroup per CU, up to kResMaxG per KV group, >= 128 keys each
  // (below 64 x kResMinKeysPerWg keys fewer workgroups per group, each with at least that many keys)
  p.rG = 0;
  p.rvres = p.rstream = false;
  const int rcap = resident_max_workgroups(kfmt, vfmt);
  const bool rsync_fits = kResSyncOffset + ((size_t)nkv * kResGroupLines + 1) * kCounterStride * sizeof(unsigned) <= kSyncBytes;
  const bool rtags_fit = kResTagOffset + (size_t)nh * kResMaxGroupWgs * 3 * sizeof(unsigned long long) <= kResSyncOffset;
  if (rcap >= nkv && rsync_fits && rtags_fit) {
    const int64_t gmax = std::min<int64_t>(rcap / nkv, kResMaxGroupWgs);
    const int64_t kpw = cdiv(n, std::min<int64_t>(gmax, cdiv(n, kResMinKeysPerWg)));
    // paged: a workgroup's keys must span at most kResPgMax pages (the kernel's LDS page table)
    const bool pages_fit = page <= 0 || cdiv(kpw, page) + 1 <= kResPgMax;
    if (kpw <= (int64_t)kResMaxPass * kResNT && pages_fit) {
      p.rkpw = (int)kpw;
      p.rG = (int)cdiv(n, kpw);
      p.rvres = vfmt == BKV_Q8_0 && kfmt == BKV_Q8_0 && kpw <= kResNT + kResTail;
      // the stream kernel: q8_0 V with q8_0 or fp16 K, one pass plus a tail per workgroup
      p.rstream = vfmt == BKV_Q8_0 && (kfmt == BKV_Q8_0 || kfmt == BKV_F16) && kpw <= kResNT + kResTail &&
                  p.rG * nkv <= stream_max_workgroups(page > 0);
      p.r_part = kSyncBytes;
      size_t f = kSyncBytes + tagged_part;
      p.r_spec = f;   f += align256((size_t)nh * gmax * kMaxSpecial * sizeof(Special));
      p.r_e = f;      f += align256((size_t)nh * p.ld * sizeof(float));
      p.r_sum = f;    f += align256((size_t)nh * sizeof(float));
      p.r_status = f; f += align256((size_t)nh * sizeof(unsigned));
      p.r_total = f;
      total = std::max(total, f);
    }
  }
#ifdef BKV_EXPERIMENT_TS
  total = align256(total) + 262144;
  p.ts_off = total - 262144;
#endif
  p.total = total;
  return p;
}

// BKV_KEEP_INTERMEDIATES=1: the resident path also writes every e_j into the workspace (where
// bkv_debug_layout says) for parity diagnostics; the other paths always do
static bool keep_intermediates() {
  const char *e = std::getenv("BKV_KEEP_INTERMEDIATES");
  return e && std::strcmp(e, "1") == 0;
}

// which implementation a decode of this plan takes
static int choose_path(const DecodePlan &p) {
  const int f = forced_path();
  if (f == kPathSplit) return kPathSplit;
  if (f == kPathResident && p.rG > 0) return kPathResident;
  if (p.rstream) return kPathStream;
  if (p.rG > 0) return kPathResident;
  return kPathSplit;
}

static bool aligned16(const void *p) { return p && ((uintptr_t)p & 15u) == 0; }

static uint64_t slot_bytes(const bkv_cache_desc *d, int which) {
  const int fmt = which < 2 ? d->k_fmt : d->v_fmt;
  const uint64_t hd = (uint64_t)d->hd, nkv = (uint64_t)d->nkv;
  switch (which) {
    case 0: case 2: return fmt == BKV_F16 ? nkv * hd * 2 : nkv * hd;
    default: return fmt == BKV_F16 ? 0 : nkv * (hd / 32) * 2;
  }
}

static int check(const bkv_cache_desc *d) {
  if (!d) return BKV_EINVAL;
  if (d->n_layers < 1 || d->nkv < 1 || d->nh < 1 || d->hd < 1 || d->cap < 1) return BKV_EINVAL;
  if ((d->k_fmt != BKV_F16 && d->k_fmt != BKV_Q8_0) || (d->v_fmt != BKV_F16 && d->v_fmt != BKV_Q8_0))
    return BKV_EINVAL;
  // KvGeom::check (runtime_vk/kv_guard.h:103-113)
  if (d->hd % 4 || d->hd % 32 || (d->hd / 32) % 2) return BKV_ESHAPE;
  if (d->nh % d->nkv) return BKV_ESHAPE;
  if (!(std::isfinite(d->scale)) || d->scale <= 0.0f) return BKV_EINVAL;
  if (d->page_tokens < 0) return BKV_EINVAL;
  if (d->page_tokens > 0) {
    if (d->cap % d->page_tokens || d->max_pages < 1 || !d->block_table) return BKV_EINVAL;
  }
  if (!d->k_data || !d->v_data) return BKV_EINVAL;
  if (d->k_fmt == BKV_Q8_0 && !d->k_scales) return BKV_EINVAL;
  if (d->v_fmt == BKV_Q8_0 && !d->v_scales) return BKV_EINVAL;
  const void *ptrs[4] = {d->k_data, d->k_scales, d->v_data, d->v_scales};
  for (int i = 0; i < 4; ++i) {
    const uint64_t sb = slot_bytes(d, i);
    if (!sb) continue;
    if (!aligned16(ptrs[i])) return BKV_EALIGN;
    if (d->n_layers > 1 && d->layer_stride_bytes[i] < sb * (uint64_t)d->cap) return BKV_EINVAL;
    if (d->layer_stride_bytes[i] % 16) return BKV_EALIGN;
  }
  return BKV_OK;
}

// shapes the gfx950 kernels are specialised for: hd 256 and 4 query heads per KV head
static int check_kernels(const bkv_cache_desc *d) {
  if (d->hd != kHd || d->nh != kGqa * d->nkv) return BKV_EUNSUPPORTED;
  return BKV_OK;
}

static int64_t max_positions(const bkv_cache_desc *d) {
  return d->page_tokens > 0 ? (int64_t)d->max_pages * d->page_tokens : (int64_t)d->cap;
}

// where a prefill's own arrays begin: past the largest decode plan this cache allows
static size_t prefill_base(const bkv_cache_desc *d) {
  return align256(plan_decode(d->nh, d->nkv, d->k_fmt, d->v_fmt, max_positions(d), d->page_tokens).total);
}

static LayerView view(const bkv_cache_desc *d, int layer) {
  LayerView L;
  auto at = [&](void *base, int i) -> const uint8_t * {
    return base ? (const uint8_t *)base + (uint64_t)layer * d->layer_stride_bytes[i] : nullptr;
  };
  L.kd = at(d->k_data, 0);
  L.ks = at(d->k_scales, 1);
  L.vd = at(d->v_data, 2);
  L.vs = at(d->v_scales, 3);
  L.bt = d->page_tokens > 0 ? d->block_table + (int64_t)layer * d->max_pages : nullptr;
  L.page = d->page_tokens > 0 ? d->page_tokens : 0;
  L.base = 0;
  return L;
}

// q / gate: head rows qs / gs floats apart (hd for [nh][hd]; 2*hd for the engine's interleaved
// attn_q output, q then gate per head)
static int decode_common(const bkv_cache_desc *d, int layer, uint32_t nfill, const float *q,
                         const float *gate, float *out, float *out_gated, void *ws, size_t ws_bytes,
                         hipStream_t st, const AppendArgs *fused, int qs = kHd, int gs = kHd,
                         uint32_t kstart = 0) {
  int rc = check(d);
  if (rc) return rc;
  if ((rc = check_kernels(d))) return rc;
  if (layer < 0 || layer >= d->n_layers) return BKV_EINVAL;
  if (nfill == 0 || (int64_t)nfill > max_positions(d)) return BKV_ECAP;
  if (!aligned16(q) || !aligned16(out)) return q && out ? BKV_EALIGN : BKV_EINVAL;
  if ((gate == nullptr) != (out_gated == nullptr)) return BKV_EINVAL;
  if (gate && (!aligned16(gate) || !aligned16(out_gated))) return BKV_EALIGN;
  if (!ws) return BKV_EWORKSPACE;
  if (((uintptr_t)ws & 255u) != 0) return BKV_EALIGN;
  // a window [kstart, nfill): the kernels see nfill - kstart keys starting at position kstart
  if (kstart >= nfill) return BKV_EINVAL;
  nfill -= kstart;
  const DecodePlan p = plan_decode(d->nh, d->nkv, d->k_fmt, d->v_fmt, nfill, d->page_tokens);
  if (ws_bytes < p.total) return BKV_EWORKSPACE;
  char *w = (char *)ws;
  LayerView L = view(d, layer);
  L.base = kstart;

  const int path = choose_path(p);
  if (path == kPathResident || path == kPathStream) {
    ResArgs ra{};
    ra.L = L; ra.nkv = d->nkv; ra.nh = d->nh; ra.nfill = nfill; ra.scale = d->scale;
    ra.G = p.rG; ra.kpw = p.rkpw; ra.ld = p.ld; ra.q = q; ra.qs = qs; ra.gs = gs;
    if (fused) ra.ap = *fused;
    ra.gate = gate; ra.out = out; ra.out_gated = out_gated;
    ra.tstats = (unsigned long long *)(w + kResTagOffset);
    ra.trec = ra.tstats + (size_t)d->nh * kResMaxGroupWgs;
    ra.spec = (Special *)(w + p.r_spec);
    ra.e = (float *)(w + p.r_e);
    ra.keep_e = keep_intermediates() ? 1 : 0;
    ra.sum = (float *)(w + p.r_sum);
    ra.status = (unsigned *)(w + p.r_status);
    ra.part = (unsigned long long *)(w + p.r_part);
    ra.sync = (unsigned *)(w + kResSyncOffset);
#ifdef BKV_EXPERIMENT_TS
    ra.ts = (unsigned *)w + 32768;
    ra.tsw = (unsigned *)(w + p.ts_off);
#endif
    if (path == kPathStream) return hip_fail(launch_stream(ra, d->k_fmt, st));
    return hip_fail(launch_resident(ra, d->k_fmt, d->v_fmt, p.rvres, st));
  }

  QkArgs qa{};
  qa.L = L; qa.nkv = d->nkv; qa.nfill = nfill; qa.nch = p.nch_qk; qa.ld = p.ld; qa.scale = d->scale;
  qa.q = q;
  qa.qs = qs;
  qa.score = (float *)(w + p.off_score);
  qa.stats = (float2 *)(w + p.off_stats);
  qa.counters = (unsigned *)(w + p.off_cnt);
  if (fused) qa.ap = *fused;
  EArgs ea{};
  ea.nh = d->nh; ea.nfill = nfill; ea.nch_qk = p.nch_qk; ea.qk_chunk = p.qk_chunk; ea.nch = p.nch_e;
  ea.ld = p.ld; ea.scale = d->scale; ea.score = qa.score; ea.stats = qa.stats;
  ea.e = (float *)(w + p.off_e);
  ea.rec = (ChunkRec *)(w + p.off_rec);
  ea.spec = (Special *)(w + p.off_spec);
  ea.counters = qa.counters;
  ea.sum = (float *)(w + p.off_sum);
  ea.status = (unsigned *)(w + p.off_status);
  ea.dbg = (unsigned long long *)(w + p.off_dbg);
  PvArgs pa{};
  pa.L = L; pa.nkv = d->nkv; pa.nh = d->nh; pa.nfill = nfill; pa.chunk = p.pv_chunk;
  pa.nch = p.nch_pv; pa.ld = p.ld; pa.e = ea.e; pa.sum = ea.sum;
  pa.part = (float *)(w + p.off_part);
  RedArgs ra{};
  ra.nh = d->nh; ra.nch = p.nch_pv; ra.part = pa.part; ra.gate = gate; ra.gs = gs; ra.out = out;
  ra.out_gated = out_gated;
  return hip_fail(launch_decode(qa, ea, pa, ra, d->k_fmt, d->v_fmt, fused != nullptr, st));
}

}  // namespace bkv

using namespace bkv;

extern "C" {

int bkv_geom_check(const bkv_cache_desc *d) { return check(d); }

uint64_t bkv_slot_bytes(const bkv_cache_desc *d, int which) {
  if (!d || which < 0 || which > 3) return 0;
  return slot_bytes(d, which);
}

int64_t bkv_max_positions(const bkv_cache_desc *d) {
  if (check(d)) return 0;
  return max_positions(d);
}

int bkv_kv_append(const bkv_cache_desc *d, int layer, uint32_t pos, int n_tok, const float *k,
                  const float *v, hipStream_t stream) {
  int rc = check(d);
  if (rc) return rc;
  if ((rc = check_kernels(d))) return rc;
  if (layer < 0 || layer >= d->n_layers || n_tok < 0) return BKV_EINVAL;
  if (n_tok == 0) return BKV_OK;
  if ((int64_t)pos + n_tok > max_positions(d)) return BKV_ECAP;
  if (!k || !v) return BKV_EINVAL;
  if (!aligned16(k) || !aligned16(v)) return BKV_EALIGN;
  AppendArgs a{};
  a.L = view(d, layer);
  a.nkv = d->nkv;
  a.pos = pos;
  a.k = k;
  a.v = v;
  return hip_fail(launch_append(a, d->k_fmt, d->v_fmt, n_tok, stream));
}

int bkv_qk_norm_rope_append(const bkv_cache_desc *d, int layer, uint32_t pos0, int n_tok,
                            const float *q_in, const float *k_in, const float *v_in,
                            const float *qn_w, const float *kn_w, int nrot, float eps,
                            float freq_base, float *q_out, hipStream_t stream) {
  int rc = check(d);
  if (rc) return rc;
  if ((rc = check_kernels(d))) return rc;
  if (layer < 0 || layer >= d->n_layers || n_tok < 0) return BKV_EINVAL;
  if (nrot < 0 || nrot > d->hd || (nrot & 1)) return BKV_EINVAL;
  if (!(eps >= 0.0f) || !std::isfinite(freq_base) || freq_base <= 0.0f) return BKV_EINVAL;
  if (n_tok == 0) return BKV_OK;
  if ((int64_t)pos0 + n_tok > max_positions(d)) return BKV_ECAP;
  const void *ptrs[6] = {q_in, k_in, v_in, qn_w, kn_w, q_out};
  for (const void *p : ptrs) {
    if (!p) return BKV_EINVAL;
    if (!aligned16(p)) return BKV_EALIGN;
  }
  NormRopeArgs a{};
  a.L = view(d, layer);
  a.nkv = d->nkv;
  a.nh = d->nh;
  a.nrot = nrot;
  a.pos0 = pos0;
  a.eps = eps;
  a.freq_base = freq_base;
  a.q_in = q_in; a.k_in = k_in; a.v_in = v_in;
  a.qn_w = qn_w; a.kn_w = kn_w;
  a.q_out = q_out;
  return hip_fail(launch_norm_rope_append(a, d->k_fmt, d->v_fmt, n_tok, stream));
}

int bkv_attn_decode(const bkv_cache_desc *d, int layer, uint32_t nfill, const float *q,
                    const float *gate, float *out, float *out_gated, void *workspace,
                    size_t ws_bytes, hipStream_t stream) {
  return decode_common(d, layer, nfill, q, gate, out, out_gated, workspace, ws_bytes, stream,
                       nullptr);
}

static int decode_step_common(const bkv_cache_desc *d, int layer, uint32_t pos, const float *k,
                              const float *v, const float *q, const float *gate, float *out,
                              float *out_gated, void *workspace, size_t ws_bytes, hipStream_t stream,
                              int qs, int gs) {
  int rc = check(d);
  if (rc) return rc;
  if (layer < 0 || layer >= d->n_layers) return BKV_EINVAL;
  if ((int64_t)pos + 1 > max_positions(d)) return BKV_ECAP;
  if (!k || !v) return BKV_EINVAL;
  if (!aligned16(k) || !aligned16(v)) return BKV_EALIGN;
  AppendArgs a{};
  a.L = view(d, layer);
  a.nkv = d->nkv;
  a.pos = pos;
  a.k = k;
  a.v = v;
  return decode_common(d, layer, pos + 1, q, gate, out, out_gated, workspace, ws_bytes, stream, &a,
                       qs, gs);
}

int bkv_decode_step(const bkv_cache_desc *d, int layer, uint32_t pos, const float *k,
                    const float *v, const float *q, const float *gate, float *out,
                    float *out_gated, void *workspace, size_t ws_bytes, hipStream_t stream) {
  return decode_step_common(d, layer, pos, k, v, q, gate, out, out_gated, workspace, ws_bytes,
                            stream, kHd, kHd);
}

// the _qg variants read Q and the gate from the engine's attn_q output: per head, hd values of q
// then hd values of the gate (the layout deint_qg splits, runtime_vk/shaders/deint_qg.comp)
int bkv_attn_decode_window(const bkv_cache_desc *d, int layer, uint32_t kstart, uint32_t nfill,
                           const float *q, const float *gate, float *out, float *out_gated,
                           void *workspace, size_t ws_bytes, hipStream_t stream) {
  return decode_common(d, layer, nfill, q, gate, out, out_gated, workspace, ws_bytes, stream,
                       nullptr, kHd, kHd, kstart);
}

int bkv_attn_decode_qg(const bkv_cache_desc *d, int layer, uint32_t nfill, const float *qg,
                       float *out, float *out_gated, void *workspace, size_t ws_bytes,
                       hipStream_t stream) {
  if (!qg) return BKV_EINVAL;
  return decode_common(d, layer, nfill, qg, out_gated ? qg + kHd : nullptr, out, out_gated,
                       workspace, ws_bytes, stream, nullptr, 2 * kHd, 2 * kHd);
}

int bkv_decode_step_qg(const bkv_cache_desc *d, int layer, uint32_t pos, const float *k,
                       const float *v, const float *qg, float *out, float *out_gated,
                       void *workspace, size_t ws_bytes, hipStream_t stream) {
  if (!qg) return BKV_EINVAL;
  return decode_step_common(d, layer, pos, k, v, qg, out_gated ? qg + kHd : nullptr, out, out_gated,
                            workspace, ws_bytes, stream, 2 * kHd, 2 * kHd);
}

static int prefill_common(const bkv_cache_desc *d, int layer, uint32_t pos0, int n_q,
                          const float *q, const float *gate, float *out, float *out_gated,
                          void *workspace, size_t ws_bytes, hipStream_t stream, int qs, int gs) {
  int rc = check(d);
  if (rc) return rc;
  if ((rc = check_kernels(d))) return rc;
  if (layer < 0 || layer >= d->n_layers) return BKV_EINVAL;
  if (n_q < 0 || n_q > BKV_PREFILL_MAX_Q) return BKV_EINVAL;
  if (n_q == 0) return BKV_OK;
  if ((int64_t)pos0 + n_q > max_positions(d)) return BKV_ECAP;
  if (!aligned16(q) || !aligned16(out)) return q && out ? BKV_EALIGN : BKV_EINVAL;
  if ((gate == nullptr) != (out_gated == nullptr)) return BKV_EINVAL;
  if (gate && (!aligned16(gate) || !aligned16(out_gated))) return BKV_EALIGN;
  if (!workspace) return BKV_EWORKSPACE;
  if (((uintptr_t)workspace & 255u) != 0) return BKV_EALIGN;
  const size_t base = prefill_base(d);
  if (!prefill_mfma_requested() && n_q >= kPxMinQ) {
    // the exact kernel, in slices of at most kPxSlice queries
    const int64_t ld = cdiv((int64_t)pos0 + n_q, kPxTile) * kPxTile + kPxTile;
    if (ws_bytes < prefill_exact_workspace(d->nh, d->nkv, (int64_t)pos0 + n_q, base)) return BKV_EWORKSPACE;
    char *w = (char *)workspace;
    PrefillXArgs a{};
    a.L = view(d, layer);
    a.nkv = d->nkv;
    a.nh = d->nh;
    a.pos0 = pos0;
    a.chunk_q = n_q;
    a.scale = d->scale;
    a.ld = ld;
    a.q = q;
    a.qs = qs;
    a.gs = gs;
    a.sc = (float *)(w + base);
    {
      const size_t scb = align256((size_t)d->nkv * (kPxSlice / kPxQ) * (size_t)ld * kPxRows * sizeof(float));
      a.sums = (float *)(w + base + scb);
      a.part = (float *)(w + base + scb + align256((size_t)d->nkv * (kPxSlice / kPxQ) * kPxRows * sizeof(float)));
    }
    a.gate = gate;
    a.out = out;
    a.out_gated = out_gated;
#ifdef BKV_EXPERIMENT_TS
    a.ts = (unsigned *)w + 32768;
#endif
    for (int qb = 0; qb < n_q; qb += kPxSlice) {
      a.q_base = qb;
      a.n_q = std::min(kPxSlice, n_q - qb);
      a.nqb = (int)cdiv(a.n_q, kPxQ);
      if ((rc = hip_fail(launch_prefill_exact(a, d->k_fmt, d->v_fmt, stream)))) return rc;
    }
    return BKV_OK;
  }
  if (!prefill_mfma_requested()) {
    // short chunks: every row is the decode row at nfill = pos0 + i + 1
    const size_t rs = (size_t)d->nh * d->hd;
    for (int i = 0; i < n_q; ++i) {
      rc = decode_common(d, layer, pos0 + (uint32_t)i + 1u, q + i * (size_t)d->nh * qs,
                         gate ? gate + i * (size_t)d->nh * gs : nullptr, out + i * rs,
                         out_gated ? out_gated + i * rs : nullptr, workspace, ws_bytes, stream,
                         nullptr, qs, gs);
      if (rc) return rc;
    }
    return BKV_OK;
  }
  const PrefillPlan p = plan_prefill(d->nh, d->nkv, pos0, n_q, base);
  if (ws_bytes < p.total) return BKV_EWORKSPACE;
  char *w = (char *)workspace;
  PrefillArgs a{};
  a.L = view(d, layer);
  a.nkv = d->nkv;
  a.nh = d->nh;
  a.pos0 = pos0;
  a.n_q = n_q;
  a.scale = d->scale;
  a.nqb = p.nqb;
  a.nsplit = p.nsplit;
  a.q = q;
  a.gate = gate;
  a.out = out;
  a.out_gated = out_gated;
  a.stats = (float2 *)(w + p.off_stats);
  a.part = p.nsplit > 1 ? (float *)(w + p.off_part) : nullptr;
  a.qs = qs;
  a.gs = gs;
  return hip_fail(launch_prefill(a, d->k_fmt, d->v_fmt, stream));
}

int bkv_attn_prefill_chunk(const bkv_cache_desc *d, int layer, uint32_t pos0, int n_q,
                           const float *q, const float *gate, float *out, float *out_gated,
                           void *workspace, size_t ws_bytes, hipStream_t stream) {
  return prefill_common(d, layer, pos0, n_q, q, gate, out, out_gated, workspace, ws_bytes, stream,
                        kHd, kHd);
}

int bkv_prefill_step(const bkv_cache_desc *d, int layer, uint32_t pos0, int n_q, const float *k,
                     const float *v, const float *q, const float *gate, float *out,
                     float *out_gated, void *workspace, size_t ws_bytes, hipStream_t stream) {
  int rc = check(d);
  if (rc) return rc;
  if (n_q < 0 || n_q > BKV_PREFILL_MAX_Q) return BKV_EINVAL;
  if (layer < 0 || layer >= d->n_layers) return BKV_EINVAL;
  if ((int64_t)pos0 + n_q > max_positions(d)) return BKV_ECAP;
  if (!workspace) return BKV_EWORKSPACE;
  if (((uintptr_t)workspace & 255u) != 0) return BKV_EALIGN;
  if (!q || !out) return BKV_EINVAL;
  if ((rc = bkv_kv_append(d, layer, pos0, n_q, k, v, stream))) return rc;
  return bkv_attn_prefill_chunk(d, layer, pos0, n_q, q, gate, out, out_gated, workspace, ws_bytes,
                                stream);
}

int bkv_attn_prefill_chunk_qg(const bkv_cache_desc *d, int layer, uint32_t pos0, int n_q,
                              const float *qg, float *out, float *out_gated, void *workspace,
                              size_t ws_bytes, hipStream_t stream) {
  if (!qg) return BKV_EINVAL;
  return prefill_common(d, layer, pos0, n_q, qg, out_gated ? qg + kHd : nullptr, out, out_gated,
                        workspace, ws_bytes, stream, 2 * kHd, 2 * kHd);
}

size_t bkv_workspace_bytes(const bkv_cache_desc *d, int op, uint32_t max_ctx) {
  if (check(d) || max_ctx == 0) return 0;
  if (op == BKV_OP_PREFILL)
    return std::max(prefill_workspace_bound(d->nh, d->nkv, prefill_base(d)),
                    prefill_exact_workspace(d->nh, d->nkv, max_ctx, prefill_base(d)));
  if (op != BKV_OP_DECODE) return 0;
  return plan_decode(d->nh, d->nkv, d->k_fmt, d->v_fmt, max_ctx, d->page_tokens).total;
}

const char *bkv_strerror(int err) {
  switch (err) {
    case BKV_OK: return "ok";
    case BKV_EINVAL: return "invalid argument";
    case BKV_ESHAPE: return "cache geometry rule broken (hd%4, hd%32, hd/32 even, nh%nkv)";
    case BKV_ECAP: return "position outside the cache (pos >= cap) or empty context";
    case BKV_EALIGN: return "pointer or stride not aligned (16 B; workspace 256 B)";
    case BKV_EWORKSPACE: return "workspace missing or smaller than bkv_workspace_bytes()";
    case BKV_ESCRATCH: return "decode plan larger than the static scratch (bkv_static_scratch_bytes())";
    case BKV_EHIP: return "HIP runtime error (see bkv_last_hip_error)";
    case BKV_EUNSUPPORTED: return "shape not supported by the gfx950 kernels (hd 256, nh = 4*nkv)";
    case BKV_ETIMEOUT: return "a decode kernel's workgroup wait timed out (its output is not valid)";
    default: return "unknown error";
  }
}

// byte offset of the single-launch kernels' error word (past their sync lines)
static uint64_t error_word_offset(int nkv) {
  return kResSyncOffset + (uint64_t)nkv * kResGroupLines * kCounterStride * sizeof(unsigned);
}

int bkv_error_words(const bkv_cache_desc *d, uint64_t out[1]) {
  const int rc = check(d);
  if (rc) return rc;
  if (!out) return BKV_EINVAL;
  out[0] = error_word_offset(d->nkv);
  return BKV_OK;
}

int bkv_workspace_error(const bkv_cache_desc *d, void *workspace, size_t ws_bytes, hipStream_t stream) {
  const int rc = check(d);
  if (rc) return rc;
  if (!workspace || ws_bytes < kSyncBytes) return BKV_EWORKSPACE;
  const uint64_t off[1] = {error_word_offset(d->nkv)};
  hipError_t e = hipStreamSynchronize(stream);
  if (e != hipSuccess) return hip_fail(e);
  int result = BKV_OK;
  for (uint64_t o : off) {
    unsigned v = 0;
    char *p = static_cast<char *>(workspace) + o;
    if ((e = hipMemcpy(&v, p, sizeof v, hipMemcpyDeviceToHost)) != hipSuccess) return hip_fail(e);
    if (v) result = BKV_ETIMEOUT;
  }
  if (result == BKV_ETIMEOUT) {
    // a call that gave up left its counters and tags mid-protocol: start the workspace afresh (this
    // also clears the error word), as bkv_workspace_init does
    if ((e = launch_workspace_init((unsigned *)workspace, ws_bytes / sizeof(unsigned), stream)) != hipSuccess ||
        (e = hipStreamSynchronize(stream)) != hipSuccess)
      return hip_fail(e);
  }
  return result;
}

int bkv_debug_layout(const bkv_cache_desc *d, uint32_t nfill, uint64_t out[6]) {
  const int rc = check(d);
  if (rc) return rc;
  if (!out || nfill == 0) return BKV_EINVAL;
  const DecodePlan p = plan_decode(d->nh, d->nkv, d->k_fmt, d->v_fmt, nfill, d->page_tokens);
  const int path = choose_path(p);
  out[0] = (uint64_t)p.ld;
  out[1] = path == kPathSplit ? p.off_score : 0;
  const bool res = path == kPathResident || path == kPathStream;
  out[2] = res ? p.r_e : p.off_e;
  out[3] = res ? p.r_sum : p.off_sum;
  out[4] = res ? p.r_status : p.off_status;
  out[5] = p.total;
  return BKV_OK;
}

int bkv_workspace_init(const bkv_cache_desc *d, void *workspace, size_t ws_bytes, hipStream_t stream) {
  const int rc = check(d);
  if (rc) return rc;
  if (!workspace) return BKV_EWORKSPACE;
  if (((uintptr_t)workspace & 255u) != 0) return BKV_EALIGN;
  if (ws_bytes < kSyncBytes) return BKV_EWORKSPACE;
  // the whole workspace: the sync words, and the tagged partials of the resident path (a tag is
  // the call generation, which starts at 1)
  return hip_fail(launch_workspace_init((unsigned *)workspace, ws_bytes / sizeof(unsigned), stream));
}

int bkv_kv_fill_synthetic(const bkv_cache_desc *d, hipStream_t stream) {
  const int rc = check(d);
  if (rc) return rc;
  const size_t slots = (size_t)d->cap * d->nkv;
  const size_t rows[4] = {slots * (size_t)row_bytes(d->k_fmt), slots * kScaleRowBytes,
                          slots * (size_t)row_bytes(d->v_fmt), slots * kScaleRowBytes};
  void *bases[4] = {d->k_data, d->k_scales, d->v_data, d->v_scales};
  for (int i = 0; i < 4; ++i) {
    if (!bases[i]) continue;
    for (int l = 0; l < d->n_layers; ++l) {
      unsigned *p = (unsigned *)((char *)bases[i] + (uint64_t)l * d->layer_stride_bytes[i]);
      const hipError_t e = launch_fill_words(p, rows[i] / 4, 0x3C003C00u, stream);
      if (e != hipSuccess) return hip_fail(e);
    }
  }
  return BKV_OK;
}

int bkv_decode_path(const bkv_cache_desc *d, uint32_t nfill) {
  if (check(d) || nfill == 0) return -1;
  return choose_path(plan_decode(d->nh, d->nkv, d->k_fmt, d->v_fmt, nfill, d->page_tokens));
}

const char *bkv_last_hip_error(void) { return g_hip_err; }

const char *bkv_version(void) { return "bkv 0.1 gfx950"; }

}  // extern "C"
