// bkv_resident.hip - the default decode kernel: one launch per layer and token, one 512-thread
// workgroup per CU, every workgroup resident for the whole call.
//
// Workgroup w serves KV group g = w % nkv and the kpw consecutive keys starting at (w / nkv) * kpw,
// one key per thread and pass (at most kResMaxPass passes). Per call:
//  1. The workgroup whose range holds pos appends the new token (decode_step). Each wave stages
//     its 64 K rows through a private LDS tile with coalesced loads; q16 of the group's 4 query heads
//     sits in registers, and each lane computes its key's 4 scores in the reference's order. For
//     q8_0 V with kpw <= 32 * kResVSlots, the V rows are loaded into registers right behind the K
//     rows, so the V stream overlaps the QK arithmetic and the barriers.
//  2. Barrier A (the group's workgroups): per-workgroup (max, sum exp) give the global max and
//     each workgroup's fp64 position on the running sum.
//  3. e_j = exp(s_j*scale - max) correctly rounded, each step of the serial fp32 sum classified as
//     an exact integer increment or a special; per-workgroup record and specials.
//  4. Barrier B: every workgroup walks the group's records itself to the exact serial sums (no
//     second hand-off for the result).
//  5. p16 = f16(e/sum) into LDS, PV over the workgroup's rows (from registers, or streamed), one
//     [4][256] partial per workgroup.
//  6. Barrier C: workgroup i sums slice i of the group's partials in workgroup order and applies the
//     gate.
// Barriers count arrivals on per-group counters (two sets, alternating by call parity; each call
// clears the set the next one uses). Every wait is bounded and records an error word on timeout.
#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <cstring>
#include <type_traits>

#include "bkv_common.h"
#include "bkv_device.h"
#include "bkv_exp.h"
#include "bkv_pv8.h"
#include "bkv_internal.h"
#include "bkv_res_shared.h"

namespace bkv {

constexpr int kResVTiles = 16;                // resident V row slots per lane (32 rows each)

// the register-resident variant: lane (wave, vkk, vsub) slot s holds bytes 16*vsub.. of row
// 32 s + 4 wave + vkk and that row's block-pair scale word (rows >= nk repeat row nk-1). XE: also
// xd / xs, the same for row 32 kResVTiles + 4 wave + vkk, the streamed slot past the resident rows
// (always loaded, so the count of loads in flight is fixed)
template <bool PG, bool XE>
__device__ __forceinline__ void load_v_regs(uint4 (&vd)[kResVTiles], uint32_t (&vs)[kResVTiles], uint4 &xd, uint32_t &xs,
                                            const SlotMap &sm, int nkv, int g, int nk) {
  const LayerView &L = *sm.L;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, vsub = lane & 15, vkk = lane >> 4;
#pragma unroll
  for (int s = 0; s < kResVTiles; ++s) {
    const int64_t slot = slot_k<PG>(sm, min(s * 32 + wave * 4 + vkk, nk - 1));
    vd[s] = *reinterpret_cast<const uint4 *>(L.vd + (slot * nkv + g) * kHd + vsub * 16);
    vs[s] = *reinterpret_cast<const uint32_t *>(L.vs + (slot * nkv + g) * kScaleRowBytes + (vsub >> 2) * 4);
  }
  if constexpr (XE) {
    const int64_t slot = slot_k<PG>(sm, min(kResVTiles * 32 + wave * 4 + vkk, nk - 1));
    xd = *reinterpret_cast<const uint4 *>(L.vd + (slot * nkv + g) * kHd + vsub * 16);
    xs = *reinterpret_cast<const uint32_t *>(L.vs + (slot * nkv + g) * kScaleRowBytes + (vsub >> 2) * 4);
  }
}
// vector loads load_v_regs issues per wave
template <bool XE>
constexpr int kVLoads = 2 * kResVTiles + (XE ? 2 : 0);

// PV over the resident slots, waiting for slot S only: out += p16 * V for the wave's rows
// 32 s + 4 wave + vkk, 16 elements per lane (attn_vk.h:194-205; q8_0 V = f16(scale) * int8)
template <int S>
struct VSlots {
  static __device__ __forceinline__ void run(const uint4 *kt, const uint32_t *tsc, int nk, int wave, int vkk,
                                             int vsub, int lane, const uint2 *s_p16,
                                             float (&acc)[kGqa][16]) {
    VSlots<S - 1>::run(kt, tsc, nk, wave, vkk, vsub, lane, s_p16, acc);
    constexpr int s = S - 1;
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kResVTiles - 1 - s) : "memory");
    if (s * 32 < nk) {
      const int k = s * 32 + wave * 4 + vkk;
      const uint2 pw = k < nk ? s_p16[k] : make_uint2(0u, 0u);
      const float p[kGqa] = {f16_to_f32(pw.x & 0xFFFFu), f16_to_f32(pw.x >> 16), f16_to_f32(pw.y & 0xFFFFu),
                             f16_to_f32(pw.y >> 16)};
      const uint32_t sw = tsc[(s * 4 + vkk) * 4 + (vsub >> 2)];
      const float vsc = k < nk ? f16_to_f32(((vsub >> 1) & 1) ? (sw >> 16) : (sw & 0xFFFFu)) : 0.0f;
      v_accum<BKV_Q8_0>(kt[s * 64 + lane], vsc, p, acc);
    }
  }
};
template <>
struct VSlots<0> {
  static __device__ __forceinline__ void run(const uint4 *, const uint32_t *, int, int, int, int, int, const uint2 *,
                                             float (&)[kGqa][16]) {}
};


// no lane of the wave needs is skipped.
template <bool DELTA>
__device__ __forceinline__ void pv_res_slots(const uint4 (&vd)[kResVTiles], const uint32_t (&vsw)[kResVTiles],
                                             const uint2 *p16, const uint2 *q16, int nk, int wave, int vkk,
                                             int vsub, float (&acc)[kGqa][KRow<BKV_Q8_0>::EPL]) {
  // each slot's probabilities are read from LDS one slot ahead (a read and its wait back to back
  // would stall every slot); keys past nk get zero weights by a select, not a branch
  const int kw = wave * 4 + vkk;
  uint2 pn = p16[kw], qn = DELTA ? q16[kw] : make_uint2(0u, 0u);
#pragma unroll
  for (int s = 0; s < kResVTiles; ++s) {
    if (s * 32 >= nk) break;
    const int k = s * 32 + kw;
    const bool live = k < nk;
    uint2 pw = pn, qw = qn;
    if (s + 1 < kResVTiles) {
      pn = p16[k + 32];
      if constexpr (DELTA) qn = q16[k + 32];
    }
    pw.x = live ? pw.x : 0u;
    pw.y = live ? pw.y : 0u;
    float p[kGqa] = {f16_to_f32(pw.x & 0xFFFFu), f16_to_f32(pw.x >> 16), f16_to_f32(pw.y & 0xFFFFu),
                     f16_to_f32(pw.y >> 16)};
    if constexpr (DELTA) {
      qw.x = live ? qw.x : 0u;
      qw.y = live ? qw.y : 0u;
      if (!__any(pw.x != qw.x || pw.y != qw.y)) continue;
      p[0] -= f16_to_f32(qw.x & 0xFFFFu);
      p[1] -= f16_to_f32(qw.x >> 16);
      p[2] -= f16_to_f32(qw.y & 0xFFFFu);
      p[3] -= f16_to_f32(qw.y >> 16);
    }
    const float vsc = live ? f16_to_f32(((vsub >> 1) & 1) ? (vsw[s] >> 16) : (vsw[s] & 0xFFFFu)) : 0.0f;
    v_accum<BKV_Q8_0>(vd[s], vsc, p, acc);
  }
}

template <int KF, int VF, bool VRES, bool PG>
__global__ __launch_bounds__(kResNT, 1) void resident_kernel(ResArgs a) {
  constexpr int NT = kResNT, NW = kResNW;
  // VRES: one pass of NT keys plus a tail of at most kResTail keys (wave 0, one lane per key and head).
  // The multi-pass form also ends in a tail when the keys past its whole passes are at most
  // kResTail, instead of a pass for them.
  constexpr int MP = VRES ? 1 : kResMaxPass;
  constexpr bool TAIL = true;
  constexpr int SB = MP * NT + (TAIL ? kResTail : 0);   // binade-map row per head
  using VR = KRow<VF>;
  static_assert(!VRES || (VF == BKV_Q8_0 && KF == BKV_Q8_0), "register V rows and the tail: q8_0 K and V only");
  // T: per-wave K tiles (64 rows x kUPR uint4 each); after the scores, each wave's q8_0 V rows
  // (68 rows x 256 B, the same bytes) and at the end the PV reduction and the merge.
  // X: the binade map, then the walk scratch, then the fp16 probabilities.
  using WS = WalkScratchT<kResMaxGroupWgs, 192>;
  __shared__ __attribute__((aligned(1024))) uint4 lds[NW * 64 * kUPR];
  static_assert(64 * kUPR * 16 == kPv8Region, "a wave's K tile holds its PV region");
  __shared__ uint4 ldx[kResXBytes / 16];
  static_assert(64 * kUPR * 16 == kResVTiles * 1024 + 64 * 16, "a wave's V rows and scales fill its K tile");
  static_assert(kResTail <= 16 && NT == 32 * kResVTiles, "the tail rows are the streamed slot");
  static_assert(kGqa * SB + kGqa * kMaxSpecial * sizeof(Special) <= sizeof(ldx), "binade map and staged specials must fit");
  static_assert(kGqa * sizeof(WS) <= sizeof(ldx), "walk scratch must fit");
  static_assert(SB * sizeof(uint2) <= sizeof(ldx), "p16 buffer must fit");
  static_assert(NW * kGqa * kHd * sizeof(float) <= sizeof(lds), "PV reduction must fit");
  __shared__ float2 s_ml[NW * kGqa];            // each wave's (max, sum of exps against it) per head
  __shared__ float4 s_wf[NW];
  __shared__ double s_wd[NW * kGqa];
  __shared__ int s_wc[NW * kGqa];
  __shared__ float s_M[kGqa], s_S[kGqa], s_Sa[kGqa];
  __shared__ double s_P0[kGqa];
  __shared__ int s_ok[kGqa];
  __shared__ long long s_tt[kGqa];
  __shared__ int s_tc[kGqa];
  __shared__ double s_t2[32];               // 2^(j/32), the table exp's
  __shared__ unsigned s_wide;                // q8_0 K: the digits do not fit (fp64 score path)

  // workgroups are dealt to the 8 XCDs round-robin by index; when the grid allows, the nkv groups
  // of one key range share an XCD, so the cache lines they split (each 64 B scale line holds all
  // groups' scales of a slot) are fetched once into that XCD's L2
  const int w = blockIdx.x, nkv = a.nkv, G = a.G;
  int g, wi;
  if ((G & 7) == 0 && ((int)gridDim.x & 7) == 0) {
    const int x = w & 7, loc = w >> 3;
    g = loc % nkv;
    wi = x * (G >> 3) + loc / nkv;
  } else {
    g = w % nkv;
    wi = w / nkv;
  }
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // the exp table: loaded here, stored to LDS once the scores are done (a wait for it here would
  // hold the K stream back by a round trip)
  const double t2v = tid < 32 ? kExp2Tab[tid] : 0.0;
  if (tid == 0) s_wide = 0u;                   // (read after the barrier that follows the digits)
  const int64_t kb = (int64_t)wi * a.kpw;
  const int64_t ke = min((int64_t)a.nfill, kb + (int64_t)a.kpw);
  const int nk = (int)max((int64_t)0, ke - kb);
  const LayerView &L = a.L;

  // sync lines of group g: generation, then counters A, B, C, F of parity 0 and of parity 1
  unsigned *gs = a.sync + (size_t)g * kResGroupLines * kCounterStride;
  unsigned *err = a.sync + (size_t)nkv * kResGroupLines * kCounterStride;
  const unsigned gen0 = ld_agent(gs);          // (first used after the scores, for the same reason)
  constexpr int GM = kResMaxGroupWgs;
  unsigned long long *tstats = a.tstats + (size_t)g * kGqa * GM;        // [kGqa][GM]
  unsigned long long *trec = a.trec + (size_t)g * kGqa * GM * 2;        // [kGqa][GM][2]
  if (wi == 0)                                  // entries of workgroups this call does not run
    for (int i = tid; i < kGqa * (GM - G); i += NT) {
      const int h = i / (GM - G), c = G + i % (GM - G);
      st_agent(tstats + h * GM + c, 0ull);
      st_agent(trec + (h * GM + c) * 2, 0ull);
      st_agent(trec + (h * GM + c) * 2 + 1, 0ull);
    }
  RTS(0);

  // decode_step: the workgroup whose keys hold the new token appends it, and only that workgroup
  // reads the row back (the others need not wait for anything before their first tile)
  const bool appender = a.ap.k && (int64_t)a.ap.pos >= kb && (int64_t)a.ap.pos < ke;
  // paged: the block-table entries of this workgroup's keys into LDS (the append's wait and
  // barrier below also cover these loads when it runs)
  __shared__ int s_pg[kResPgMax];
  SlotMap sm{&L, kb, s_pg, 0u};
  if constexpr (PG) {
    const uint32_t pgs = (uint32_t)L.page, pg0 = (uint32_t)(kb + L.base) / pgs,
                   pg1 = (uint32_t)(kb + max(nk, 1) - 1 + L.base) / pgs;
    sm.pf = pg0;
    if (tid <= (int)min(pg1 - pg0, (uint32_t)kResPgMax - 1u)) s_pg[tid] = L.bt[pg0 + tid];
    if (!appender) __syncthreads();
  }

  if (appender) {
    if (wave == 0) append_token<KF, VF, false>(a.ap, a.ap.pos, 0, g, lane);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }

  // ---------------------------------------------------------------- QK
  // the first pass's K tile goes out before q is read, so both arrive in one round trip (the wait
  // for q, issued after the tile, also covers it: loads complete in order)
  const int vsub = lane % VR::LPR, vkk = lane / VR::LPR;
  uint4 *kt = lds + wave * 64 * kUPR;
  const int n_first = (int)max((int64_t)0, min((int64_t)64, ke - (kb + wave * 64)));
  if (n_first > 0) stage_k_wave<KF, PG>(kt, sm, nkv, g, wave * 64, n_first, 0);
  // the tail's rows (keys NT .., wave 0) into the exchange area, free until the e phase
  // tb: the keys the passes cover, and the first tail key (the tail holds keys tb .. nk-1); the
  // forms whose tail is fixed keep constants (VRES: one pass, its tail starts at NT; no tail: nk)
  constexpr bool MTAIL = TAIL && !VRES;
  const int tb = MTAIL ? (nk > NT && nk % NT <= kResTail ? nk - nk % NT : nk) : VRES ? NT : nk;
  const int tpk = MTAIL ? tb : nk;         // pass keys are those below tpk
  const int tn = TAIL ? max(0, nk - tb) : 0;
  uint4 *tail_t = ldx;
  if (TAIL && tn > 0 && wave == 0) stage_k_wave<KF, PG>(tail_t, sm, nkv, g, tb, tn, 0);
  // q8_0 K: the digits of the group's q rows (int8 matrix cores, bkv_q8dot.h) in the exchange area
  // past the tail rows, free until the e phase; fp16 K: the q rows rounded to q16 for the score
  // chains ([head][256] fp32), past the whole 64-row tile the tail's staging writes (its loads may
  // still land while q16 is written: no barrier drains them first)
  const float *qg = a.q + (size_t)g * kGqa * a.qs;
  float *q16 = reinterpret_cast<float *>(reinterpret_cast<char *>(ldx) + 64 * kUPR * 16);
  static_assert(64 * kUPR * 16 + kGqa * kHd * 4 <= sizeof(ldx), "q16 beside the tail tile");
  Q8Lim qlim;
  bool wide = false;
  if constexpr (KF == BKV_Q8_0) {
    int8_t *s_lim = reinterpret_cast<int8_t *>(ldx) + kResTail * kUPR * 16;
    int *s_lt = reinterpret_cast<int *>(s_lim + kLimBytes);
    static_assert(kResTail * kUPR * 16 + kLimBytes + kGqa * 4 <= sizeof(ldx), "digits beside the tail rows");
    __syncthreads();                             // s_wide cleared
    q8lim_build(qg, a.qs, s_lim, s_lt, &s_wide, tid, NT);
    __syncthreads();
    q8lim_load(s_lim, s_lt, qlim);
    wide = s_wide != 0u;
  } else {
    for (int i = tid; i < kGqa * kHd; i += NT) q16[i] = round_f16(qg[(size_t)(i / kHd) * a.qs + i % kHd]);
    __syncthreads();
  }

  // VRES: this wave's V rows 32 s + 4 wave + vkk (s < kResVTiles) and their block-pair scale words,
  // loaded right behind the first K tile so that they stream in during the scores
  uint4 vd[VRES ? kResVTiles : 1];
  uint32_t vsw[VRES ? kResVTiles : 1];
  // XE (q8_0 K, contiguous: the variant with registers to spare): the streamed slot's V row loads
  // with the resident ones instead of at the start of PV, where its latency would sit on the
  // critical path
  constexpr bool XE = VRES && KF == BKV_Q8_0 && !PG;
  uint4 xw = make_uint4(0u, 0u, 0u, 0u);
  uint32_t xs = 0u;
  float sc[MP][kGqa];
  float mloc[kGqa];
#pragma unroll
  for (int h = 0; h < kGqa; ++h) mloc[h] = -INFINITY;
#pragma unroll
  for (int r = 0; r < MP; ++r) {
#pragma unroll
    for (int h = 0; h < kGqa; ++h) sc[r][h] = 0.0f;
    const int64_t j0 = kb + (int64_t)r * NT + wave * 64;
    const int k0 = r * NT + wave * 64;
    const int n = (int)max((int64_t)0, min((int64_t)64, kb + tpk - j0));
    if (n > 0) {
      float acc[kGqa];
#pragma unroll
      for (int h = 0; h < kGqa; ++h) acc[h] = 0.0f;
      if (r > 0) stage_k_wave<KF, PG>(kt, sm, nkv, g, k0, n, 0);
      if (VRES && r == 0) {
        if constexpr (VRES) load_v_regs<PG, XE>(vd, vsw, xw, xs, sm, nkv, g, nk);
        wait_vm<kVLoads<XE>>();                // the K tile has landed; the V rows stay in flight
      } else {
        wait_vm<0>();
      }
      if constexpr (KF == BKV_Q8_0) {
        if (!wide)
          q8_score64(kt, kUPR, qlim, acc);
        else
          q8_score_key_slow(kt + lane * kUPR, qg, a.qs, acc);
      } else {
        // the chains on the fp32 matrix cores (bkv_res_shared.h), half row 0, the tile restaged with
        // half row 1
        fv4_t a4 = fv4_t{0.0f, 0.0f, 0.0f, 0.0f};
        qk_f16_mfma<0, 8>(kt + lane * kUPR, q16, a4);
        wave_lds_sync();
        stage_k_wave<KF, PG>(kt, sm, nkv, g, k0, n, 1);
        wait_vm<0>();
        qk_f16_mfma<128, 8>(kt + lane * kUPR, q16, a4);
#pragma unroll
        for (int h = 0; h < kGqa; ++h) acc[h] = a4[h];
      }
      wave_lds_sync();
#pragma unroll
      for (int h = 0; h < kGqa; ++h) {
        sc[r][h] = acc[h];
        if (lane < n) mloc[h] = fmaxf(mloc[h], acc[h] * a.scale);
      }
    } else if (r == 0) {
      if constexpr (VRES) load_v_regs<PG, XE>(vd, vsw, xw, xs, sm, nkv, g, nk);
    }
  }
  // the tail (keys NT .. nk-1, at most kResTail): wave 0, lane = 16 h + t scores key NT + t against
  // head h, with its own head's q16 broadcast along the lane's DPP row (fp16 K: qt[j] = q16[h][16 j +
  // lane % 16]); its rows were staged with the first tile, so only the V loads (issued after them)
  // may still be in flight
  const int th = lane >> 4, tt = lane & 15;
  float sct = 0.0f;
  if (TAIL && tn > 0 && wave == 0) {
    wait_vm<kVLoads<XE>>();
    float acc1 = 0.0f;
    if constexpr (KF == BKV_Q8_0) {
      // the MFMA key group's lane (key tt, head th) is this lane's (key, head)
      const uint4 *trow = tail_t + min(tt, tn - 1) * kUPR;
      if (!wide) {
        acc1 = q8_score16(trow, qlim);
      } else {
        float a4[kGqa];
        q8_score_key_slow(trow, qg, a.qs, a4);
        acc1 = pick4(a4, th);
      }
    } else {                               // fp16 rows: the second half row follows the first
      float qt[kHd / 16];
#pragma unroll
      for (int j = 0; j < kHd / 16; ++j) qt[j] = q16[th * kHd + 16 * j + tt];
#pragma unroll
      for (int j = 0; j < kHd / 16; ++j) asm volatile("" : "+v"(qt[j]));
      asm volatile("s_nop 4");                 // (the DPP reads of qt come from inline asm)
      qk_f16_half1<0>(tail_t + tt * kUPR, qt, acc1);
      wave_lds_sync();
      stage_k_wave<KF, PG>(tail_t, sm, nkv, g, tb, tn, 1);
      wait_vm<0>();
      qk_f16_half1<1>(tail_t + tt * kUPR, qt, acc1);
    }
    sct = acc1;
    if (tt < tn)
#pragma unroll
      for (int h = 0; h < kGqa; ++h)
        if (th == h) mloc[h] = fmaxf(mloc[h], sct * a.scale);
  }
  // q8_0 V without the register V form (more than one pass, or fp16 K): the PV runs on the int8
  // matrix cores after the walk (bkv_pv8.h). Once the statistics are out, the first pass's rows of
  // the wave's keys 64 wave .. + 63 go into its K tile by direct-to-LDS loads (the region layout),
  // and the second pass's rows into registers (keys NT + 64 wave + 4 i + lane / 16), so that both
  // stream in during barrier A, the e pass and the walk
  constexpr bool VPF = !VRES && VF == BKV_Q8_0;
  u32x4 pv_w[VPF ? 16 : 1];
  uint32_t pv_s[VPF ? 16 : 1];
  static_assert(kResTail == 16, "the tail fills blocks 0..3 of wave 0's region");
  u32x4 tl_w[VPF ? kResTail / 4 : 1];       // VPF: the tail rows (wave 0)
  uint32_t tl_s[VPF ? kResTail / 4 : 1];
  auto pv_regs = [&](int r) {                // pass r's rows of this wave into pv_w / pv_s
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int kl = r * NT + 64 * wave + 4 * i + vkk;
      const int64_t slot = slot_k<PG>(sm, min(kl, nk - 1));
      pv_w[i] = *reinterpret_cast<const u32x4 *>(L.vd + (slot * nkv + g) * kHd + vsub * 16);
      pv_s[i] = *reinterpret_cast<const uint32_t *>(L.vs + (slot * nkv + g) * kScaleRowBytes + (vsub >> 2) * 4);
    }
  };
  RTS(1);

  // the workgroup's (max of s*scale, sum of exp(s*scale - max)) per head
  if (tid < 32) s_t2[tid] = t2v;           // (published by the reductions' barriers)
  const unsigned gen = gen0 + 1u;
  unsigned *cnt = gs + (1 + (gen & 1u) * 4) * kCounterStride;
  if (wi == 0 && tid < 4) st_agent(gs + (1 + ((gen + 1u) & 1u) * 4 + tid) * kCounterStride, 0u);
  const unsigned tag = 1u + (gen & 1u);
  // Two barriers: each wave's maximum per head and its sum of exps against that maximum go to LDS;
  // after the first barrier (also: every wave is done with its K tile) every lane takes the maximum
  // over the waves, and wave 0 rescales the waves' sums to it (lane 4 i + h: wave i, head h); the
  // second keeps the later loads behind the statistics' store. (The sum feeds S_a and the
  // workgroups' positions, estimates whose margins are far above the roundings this adds; the
  // exact sum is the walk's.)
  {
    float wm[kGqa], lw[kGqa];
#pragma unroll
    for (int h = 0; h < kGqa; ++h)
      wm[h] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wave_max_l63(mloc[h])), 63));
#pragma unroll
    for (int h = 0; h < kGqa; ++h) {
      float l = 0.0f;
#pragma unroll
      for (int r = 0; r < MP; ++r)
        if (r * NT + tid < tpk) l += __expf(sc[r][h] * a.scale - wm[h]);
      if (TAIL && wave == 0 && th == h && tt < tn) l += __expf(sct * a.scale - wm[h]);
      lw[h] = wave_sum_l63(l);
    }
    if (lane == 63)
#pragma unroll
      for (int h = 0; h < kGqa; ++h) s_ml[wave * kGqa + h] = make_float2(wm[h], lw[h]);
    __syncthreads();
#pragma unroll
    for (int h = 0; h < kGqa; ++h) {
      float r = s_ml[h].x;
#pragma unroll
      for (int i = 1; i < NW; ++i) r = fmaxf(r, s_ml[i * kGqa + h].x);
      mloc[h] = r;
    }
    if (wave == 0) {
      const int hh = lane & 3;
      const float M = pick4(mloc, hh);
      const float2 x = lane < NW * kGqa ? s_ml[lane] : make_float2(-INFINITY, 0.0f);
      float r = x.x != -INFINITY ? x.y * __expf(x.x - M) : 0.0f;
      r += __shfl_xor(r, 4);
      r += __shfl_xor(r, 8);
      r += __shfl_xor(r, 16);
      if (lane < kGqa) st_agent(tstats + lane * GM + wi, pack_stats(M, r, tag));
    }
    __syncthreads();
  }
  // VPF: the first pass's V rows once the statistics are out (every wave is done with its K tile:
  // the reductions above synchronise the workgroup), so that the K stream of the later passes and
  // the statistics do not wait behind them. (Issued by waves kGqa.. once barrier A has passed, with
  // the e pass's barriers LDS-only, config 4 q8_0 took 487 against 467 us per token.)
  if constexpr (VPF) {
    if (64 * wave < tpk) {
      const uint32_t region = __builtin_amdgcn_readfirstlane(lds_addr(kt));
      pv8_dma_region(
          region,
          [&](int k) {
            const int64_t slot = slot_k<PG>(sm, min(64 * wave + k, nk - 1));
            return L.vd + (slot * nkv + g) * kHd;
          },
          [&](int k) {
            const int64_t slot = slot_k<PG>(sm, min(64 * wave + k, nk - 1));
            return L.vs + (slot * nkv + g) * kScaleRowBytes;
          });
    }
  }
  // the second pass's rows and the tail's go out once the records are (after barrier A: its polls
  // would wait behind them; after the record stores: the wait that orders the specials before the
  // record would too). Requested after the walk instead, config 4 q8_0 took 477 against 467 us per
  // token: the PV then waits for them.
  auto request_later_v = [&]() {
    if constexpr (VPF) {
      if (NT < tpk) pv_regs(1);
      if (tn > 0 && wave == 0)                 // the tail keys tb + 4 i + lane / 16 (wave 0)
#pragma unroll
        for (int i = 0; i < kResTail / 4; ++i) {
          const int64_t slot = slot_k<PG>(sm, min(tb + 4 * i + vkk, nk - 1));
          tl_w[i] = *reinterpret_cast<const u32x4 *>(L.vd + (slot * nkv + g) * kHd + vsub * 16);
          tl_s[i] = *reinterpret_cast<const uint32_t *>(L.vs + (slot * nkv + g) * kScaleRowBytes + (vsub >> 2) * 4);
        }
    }
  };

  // ---------------------------------------------------------------- barrier A: global max
  // wave h polls head h's statistics of every workgroup of the group: the global max and this
  // workgroup's approximate position on the running sum come with them
  if (wave < kGqa) {
    unsigned long long v[2];
    poll_tagged(tstats + wave * GM, 1, 1, G, tag, v, err);
    const float mw = lane < G ? __uint_as_float((unsigned)(v[0] >> 32)) : -INFINITY;
    const float lw = lane < G ? __uint_as_float((unsigned)v[0] & ~3u) : 0.0f;
    // the max and the prefix sums by DPP (max scan / add scan, then readlane): no LDS round trips
    // (lanes without a source read -inf)
    auto dmax = [](float v, auto ctl) {
      constexpr int C = decltype(ctl)::c, RM = decltype(ctl)::rm;
      const int ninf = (int)0xFF800000u;
      return fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(ninf, __float_as_int(v), C, RM, 0xF, false)));
    };
    float mx = mw;
    mx = dmax(mx, DppCtl<0x111, 0xF>{});
    mx = dmax(mx, DppCtl<0x112, 0xF>{});
    mx = dmax(mx, DppCtl<0x114, 0xF>{});
    mx = dmax(mx, DppCtl<0x118, 0xF>{});
    mx = dmax(mx, DppCtl<0x142, 0xA>{});
    mx = dmax(mx, DppCtl<0x143, 0xC>{});
    const float m = rd_lane(mx, 63);
    const double lx = lane < G ? (double)lw * exp((double)mw - (double)m) : 0.0;
    const double sx = wave_incl_scan_dpp(lx);
    const double p = wi > 0 ? rd_lane(sx, wi - 1) : 0.0, t = rd_lane(sx, 63);
    if (lane == 0) {
      s_M[wave] = m;
      s_P0[wave] = p;
      s_Sa[wave] = (float)t;   // the sum from the statistics: within ~1e-6 of the exact one
    }
  }
  __syncthreads();
  RTS(2);
  RTS(9);
  // ---------------------------------------------------------------- e, classification, records
  int8_t *s_bin = reinterpret_cast<int8_t *>(ldx);   // [kGqa][SB] binade, kNoBin8: special
  Special *s_spec = reinterpret_cast<Special *>(ldx + (kGqa * SB + 15) / 16);   // [kGqa][kMaxSpecial]
  float ev[MP][kGqa];
  long long itot[kGqa];
  int nspc[kGqa];
  double carry[kGqa];
  float Mh[kGqa];
#pragma unroll
  for (int h = 0; h < kGqa; ++h) { itot[h] = 0; nspc[h] = 0; carry[h] = s_P0[h]; Mh[h] = s_M[h]; }
  Special *spec_g = a.spec + (size_t)(g * kGqa) * G * kMaxSpecial;
#pragma unroll
  for (int r = 0; r < MP; ++r) {
#pragma unroll
    for (int h = 0; h < kGqa; ++h) ev[r][h] = 0.0f;
    if (r * NT < tpk) {
      const int kl = r * NT + tid;
      const bool valid = kl < tpk;
      const int64_t j = kb + kl;
      // the key's position on the running sum: the fp64 start of this workgroup plus an fp32
      // exclusive scan inside it (relative error ~1e-7, far inside the classification margin)
      {
        // the 4 heads' exps together, branch-free (table reads in flight at once); the rare cases
        // the table path leaves to the library afterwards
        float xh[kGqa];
        bool slow[kGqa], any = false;
#pragma unroll
        for (int h = 0; h < kGqa; ++h) {
          xh[h] = sc[r][h] * a.scale - Mh[h];
          ev[r][h] = exp_t_fast(xh[h], s_t2, slow[h]);
          any = any || (valid && slow[h]);
        }
        if (any) {
#pragma unroll
          for (int h = 0; h < kGqa; ++h)
            if (slow[h]) ev[r][h] = exp_t_slow(xh[h]);
        }
      }
#pragma unroll
      for (int h = 0; h < kGqa; ++h) {
        ev[r][h] = valid ? ev[r][h] : 0.0f;
        if (valid && a.keep_e) a.e[(size_t)(g * kGqa + h) * a.ld + j] = ev[r][h];
      }
      float fin[kGqa];
#pragma unroll
      for (int h = 0; h < kGqa; ++h) fin[h] = wave_incl_scan_dpp(ev[r][h]);
      if (lane == 63) s_wf[wave] = make_float4(fin[0], fin[1], fin[2], fin[3]);
      __syncthreads();
      float fb[kGqa], ft[kGqa];
#pragma unroll
      for (int h = 0; h < kGqa; ++h) xwave_prefix(reinterpret_cast<const float *>(s_wf), h, wave, fb[h], ft[h]);
      // per head: the step's exact increment (an integer below 2^40 in units of 2^-40: fp64 sums of
      // a workgroup's increments stay exact) or a special
      bool sp[kGqa];
      double dinc[kGqa], din[kGqa];
      unsigned long long msk[kGqa];
#pragma unroll
      for (int h = 0; h < kGqa; ++h) {
        const double ab = carry[h] + (double)(fb[h] + fin[h] - ev[r][h]);
        int bin;
        classify_d(ab, ab + (double)ev[r][h], ev[r][h], sp[h], bin, dinc[h]);
        sp[h] = sp[h] && valid;
        if (!valid) dinc[h] = 0.0;
        carry[h] += (double)ft[h];
        s_bin[h * SB + kl] = (valid && !sp[h]) ? (int8_t)bin : kNoBin8;
        msk[h] = __ballot(sp[h]);
        din[h] = wave_incl_scan_dpp(dinc[h]);
      }
      if (lane == 63)
#pragma unroll
        for (int h = 0; h < kGqa; ++h) {
          s_wd[wave * kGqa + h] = din[h];
          s_wc[wave * kGqa + h] = __popcll(msk[h]);
        }
      __syncthreads();                     // also publishes s_bin
      // (pass timestamp removed)
#pragma unroll
      for (int h = 0; h < kGqa; ++h) {
        double ib, it;
        int cb, ct;
        xwave_prefix(s_wd, h, wave, ib, it);
        xwave_prefix(s_wc, h, wave, cb, ct);
        if (sp[h]) {
          const int id = nspc[h] + cb + (int)__builtin_amdgcn_mbcnt_hi((unsigned)(msk[h] >> 32), __builtin_amdgcn_mbcnt_lo((unsigned)msk[h], 0u));
          if (id < kMaxSpecial) {
            const int8_t bp8 = kl > 0 ? s_bin[h * SB + kl - 1] : (int8_t)0;
            const int bprev = kl > 0 ? (bp8 == kNoBin8 ? kNoBinade : bp8) : 127;
            Special x;
            x.ipre = itot[h] + (long long)(ib + din[h] - dinc[h]);
            x.e = ev[r][h];
            x.meta = kl | ((bprev == kNoBinade ? 0 : (bprev + 128)) << 16);
            s_spec[h * kMaxSpecial + id] = x;
          }
        }
        itot[h] += (long long)it;
        nspc[h] += ct;
      }
    }
  }
  RTS(10);
  // TAIL: the passes' specials go out now, so that their stores have landed by the time the record
  // (which must not be seen before them) is written after the tail
  int ns_main = 0;
  if (TAIL && tn > 0) __syncthreads();    // s_spec holds every pass's specials (tn: uniform)
  if (TAIL && tn > 0 && wave < kGqa) {
    const int h = wave;
    ns_main = min(pick4(nspc, h), kMaxSpecial);
    if (lane < ns_main) st_spec(&spec_g[((size_t)h * G + wi) * kMaxSpecial + lane], s_spec[h * kMaxSpecial + lane]);
  }
  // the tail's steps come after every key of the passes: wave 0 places them with DPP-row scans
  // (lane 16 h + t: key NT + t, head h) on the running sums carried so far
  float evt = 0.0f;
  if (TAIL) {
    if (wave == 0) {
      long long tot_l = 0;
      int tot_c = 0;
      if (tn > 0) {
        const bool valid = tt < tn;
        float Mt = Mh[0];
        double ct = carry[0];
        long long it = itot[0];
        int ns = nspc[0];
#pragma unroll
        for (int h = 1; h < kGqa; ++h)
          if (th == h) { Mt = Mh[h]; ct = carry[h]; it = itot[h]; ns = nspc[h]; }
        evt = valid ? exp_cr_t(sct * a.scale - Mt, s_t2) : 0.0f;
        if (valid && a.keep_e) a.e[(size_t)(g * kGqa + th) * a.ld + kb + tb + tt] = evt;
        const float fin = row_incl_scan_dpp(evt);
        const double ab = ct + (double)(fin - evt);
        bool sp;
        int bin;
        double dinc;
        classify_d(ab, ab + (double)evt, evt, sp, bin, dinc);
        sp = sp && valid;
        if (!valid) dinc = 0.0;
        s_bin[th * SB + tb + tt] = (valid && !sp) ? (int8_t)bin : kNoBin8;
        wave_lds_sync();
        const unsigned long long msk = __ballot(sp);
        const unsigned rowm = (unsigned)(msk >> (16 * th)) & 0xFFFFu;
        const double din = row_incl_scan_dpp(dinc);
        if (sp) {
          const int id = ns + __popc(rowm & ((1u << tt) - 1u));
          if (id < kMaxSpecial) {
            const int8_t bp8 = s_bin[th * SB + tb + tt - 1];
            const int bprev = bp8 == kNoBin8 ? kNoBinade : bp8;
            Special x;
            x.ipre = it + (long long)(din - dinc);
            x.e = evt;
            x.meta = (tb + tt) | ((bprev == kNoBinade ? 0 : (bprev + 128)) << 16);
            s_spec[th * kMaxSpecial + id] = x;
          }
        }
        tot_l = (long long)dpp0<0x15F, 0xF>(din);   // row_newbcast:15, the row's last lane
        tot_c = __popc(rowm);
      }
      if (tt == 0) {
        s_tt[th] = tot_l;
        s_tc[th] = tot_c;
      }
    }
    __syncthreads();
#pragma unroll
    for (int h = 0; h < kGqa; ++h) {
      itot[h] += s_tt[h];
      nspc[h] += s_tc[h];
    }
  }
  // VRES: p16' = f16(e / S_a), the probabilities with the sum barrier A already gives, into the
  // (now free) K tile area, for the speculative PV of waves kGqa.. during the walk
  uint2 *s_ps = reinterpret_cast<uint2 *>(lds);
  if constexpr (VRES) {
    static_assert(2048 * 4 >= NT * sizeof(uint2), "s_ps (one pass) must end before s_acc");
    if (tid < nk) {
      _Float16 pk[kGqa];
#pragma unroll
      for (int h = 0; h < kGqa; ++h) pk[h] = (_Float16)(ev[0][h] / s_Sa[h]);
      s_ps[tid] = make_uint2((uint32_t)__builtin_bit_cast(uint16_t, pk[0]) | ((uint32_t)__builtin_bit_cast(uint16_t, pk[1]) << 16),
                             (uint32_t)__builtin_bit_cast(uint16_t, pk[2]) | ((uint32_t)__builtin_bit_cast(uint16_t, pk[3]) << 16));
    }
  }
  RTS(11);
  __syncthreads();                         // s_spec complete (and s_ps)
  // (spec timestamp removed)
  // wave h writes head h's specials (staged in LDS) and record: only waves 0..3 store anything
  // barrier B waits for
  if (wave < kGqa) {
    const int h = wave, ns = min(pick4(nspc, h), kMaxSpecial);
    if (lane >= ns_main && lane < ns) st_spec(&spec_g[((size_t)h * G + wi) * kMaxSpecial + lane], s_spec[h * kMaxSpecial + lane]);
    if (ns > 0) __builtin_amdgcn_s_waitcnt(0);   // the specials are visible before the record is
    if (lane == 0) {
      ChunkRec rc;
      rc.tot = pick4(itot, h);
      rc.nsp = pick4(nspc, h);
      rc.blast = (nk > 0 && s_bin[h * SB + nk - 1] != kNoBin8) ? s_bin[h * SB + nk - 1] : kNoBinade;
      unsigned long long w0, w1;
      pack_rec(rc, tag, w0, w1);
      st_agent(trec + (h * GM + wi) * 2, w0);
      st_agent(trec + (h * GM + wi) * 2 + 1, w1);
    }
  }
  request_later_v();
  RTS(3);
  // VRES: waves kGqa.. (idle through barrier B and the walk) accumulate PV over their register
  // rows with p16', and park the partial in the K tile area; after the walk they add
  // (p16 - p16') only for the keys whose rounding the exact sum changes
  float *s_acc = reinterpret_cast<float *>(lds) + 2048;   // [kGqa*EPL][NW-kGqa][64], past s_ps
  if constexpr (VRES) {
    static_assert((2048 + kGqa * VR::EPL * (NW - kGqa) * 64) * 4 <= sizeof(lds), "s_acc must fit");
    if (wave >= kGqa) {
      float sacc[kGqa][VR::EPL];
#pragma unroll
      for (int h = 0; h < kGqa; ++h)
#pragma unroll
        for (int i = 0; i < VR::EPL; ++i) sacc[h][i] = 0.0f;
      pv_res_slots<false>(vd, vsw, s_ps, nullptr, nk, wave, vkk, vsub, sacc);
#pragma unroll
      for (int h = 0; h < kGqa; ++h)
#pragma unroll
        for (int i = 0; i < VR::EPL; ++i) s_acc[((h * VR::EPL + i) * (NW - kGqa) + wave - kGqa) * 64 + lane] = sacc[h][i];
    }
  }

  // ---------------------------------------------------------------- barrier B: the exact sums
  // wave h polls head h's records of every workgroup, then walks them (every workgroup of the
  // group walks the same records to the same sums: no second hand-off)
  if (wave < kGqa) {
    const int hh = g * kGqa + wave;
    unsigned long long v[2];
    poll_tagged(trec + wave * GM * 2, 2, 2, G, tag, v, err);
    RTS(4);
    const ChunkRec x = unpack_rec(v[0], v[1]);
    float sres;
    bool gres;
    walk_one<WS, false>(x, a.spec + (size_t)hh * G * kMaxSpecial, G, (int64_t)a.kpw, (int64_t)a.nfill,
                 reinterpret_cast<WS *>(ldx)[wave], sres, gres);
    if (lane == 0) {
      s_S[wave] = sres;
      s_ok[wave] = gres ? 1 : 0;
    }
  }
  __syncthreads();
  if (!(s_ok[0] && s_ok[1] && s_ok[2] && s_ok[3])) {
    // a classification assumption failed (the same in every workgroup of the group, since all
    // walk the same records): publish e device-wide and run the serial loop itself
    if (!a.keep_e) {
#pragma unroll
      for (int r = 0; r < MP; ++r)
        if (r * NT + tid < tpk)
#pragma unroll
          for (int h = 0; h < kGqa; ++h) a.e[(size_t)(g * kGqa + h) * a.ld + kb + r * NT + tid] = ev[r][h];
      if (TAIL && wave == 0 && tt < tn) a.e[(size_t)(g * kGqa + th) * a.ld + kb + tb + tt] = evt;
    }
    __threadfence();
    group_barrier(cnt + 3 * kCounterStride, (unsigned)G, err);
    if (wave < kGqa && !s_ok[wave]) {
      const int hh = g * kGqa + wave;
      float ss = 0.0f;
      for (int64_t b0 = 0; b0 < (int64_t)a.nfill; b0 += 64) {
        const int nb = (int)min((int64_t)64, (int64_t)a.nfill - b0);
        const float x = lane < nb ? ld_agent(&a.e[(size_t)hh * a.ld + b0 + lane]) : 0.0f;
        for (int i = 0; i < nb; ++i) ss = __fadd_rn(ss, __shfl(x, i));
      }
      if (lane == 0) s_S[wave] = ss;
    }
    __syncthreads();
  }
  if (wi == 0 && tid < kGqa) {
    a.sum[g * kGqa + tid] = s_S[tid];
    a.status[g * kGqa + tid] = s_ok[tid] ? 0u : 1u;
  }
  RTS(5);

  // ---------------------------------------------------------------- p16 and PV
  // p16 = f16_rne(e / sum) (attn_vk.h:188 and the fp16 operand cast, :295-296), the 4 heads of a
  // key side by side in LDS; out += p16 * V over this workgroup's rows, 4 heads per V row read
  uint2 *s_p16 = reinterpret_cast<uint2 *>(ldx);
  {
    float S[kGqa];
#pragma unroll
    for (int h = 0; h < kGqa; ++h) S[h] = s_S[h];
#pragma unroll
    for (int r = 0; r < MP; ++r) {
      if (r * NT < tpk) {
        const int kl = r * NT + tid;
        _Float16 pk[kGqa];
#pragma unroll
        for (int h = 0; h < kGqa; ++h) pk[h] = (_Float16)(kl < tpk ? ev[r][h] / S[h] : 0.0f);
        uint2 pw;
        pw.x = (uint32_t)__builtin_bit_cast(uint16_t, pk[0]) | ((uint32_t)__builtin_bit_cast(uint16_t, pk[1]) << 16);
        pw.y = (uint32_t)__builtin_bit_cast(uint16_t, pk[2]) | ((uint32_t)__builtin_bit_cast(uint16_t, pk[3]) << 16);
        s_p16[kl] = pw;
      }
    }
    if (TAIL && wave == 0 && tt < tn) {
      float St = S[0];
#pragma unroll
      for (int h = 1; h < kGqa; ++h)
        if (th == h) St = S[h];
      reinterpret_cast<_Float16 *>(s_p16 + tb + tt)[th] = (_Float16)(evt / St);
    }
  }
  __syncthreads();
  float acc[kGqa][VR::EPL];
  float pvp[16];                           // VPF: the matrix cores' part, head lane / 16, dim 16 t + lane % 16
#pragma unroll
  for (int t = 0; t < 16; ++t) pvp[t] = 0.0f;
  RTS(12);
#pragma unroll
  for (int h = 0; h < kGqa; ++h)
#pragma unroll
    for (int i = 0; i < VR::EPL; ++i) acc[h][i] = 0.0f;
  auto probs = [&](int k, float (&p)[kGqa]) {
    const uint2 pw = k < nk ? s_p16[k] : make_uint2(0u, 0u);
    p[0] = f16_to_f32(pw.x & 0xFFFFu);
    p[1] = f16_to_f32(pw.x >> 16);
    p[2] = f16_to_f32(pw.y & 0xFFFFu);
    p[3] = f16_to_f32(pw.y >> 16);
  };
  if constexpr (VRES) {
    // rows 32*kResVTiles.. (at most one slot) are not resident: this wave's row of that slot
    const int kx = kResVTiles * 32 + wave * 4 + vkk;
    if (!XE && kResVTiles * 32 < nk) {
      const int64_t slot = slot_k<PG>(sm, min(kx, nk - 1));
      xw = *reinterpret_cast<const uint4 *>(L.vd + (slot * nkv + g) * kHd + vsub * 16);
      xs = *reinterpret_cast<const uint32_t *>(L.vs + (slot * nkv + g) * kScaleRowBytes + (vsub >> 2) * 4);
    }
    if (wave < kGqa) {
      pv_res_slots<false>(vd, vsw, s_p16, nullptr, nk, wave, vkk, vsub, acc);
    } else {
#pragma unroll
      for (int h = 0; h < kGqa; ++h)
#pragma unroll
        for (int i = 0; i < VR::EPL; ++i) acc[h][i] = s_acc[((h * VR::EPL + i) * (NW - kGqa) + wave - kGqa) * 64 + lane];
      pv_res_slots<true>(vd, vsw, s_p16, s_ps, nk, wave, vkk, vsub, acc);
    }
    if (kResVTiles * 32 < nk) {
      float p[kGqa];
      probs(kx, p);
      const float vsc = kx < nk ? f16_to_f32(((vsub >> 1) & 1) ? (xs >> 16) : (xs & 0xFFFFu)) : 0.0f;
      v_accum<BKV_Q8_0>(xw, vsc, p, acc);
    }
  } else {
    constexpr int RS = NW * VR::KPW;        // rows per workgroup step
    constexpr int U = 4;                    // row loads in flight per lane
    constexpr int RB = row_bytes(VF);
    int base0 = 0;
    if constexpr (VPF) {
      // out += p16 * V over the passes on the int8 matrix cores: each wave over its keys
      // 64 wave .. + 63 of each pass, in its region (pass 0 loaded there directly, pass 1 from
      // registers, later passes loaded now), two rounds of 32 keys per pass; 2^sig(h) keeps every
      // p16 * scale of the pass below 2^29 (p16 <= the workgroup's largest e over the exact sum,
      // plus a margin; the scale <= the wave's largest of the pass)
      const Pv8Sel z = pv8_sel();
      const int ia = lane & 3, ha = (lane & 15) >> 2, kq = lane >> 4;
      char *region = reinterpret_cast<char *>(kt);
      const uint32_t rg = __builtin_amdgcn_readfirstlane(lds_addr(kt));
      int ep[kGqa];
#pragma unroll
      for (int h = 0; h < kGqa; ++h) {
        const float pb = __expf(mloc[h] - s_M[h]) / s_S[h] * 1.002f;
        ep[h] = max(-30, (int)((__float_as_uint(pb) >> 23) & 0xFFu) - 127);
      }
      wait_vm<0>();                            // pass 0's direct-to-LDS rows, pass 1's registers
      // one part (a pass's 64 keys of this wave, or the tail on wave 0) already in the region:
      // keys kw0 + k (k < 64) with probabilities below kend
      auto part = [&](int kw0, int kend) __attribute__((always_inline)) {
        const uint4 sr = *reinterpret_cast<const uint4 *>(region + kPv8Scales + 16 * lane);
        const uint32_t dm = kw0 + lane < kend ? f16_row_max(sr) : 0u;
        const int ed = f16_exp_bound(__builtin_bit_cast(uint16_t, (_Float16)rd_lane(wave_max_l63(f16_to_f32(dm)), 63)));
        int sig[kGqa];
#pragma unroll
        for (int h = 0; h < kGqa; ++h) sig[h] = min(100, 27 - ep[h] - ed);
        const float sga = __builtin_ldexpf(1.0f, pick4(sig, ha));
        // two halves of 8 dim tiles (blocks 0..3, 4..7): half the accumulators live at a time
        auto half = [&](auto hc) __attribute__((always_inline)) {
          constexpr int hf = decltype(hc)::value;
          v4i_t pacc[8];
          auto round = [&](auto rc) __attribute__((always_inline)) {
            constexpr int rd = decltype(rc)::value;
            const int ka = 32 * rd + 8 * kq + 2 * ia;
            auto pf = [&](int k) {
              if (kw0 + k >= kend) return 0.0f;
              const uint2 pw = s_p16[kw0 + k];
              const uint32_t w2 = ha < 2 ? pw.x : pw.y;
              return f16_half(w2, ha & 1) * sga;   // exact: a power of two
            };
            const float pa = pf(ka), pb = pf(ka + 1);
            const uint4 sa = *reinterpret_cast<const uint4 *>(region + kPv8Scales + 16 * ka);
            const uint4 sb = *reinterpret_cast<const uint4 *>(region + kPv8Scales + 16 * (ka + 1));
            long A[4];
            pv8_prep<4 * hf, 4>(pa, pb, sa, sb, z, A);
            pv8_round_region<rd == 0, 8 * hf, 8>(rg, rd, A, pacc);
          };
          round(std::integral_constant<int, 0>{});
          if (kw0 + 32 < kend) round(std::integral_constant<int, 1>{});
          const int nsig = -pick4(sig, lane >> 4);
#pragma unroll
          for (int t = 0; t < 8; ++t) pvp[8 * hf + t] += pv8_value(pacc[t], nsig);
        };
        half(std::integral_constant<int, 0>{});
        half(std::integral_constant<int, 1>{});
      };
#pragma unroll 1
      for (int r = 0; r < MP; ++r) {
        if (r * NT >= tpk) break;
        const int kw0 = r * NT + 64 * wave;
        if (r >= 1) {
          if (r >= 2) {
            pv_regs(r);
            wait_vm<0>();
          }
          wave_lds_sync();                     // the previous part's reads of the region are done
          pv8_store_region(region, pv_w, pv_s);
          wave_lds_sync();
        }
        if (kw0 < tpk) part(kw0, tpk);         // (uniform)
      }
      if (tn > 0 && wave == 0) {               // the tail keys tb .. nk - 1 as blocks 0..3 of the region
        wave_lds_sync();
#pragma unroll
        for (int i = 0; i < kResTail / 4; ++i) {
          *reinterpret_cast<u32x4 *>(region + 1024 * i + 64 * (vsub ^ (i & 3)) + 16 * vkk) = tl_w[i];
          if ((vsub & 3) == 0) *reinterpret_cast<uint32_t *>(region + kPv8Scales + 16 * (4 * i + vkk) + 4 * (vsub >> 2)) = tl_s[i];
        }
        wave_lds_sync();
        part(tb, nk);
      }
      base0 = nk;
    }
    for (int base = base0; base < nk; base += RS * U) {
      uint4 wv[U];
      uint32_t sw[U];
      int kl[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        kl[u] = base + u * RS + wave * VR::KPW + vkk;
        const int64_t slot = slot_k<PG>(sm, min(kl[u], nk - 1));
        wv[u] = *reinterpret_cast<const uint4 *>(L.vd + (slot * nkv + g) * RB + vsub * 16);
        sw[u] = 0u;
        if (VF == BKV_Q8_0)
          sw[u] = *reinterpret_cast<const uint32_t *>(L.vs + (slot * nkv + g) * kScaleRowBytes + (vsub >> 2) * 4);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        float p[kGqa];
        probs(kl[u], p);
        float vsc = 1.0f;
        if (VF == BKV_Q8_0) vsc = f16_to_f32(((vsub >> 1) & 1) ? (sw[u] >> 16) : (sw[u] & 0xFFFFu));
        if (kl[u] >= nk) {
          vsc = 0.0f;
          wv[u] = make_uint4(0u, 0u, 0u, 0u);
        }
        v_accum<VF>(wv[u], vsc, p, acc);
      }
    }
  }
  RTS(13);
  RTSW(15, 7);
  // the 4 row groups' sums: q8_0 V (16-lane rows) by a reduce-scatter that leaves row group r with
  // head r's totals in red[i]; fp16 V (two 32-lane rows) by one swap, both rows with every head
  float red[VR::EPL];
  if constexpr (VR::LPR == 16) {
#pragma unroll
    for (int i = 0; i < VR::EPL; ++i) {
      // permlane32_swap(x, y) pairs lanes l < 32 of y with lanes l + 32 of x: the two halves' sums
      // of head 0 (head 1) land in lanes 0-31, those of head 2 (head 3) in lanes 32-63
      const auto s02 = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[0][i]), __float_as_uint(acc[2][i]), false, false);
      const auto s13 = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[1][i]), __float_as_uint(acc[3][i]), false, false);
      const float za = __uint_as_float(s02[0]) + __uint_as_float(s02[1]);
      const float zb = __uint_as_float(s13[0]) + __uint_as_float(s13[1]);
      // permlane16_swap(x, y) pairs odd rows of x with even rows of y: row r then holds head r's sum
      const auto t = __builtin_amdgcn_permlane16_swap(__float_as_uint(za), __float_as_uint(zb), false, false);
      red[i] = __uint_as_float(t[0]) + __uint_as_float(t[1]);
    }
  } else {
#pragma unroll
    for (int h = 0; h < kGqa; ++h)
#pragma unroll
      for (int i = 0; i < VR::EPL; ++i) {
        const auto a2 = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[h][i]), __float_as_uint(acc[h][i]), false, false);
        acc[h][i] = __uint_as_float(a2[0]) + __uint_as_float(a2[1]);
      }
  }
  RTS(14);
  __syncthreads();                         // every wave is done with its V rows
  // [NW][kGqa][EPL][LPR]: element d = LPR-chunk vsub, index i of head h. After the row reduction
  // every row group holds the sums; row group h writes head h's, one float per lane per store,
  // consecutive lanes to consecutive words (no bank conflicts)
  float *s_red = reinterpret_cast<float *>(lds);
  static_assert(VR::LPR * VR::EPL == kHd && (VR::LPR != 16 || 64 / VR::LPR == kGqa), "partial layout");
  if constexpr (VR::LPR == 16) {
    if constexpr (VPF) {                   // element (head lane / 16, dim 16 t + lane % 16)
#pragma unroll
      for (int t = 0; t < 16; ++t) s_red[((wave * kGqa + (lane >> 4)) * VR::EPL + (lane & 15)) * VR::LPR + t] = pvp[t];
    } else {
#pragma unroll
      for (int i = 0; i < VR::EPL; ++i) s_red[((wave * kGqa + vkk) * VR::EPL + i) * VR::LPR + vsub] = red[i];
    }
  } else if (vkk == 0) {
#pragma unroll
    for (int h = 0; h < kGqa; ++h)
#pragma unroll
      for (int i = 0; i < VR::EPL; ++i) s_red[((wave * kGqa + h) * VR::EPL + i) * VR::LPR + vsub] = acc[h][i];
  }
  __syncthreads();
  // the partial, each element tagged with the call's generation: {float bits, gen} in one 64-bit
  // store, so the merge below polls the data itself (no arrival counter, no stale match: the
  // generation only grows)
  unsigned long long *part_g = a.part + (size_t)g * G * kGqa * kHd;
  {
    static_assert(kGqa * kHd == 2 * NT, "two partial elements per thread");
    float2 v = make_float2(0.0f, 0.0f);
    const int hh = (2 * tid) / kHd, dd = (2 * tid) % kHd;   // elements (hh, dd) and (hh, dd + 1)
    const int ro = (hh * VR::EPL + dd % VR::EPL) * VR::LPR + dd / VR::EPL;
#pragma unroll
    for (int wv = 0; wv < NW; ++wv) {
      v.x += s_red[wv * kGqa * kHd + ro];
      v.y += s_red[wv * kGqa * kHd + ro + VR::LPR];
    }
    unsigned long long *dst = part_g + (size_t)wi * kGqa * kHd + 2 * tid;
    st_agent(dst, (unsigned long long)__float_as_uint(v.x) | ((unsigned long long)gen << 32));
    st_agent(dst + 1, (unsigned long long)__float_as_uint(v.y) | ((unsigned long long)gen << 32));
  }
  RTS(6);

  // ---------------------------------------------------------------- merge + gate
  // workgroup wi sums slice wi of the group's partials in workgroup order, polling each element
  // until it carries this call's generation
  {
    constexpr int E = kGqa * kHd;
    const int sl = (E + G - 1) / G;                      // elements per workgroup
    const int e0 = wi * sl, ecount = max(0, min(E, e0 + sl) - e0);
    for (int c0 = 0; c0 < ecount; c0 += NT) {
      const int ne = min(NT, ecount - c0);
      const int ngrp = NT / ne;                          // threads per element
      const int el = tid % ne, grp = tid / ne;
      constexpr int B = 8;
      float sacc = 0.0f;
      if (grp < ngrp) {
        for (int w0 = grp; w0 < G; w0 += ngrp * B) {
          unsigned long long t[B];
          unsigned spins = 0;
          for (;;) {
            bool ok = true;
#pragma unroll
            for (int u = 0; u < B; ++u) {
              const int ww = w0 + u * ngrp;
              t[u] = ww < G ? ld_agent(&part_g[(size_t)ww * E + e0 + c0 + el]) : ((unsigned long long)gen << 32);
              ok = ok && (unsigned)(t[u] >> 32) == gen;
            }
            if (ok) break;
            __builtin_amdgcn_s_sleep(1);
            if (++spins > kResSpin) {
              atomicOr(err, 1u);
              break;
            }
          }
#pragma unroll
          for (int u = 0; u < B; ++u) sacc += __uint_as_float((unsigned)t[u]);
        }
        s_red[grp * ne + el] = sacc;
      }
      __syncthreads();
      if (tid < ne) {
        float v = 0.0f;
        for (int j = 0; j < ngrp; ++j) v += s_red[j * ne + tid];
        const int eg = e0 + c0 + tid;
        const size_t oi = (size_t)g * E + eg;           // out is [nh][hd], head g*kGqa + eg/hd
        a.out[oi] = v;
        if (a.gate) a.out_gated[oi] = v * (1.0f / (1.0f + exp_cr(-a.gate[gate_index(oi, a.gs)])));
      }
      __syncthreads();
    }
  }
  RTS(7);
  // every workgroup of the group has written its partial, so all have read the generation
  if (wi == 0 && tid == 0) st_agent(gs, gen);
  RTS(8);
}

// workgroups of one variant resident at once on the current device
template <typename K>
static int occupancy_of(K kernel, int dev) {
  int per = 0;
  hipDeviceProp_t pr;
  if (hipGetDeviceProperties(&pr, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kernel, kResNT, 0) != hipSuccess)
    return 0;
  return per * pr.multiProcessorCount;
}

// the grid the launches may use on the current device: the smallest occupancy over every variant
// of this format pair that launch_resident can launch (register V or not, paged or not), queried
// once per device
template <int KF, int VF>
static int resident_capacity() {
  // per device, published once computed (value + 1; 0: not yet): threads that race here compute
  // the same value
  constexpr int kMaxDev = 64;
  static std::atomic<int> cached[kMaxDev];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) return 0;
  const int known = cached[dev].load(std::memory_order_acquire);
  if (known > 0) return known - 1;
  int c = std::min(occupancy_of(resident_kernel<KF, VF, false, false>, dev),
                   occupancy_of(resident_kernel<KF, VF, false, true>, dev));
  if constexpr (KF == BKV_Q8_0 && VF == BKV_Q8_0)
    c = std::min({c, occupancy_of(resident_kernel<KF, VF, true, false>, dev),
                   occupancy_of(resident_kernel<KF, VF, true, true>, dev)});
  c = std::max(c, 0);
  cached[dev].store(c + 1, std::memory_order_release);
  return c;
}

int resident_max_workgroups(int kf, int vf) {
  BKV_FMT_SWITCH(kf, vf, { return resident_capacity<KF_, VF_>(); });
  return 0;
}

template <int KF, int VF, bool VRES>
static void launch_res(const ResArgs &a, hipStream_t st) {
  const dim3 grid(a.G * a.nkv), block(kResNT);
  if (a.L.page) hipLaunchKernelGGL((resident_kernel<KF, VF, VRES, true>), grid, block, 0, st, a);
  else hipLaunchKernelGGL((resident_kernel<KF, VF, VRES, false>), grid, block, 0, st, a);
}

// The grid never exceeds what the occupancy query says is resident at once (one workgroup per CU),
// so on a device not held by other long-running kernels every wait is reached by its producers.
hipError_t launch_resident(const ResArgs &a, int kf, int vf, bool vres, hipStream_t st) {
  BKV_FMT_SWITCH(kf, vf, {
    if constexpr (VF_ == BKV_Q8_0 && KF_ == BKV_Q8_0) {
      if (vres) {
        launch_res<KF_, VF_, true>(a, st);
        return hipGetLastError();
      }
    }
    launch_res<KF_, VF_, false>(a, st);
  });
  return hipGetLastError();
}

}  // namespace bkv
