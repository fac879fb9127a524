// bkv_stream.hip - the default decode kernel for q8_0 K and V when a KV group's keys fit 64
// workgroups of at most 512 + kResTail keys: one launch per layer and token, one 512-thread
// workgroup per CU, every workgroup resident for the whole call.
//
// Every wave requests its share of the whole K and V stream up front (a K tile of 64 rows into LDS
// by direct-to-LDS loads, 17 slots of V rows into registers), so the stream runs at full bandwidth
// and has landed by the time the scores are done. A wave's vector load completes only after every
// older load of its CU's queue, so the cross-workgroup polls (waves 0..3) come after the stream.
//
// Per call:
//  1. Loads; wave 0 also brings q (and decode_step's new K and V) into LDS. The new token is
//     quantised into the cache and patched into the LDS tile (no round trip through memory).
//  2. Scores in the reference's order (attn_vk.h:156-170), one key per lane and wave; the tail keys
//     (past 512, at most kResTail) 8 lanes per (key, head), one per 32-element block. The
//     workgroup's (max, sum exp) per head go out as tagged words; barrier A gives the global max M,
//     the sum estimate S_a and the workgroup's position on the running sum.
//  3. e = exp(s*scale - M) correctly rounded, positions by fp32 DPP scans, each step of the serial
//     fp32 sum classified as an exact integer increment in its binade or a special; the workgroup's
//     record and specials go out. p16' = f16(e / S_a); the keys whose p16 the exact sum may still
//     change ("at risk") keep their V rows in LDS.
//  4. Every wave: PV over its slots with p16'. Waves 0..3 then poll the records (barrier B), walk
//     them to the exact serial sums (every workgroup walks the group's records itself), form
//     p16 = f16(e / sum) and add (p16 - p16') * v for the keys whose rounding changed.
//  5. The workgroup's [4][256] partial goes out as tagged words, and workgroup i sums slice i of
//     the group's partials in workgroup order (+ gate).
#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <type_traits>
#include <utility>

#include "bkv_exp.h"
#include "bkv_pv8.h"
#include "bkv_res_shared.h"

namespace bkv {

constexpr int kSwKW = 4;                 // waves 0..3 poll, walk and correct
constexpr int kSwNP = kResNT;            // pass keys per workgroup (one per thread)
constexpr int kSwKeys = kSwNP + kResTail;
constexpr int kSwTailLoads = (kResTail * kUPR + 63) / 64;   // direct-to-LDS loads of the tail rows
constexpr int kSwBlocks = kSwNP / 64 + 1;                  // e-pass blocks: 8 of 64 keys, the tail
constexpr int kSwRisk = 32;              // at-risk V rows the LDS keeps (more: re-read from the cache)
// relative distance from S_a inside which the exact sum is expected: the serial fp32 sum departs
// from the exact one by up to ~7e-6 relative at 32K keys (2e-6 median), and S_a adds its own ~1e-6;
// a key is at risk when p16' would round differently anywhere within twice this distance of it
constexpr float kSwRiskBand = 0x1p-16f;

// rows [0, n) of the tail (keys k0 ..) into tt (kUPR uint4 per row), lanes past the rows masked
template <bool PG>
__device__ __forceinline__ void stage_tail(uint4 *tt, const SlotMap &sm, int nkv, int g, int k0, int n) {
  const int lane = threadIdx.x & 63;
  const uint32_t base = __builtin_amdgcn_readfirstlane(lds_addr(tt));
#pragma unroll
  for (int i = 0; i < kSwTailLoads; ++i) {
    const int slotx = 64 * i + lane, row = slotx / kUPR, col = slotx - row * kUPR;
    const int64_t sl = slot_k<PG>(sm, k0 + min(row, n - 1));
    const uint8_t *src = col == 16 ? sm.L->ks + (sl * nkv + g) * kScaleRowBytes
                                   : sm.L->kd + (sl * nkv + g) * kHd + col * 16;
    if (slotx < kResTail * kUPR)
      asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(base + 1024u * i)
                   : "memory", "m0");
  }
}

// The new token's row of one tensor for group g, quantised (q8_0, round half to even): lanes
// s = 0..15 of each 32-lane half own elements 16 s .. 16 s + 15 (lanes 0..31: K, 32..63: V). d gets
// the lane's 16 data bytes, sw (lanes s % 4 == 0) the scale word of blocks s/2 and s/2 + 1. The rows
// are stored to the cache slot here (attn_norm_rope2.comp:184-217 for the arithmetic).
// K16: the K row in fp16 instead (lanes 0..31, 8 elements each; d gets the lane's 16 bytes).
template <bool K16>
__device__ __forceinline__ void append_q8_rows(const AppendArgs &ap, int64_t slot, const float *xk, const float *xv,
                                               int g, int lane, uint4 &d, uint32_t &sw) {
  if (K16 && lane < 32) {
    const float *x = xk + 8 * lane;
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = f32_to_f16_rne(x[2 * i]) | (f32_to_f16_rne(x[2 * i + 1]) << 16);
    d = make_uint4(w[0], w[1], w[2], w[3]);
    sw = 0u;
    uint8_t *dr = const_cast<uint8_t *>(ap.L.kd) + (slot * ap.nkv + g) * row_bytes(BKV_F16);
    *reinterpret_cast<uint4 *>(dr + 16 * lane) = d;
    return;
  }
  const int s = lane & 15;
  const float *x = (lane < 32 ? xk : xv) + 16 * s;
  float v[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) v[i] = x[i];
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(v[i]));
  amax = fmaxf(amax, __shfl_xor(amax, 1));
  const float id = q8_iscale(amax);
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    w[i] = q8_byte<false>(v[4 * i], id) | (q8_byte<false>(v[4 * i + 1], id) << 8) |
           (q8_byte<false>(v[4 * i + 2], id) << 16) | (q8_byte<false>(v[4 * i + 3], id) << 24);
  const uint32_t h = f32_to_f16_rne(q8_scale(amax));
  const uint32_t hn = __shfl_down(h, 2);
  d = make_uint4(w[0], w[1], w[2], w[3]);
  sw = h | (hn << 16);
  if ((lane & 31) < 16) {
    const bool isk = lane < 32;
    uint8_t *dr = const_cast<uint8_t *>(isk ? ap.L.kd : ap.L.vd) + (slot * ap.nkv + g) * kHd;
    uint8_t *sr = const_cast<uint8_t *>(isk ? ap.L.ks : ap.L.vs) + (slot * ap.nkv + g) * kScaleRowBytes;
    *reinterpret_cast<uint4 *>(dr + 16 * s) = d;
    if ((s & 3) == 0) *reinterpret_cast<uint32_t *>(sr + (s >> 2) * 4) = sw;
  }
}

// binade classification of one step of the running sum from its fp32 position before and after
// (the fp32 error of a position is far inside the 2^-14 relative margin): B and the step's exact
// increment in ulps of that binade (an integer below 2^24), or a special
__device__ __forceinline__ void classify_i(float abefore, float aafter, float e, bool &special, int &bin, int &inc) {
  const int B = (int)((__float_as_uint(aafter) >> 23) & 0xFF) - 127;
  const float lo = __uint_as_float((uint32_t)min(max(B + 127, 1), 254) << 23);
  const float t = ldexpf(e, 23 - B);
  const float r = __builtin_rintf(t);
  const bool ok = aafter >= 0x1p-17f && aafter < 0x1p22f && !(aafter > 2.0f * lo * (float)(1.0 - kMargin)) &&
                  !(abefore < lo * (float)(1.0 + kMargin)) && (t - __builtin_floorf(t) != 0.5f);
  special = !ok;
  bin = B;
  inc = ok ? (int)r : 0;
}

// inner[h] = sum of q16[h][32 b + i] * x[i], i ascending (one fma per product: every product is
// exact), for the block b of the lane's 16-lane row; q16[h][32 b + 16 c + j] sits in lane j of
// the row, register q[h][c], and reaches the other lanes by row_newbcast
template <int I>
struct BlockChain {
  static __device__ __forceinline__ void run(float (&inner)[kGqa], const float (&q)[kGqa][2], const float (&x)[32]) {
    BlockChain<I - 1>::run(inner, q, x);
#pragma unroll
    for (int h = 0; h < kGqa; ++h) fmac_bc<(I - 1) % 16>(inner[h], q[h][(I - 1) / 16], x[I - 1]);
  }
};
template <>
struct BlockChain<0> {
  static __device__ __forceinline__ void run(float (&)[kGqa], const float (&)[kGqa][2], const float (&)[32]) {}
};

// s_waitcnt vmcnt(n) for a runtime n (a branch per value; an n the compiler knows folds away)
__device__ __forceinline__ void wait_vm_n(int n) {
  switch (n) {
#define BKV_WAIT_CASE(i) case i: wait_vm<i>(); break;
    BKV_WAIT_CASE(0) BKV_WAIT_CASE(1) BKV_WAIT_CASE(2) BKV_WAIT_CASE(3) BKV_WAIT_CASE(4) BKV_WAIT_CASE(5)
    BKV_WAIT_CASE(6) BKV_WAIT_CASE(7) BKV_WAIT_CASE(8) BKV_WAIT_CASE(9) BKV_WAIT_CASE(10) BKV_WAIT_CASE(11)
    BKV_WAIT_CASE(12) BKV_WAIT_CASE(13) BKV_WAIT_CASE(14) BKV_WAIT_CASE(15) BKV_WAIT_CASE(16) BKV_WAIT_CASE(17)
    BKV_WAIT_CASE(18) BKV_WAIT_CASE(19) BKV_WAIT_CASE(20) BKV_WAIT_CASE(21) BKV_WAIT_CASE(22) BKV_WAIT_CASE(23)
    BKV_WAIT_CASE(24) BKV_WAIT_CASE(25) BKV_WAIT_CASE(26) BKV_WAIT_CASE(27) BKV_WAIT_CASE(28) BKV_WAIT_CASE(29)
    BKV_WAIT_CASE(30) BKV_WAIT_CASE(31) BKV_WAIT_CASE(32) BKV_WAIT_CASE(33) BKV_WAIT_CASE(34) BKV_WAIT_CASE(35)
    BKV_WAIT_CASE(36) BKV_WAIT_CASE(37) BKV_WAIT_CASE(38) BKV_WAIT_CASE(39) BKV_WAIT_CASE(40)
#undef BKV_WAIT_CASE
    default: wait_vm<0>(); break;
  }
}

// LDS flags between the roles. A K-wave barrier: each K wave adds one to *ctr and waits until it
// reaches target (the V waves are busy elsewhere). A flag: the K waves each add one once their part
// is in LDS; a V wave waits until it reaches target. LDS operations of one wave complete in order,
// so whatever a wave wrote before its add is in LDS once the add is seen.
__device__ __forceinline__ unsigned lds_ld(const unsigned *p) {
  return __hip_atomic_load(const_cast<unsigned *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_arrive(unsigned *ctr) {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  if ((threadIdx.x & 63) == 0) atomicAdd(ctr, 1u);
}
__device__ __forceinline__ void lds_wait(const unsigned *ctr, unsigned target) {
  while (lds_ld(ctr) < target) __builtin_amdgcn_s_sleep(1);
  asm volatile("" ::: "memory");
}
__device__ __forceinline__ void kwave_sync(unsigned *ctr, unsigned target) {
  lds_arrive(ctr);
  lds_wait(ctr, target);
}

// the wave's max / sum of one value per head over its 64 lanes, in every lane
__device__ __forceinline__ float wave_max64(float v) { return rd_lane(wave_max_l63(v), 63); }
__device__ __forceinline__ float wave_sum64(float v) { return rd_lane(wave_sum_l63(v), 63); }
__device__ __forceinline__ int wave_sum64_i(int v) { return __builtin_amdgcn_readlane(wave_scan_i32(v), 63); }

// SHORT: a plan of at most 128 keys per workgroup (every workgroup then has no tail keys); its own
// instantiation, so that the block-split scores and e pass leave the full-pass code as it is
// KF: the K format, q8_0 (scores on the int8 matrix cores) or fp16 (the reference's own cache
// format, kv_guard.h:118-130: scores as DPP chains in the reference's order, attn_vk.h:156-170,
// over half rows staged twice); V is q8_0.
template <int KF, bool PG, bool SHORT>
__global__ __launch_bounds__(kResNT, 1) void stream_kernel(ResArgs a) {
  constexpr int NT = kResNT, NW = kResNW, NP = kSwNP, KS = kSwKeys;
  constexpr bool K16 = KF == BKV_F16;
  using WS = WalkScratchT<kResMaxGroupWgs, 192>;
  using VR = KRow<BKV_Q8_0>;
  // LDS. kt: the K tiles (pass key k at row k: kt + k * kUPR); once every tile is scored the same
  // bytes hold the e values, probabilities, binade map, specials, walk scratch, the at-risk V rows
  // and the PV reduction.
  __shared__ uint4 kt[NP * kUPR];
  __shared__ uint4 vsc[NW * 64];            // V scale rows: pass key k of wave w at [w][k - NKW w]
  __shared__ uint4 ttl[kResTail * kUPR];    // the tail's K rows
  __shared__ float4 s_q[kGqa * kHd / 4];    // the group's q rows (fp32)
  __shared__ uint4 s_x[2 * kHd / 4];        // decode_step: the new token's K and V (fp32), then its V row
  __shared__ float s_tsc[kResTail * kGqa];  // the tail's scores [key][head]
  __shared__ uint32_t s_tsw[kResTail * 4];  // the tail's V scale rows
  __shared__ int s_pg[kResPgMax];
  __shared__ double s_t2[32];               // 2^(j/32)
  __shared__ float2 s_ml[NW * kGqa];            // each wave's (max, sum of exps against it) per head
  __shared__ float s_M[kGqa], s_Sa[kGqa], s_S[kGqa];
  __shared__ double s_P0[kGqa];
  __shared__ int s_ok[kGqa];
  __shared__ float4 s_bt[kSwBlocks];        // e-pass block totals of e (positions), per head
  __shared__ double s_bu[kSwBlocks * kGqa]; // block totals of the increments (units of 2^-40)
  __shared__ int s_bc[kSwBlocks * kGqa];    // block counts of specials
  __shared__ int s_nrisk;
  __shared__ unsigned long long s_rb[kSwBlocks];   // at-risk keys: bit k % 64 of word k / 64 (tail: word 8)
  __shared__ unsigned s_kctr;               // the K waves' spin barrier
  __shared__ unsigned s_pvctr;              // waves done reading their PV staging rows
  __shared__ unsigned s_stg1;               // K waves done staging their round-1 PV rows
  __shared__ int s_lt[kGqa];                // q8_0 K digits: the exponent of each head
  __shared__ unsigned s_wide;               // the q8_0 K digits do not fit (fp64 score path)

  // workgroups are dealt to the 8 XCDs round-robin by index; when the grid allows, the nkv groups
  // of one key range share an XCD (each 64 B scale line holds all groups' scales of a slot)
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
  const bool kwave = wave < kSwKW;
  const int64_t kb = (int64_t)wi * a.kpw;
  const int64_t ke = min((int64_t)a.nfill, kb + (int64_t)a.kpw);
  const int nk = (int)max((int64_t)1, ke - kb);        // the plan gives every workgroup keys
  const int np = min(nk, NP), tn = max(0, nk - NP);     // pass keys, tail keys (tn <= kResTail)
  const LayerView &L = a.L;

  // ---------------------------------------------------------------- set-up
  unsigned *gs = a.sync + (size_t)g * kResGroupLines * kCounterStride;
  unsigned *err = a.sync + (size_t)nkv * kResGroupLines * kCounterStride;
  const unsigned gen = ld_agent(gs) + 1u;
  unsigned *cnt = gs + (1 + (gen & 1u) * 4) * kCounterStride;
  if (wi == 0 && tid < 4) st_agent(gs + (1 + ((gen + 1u) & 1u) * 4 + tid) * kCounterStride, 0u);
  const unsigned tag = 1u + (gen & 1u);
  constexpr int GM = kResMaxGroupWgs;
  unsigned long long *tstats = a.tstats + (size_t)g * kGqa * GM;
  unsigned long long *trec = a.trec + (size_t)g * kGqa * GM * 2;
  // the group's specials [head][workgroup][kMaxSpecial], stored where the e pass finds them
  Special *spec_g = a.spec + (size_t)(g * kGqa) * G * kMaxSpecial;
  if (wi == 0)                                 // entries of workgroups this call does not run
    for (int i = tid; i < kGqa * (GM - G); i += NT) {
      const int h = i / (GM - G), c = G + i % (GM - G);
      st_agent(tstats + h * GM + c, 0ull);
      st_agent(trec + (h * GM + c) * 2, 0ull);
      st_agent(trec + (h * GM + c) * 2 + 1, 0ull);
    }
  if (tid == 0) { s_kctr = 0u; s_pvctr = 0u; s_stg1 = 0u; s_nrisk = 0; s_wide = 0u; }
  if (tid < kSwBlocks) s_rb[tid] = 0ull;
  if (tid < kGqa) {                            // the tail block's totals when there is no tail
    s_bu[(kSwBlocks - 1) * kGqa + tid] = 0.0;
    s_bc[(kSwBlocks - 1) * kGqa + tid] = 0;
  }
  if (tid == 0) s_bt[kSwBlocks - 1] = make_float4(0.f, 0.f, 0.f, 0.f);
  if (tid >= 64 && tid < 96) s_t2[tid - 64] = kExp2Tab[tid - 64];
  RTS(0);

  const bool appender = a.ap.k && (int64_t)a.ap.pos >= kb && (int64_t)a.ap.pos < ke;
  const int kp = appender ? (int)((int64_t)a.ap.pos - kb) : -1;     // the new token's key in this workgroup
  // pass key k sits in wave k / 64 (its K tile) and, for the PV, in wave k / NKW (V slot
  // (k % NKW) / 4, row group k % 4); tail key NP + t: its K row on wave t / 2, its V row on wave
  // t / 4 (the tail slot)
  const int aw = kp < 0 ? -1 : (kp < NP ? kp >> 6 : (kp - NP) >> 1);   // the wave that appends it
  SlotMap sm{&L, kb, s_pg, 0u};
  if constexpr (PG) {
    const uint32_t pgs = (uint32_t)L.page, pg0 = (uint32_t)(kb + L.base) / pgs,
                   pg1 = (uint32_t)(kb + nk - 1 + L.base) / pgs;
    sm.pf = pg0;
    if (tid <= (int)min(pg1 - pg0, (uint32_t)kResPgMax - 1u)) s_pg[tid] = L.bt[pg0 + tid];
  }
  __syncthreads();                             // flags, table, page table

  // scratch carved from the K tiles once every tile is scored
  char *xb = reinterpret_cast<char *>(kt);
  float *s_e = reinterpret_cast<float *>(xb);                         // [kGqa][KS]
  uint2 *s_ps = reinterpret_cast<uint2 *>(xb + kGqa * KS * 4);        // [KS] p16' (4 heads per key)
  uint2 *s_p16 = s_ps + KS;                                           // [KS] p16
  int8_t *s_bin = reinterpret_cast<int8_t *>(s_p16 + KS);             // [kGqa][KS]
  int16_t *s_ridx = reinterpret_cast<int16_t *>(s_bin + kGqa * KS);   // [KS] at-risk row index, -1: none
  // (24576 .. : room for [kGqa][kMaxSpecial] specials, which now go straight to global memory)
  WS *s_walk = reinterpret_cast<WS *>(xb + 24576 + kGqa * kMaxSpecial * sizeof(Special));
  constexpr int kStg = 53248 + kSwRisk * 256;                         // the PV staging rows, 8 waves
  constexpr int kStgW = kPv8Rows * kPv8Stride;
  uint4 *s_rrow = reinterpret_cast<uint4 *>(xb + 53248);              // [kSwRisk][16] at-risk V rows
  // [wave][head][dim]: each wave's PV partial; over the staging rows of waves 0..3, written once
  // every wave has finished reading its staging rows (s_pvctr)
  float *s_red = reinterpret_cast<float *>(xb + kStg);
  int16_t *s_rl = reinterpret_cast<int16_t *>(xb + kStg + NW * kStgW);   // [K wave][KS]
  static_assert(kGqa * KS * 4 + 2 * KS * 8 + kGqa * KS + 2 * KS <= 24576, "e, p16', p16, binade map, risk index");
  static_assert(24576 + kGqa * kMaxSpecial * sizeof(Special) + kGqa * sizeof(WS) <= 53248, "specials, walk scratch");
  static_assert(NW * kGqa * kHd * 4 <= NW * kStgW, "the PV partials over the staging rows");
  static_assert(kStg + NW * kStgW + kSwKW * KS * 2 <= sizeof(kt), "at-risk rows, PV staging, at-risk key lists");
  const int th = lane >> 4, tt = lane & 15;   // tail e pass: lane 16 h + t takes tail key t, head h
  const int vsub = lane & 15, vkk = lane >> 4;
  // the PV's pass keys per wave (kw0 = NKW w ..) and V slots per lane (slot s: key kw0 + 4 s + vkk,
  // its 16-byte chunk vsub), staged for the matrix cores in rounds of 32 keys
  constexpr int NKW = SHORT ? 16 : 64, NS = NKW / 4, NR = (NKW + kPv8Rows - 1) / kPv8Rows;
  const int kw0 = NKW * wave;
  auto vsc_row = [&](int k) { return SHORT ? (k / NKW) * 64 + k % NKW : k; };   // pass key k's V scale row

  // ---------------------------------------------------------------- loads
  // Wave 0 first brings q (and decode_step's new K and V) into LDS; every wave then stages its K
  // tile (pass keys 64 w ..) and its tail K rows (tail keys 2 w, 2 w + 1) by direct-to-LDS loads,
  // its V scale rows into LDS and its V rows into registers: the whole stream is requested up front.
  // The direct-to-LDS loads bypass the compiler's wait counting; each wait below names how many loads
  // were issued after the ones it needs (the V loads are the compiler's and come last).
  const bool t0 = 64 * wave < np;              // the wave's K tile holds keys
  const int tr = min(2, max(0, tn - 2 * wave));   // the wave's tail K rows
  const bool vt = !SHORT && wave < 4;          // the wave holds a tail V slot
  if (wave == 0) {
    const uint32_t qb = __builtin_amdgcn_readfirstlane(lds_addr(s_q));
    const float *qsrc = a.q + (size_t)g * kGqa * a.qs;
#pragma unroll
    for (int i = 0; i < kGqa; ++i)             // head i's 256 floats: 64 lanes x 16 B
      asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(qsrc + (size_t)i * a.qs + 4 * lane),
                   "s"(qb + 1024u * i) : "memory", "m0");
    if (appender) {
      const uint32_t xbs = __builtin_amdgcn_readfirstlane(lds_addr(s_x));
      asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(a.ap.k + (size_t)g * kHd + 4 * lane),
                   "s"(xbs) : "memory", "m0");
      asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(a.ap.v + (size_t)g * kHd + 4 * lane),
                   "s"(xbs + 1024u) : "memory", "m0");
    }
  }
  // (fp16 K: half row ch, dims 128 ch .., of each key; column 16 an unused copy. Full plans: quarter
  // rows instead, quarters 0 and 1 here, quarters 2 and 3 once the chains have passed 0 and 1)
  constexpr bool KQ = K16 && !SHORT;
  auto stage_tile = [&](int ch) {
    if (t0) {
      if constexpr (KQ) {
        stage_k16_quarter<PG>(kt + 64 * wave * kUPR, sm, nkv, g, 64 * wave, min(64, np - 64 * wave), 2 * ch, 0);
        stage_k16_quarter<PG>(kt + 64 * wave * kUPR, sm, nkv, g, 64 * wave, min(64, np - 64 * wave), 2 * ch + 1, 1);
      } else {
        stage_k_wave<KF, PG>(kt + 64 * wave * kUPR, sm, nkv, g, 64 * wave, min(64, np - 64 * wave), ch);
      }
    }
  };
  auto stage_tail = [&](int ch) {
    if (tr > 0) {                              // 2 rows x 17 uint4: lanes 0..33
      const uint32_t tb = __builtin_amdgcn_readfirstlane(lds_addr(ttl + 2 * wave * kUPR));
      const int row = lane / kUPR, col = lane - row * kUPR;
      const int64_t sl = slot_k<PG>(sm, NP + 2 * wave + min(row, tr - 1));
      const uint8_t *src = K16 ? L.kd + (sl * nkv + g) * row_bytes(KF) + (ch * 16 + (col & 15)) * 16
                         : col == 16 ? L.ks + (sl * nkv + g) * kScaleRowBytes : L.kd + (sl * nkv + g) * kHd + col * 16;
      if (lane < 2 * kUPR)
        asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(tb) : "memory", "m0");
    }
  };
  stage_tile(0);
  stage_tail(0);
  // q (and x) are read by every wave: wave 0 waits for them (the K loads it issued after them may
  // still be in flight), then the workgroup syncs once; each wave then waits for its own K rows only
  // and scores them while the other waves' tiles are still landing
  if (wave == 0) wait_vm_n((t0 ? (KQ ? 16 : kUPR) : 0) + (tr > 0 ? 1 : 0));
  __syncthreads();                             // s_q (and s_x) visible to every wave
  // the q8_0 K digits of the group's q rows, in the V scale rows' LDS (their loads come after the
  // scores, once every wave has read its A operands)
  // (fp16 K: the q rows rounded to q16 in place, read from LDS by the score chains)
  int8_t *s_lim = reinterpret_cast<int8_t *>(vsc);
  static_assert(kLimBytes <= (int)sizeof(vsc), "digits in the V scale rows");
  Q8Lim qlim;
  float *const q16 = reinterpret_cast<float *>(s_q);
  if constexpr (!K16) {
    q8lim_build(q16, kHd, s_lim, s_lt, &s_wide, tid, NT);
    __syncthreads();
    q8lim_load(s_lim, s_lt, qlim);
  } else {
    for (int i = tid; i < kGqa * kHd; i += NT) q16[i] = round_f16(q16[i]);
    __syncthreads();
  }
  // the DPP chains' q operand (short plans and tail keys): qt[j] = q16[h][16 j + lane % 16]
  auto load_qt = [&](int h, float (&qt)[kHd / 16]) {
#pragma unroll
    for (int j = 0; j < kHd / 16; ++j) qt[j] = q16[h * kHd + 16 * j + (lane & 15)];
#pragma unroll
    for (int j = 0; j < kHd / 16; ++j) asm volatile("" : "+v"(qt[j]));
    asm volatile("s_nop 4");                   // (the DPP reads of qt come from inline asm)
  };
  const bool wide = !K16 && s_wide != 0u;
  wait_vm<0>();                                // this wave's K tile
  RTSV(0);

  // ---------------------------------------------------------------- scores
  // q8_0 K on the int8 matrix cores (bkv_q8dot.h): each wave scores its 64 keys as four MFMA key
  // groups and transposes them to one key per lane, 4 heads each; the tail keys 2 w, 2 w + 1 are
  // one more (partly empty) key group.
  float sc[kGqa];
  float sv_short = 0.0f;                       // SHORT: the score of key 16 w + lane % 16, head lane / 16
  float mloc[kGqa];
#pragma unroll
  for (int h = 0; h < kGqa; ++h) { mloc[h] = -INFINITY; sc[h] = 0.0f; }
  const int kl = 64 * wave + lane;             // this lane's pass key
  constexpr bool bsplit = SHORT;               // short workgroups: all 8 waves score and run the e pass
  {
    // decode_step: the wave that holds the new token's K row quantises the token (both rows stored
    // to the cache here), patches its K row into the tile and leaves its V row in s_x
    uint4 ad = make_uint4(0u, 0u, 0u, 0u);
    uint32_t asw = 0u;
    if (wave == aw) {
      const float *xf = reinterpret_cast<const float *>(s_x);
      append_q8_rows<K16>(a.ap, slot_k<PG>(sm, kp), xf, xf + kHd, g, lane, ad, asw);   // (decode_step: base 0)
      wave_lds_sync();
      __builtin_amdgcn_wave_barrier();
      if (lane >= 32 && lane < 48) {           // the V patch row: 16 data uint4, then the scale row
        s_x[lane - 32] = ad;
        if (((lane - 32) & 3) == 0) reinterpret_cast<uint32_t *>(&s_x[16])[(lane - 32) >> 2] = asw;
      }
    }
    auto patch_k = [&](uint4 *row, int ch) {  // the appended K row (fp16: half row ch) over its staged copy
      if constexpr (K16) {
        if (lane >= 16 * ch && lane < 16 * ch + 16) row[lane - 16 * ch] = ad;
      } else if (lane < 16) {
        row[lane] = ad;
        if ((lane & 3) == 0) reinterpret_cast<uint32_t *>(&row[16])[lane >> 2] = asw;
      }
      wave_lds_sync();
    };
    asm volatile("s_nop 4");
    RTSV(5);
    RTSC(6);
    if (bsplit) {
      // at most 2 x 64 keys: every wave scores one MFMA key group of 16
      RTS(14);
      if (wave == aw && kp < NP) patch_k(kt + kp * kUPR, 0);
      __syncthreads();                         // both tiles (and the patched row) are in LDS
      // wave w: keys 16 w + lane % 16 against head lane / 16 (the scores go to s_e, over the K
      // tiles, once every wave has scored)
      const int i16 = lane & 15, hg = lane >> 4, key = 16 * wave + i16;
      float v = 0.0f;
      if constexpr (K16) {
        // one chain per lane over both half rows: the second half is staged once every wave has
        // taken the first
        float qt[kHd / 16];
        load_qt(hg, qt);
        const uint4 *row = kt + min(key, np - 1) * kUPR;
        if (16 * wave < np) qk_f16_half1<0>(row, qt, v);   // (uniform)
        __syncthreads();
        stage_tile(1);
        wait_vm<0>();
        if (wave == aw && kp < NP) patch_k(kt + kp * kUPR, 1);
        __syncthreads();
        if (16 * wave < np) qk_f16_half1<1>(row, qt, v);
      } else if (16 * wave < np) {             // (uniform)
        const uint4 *row = kt + min(key, np - 1) * kUPR;
        if (!wide) {
          v = q8_score16(row, qlim);
        } else {
          float a4[kGqa];
          q8_score_key_slow(row, q16, kHd, a4);
          v = pick4(a4, hg);
        }
      }
      const bool live = key < np;
#pragma unroll
      for (int h = 0; h < kGqa; ++h) mloc[h] = (live && h == hg) ? v * a.scale : -INFINITY;
      sv_short = live ? v : 0.0f;
      __syncthreads();
      if (live) s_e[hg * KS + key] = v;        // for the e pass, which reads them by (key, head)
      RTSV(1);
    } else if (t0) {
      RTS(14);
      if constexpr (!KQ)
        if (wave == aw && kp < NP) patch_k(kt + kp * kUPR, 0);
      float acc1[kGqa];
      if constexpr (K16) {
        // the chains on the fp32 matrix cores over quarter rows 0 and 1 (slots 0, 1 of the wave's
        // tile region); each slot is restaged with quarter 2 / 3 as soon as the chains have read it
        // (attn_vk.h:156-170: one chain per key and head in ascending d)
        char *reg = reinterpret_cast<char *>(kt + 64 * wave * kUPR);
        const uint4 *myrow = reinterpret_cast<const uint4 *>(reg + 128 * (lane & 63));
        auto patch_q = [&](int Q, int S) {       // the appended K row's quarter Q over its staged copy
          if (wave == aw && kp < NP) {
            if (lane >= 8 * Q && lane < 8 * Q + 8)
              reinterpret_cast<uint4 *>(reg + 8192 * S + 128 * (kp - 64 * wave))[lane - 8 * Q] = ad;
            wave_lds_sync();
          }
        };
        patch_q(0, 0);
        patch_q(1, 1);
        fv4_t acc = fv4_t{0.0f, 0.0f, 0.0f, 0.0f};
        qk_f16_mfma<0, 4>(myrow, q16, acc);
        wave_lds_sync();
        stage_k16_quarter<PG>(kt + 64 * wave * kUPR, sm, nkv, g, 64 * wave, min(64, np - 64 * wave), 2, 0);
        qk_f16_mfma<64, 4>(myrow + 512, q16, acc);
        wave_lds_sync();
        stage_k16_quarter<PG>(kt + 64 * wave * kUPR, sm, nkv, g, 64 * wave, min(64, np - 64 * wave), 3, 1);
        wait_vm<8>();
        patch_q(2, 0);
        qk_f16_mfma<128, 4>(myrow, q16, acc);
        wait_vm<0>();
        patch_q(3, 1);
        qk_f16_mfma<192, 4>(myrow + 512, q16, acc);
#pragma unroll
        for (int h = 0; h < kGqa; ++h) acc1[h] = acc[h];
      } else if (!wide) {
        // four MFMA key groups of 16 (lane: key 16 c + lane % 16, head lane / 16), then transposed
        // to one key per lane
        q8_score64(kt + 64 * wave * kUPR, kUPR, qlim, acc1);
      } else {
        q8_score_key_slow(kt + kl * kUPR, q16, kHd, acc1);
      }
#pragma unroll
      for (int h = 0; h < kGqa; ++h) {
        sc[h] = acc1[h];
        if (kl < np) mloc[h] = fmaxf(mloc[h], acc1[h] * a.scale);
      }
      RTSV(1);
    }
    if (tr > 0) {
      if (wave == aw && kp >= NP) patch_k(ttl + (kp - NP) * kUPR, 0);
      // the wave's tail keys 2 w, 2 w + 1 (lane: key lane % 16, head lane / 16; q8_0 K: as MFMA
      // columns 0, 1)
      const int n16 = lane & 15, hg = lane >> 4, t = 2 * wave + n16;
      const uint4 *row = ttl + (2 * wave + min(n16, tr - 1)) * kUPR;
      float v[kGqa];
      if constexpr (K16) {
        float qt[kHd / 16];
        load_qt(hg, qt);
        float x = 0.0f;
        qk_f16_half1<0>(row, qt, x);
        wave_lds_sync();
        stage_tail(1);
        wait_vm<0>();
        if (wave == aw && kp >= NP) patch_k(ttl + (kp - NP) * kUPR, 1);
        qk_f16_half1<1>(row, qt, x);
#pragma unroll
        for (int h = 0; h < kGqa; ++h) v[h] = x;
      } else if (!wide) {
        const float x = q8_score16(row, qlim);
#pragma unroll
        for (int h = 0; h < kGqa; ++h) v[h] = x;
      } else {
        q8_score_key_slow(row, q16, kHd, v);
      }
      const bool tv = n16 < tr;
      if (!wide) {
        if (tv) s_tsc[t * kGqa + hg] = v[0];
      } else if (tv && hg == 0) {
#pragma unroll
        for (int h = 0; h < kGqa; ++h) s_tsc[t * kGqa + h] = v[h];
      }
#pragma unroll
      for (int hh = 0; hh < kGqa; ++hh) {      // fold the tail scores into the lane maxima
        const bool on = tv && (wide ? hg == 0 : hg == hh);
        mloc[hh] = fmaxf(mloc[hh], on ? v[wide ? hh : 0] * a.scale : -INFINITY);
      }
    }
  }
  RTSC(7);
  RTS(1);
  RTSV(2);
  // the workgroup's (max of s*scale, sum of exp(s*scale - max)) per head, with one barrier: each
  // wave's maximum and its sum of exps against it go to LDS; every lane takes the maximum over the
  // waves (mloc, which the PV's scale bound reads), and the lanes that store the statistics rescale
  // the waves' sums to it. (The sum feeds S_a and the workgroups' positions, estimates whose
  // margins are far above the few fp32 roundings this adds; the exact sum is the walk's.)
  {
    float wm[kGqa];
#pragma unroll
    for (int h = 0; h < kGqa; ++h)
      wm[h] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wave_max_l63(mloc[h])), 63));
    float lw[kGqa];
#pragma unroll
    for (int h = 0; h < kGqa; ++h) {
      float l;
      if constexpr (SHORT) {
        l = (16 * wave + (lane & 15) < np && h == (lane >> 4)) ? __expf(sv_short * a.scale - wm[h]) : 0.0f;
      } else {
        l = (t0 && kl < np) ? __expf(sc[h] * a.scale - wm[h]) : 0.0f;
      }
      lw[h] = wave_sum_l63(l);
    }
    if (lane == 63)
#pragma unroll
      for (int h = 0; h < kGqa; ++h) s_ml[wave * kGqa + h] = make_float2(wm[h], lw[h]);
    __syncthreads();
    RTSV(3);
#pragma unroll
    for (int h = 0; h < kGqa; ++h) {
      float r = s_ml[h].x;
#pragma unroll
      for (int i = 1; i < NW; ++i) r = fmaxf(r, s_ml[i * kGqa + h].x);
      mloc[h] = r;
    }
    // wave 0: the waves' sums rescaled to the maximum (lane 4 i + h: wave i < NW, head h) and the
    // tail keys (several waves scored them: read after the barrier; lane 16 h + t), summed per head
    if (wave == 0) {
      const int hh = lane & 3;
      const float M = pick4(mloc, hh);
      const float2 x = lane < NW * kGqa ? s_ml[lane] : make_float2(-INFINITY, 0.0f);
      float r = x.x != -INFINITY ? x.y * __expf(x.x - M) : 0.0f;
      r += __shfl_xor(r, 4);
      r += __shfl_xor(r, 8);
      r += __shfl_xor(r, 16);
      const float tx = row16_sum(tt < tn ? __expf(s_tsc[tt * kGqa + th] * a.scale - pick4(mloc, th)) : 0.0f);
      const float L = r + __shfl(tx, 16 * hh);
      if (lane < kGqa) st_agent(tstats + lane * GM + wi, pack_stats(M, L, tag));
    }
    __syncthreads();                           // the statistics go out ahead of every wave's V requests
  }
  RTS(9);
  // V after the statistics: the K stream (which the scores wait for) is not shared with the V
  // stream (which only the PV needs), and the statistics do not wait behind the V requests, whose
  // issue stalls a wave while its CU's memory queue is full. (Polling waves that request theirs
  // only after barrier A hold up the e pass: 288 against 280 us per token.) The digits in vsc were
  // read before the statistics' barrier.
  // (vector types: copies of HIP's uint4 struct into LDS are memcpys, which keep the array in
  // scratch memory)
  u32x4 vd[NS];                                // slot s: row kw0 + 4 s + vkk
  u32x4 vtl = u32x4{0u, 0u, 0u, 0u};           // the tail slot (waves 0..3): row NP + 4 w + vkk
  uint32_t xs = 0u;                            // the tail slot's scale word
  // V1 (slots of the first round, and the scale rows) before barrier A; the rest once the records
  // are out (the barrier-A polls wait behind every load their CU has queued, and only the PV reads
  // the later slots)
  constexpr int NS1 = NS < 8 ? NS : 8;
  auto request_v = [&]() {
    {
      const uint32_t sb = __builtin_amdgcn_readfirstlane(lds_addr(vsc + wave * 64));
      const int64_t sl = slot_k<PG>(sm, min(kw0 + (lane & (NKW - 1)), nk - 1));
      asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(L.vs + (sl * nkv + g) * kScaleRowBytes),
                   "s"(sb) : "memory", "m0");
    }
#pragma unroll
    for (int s = 0; s < NS1; ++s) {
      const int64_t sl = slot_k<PG>(sm, min(kw0 + 4 * s + vkk, nk - 1));
      vd[s] = *reinterpret_cast<const u32x4 *>(L.vd + (sl * nkv + g) * kHd + vsub * 16);
    }
    if (vt) {
      const int64_t sl = slot_k<PG>(sm, min(NP + 4 * wave + vkk, nk - 1));
      xs = *reinterpret_cast<const uint32_t *>(L.vs + (sl * nkv + g) * kScaleRowBytes + (vsub >> 2) * 4);
      vtl = *reinterpret_cast<const u32x4 *>(L.vd + (sl * nkv + g) * kHd + vsub * 16);
    }
  };
  // (the tail slot goes with V1: loads only some waves issue, between the two groups, would make
  // the compiler's wait for the first round's rows also wait for part of V2 on those waves)
  auto request_v2 = [&]() {
#pragma unroll
    for (int s = NS1; s < NS; ++s) {
      const int64_t sl = slot_k<PG>(sm, min(kw0 + 4 * s + vkk, nk - 1));
      vd[s] = *reinterpret_cast<const u32x4 *>(L.vd + (sl * nkv + g) * kHd + vsub * 16);
    }
  };
  if (kwave) request_v();

  // ---------------------------------------------------------------- barrier A: global max
  // wave h polls head h's statistics of every workgroup of the group (the V stream has landed by
  // now: a poll's load would wait for it)
  if (kwave) {
    unsigned long long v[2];
    poll_tagged(tstats + wave * GM, 1, 1, G, tag, v, err);
    const float mw = lane < G ? __uint_as_float((unsigned)(v[0] >> 32)) : -INFINITY;
    const float lw = lane < G ? __uint_as_float((unsigned)v[0] & ~3u) : 0.0f;
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
      s_Sa[wave] = (float)t;
    }
  }
  __syncthreads();
  RTS(2);
  // waves kGqa.. request their first V group now: their PV starts only after the e pass, and in
  // front of the barrier-A polls the loads would hold the polls up
  if (!kwave) request_v();

  // ---------------------------------------------------------------- e, classification, records
  // Block w = keys 64 w .. 64 w + 63 (wave w); wave 0 also the tail (block 8, lane 16 h + t: key
  // NP + t, head h). Each step of the serial sum is placed on its fp32 position: the workgroup's
  // fp64 start rounded to fp32 (the classification margin is 2^-14 relative, far above the fp32
  // error of a position), plus the blocks before and the lane's scan.
  float Mh[kGqa], rSa[kGqa], P0f[kGqa], ev[kGqa], fin[kGqa];
#pragma unroll
  for (int h = 0; h < kGqa; ++h) { Mh[h] = s_M[h]; rSa[h] = 1.0f / s_Sa[h]; P0f[h] = (float)s_P0[h]; }
  // p16' = f16(e * (1/S_a)) (a speculative value: any rounding of it serves, the corrections
  // subtract exactly what the PV added); at risk: p16' would round differently somewhere within
  // 2 kSwRiskBand of it
  auto risky = [](float p) {
    const _Float16 a = (_Float16)(p * (1.0f - 2.0f * kSwRiskBand)), b = (_Float16)(p * (1.0f + 2.0f * kSwRiskBand));
    return __builtin_bit_cast(uint16_t, a) != __builtin_bit_cast(uint16_t, b);
  };
  if (!bsplit) {
  const bool valid = kl < np;
  {
    // the 4 heads' exps together, branch-free (their table reads in flight at once), the rare
    // cases the table path leaves to the library afterwards
    float xh[kGqa];
    bool slow[kGqa], any = false;
#pragma unroll
    for (int h = 0; h < kGqa; ++h) {
      xh[h] = sc[h] * a.scale - Mh[h];
      ev[h] = exp_t_fast(xh[h], s_t2, slow[h]);
      any = any || (valid && slow[h]);
    }
    if (any) {
#pragma unroll
      for (int h = 0; h < kGqa; ++h)
        if (slow[h]) ev[h] = exp_t_slow(xh[h]);
    }
#pragma unroll
    for (int h = 0; h < kGqa; ++h) ev[h] = valid ? ev[h] : 0.0f;
  }
#pragma unroll
  for (int h = 0; h < kGqa; ++h) {
    fin[h] = wave_incl_scan_dpp(ev[h]);
    if (valid) s_e[h * KS + kl] = ev[h];
  }
  if (lane == 63) s_bt[wave] = make_float4(fin[0], fin[1], fin[2], fin[3]);
  if (a.keep_e && valid)
#pragma unroll
    for (int h = 0; h < kGqa; ++h) a.e[(size_t)(g * kGqa + h) * a.ld + kb + kl] = ev[h];
  float evt = 0.0f, fint = 0.0f;
  const bool tl = wave == 0 && tn > 0;
  const bool tvalid = tl && tt < tn;
  if (tl) {
    evt = tvalid ? exp_cr_t(s_tsc[min(tt, kResTail - 1) * kGqa + th] * a.scale - pick4(Mh, th), s_t2) : 0.0f;
    fint = row_incl_scan_dpp(evt);
    if (tvalid) s_e[th * KS + NP + tt] = evt;
    if (tt == 15) reinterpret_cast<float *>(&s_bt[kSwBlocks - 1])[th] = fint;
    if (a.keep_e && tvalid) a.e[(size_t)(g * kGqa + th) * a.ld + kb + NP + tt] = evt;
  }
  __syncthreads();
  bool sp[kGqa];
  double din[kGqa], dinc[kGqa];
  unsigned long long msk[kGqa];
  {
    float fb[kGqa] = {0.f, 0.f, 0.f, 0.f};
    for (int b = 0; b < wave; ++b) {
      const float4 t = s_bt[b];
      fb[0] += t.x; fb[1] += t.y; fb[2] += t.z; fb[3] += t.w;
    }
#pragma unroll
    for (int h = 0; h < kGqa; ++h) {
      const float ab = P0f[h] + (fb[h] + (fin[h] - ev[h]));
      int bin, inc;
      bool spx;
      classify_i(ab, ab + ev[h], ev[h], spx, bin, inc);
      spx = spx && valid;
      sp[h] = spx;
      if (valid) s_bin[h * KS + kl] = spx ? kNoBin8 : (int8_t)bin;
      msk[h] = __ballot(spx);
      // a block whose steps all sit in one binade and hold no special sums its increments as
      // integers; otherwise an fp64 scan (exact: a workgroup's increments are integers below 2^50
      // in units of 2^-40)
      const int b0 = __builtin_amdgcn_readfirstlane(bin);
      const bool uni = msk[h] == 0 && __ballot(valid && bin != b0) == 0;
      if (uni) {
        const int t = wave_sum64_i(valid ? inc : 0);
        din[h] = 0.0;
        dinc[h] = 0.0;
        if (lane == 63) s_bu[wave * kGqa + h] = ldexp((double)t, b0 + 17);
      } else {
        dinc[h] = (valid && !spx) ? ldexp((double)inc, bin + 17) : 0.0;
        din[h] = wave_incl_scan_dpp(dinc[h]);
        if (lane == 63) s_bu[wave * kGqa + h] = din[h];
      }
      if (lane == 63) s_bc[wave * kGqa + h] = __popcll(msk[h]);
    }
  }
  bool spt = false;
  double dint = 0.0, dinct = 0.0;
  unsigned rowm = 0u;
  if (tl) {
    float fb = 0.0f;
#pragma unroll
    for (int b = 0; b < kSwBlocks - 1; ++b) fb += reinterpret_cast<const float *>(&s_bt[b])[th];
    const float ab = pick4(P0f, th) + (fb + (fint - evt));
    int bin, inc;
    classify_i(ab, ab + evt, evt, spt, bin, inc);
    spt = spt && tvalid;
    dinct = (tvalid && !spt) ? ldexp((double)inc, bin + 17) : 0.0;
    if (tvalid) s_bin[th * KS + NP + tt] = spt ? kNoBin8 : (int8_t)bin;
    rowm = (unsigned)(__ballot(spt) >> (16 * th)) & 0xFFFFu;
    dint = row_incl_scan_dpp(dinct);
    if (tt == 15) {
      s_bu[(kSwBlocks - 1) * kGqa + th] = dint;
      s_bc[(kSwBlocks - 1) * kGqa + th] = __popc(rowm);
    }
  }
  __syncthreads();                             // block totals, the binade map
  // specials into LDS (at most kMaxSpecial per head)
#pragma unroll
  for (int h = 0; h < kGqa; ++h) {
    if (sp[h]) {
      int cb = 0;
      double ib = 0.0;
      for (int b = 0; b < wave; ++b) { cb += s_bc[b * kGqa + h]; ib += s_bu[b * kGqa + h]; }
      const int id = cb + (int)__builtin_amdgcn_mbcnt_hi((unsigned)(msk[h] >> 32), __builtin_amdgcn_mbcnt_lo((unsigned)msk[h], 0u));
      if (id < kMaxSpecial) {
        const int8_t bp8 = kl > 0 ? s_bin[h * KS + kl - 1] : (int8_t)0;
        const int bprev = kl > 0 ? (bp8 == kNoBin8 ? kNoBinade : bp8) : 127;
        Special x;
        x.ipre = (long long)(ib + (din[h] - dinc[h]));
        x.e = ev[h];
        x.meta = kl | ((bprev == kNoBinade ? 0 : (bprev + 128)) << 16);
        st_spec(&spec_g[((size_t)h * G + wi) * kMaxSpecial + id], x);
      }
    }
  }
  if (spt) {
    int cb = 0;
    double ib = 0.0;
    for (int b = 0; b < kSwBlocks - 1; ++b) { cb += s_bc[b * kGqa + th]; ib += s_bu[b * kGqa + th]; }
    const int id = cb + __popc(rowm & ((1u << tt) - 1u));
    if (id < kMaxSpecial) {
      const int8_t bp8 = s_bin[th * KS + NP + tt - 1];
      const int bprev = bp8 == kNoBin8 ? kNoBinade : bp8;
      Special x;
      x.ipre = (long long)(ib + (dint - dinct));
      x.e = evt;
      x.meta = (NP + tt) | ((bprev == kNoBinade ? 0 : (bprev + 128)) << 16);
      st_spec(&spec_g[((size_t)th * G + wi) * kMaxSpecial + id], x);
    }
  }
  {
    bool rk = false;
    if (valid) {
      _Float16 pk[kGqa];
      bool r = false;
#pragma unroll
      for (int h = 0; h < kGqa; ++h) {
        const float p = ev[h] * rSa[h];
        pk[h] = (_Float16)p;
        r = r || risky(p);
      }
      s_ps[kl] = make_uint2((uint32_t)__builtin_bit_cast(uint16_t, pk[0]) | ((uint32_t)__builtin_bit_cast(uint16_t, pk[1]) << 16),
                            (uint32_t)__builtin_bit_cast(uint16_t, pk[2]) | ((uint32_t)__builtin_bit_cast(uint16_t, pk[3]) << 16));
      int ri = -1;
      rk = r;
      if (r) {
        ri = atomicAdd(&s_nrisk, 1);
        if (ri >= kSwRisk) ri = -1;
      }
      s_ridx[kl] = (int16_t)ri;
    } else {
      s_ridx[kl] = -1;
    }
    if (wave == 1 && lane < kResTail) s_ridx[NP + lane] = -1;
    {
      const unsigned long long rbw = __ballot(rk);
      if (lane == 0) s_rb[wave] = rbw;
      if (wave == 0 && lane == 1 && tn == 0) s_rb[kSwBlocks - 1] = 0ull;
    }
    __syncthreads();
    if (tl) {                                  // the tail: one head per lane
      const float p = evt * pick4(rSa, th);
      if (tvalid) reinterpret_cast<_Float16 *>(s_ps + NP + tt)[th] = (_Float16)p;
      const unsigned long long rm = __ballot(tvalid && risky(p));
      const bool r = ((rm >> tt) | (rm >> (tt + 16)) | (rm >> (tt + 32)) | (rm >> (tt + 48))) & 1ull;
      if (th == 0 && tt < tn && r) {
        const int ri = atomicAdd(&s_nrisk, 1);
        s_ridx[NP + tt] = (int16_t)(ri < kSwRisk ? ri : -1);
      }
      const unsigned long long rbt = __ballot(th == 0 && tt < tn && r);
      if (lane == 0) s_rb[kSwBlocks - 1] = rbt;
    }
  }
  } else {
    // At most 128 keys: the e pass on all eight waves with the tail's mapping, lane 16 h + i: key
    // 16 w + i, head h. Block w = keys 16 w .. 16 w + 15, positions by row scans; the score of
    // (key, head) sits in s_e, where the block-split scores left it, and e replaces it.
    const int hh = lane >> 4, i16 = lane & 15, kk = 16 * wave + i16;
    const bool sv = kk < np;
    for (int i = tid; i < KS; i += NT) s_ridx[i] = -1;
    const float evs = sv ? exp_cr_t(s_e[hh * KS + kk] * a.scale - pick4(Mh, hh), s_t2) : 0.0f;
    const float fins = row_incl_scan_dpp(evs);
    if (sv) s_e[hh * KS + kk] = evs;
    if (i16 == 15) reinterpret_cast<float *>(&s_bt[wave])[hh] = fins;
    if (a.keep_e && sv) a.e[(size_t)(g * kGqa + hh) * a.ld + kb + kk] = evs;
    __syncthreads();
    float fb = 0.0f;
    for (int b = 0; b < wave; ++b) fb += reinterpret_cast<const float *>(&s_bt[b])[hh];
    const float ab = pick4(P0f, hh) + (fb + (fins - evs));
    int bin, inc;
    bool sps;
    classify_i(ab, ab + evs, evs, sps, bin, inc);
    sps = sps && sv;
    const double dincs = (sv && !sps) ? ldexp((double)inc, bin + 17) : 0.0;
    if (sv) s_bin[hh * KS + kk] = sps ? kNoBin8 : (int8_t)bin;
    const unsigned rowms = (unsigned)(__ballot(sps) >> (16 * hh)) & 0xFFFFu;
    const double dins = row_incl_scan_dpp(dincs);
    if (i16 == 15) {
      s_bu[wave * kGqa + hh] = dins;
      s_bc[wave * kGqa + hh] = __popc(rowms);
    }
    __syncthreads();                           // block totals, the binade map
    if (sps) {
      int cb = 0;
      double ib = 0.0;
      for (int b = 0; b < wave; ++b) { cb += s_bc[b * kGqa + hh]; ib += s_bu[b * kGqa + hh]; }
      const int id = cb + __popc(rowms & ((1u << i16) - 1u));
      if (id < kMaxSpecial) {
        const int8_t bp8 = kk > 0 ? s_bin[hh * KS + kk - 1] : (int8_t)0;
        const int bprev = kk > 0 ? (bp8 == kNoBin8 ? kNoBinade : bp8) : 127;
        Special x;
        x.ipre = (long long)(ib + (dins - dincs));
        x.e = evs;
        x.meta = kk | ((bprev == kNoBinade ? 0 : (bprev + 128)) << 16);
        st_spec(&spec_g[((size_t)hh * G + wi) * kMaxSpecial + id], x);
      }
    }
    const float p = evs * pick4(rSa, hh);
    if (sv) reinterpret_cast<_Float16 *>(s_ps + kk)[hh] = (_Float16)p;
    const unsigned long long rm = __ballot(sv && risky(p));
    const bool r = ((rm >> i16) | (rm >> (i16 + 16)) | (rm >> (i16 + 32)) | (rm >> (i16 + 48))) & 1ull;
    if (hh == 0 && sv && r) {
      const int ri = atomicAdd(&s_nrisk, 1);
      s_ridx[kk] = (int16_t)(ri < kSwRisk ? ri : -1);
      atomicOr(&s_rb[kk >> 6], 1ull << (kk & 63));
    }
  }
  // every wave's specials are stored (before the records that announce them) and its V scale rows
  // are in LDS: the first V group and the specials were issued long enough ago for this wait to be short
  wait_vm<0>();
  __syncthreads();                             // p16', the risk index, the V scale rows
  RTS(3);

  // ---------------------------------------------------------------- records (K waves)
  if (kwave) {
    const int h = wave;
    int nsp = 0;
    double t = 0.0;
    for (int b = 0; b < kSwBlocks; ++b) { nsp += s_bc[b * kGqa + h]; t += s_bu[b * kGqa + h]; }
    if (lane == 0) {
      ChunkRec rc;
      rc.tot = (long long)t;
      rc.nsp = nsp;
      const int8_t bl = s_bin[h * KS + nk - 1];
      rc.blast = bl != kNoBin8 ? bl : kNoBinade;
      unsigned long long w0, w1;
      pack_rec(rc, tag, w0, w1);
      st_agent(trec + (h * GM + wi) * 2, w0);
      st_agent(trec + (h * GM + wi) * 2 + 1, w1);
    }
  }
  request_v2();

  // ---------------------------------------------------------------- the speculative PV (every wave)
  // out += p16' * V over the wave's pass keys on the int8 matrix cores (bkv_pv8.h), in rounds of 32
  // keys staged from the V registers into LDS; the rows of at-risk keys are kept in LDS for the
  // corrections. Waves 0..3 add the tail slot on the VALU (acc, which later takes the corrections).
  float acc[kGqa][VR::EPL];
#pragma unroll
  for (int h = 0; h < kGqa; ++h)
#pragma unroll
    for (int i = 0; i < VR::EPL; ++i) acc[h][i] = 0.0f;
  auto p4 = [](uint2 pw, float (&p)[kGqa]) {
    p[0] = f16_to_f32(pw.x & 0xFFFFu);
    p[1] = f16_to_f32(pw.x >> 16);
    p[2] = f16_to_f32(pw.y & 0xFFFFu);
    p[3] = f16_to_f32(pw.y >> 16);
  };
  // the appended row (decode_step) replaces the loaded copy, which may predate it
  const u32x4 pd = reinterpret_cast<const u32x4 *>(s_x)[vsub];
  const uint32_t pws = reinterpret_cast<const uint32_t *>(&s_x[16])[vsub >> 2];
  const float pscale = f16_to_f32(((vsub >> 1) & 1) ? (pws >> 16) : (pws & 0xFFFFu));
  float pvp[16];                               // the wave's partial: head lane / 16, dim 16 t + lane % 16
  RTSV(13);
  if constexpr (SHORT) {
    // short plans: 16 keys per wave on the VALU (with so few keys the matrix-core form's fixed
    // costs and LDS round trips take longer)
    const unsigned rbw = (unsigned)(s_rb[kw0 >> 6] >> (kw0 & 63)) & 0xFFFFu;
#pragma unroll
    for (int sl = 0; sl < NS; ++sl) {
      const int key = kw0 + 4 * sl + vkk;
      const bool live = key < np;
      float p[kGqa];
      p4(live ? s_ps[key] : make_uint2(0u, 0u), p);
      const uint32_t sw = reinterpret_cast<const uint32_t *>(vsc + wave * 64 + 4 * sl + vkk)[vsub >> 2];
      const u32x4 rv = key == kp ? pd : vd[sl];
      const uint4 row = make_uint4(rv.x, rv.y, rv.z, rv.w);
      const float vs = key == kp ? pscale : f16_to_f32(((vsub >> 1) & 1) ? (sw >> 16) : (sw & 0xFFFFu));
      v_accum<BKV_Q8_0>(row, live ? vs : 0.0f, p, acc);
      if ((rbw >> (4 * sl + vkk)) & 1u) {      // (rare) an at-risk key: its row for the corrections
        const int ri = s_ridx[key];
        if (ri >= 0) s_rrow[ri * 16 + vsub] = row;
      }
    }
#pragma unroll
    for (int t = 0; t < 16; ++t) pvp[t] = 0.0f;
    lds_arrive(&s_pvctr);
  } else {
  {
    // 2^sig(h): every p16' * scale of the wave's keys times it stays below 2^29 (p16' <= the
    // workgroup's largest e, exp(mloc - M), times 1 / S_a, plus a margin for the roundings; the
    // scale <= the largest of the wave's V scale rows)
    const bool apw = kp >= 0 && kp < NP && wave == kp / NKW;   // the appended key is one of this wave's
    if (apw && lane == 0) vsc[vsc_row(kp)] = s_x[16];        // its scale row over the loaded one
    wave_lds_sync();
    int sig[kGqa], ep[kGqa];
    {
      const uint32_t dm = f16_row_max(vsc[wave * 64 + (lane & (NKW - 1))]);
      const int ed = f16_exp_bound(__builtin_bit_cast(uint16_t, (_Float16)wave_max64(f16_to_f32(dm))));
#pragma unroll
      for (int h = 0; h < kGqa; ++h) {
        const float pb = __expf(mloc[h] - Mh[h]) * rSa[h] * 1.002f;
        ep[h] = max(-30, (int)((__float_as_uint(pb) >> 23) & 0xFFu) - 127);
        sig[h] = min(100, 27 - ep[h] - ed);
      }
    }
    const Pv8Sel z = pv8_sel();
    v4i_t pacc[16];
    const uint32_t stg = __builtin_amdgcn_readfirstlane(lds_addr(xb + kStg + wave * kStgW));
    const int ia = lane & 3, ha = (lane & 15) >> 2, kq = lane >> 4;
    const float sga = __builtin_ldexpf(1.0f, pick4(sig, ha));
    const int lim = min(np, kw0 + NKW);
    // round r's rows of this wave into its staging rows (the appended row over its loaded copy, the
    // at-risk keys' rows kept for the corrections)
    auto stage_rows = [&](auto rc) __attribute__((always_inline)) {
      constexpr int r = decltype(rc)::value;
      auto stage = [&](auto jc) __attribute__((always_inline)) {
        constexpr int j = decltype(jc)::value, sl = 8 * r + j;
        if constexpr (sl < NS)
          *reinterpret_cast<u32x4 *>(xb + kStg + wave * kStgW + (4 * j + vkk) * kPv8Stride + 16 * vsub) = vd[sl];
      };
      [&]<int... J>(std::integer_sequence<int, J...>) __attribute__((always_inline)) {
        (stage(std::integral_constant<int, J>{}), ...);
      }(std::make_integer_sequence<int, 8>{});
      const int k0 = kw0 + kPv8Rows * r;
      if (apw && kp >= k0 && kp < k0 + kPv8Rows && vkk == ((kp - k0) & 3))   // the appended row over its loaded copy
        *reinterpret_cast<u32x4 *>(xb + kStg + wave * kStgW + (kp - k0) * kPv8Stride + 16 * vsub) = pd;
      // (rare) at-risk keys: their rows kept for the corrections
      const unsigned rb32 = (unsigned)(s_rb[k0 >> 6] >> (k0 & 63)) & (NKW < 32 ? 0xFFFFu : 0xFFFFFFFFu);
      if (rb32 != 0u) {
#pragma unroll 1
        for (int j = 0; j < NKW / 4 && j < 8; ++j) {
          const int key = k0 + 4 * j + vkk;
          if ((rb32 >> (4 * j + vkk)) & 1u) {
            const int ri = s_ridx[key];
            if (ri >= 0)
              reinterpret_cast<u32x4 *>(s_rrow)[ri * 16 + vsub] = *reinterpret_cast<const u32x4 *>(xb + kStg + wave * kStgW + (4 * j + vkk) * kPv8Stride + 16 * vsub);
          }
        }
      }
      asm volatile("" ::: "memory");
    };
    // the matrix-core part of a round: keys k0 .. k0 + 31 of wave bw's keys (its scale rows, its
    // staging rows at stgb; keys from lmb on weigh 0), scaled by sgab
    auto comp = [&](auto fc, int bw, int k0, int lmb, float sgab, uint32_t stgb) __attribute__((always_inline)) {
      const int ka = k0 + 8 * kq + 2 * ia;
      auto pf = [&](int k) {
        if (k >= lmb) return 0.0f;
        const uint2 pw = s_ps[k];
        const uint32_t w = ha < 2 ? pw.x : pw.y;
        return f16_half(w, ha & 1) * sgab;     // exact: a power of two
      };
      const float pa = pf(ka), pb = pf(ka + 1);
      const int kwb = NKW * bw;
      const uint4 sa = vsc[bw * 64 + min(ka - kwb, NKW - 1)], sb = vsc[bw * 64 + min(ka + 1 - kwb, NKW - 1)];
      long A[8];
      pv8_prep(pa, pb, sa, sb, z, A);
      pv8_round<decltype(fc)::value>(stgb, A, pacc);
      asm volatile("" ::: "memory");
    };
    // Waves 0..3 run round 0 only and stage round 1's rows for wave + kGqa, which runs them after its
    // own two rounds: the K waves reach barrier B and the walk a round earlier, while waves kGqa..
    // would idle through the walk.
    if (kw0 < np) {                            // (uniform) the wave holds keys
      stage_rows(std::integral_constant<int, 0>{});
      comp(std::true_type{}, wave, kw0, lim, sga, stg);
      RTSV(14);
      if constexpr (NR > 1) {
        if (kw0 + kPv8Rows < np) {
          if (kwave) {
            wave_lds_sync();                   // round 0's staging reads are done
            stage_rows(std::integral_constant<int, 1>{});
          } else {
            stage_rows(std::integral_constant<int, 1>{});
            comp(std::false_type{}, wave, kw0 + kPv8Rows, lim, sga, stg);
          }
        }
      }
      const int nsig = -pick4(sig, lane >> 4);
#pragma unroll
      for (int t = 0; t < 16; ++t) pvp[t] = pv8_value(pacc[t], nsig);
      RTSV(15);
    } else {
#pragma unroll
      for (int t = 0; t < 16; ++t) pvp[t] = 0.0f;
    }
    if (kwave) {
      lds_arrive(&s_stg1);                     // round 1's rows staged (or none to stage)
    } else if constexpr (NR > 1) {
      const int bw = wave - kSwKW, kwb = NKW * bw;
      if (kwb + kPv8Rows < np) {               // (uniform) wave bw's round 1, with its own 2^sig
        int sig2[kGqa];
        const uint32_t dm = f16_row_max(vsc[bw * 64 + (lane & (NKW - 1))]);
        const int ed2 = f16_exp_bound(__builtin_bit_cast(uint16_t, (_Float16)wave_max64(f16_to_f32(dm))));
#pragma unroll
        for (int h = 0; h < kGqa; ++h) sig2[h] = min(100, 27 - ep[h] - ed2);
        lds_wait(&s_stg1, kSwKW);
        const uint32_t stgb = __builtin_amdgcn_readfirstlane(lds_addr(xb + kStg + bw * kStgW));
        comp(std::true_type{}, bw, kwb + kPv8Rows, min(np, kwb + NKW), __builtin_ldexpf(1.0f, pick4(sig2, ha)), stgb);
        const int nsig2 = -pick4(sig2, lane >> 4);
#pragma unroll
        for (int t = 0; t < 16; ++t) pvp[t] += pv8_value(pacc[t], nsig2);
      }
    }
    lds_arrive(&s_pvctr);                      // (waits for this wave's staging reads)
  }
  }
  if (vt && tn > 0) {                          // the tail slot: key NP + 4 w + vkk
    const int key = NP + 4 * wave + vkk;
    const bool live = key < nk;
    float p[kGqa];
    p4(live ? s_ps[key] : make_uint2(0u, 0u), p);
    const u32x4 rv = key == kp ? pd : vtl;
    const uint4 row = make_uint4(rv.x, rv.y, rv.z, rv.w);
    const float vs = key == kp ? pscale : f16_to_f32(((vsub >> 1) & 1) ? (xs >> 16) : (xs & 0xFFFFu));
    v_accum<BKV_Q8_0>(row, live ? vs : 0.0f, p, acc);
    const int ri = s_ridx[min(key, KS - 1)];
    if (live && ri >= 0) s_rrow[ri * 16 + vsub] = row;
  }
  if (vt && (vsub & 3) == 0) s_tsw[(4 * wave + vkk) * 4 + (vsub >> 2)] = xs;
  if (!kwave && !SHORT) {                      // the partial goes out once every wave has read its staging
    lds_wait(&s_pvctr, NW);
#pragma unroll
    for (int t = 0; t < 16; ++t) s_red[(wave * kGqa + (lane >> 4)) * kHd + 16 * t + (lane & 15)] = pvp[t];
  }
  RTS(13);
  RTSV(4);

  if (kwave) {
    // ---------------------------------------------------------------- barrier B, the walk
    const int h = wave;
    __builtin_amdgcn_s_setprio(2);
    {
      unsigned long long v[2];
      poll_tagged(trec + h * GM * 2, 2, 2, G, tag, v, err);
      RTS(4);
      const ChunkRec x = unpack_rec(v[0], v[1]);
      float sres;
      bool gres;
      walk_one<WS>(x, a.spec + (size_t)(g * kGqa + h) * G * kMaxSpecial, G, (int64_t)a.kpw, (int64_t)a.nfill,
                   s_walk[h], sres, gres,
                   a.tsw ? a.tsw + (blockIdx.x * 8 + wave) * 16 + 8 : nullptr);
      if (lane == 0) {
        s_S[h] = sres;
        s_ok[h] = gres ? 1 : 0;
      }
    }
    __builtin_amdgcn_s_setprio(0);
    unsigned kc = kSwKW;                       // K-wave spin barrier target
    kwave_sync(&s_kctr, kc);
    RTS(5);
    if (!(s_ok[0] && s_ok[1] && s_ok[2] && s_ok[3])) {
      // a classification assumption failed (in every workgroup of the group alike, since all walk
      // the same records): publish e device-wide and run the serial loop (K waves only)
      if (!a.keep_e)
        for (int i = lane; i < nk; i += 64) a.e[(size_t)(g * kGqa + h) * a.ld + kb + i] = s_e[h * KS + i];
      __builtin_amdgcn_s_waitcnt(0);
      __threadfence();
      kwave_sync(&s_kctr, kc += kSwKW);
      if (tid == 0) {
        unsigned *c3 = cnt + 3 * kCounterStride;
        atomicAdd(c3, 1u);
        unsigned spins = 0;
        while (ld_agent(c3) < (unsigned)G) {
          __builtin_amdgcn_s_sleep(1);
          if (++spins > kResSpin) {
            atomicOr(err, 1u);
            break;
          }
        }
      }
      kwave_sync(&s_kctr, kc += kSwKW);
      if (!s_ok[h]) {
        const int hh = g * kGqa + h;
        float ss = 0.0f;
        for (int64_t b0 = 0; b0 < (int64_t)a.nfill; b0 += 64) {
          const int nb = (int)min((int64_t)64, (int64_t)a.nfill - b0);
          const float x = lane < nb ? ld_agent(&a.e[(size_t)hh * a.ld + b0 + lane]) : 0.0f;
          for (int i = 0; i < nb; ++i) ss = __fadd_rn(ss, __shfl(x, i));
        }
        if (lane == 0) s_S[h] = ss;
      }
    }
    const float S = s_S[h];
    if (wi == 0 && lane == 0) {
      a.sum[g * kGqa + h] = S;
      a.status[g * kGqa + h] = s_ok[h] ? 0u : 1u;
    }
    // (p16 - p16') * v for up to 4 keys whose rounding the exact sum changed (row group vkk takes
    // kq[vkk]; -1: none): the at-risk row from LDS, the appended row from s_x, or (a changed key not
    // at risk) the cache
    auto correct4 = [&](const int (&kq)[4]) {
      const int kc4 = kq[vkk];
      uint4 d = make_uint4(0u, 0u, 0u, 0u);
      float vs = 0.0f, p[kGqa] = {0.f, 0.f, 0.f, 0.f};
      if (kc4 >= 0) {
        float q[kGqa];
        p4(s_p16[kc4], p);
        p4(s_ps[kc4], q);
#pragma unroll
        for (int hh = 0; hh < kGqa; ++hh) p[hh] -= q[hh];
        if (kc4 == kp) {
          d = make_uint4(pd.x, pd.y, pd.z, pd.w);
          vs = pscale;
        } else {
          const int ri = s_ridx[kc4];
          const uint32_t sw = kc4 < NP ? reinterpret_cast<const uint32_t *>(vsc + vsc_row(kc4))[vsub >> 2]
                                       : s_tsw[(kc4 - NP) * 4 + (vsub >> 2)];
          vs = f16_to_f32(((vsub >> 1) & 1) ? (sw >> 16) : (sw & 0xFFFFu));
          if (ri >= 0) {
            d = s_rrow[ri * 16 + vsub];
          } else {
            const int64_t sl = slot_k<PG>(sm, kc4);
            d = *reinterpret_cast<const uint4 *>(L.vd + (sl * nkv + g) * kHd + vsub * 16);
          }
        }
      }
      v_accum<BKV_Q8_0>(d, vs, p, acc);
    };
    // When every head's exact sum lies within kSwRiskBand of S_a (relative), a key whose p16' rounds
    // the same anywhere within 2 kSwRiskBand of it (not at risk) has p16 = p16' (the fp32 roundings
    // of e / sum and e * (1 / S_a) move the quotient by a few 2^-24 at most), so only the at-risk keys
    // need the exact p16. Otherwise every key's p16 is formed and compared.
    bool fast = true;
#pragma unroll
    for (int hh = 0; hh < kGqa; ++hh)
      fast = fast && s_ok[hh] && fabsf(s_S[hh] - s_Sa[hh]) <= kSwRiskBand * fminf(s_S[hh], s_Sa[hh]);
    if (fast) {
      // the at-risk keys in key order (each K wave lists them all); then 16 keys per step, lane
      // 16 h + i: key i of the step, head h; K wave w takes steps w, w + 4, ..., so the corrections
      // of every key are added by one fixed wave in key order
      int16_t *lst = s_rl + wave * KS;
      unsigned long long rbw[kSwBlocks];
#pragma unroll
      for (int wd = 0; wd < kSwBlocks; ++wd) rbw[wd] = s_rb[wd];
      int n = 0;
#pragma unroll
      for (int wd = 0; wd < kSwBlocks; ++wd) {
        const unsigned long long b = rbw[wd];
        const int pos = n + (int)__builtin_amdgcn_mbcnt_hi((unsigned)(b >> 32), __builtin_amdgcn_mbcnt_lo((unsigned)b, 0u));
        if ((b >> lane) & 1ull) lst[pos] = (int16_t)(wd < kSwBlocks - 1 ? 64 * wd + lane : NP + lane);
        n += __popcll(b);
      }
      wave_lds_sync();
      RTS(12);
      const int hh = lane >> 4;
      const float Sh = s_S[hh];
      _Float16 *p16h = reinterpret_cast<_Float16 *>(s_p16);
      const _Float16 *psh = reinterpret_cast<const _Float16 *>(s_ps);
      for (int j0 = 16 * wave; j0 < n; j0 += 16 * kSwKW) {
        const int e = j0 + (lane & 15);
        const int k = e < n ? (int)lst[e] : -1;
        bool ch = false;
        if (k >= 0) {
          // p16 = f16_rne(e / sum) (attn_vk.h:188 and the fp16 operand cast, :295-296)
          const _Float16 x = (_Float16)(s_e[hh * KS + k] / Sh);
          p16h[k * kGqa + hh] = x;
          ch = __builtin_bit_cast(uint16_t, x) != __builtin_bit_cast(uint16_t, psh[k * kGqa + hh]);
        }
        const unsigned long long cm = __ballot(ch);
        unsigned m = (unsigned)((cm | (cm >> 16) | (cm >> 32) | (cm >> 48)) & 0xFFFFull);
        wave_lds_sync();
        while (m) {
          int kq[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            kq[j] = m ? __builtin_amdgcn_readlane(k, (int)__builtin_ctz(m)) : -1;
            m &= m - 1;
          }
          correct4(kq);
        }
      }
    } else {
      // p16 = f16_rne(e / sum) (attn_vk.h:188 and the fp16 operand cast, :295-296) of head h
      _Float16 *p16h = reinterpret_cast<_Float16 *>(s_p16);
      for (int i = lane; i < KS; i += 64) {
        const bool live = i < np || (i >= NP && i < NP + tn);
        p16h[i * kGqa + h] = (_Float16)(live ? s_e[h * KS + i] / S : 0.0f);
      }
      kwave_sync(&s_kctr, kc += kSwKW);
      RTS(12);
      // K wave w checks keys 64 (w + 4 i) + lane and takes its changed ones in order, 4 at a time
#pragma unroll 1
      for (int i = 0; i < 3; ++i) {
        const int k0 = 64 * (wave + 4 * i), k = k0 + lane;
        const bool live = k < np || (k >= NP && k < NP + tn);
        const int kk = min(k, KS - 1);
        const uint2 pw = s_p16[kk], qw = s_ps[kk];
        unsigned long long m = __ballot(live && (pw.x != qw.x || pw.y != qw.y));
        while (m) {
          int kq[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            kq[j] = __builtin_amdgcn_readfirstlane(m ? k0 + (int)__builtin_ctzll(m) : -1);
            m &= m - 1;
          }
          correct4(kq);
        }
      }
    }
    RTS(15);
  }
  if (kwave || SHORT) {
    // the partial, then the VALU part (tail, corrections; short plans: all of it): the 4 row
    // groups' sums by a reduce-scatter (row group r ends with head r's totals) added to it
    lds_wait(&s_pvctr, NW);
#pragma unroll
    for (int t = 0; t < 16; ++t) s_red[(wave * kGqa + (lane >> 4)) * kHd + 16 * t + (lane & 15)] = pvp[t];
    float red[VR::EPL];
#pragma unroll
    for (int i = 0; i < VR::EPL; ++i) {
      const auto s02 = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[0][i]), __float_as_uint(acc[2][i]), false, false);
      const auto s13 = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[1][i]), __float_as_uint(acc[3][i]), false, false);
      const float za = __uint_as_float(s02[0]) + __uint_as_float(s02[1]);
      const float zb = __uint_as_float(s13[0]) + __uint_as_float(s13[1]);
      const auto t = __builtin_amdgcn_permlane16_swap(__float_as_uint(za), __float_as_uint(zb), false, false);
      red[i] = __uint_as_float(t[0]) + __uint_as_float(t[1]);
    }
    float4 *dst = reinterpret_cast<float4 *>(s_red + (wave * kGqa + vkk) * kHd + 16 * vsub);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float4 x = dst[i];
      x.x += red[4 * i];
      x.y += red[4 * i + 1];
      x.z += red[4 * i + 2];
      x.w += red[4 * i + 3];
      dst[i] = x;
    }
  }
  __syncthreads();
  RTS(10);
  unsigned long long *part_g = a.part + (size_t)g * G * kGqa * kHd;
  {
    static_assert(kGqa * kHd == 2 * NT, "two partial elements per thread");
    float2 v = make_float2(0.0f, 0.0f);
#pragma unroll
    for (int wv = 0; wv < NW; ++wv) {
      const float2 x = reinterpret_cast<const float2 *>(s_red + wv * kGqa * kHd)[tid];
      v.x += x.x;
      v.y += x.y;
    }
    unsigned long long *dst = part_g + (size_t)wi * kGqa * kHd + 2 * tid;
    st_agent(dst, (unsigned long long)__float_as_uint(v.x) | ((unsigned long long)gen << 32));
    st_agent(dst + 1, (unsigned long long)__float_as_uint(v.y) | ((unsigned long long)gen << 32));
  }
  RTS(6);
  __syncthreads();                             // s_red is reused below

  // ---------------------------------------------------------------- merge + gate
  // workgroup wi sums slice wi of the group's partials in workgroup order, polling each element
  // until it carries this call's generation
  {
    constexpr int E = kGqa * kHd;
    const int sl = (E + G - 1) / G;
    const int e0 = wi * sl, ecount = max(0, min(E, e0 + sl) - e0);
    for (int c0 = 0; c0 < ecount; c0 += NT) {
      const int ne = min(NT, ecount - c0);
      const int ngrp = NT / ne;
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
        const size_t oi = (size_t)g * E + eg;
        a.out[oi] = v;
        if (a.gate) a.out_gated[oi] = v * (1.0f / (1.0f + exp_cr(-a.gate[gate_index(oi, a.gs)])));
      }
      __syncthreads();
    }
  }
  RTS(7);
  if (wi == 0 && tid == 0) st_agent(gs, gen);
  RTS(8);
}

template <bool PG>
static int stream_capacity() {
  // every instantiation launch_stream may launch (full and short plans). Per device, published
  // once computed (value + 1; 0: not yet): threads that race here compute the same value.
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  const int known = cached[dev].load(std::memory_order_acquire);
  if (known > 0) return known - 1;
  int cap = 0, per[4] = {0, 0, 0, 0};
  hipDeviceProp_t pr;
  if (hipGetDeviceProperties(&pr, dev) == hipSuccess &&
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per[0], stream_kernel<BKV_Q8_0, PG, false>, kResNT, 0) == hipSuccess &&
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per[1], stream_kernel<BKV_Q8_0, PG, true>, kResNT, 0) == hipSuccess &&
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per[2], stream_kernel<BKV_F16, PG, false>, kResNT, 0) == hipSuccess &&
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per[3], stream_kernel<BKV_F16, PG, true>, kResNT, 0) == hipSuccess)
    cap = std::min({per[0], per[1], per[2], per[3]}) * pr.multiProcessorCount;
  cached[dev].store(cap + 1, std::memory_order_release);
  return cap;
}

int stream_max_workgroups(bool paged) { return paged ? stream_capacity<true>() : stream_capacity<false>(); }

// Every wait in the kernel relies on all workgroups being resident at once. The host sizes the grid
// from the occupancy query (stream_capacity: one workgroup per CU) and launches it as an ordinary
// kernel; a grid that is not co-resident (another kernel holding CUs) makes the bounded waits give
// up and set the workspace's error word (bkv_workspace_error). BKV_COOP=1 launches cooperatively
// instead, so that the runtime refuses such a grid up front, at about 18 us more per call.
hipError_t launch_stream(const ResArgs &a, int kf, hipStream_t st) {
  const dim3 grid(a.G * a.nkv), block(kResNT);
  static const bool coop = [] { const char *e = std::getenv("BKV_COOP"); return e && e[0] == '1'; }();
  const bool shrt = a.kpw <= 2 * 64;
  const void *fn;
#define BKV_STREAM_FN(KF)                                                                              \
  (a.L.page ? (shrt ? (const void *)stream_kernel<KF, true, true> : (const void *)stream_kernel<KF, true, false>) \
            : (shrt ? (const void *)stream_kernel<KF, false, true> : (const void *)stream_kernel<KF, false, false>))
  fn = kf == BKV_F16 ? BKV_STREAM_FN(BKV_F16) : BKV_STREAM_FN(BKV_Q8_0);
#undef BKV_STREAM_FN
  ResArgs args = a;
  void *kp[] = {&args};
  if (coop) return hipLaunchCooperativeKernel(fn, grid, block, kp, 0, st);
  return hipLaunchKernel(fn, grid, block, kp, 0, st);
}

}  // namespace bkv
