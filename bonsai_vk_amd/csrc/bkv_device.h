// bkv_device.h - device building blocks shared by the split and fused decode kernels: the
// quantise-on-write append, the DPP-broadcast dot in the reference's order, the classification of
// softmax-sum steps and the exact binade arithmetic, the write-through cross-workgroup hand-off,
// and the q8_0/fp16 V accumulation.
#pragma once

#include "bkv_common.h"
#include "bkv_internal.h"

namespace bkv {

// LDS address (32-bit, LDS aperture) of a __shared__ object
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

// ------------------------------------------------------------------ append
// One 32-lane half wave writes one head row. q8_0: lanes 0..15 each own 16 consecutive elements
// (half a block); the block absmax pairs lanes 2k and 2k+1. fp16: all 32 lanes own 8 elements.
// (attn_norm_rope2.comp:167-217 for the arithmetic; the lane mapping is this kernel's own.)
template <int FMT, bool RHAZ>
__device__ __forceinline__ void append_row(const float *__restrict__ x, uint8_t *__restrict__ drow,
                                           uint8_t *__restrict__ srow, int sub) {
  if (FMT == BKV_Q8_0) {
    const int s = sub & 15;
    const float4 *xp = reinterpret_cast<const float4 *>(x + 16 * s);
    float v[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 t = xp[i];
      v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(v[i]));
    amax = fmaxf(amax, __shfl_xor(amax, 1));
    const float id = q8_iscale(amax);
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = q8_byte<RHAZ>(v[4 * i], id) | (q8_byte<RHAZ>(v[4 * i + 1], id) << 8) |
             (q8_byte<RHAZ>(v[4 * i + 2], id) << 16) | (q8_byte<RHAZ>(v[4 * i + 3], id) << 24);
    const uint32_t h = f32_to_f16_rne(q8_scale(amax));
    const uint32_t hn = __shfl_down(h, 2);       // scale of the next block (lane s+2)
    if (sub < 16) {
      *reinterpret_cast<uint4 *>(drow + 16 * s) = make_uint4(w[0], w[1], w[2], w[3]);
      if ((s & 3) == 0) *reinterpret_cast<uint32_t *>(srow + (s >> 2) * 4) = h | (hn << 16);
    }
  } else {
    const float4 *xp = reinterpret_cast<const float4 *>(x + 8 * sub);
    const float4 a = xp[0], b = xp[1];
    const uint4 o = make_uint4(f32_to_f16_rne(a.x) | (f32_to_f16_rne(a.y) << 16),
                               f32_to_f16_rne(a.z) | (f32_to_f16_rne(a.w) << 16),
                               f32_to_f16_rne(b.x) | (f32_to_f16_rne(b.y) << 16),
                               f32_to_f16_rne(b.z) | (f32_to_f16_rne(b.w) << 16));
    *reinterpret_cast<uint4 *>(drow + 16 * sub) = o;
  }
}

// one wave: lanes 0..31 write the K row, lanes 32..63 the V row of (token t, head g)
template <int KF, int VF, bool RHAZ>
__device__ __forceinline__ void append_token(const AppendArgs &a, int64_t pos, int t, int g,
                                             int lane) {
  const int64_t slot = slot_of(a.L, pos);
  const size_t xoff = ((size_t)t * a.nkv + g) * kHd;
  if (lane < 32) {
    uint8_t *dr = const_cast<uint8_t *>(a.L.kd) + (slot * a.nkv + g) * row_bytes(KF);
    uint8_t *sr = KF == BKV_Q8_0 ? const_cast<uint8_t *>(a.L.ks) + (slot * a.nkv + g) * kScaleRowBytes
                                 : nullptr;
    append_row<KF, RHAZ>(a.k + xoff, dr, sr, lane);
  } else {
    uint8_t *dr = const_cast<uint8_t *>(a.L.vd) + (slot * a.nkv + g) * row_bytes(VF);
    uint8_t *sr = VF == BKV_Q8_0 ? const_cast<uint8_t *>(a.L.vs) + (slot * a.nkv + g) * kScaleRowBytes
                                 : nullptr;
    append_row<VF, RHAZ>(a.v + xoff, dr, sr, lane - 32);
  }
}

// ------------------------------------------------------------------ QK in the reference's order
// One thread per key, the K tile staged in LDS with 128-bit coalesced loads. Each score is a single
// accumulation chain in ascending d, exactly attn_score_row (runtime_vk/attn_vk.h:156-170): fp16 K:
// acc = acc + q16_d*k_d with exact products; q8_0 K: per 32-block inner = sum of q16_d*int8_d (exact
// products), then acc = acc + f16(scale)*inner.
// The 1024 q16 operands of the group live in 64 VGPRs: register (h, j) holds q16[h][16j + lane%16]
// in every 16-lane DPP row, and each FMA takes its operand through a row_newbcast broadcast of lane
// d%16, so the shared operand costs no LDS or scalar traffic.
template <int N>
__device__ __forceinline__ void fmac_bc(float &acc, float q, float k) {
  asm("v_fmac_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf"
      : "+v"(acc)
      : "v"(q), "v"(k), "n"(N));
}
// acc = acc + q[base+i]*x[i] for i = 0..I-1, in ascending i
template <int I>
struct Dot16 {
  static __device__ __forceinline__ void run(float &acc, float qr, const float (&x)[16]) {
    Dot16<I - 1>::run(acc, qr, x);
    fmac_bc<I - 1>(acc, qr, x[I - 1]);
  }
};
template <>
struct Dot16<0> {
  static __device__ __forceinline__ void run(float &, float, const float (&)[16]) {}
};

// The group's 4 query rows rounded to fp16 (the reference's Q16 operand), laid out for fmac_bc:
// qv[h][j] holds q16[h][16j + lane%16] in every DPP row. q: the group's first row, rows qs floats
// apart (hd for [nh][hd], 2*hd for the engine's interleaved q/gate rows).
__device__ __forceinline__ void load_q16_rows(const float *q, float (&qv)[kGqa][kHd / 16], int qs = kHd) {
  const float *qg = q + (threadIdx.x & 15);
#pragma unroll
  for (int h = 0; h < kGqa; ++h)
#pragma unroll
    for (int j = 0; j < kHd / 16; ++j) qv[h][j] = round_f16(qg[(size_t)h * qs + 16 * j]);
#pragma unroll
  for (int h = 0; h < kGqa; ++h)
#pragma unroll
    for (int j = 0; j < kHd / 16; ++j) asm volatile("" : "+v"(qv[h][j]));
}

// Scores of one cached key against the group's 4 query heads, each one accumulation chain in
// ascending d (attn_vk.h:156-170). row: the key's LDS row - q8_0: 16 data uint4 then the scale
// uint4; fp16: 32 data uint4. The caller guarantees at least two VALU cycles between writing qv and
// this call (DPP source hazard).
// the 16 steps i of several independent chains interleaved, step by step (chain c: acc[c] =
// acc[c] + q[c] (broadcast of lane i of the row) * x[c][i]), so that consecutive FMAs never depend on
// each other; each chain's own order is the reference's ascending one
template <int C, int I = 0>
struct DotIl {
  static __device__ __forceinline__ void run(float (&acc)[C], const float (&q)[C], const float (&x)[C][16]) {
#pragma unroll
    for (int c = 0; c < C; ++c) fmac_bc<I>(acc[c], q[c], x[c][I]);
    DotIl<C, I + 1>::run(acc, q, x);
  }
};
template <int C>
struct DotIl<C, 16> {
  static __device__ __forceinline__ void run(float (&)[C], const float (&)[C], const float (&)[C][16]) {}
};

// Scores of one cached fp16 K row against the group's 4 query heads, each one accumulation chain
// in ascending d (attn_vk.h:156-170): acc = acc + q16_d * k_d, every product exact. row: the key's
// 32 data uint4 in LDS. The chains of the 4 heads are interleaved. The caller guarantees at least
// two VALU cycles between writing qv and this call (DPP source hazard). (q8_0 K: bkv_q8dot.h.)
template <int KF>
__device__ __forceinline__ void qk_row_dot(const uint4 *row, const float (&qv)[kGqa][kHd / 16],
                                           float (&acc)[kGqa]) {
  static_assert(KF == BKV_F16, "q8_0 K scores: bkv_q8dot.h");
#pragma unroll
  for (int h = 0; h < kGqa; ++h) acc[h] = 0.0f;
  {
#pragma unroll
    for (int j = 0; j < kHd / 16; ++j) {
      const uint4 w0 = row[2 * j], w1 = row[2 * j + 1];
      const uint32_t u[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
      float x[kGqa][16], q[kGqa];
#pragma unroll
      for (int i = 0; i < 16; ++i) x[0][i] = f16_to_f32((u[i >> 1] >> ((i & 1) * 16)) & 0xFFFFu);
#pragma unroll
      for (int h = 0; h < kGqa; ++h) {
        q[h] = qv[h][j];
        if (h > 0)
#pragma unroll
          for (int i = 0; i < 16; ++i) x[h][i] = x[0][i];
      }
      DotIl<kGqa>::run(acc, q, x);                  // exact products
    }
  }
}

// ------------------------------------------------------------------ probabilities' numerators and the exact serial sum
// e_j = exp(s_j*scale - max) (attn_vk.h:182-186), then the reference's serial fp32 sum
// sum = sum + e_j over ascending j, reproduced exactly. The running sum is non-decreasing, so inside
// one binade [2^B, 2^(B+1)) every step adds e_j rounded to a multiple of the binade's ulp 2^(B-23):
// an integer. Each chunk places its keys on the running sum with an approximate fp64 prefix (built
// from the QK partition statistics, no cross-workgroup wait), turns every step that is safely inside
// a binade into an exact integer increment, and records the rest - binade crossings, steps within a
// relative 2^-14 of a binade edge (the fp64
// prefix stays within ~1.2e-5 of the serial sum at 64K keys), exact ties, tiny sums - as specials. The last workgroup of each
// head walks the chunk records in order, adding increments exactly and specials in fp32, and checks
// every binade assumption; if one fails it recomputes the serial loop itself.
constexpr double kMargin = 1.0 / 16384.0;
constexpr int kWalkBatch = 32;

__device__ __forceinline__ void classify(double abefore, double aafter, float e, bool &special,
                                         int &bin, long long &inc) {
  special = true;
  bin = kNoBinade;
  inc = 0;
  if (!(aafter >= 0x1p-17) || aafter >= 0x1p22) return;
  const int B = ilogb(aafter);
  const double lo = ldexp(1.0, B);
  if (aafter > 2.0 * lo * (1.0 - kMargin) || abefore < lo * (1.0 + kMargin)) return;
  const double t = ldexp((double)e, 23 - B);
  const double fl = floor(t);
  if (t - fl == 0.5) return;
  special = false;
  bin = B;
  inc = (long long)rint(t) << (B + 17);
}

// Advance a running sum s that lies in binade B by du units of 2^-40 (a multiple of that binade's
// ulp 2^(B-23)), in integer arithmetic on the float's significand. False when s is not in binade B,
// du is not a whole number of ulps, or the result leaves the binade - an assumption of the
// classification failed, and the caller falls back to the serial loop.
__device__ __forceinline__ bool advance(float &s, int B, long long du) {
  const uint32_t bits = __float_as_uint(s);
  if (B < -17 || B > 22 || (int)(bits >> 23) != B + 127) return false;
  const int sh = B + 17;
  if (du < 0 || (du & ((1ll << sh) - 1)) != 0) return false;
  const long long m = (long long)((bits & 0x7FFFFFu) | 0x800000u) + (du >> sh);
  if (m >= (1ll << 24)) return false;
  s = __uint_as_float(((uint32_t)(B + 127) << 23) | ((uint32_t)m & 0x7FFFFFu));
  return true;
}

// Cross-workgroup hand-off inside the probability kernel without L2-wide fences: everything the
// walker reads (chunk records, specials, e) is written with agent-scope relaxed atomic stores, which
// write through the XCD's L2, and read with agent-scope atomic loads, which bypass it; each producer
// waits for its stores to complete (s_waitcnt) before it counts itself in.
template <typename T>
__device__ __forceinline__ void st_agent(T *p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ T ld_agent(const T *p) {
  return __hip_atomic_load(const_cast<T *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_rec(ChunkRec *p, const ChunkRec &r) {
  st_agent(&p->tot, r.tot);
  st_agent(&p->nsp, r.nsp);
  st_agent(&p->blast, r.blast);
}
__device__ __forceinline__ ChunkRec ld_rec(const ChunkRec *p) {
  ChunkRec r;
  r.tot = ld_agent(&p->tot);
  r.nsp = ld_agent(&p->nsp);
  r.blast = ld_agent(&p->blast);
  return r;
}
__device__ __forceinline__ void st_spec(Special *p, const Special &x) {
  st_agent(&p->ipre, x.ipre);
  st_agent(&p->e, x.e);
  st_agent(&p->meta, x.meta);
}
__device__ __forceinline__ Special ld_spec(const Special *p) {
  Special x;
  x.ipre = ld_agent(&p->ipre);
  x.e = ld_agent(&p->e);
  x.meta = ld_agent(&p->meta);
  return x;
}

__device__ __forceinline__ void st_f2(float2 *p, float2 v) {
  st_agent(reinterpret_cast<unsigned long long *>(p),
           (unsigned long long)__float_as_uint(v.x) | ((unsigned long long)__float_as_uint(v.y) << 32));
}
__device__ __forceinline__ float2 ld_f2(const float2 *p) {
  const unsigned long long u = ld_agent(reinterpret_cast<const unsigned long long *>(p));
  return make_float2(__uint_as_float((uint32_t)u), __uint_as_float((uint32_t)(u >> 32)));
}

// ------------------------------------------------------------------ row staging into LDS
// Rows [0, n) of one KV head's array (COLS x 16 B per row, row_bytes_ apart per head slot) at
// positions j0.. into tile[row * STRIDE + col]; rows [n, ROWS) are zero-filled. Every load of a batch
// is issued before the first LDS store, and out-of-range rows read position j0 (or 0) so the batch
// is straight-line code: the batch costs one memory latency, not one per load.
template <int NT, int ROWS, int COLS, int STRIDE, int BATCH = 8>
__device__ __forceinline__ void stage_rows(uint4 *tile, const uint8_t *base, int row_bytes_, const LayerView &L,
                                           int nkv, int g, int64_t j0, int n) {
  static_assert((ROWS * COLS) % NT == 0, "whole rows per pass");
  constexpr int PER = ROWS * COLS / NT;
  constexpr int B = PER < BATCH ? PER : BATCH;
  static_assert(PER % B == 0, "whole batches");
#pragma unroll
  for (int b = 0; b < PER; b += B) {
    uint4 t[B];
#pragma unroll
    for (int u = 0; u < B; ++u) {
      const int i = threadIdx.x + (b + u) * NT, row = i / COLS, col = i % COLS;
      const int64_t pos = n > 0 ? j0 + min(row, n - 1) : 0;
      const uint4 v = *reinterpret_cast<const uint4 *>(base + (slot_of(L, pos) * nkv + g) * (int64_t)row_bytes_ + col * 16);
      t[u] = row < n ? v : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int u = 0; u < B; ++u) {
      const int i = threadIdx.x + (b + u) * NT, row = i / COLS, col = i % COLS;
      tile[row * STRIDE + col] = t[u];
    }
  }
}

// ------------------------------------------------------------------ PV over the fp16 probabilities
template <int VF>
struct KRow {
  static constexpr int LPR = VF == BKV_Q8_0 ? 16 : 32;   // lanes per head row
  static constexpr int EPL = kHd / LPR;                  // elements per lane (16 or 8)
  static constexpr int KPW = kWave / LPR;                // rows per wave per step (4 or 2)
};

// p16_j = f16_rne(e_j / sum) (attn_vk.h:188 and the fp16 operand cast, :295-296); out = sum_j p16_j*V_j.
// 16 lanes per q8_0 V row (32 per fp16 row) with 128-bit loads; the 4 heads of the group share each
// V tile read. Accumulation order is free here (within the tolerance).
template <int VF>
__device__ __forceinline__ void v_accum(const uint4 w, float vsc, const float (&p)[kGqa],
                                        float (&acc)[kGqa][KRow<VF>::EPL]) {
  const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
  if (VF == BKV_Q8_0) {
    float wgt[kGqa];
#pragma unroll
    for (int h = 0; h < kGqa; ++h) wgt[h] = p[h] * vsc;      // exact: two 11-bit significands
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float x = sbyte(ww[i >> 2], i & 3);
#pragma unroll
      for (int h = 0; h < kGqa; ++h) acc[h][i] = fmaf(wgt[h], x, acc[h][i]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float x = f16_to_f32((ww[i >> 1] >> ((i & 1) * 16)) & 0xFFFFu);
#pragma unroll
      for (int h = 0; h < kGqa; ++h) acc[h][i] = fmaf(p[h], x, acc[h][i]);
    }
  }
}


// ---------------------------------------------------------------- the walk (one wave, 1..NHW heads)
// Records rec[c] / specials spec[c][..] of the group's workgroups in key order, each covering kpw
// keys. The fields of every special (global key index, global increment prefix, binade of the step
// before it, the whole ulps of the segment before it) are resolved in parallel across the wave into
// LDS. The serial chain then carries only the running sum: per special, the bits of the sum advance
// by the segment's ulps (an integer add, valid while the sum stays in the recorded binade) and the
// special's e is added in fp32. The binade conditions are checked afterwards, in parallel, on the
// sums recorded before each step. A wave walks its heads' chains interleaved.
// WG: workgroups per group the scratch holds; CAP: specials per head (more: serial fallback)
template <int WG, int CAP>
struct WalkScratchT {
  static constexpr int kWg = WG, kCap = CAP;
  long long wg_ib[WG];
  int wg_off[WG + 1], wg_bp[WG];
  long long si[CAP];
  int sk[CAP];
  float se[CAP];
  int sck[CAP];                    // binade exponent field the step must start and end in, -1: no advance
  int sdu[CAP];                    // ulps the sum advances by before the special (0: none)
};

#ifdef BKV_EXPERIMENT_TS
#define WTS(q, i) do { if (tsp[q] && (threadIdx.x & 63) == 0) tsp[q][i] = (unsigned)wall_clock64(); } while (0)
#else
#define WTS(q, i) do { } while (0)
#endif

template <int NHW, typename WS>
__device__ void walk_heads(const ChunkRec *const *rec, const Special *const *spec, int nhere, int gg,
                           int64_t kpw, int64_t nfill, WS *const *ws, float *s_out, bool *good_out,
                           unsigned *const *tsp) {
  const int lane = threadIdx.x & 63;
  constexpr int kWalkWg = WS::kWg, kWalkCap = WS::kCap;
  constexpr int kRounds = (kWalkWg + 63) / 64;
  int T[NHW], blast_last[NHW];
  long long itot[NHW];
  bool ok[NHW];
  // 1. every record of every head in one round trip, then the prefix scans
  ChunkRec r[NHW][kRounds];
#pragma unroll
  for (int q = 0; q < NHW; ++q)
#pragma unroll
    for (int rr = 0; rr < kRounds; ++rr) {
      const int c = rr * 64 + lane;
      r[q][rr].tot = 0; r[q][rr].nsp = 0; r[q][rr].blast = kNoBinade;
      if (q < nhere && c < gg) r[q][rr] = ld_rec(&rec[q][c]);
    }
#pragma unroll
  for (int q = 0; q < NHW; ++q) {
    ok[q] = q < nhere && gg <= kWalkWg;
    long long ibase = 0;
    int obase = 0, blast_prev = kNoBinade;
    bool over = false;
    WS &w = *ws[q];
#pragma unroll
    for (int rr = 0; rr < kRounds; ++rr) {
      if (rr * 64 < gg) {
        const int c = rr * 64 + lane;
        const ChunkRec x = r[q][rr];
        over |= x.nsp > kMaxSpecial;
        const int cnt = min(x.nsp, kMaxSpecial);
        const long long incl = wave_incl_scan<long long>(x.tot, lane);
        const int oincl = wave_incl_scan<int>(cnt, lane);
        int bp = __shfl_up(x.blast, 1);
        if (lane == 0) bp = blast_prev;
        if (q < nhere && c < gg) {
          w.wg_ib[c] = ibase + incl - x.tot;
          w.wg_off[c] = obase + oincl - cnt;
          w.wg_bp[c] = bp;
        }
        const int nb = min(64, gg - rr * 64);
        ibase += __shfl(incl, 63);
        obase += __shfl(oincl, 63);
        blast_prev = __shfl(x.blast, nb - 1);
      }
    }
    if (q < nhere && lane == 0) w.wg_off[gg] = obase;
    ok[q] = ok[q] && !__any(over) && obase <= kWalkCap;
    T[q] = ok[q] ? obase : 0;
    itot[q] = ibase;
    blast_last[q] = blast_prev;
    WTS(q, 0);
  }
  __builtin_amdgcn_wave_barrier();
  // 2. the specials, resolved to global key index, increment prefix and starting binade (the loads
  // of all heads are issued before any is used)
  {
    int Tm = 0;
#pragma unroll
    for (int q = 0; q < NHW; ++q) Tm = max(Tm, T[q]);
    for (int o = lane; o < Tm; o += 64) {
      int lo[NHW];
      Special x[NHW];
#pragma unroll
      for (int q = 0; q < NHW; ++q) {
        const WS &w = *ws[q];
        int l = 0, hi = gg - 1;
        if (o < T[q]) {
          while (l < hi) {
            const int mid = (l + hi + 1) >> 1;
            if (w.wg_off[mid] <= o) l = mid; else hi = mid - 1;
          }
        }
        lo[q] = l;
      }
#pragma unroll
      for (int q = 0; q < NHW; ++q)
        if (o < T[q]) x[q] = ld_spec(&spec[q][(size_t)lo[q] * kMaxSpecial + (o - ws[q]->wg_off[lo[q]])]);
#pragma unroll
      for (int q = 0; q < NHW; ++q) {
        if (o < T[q]) {
          WS &w = *ws[q];
          const int bf = (x[q].meta >> 16) & 0xFF;
          w.si[o] = w.wg_ib[lo[q]] + x[q].ipre;
          w.sk[o] = (int)(lo[q] * kpw + (x[q].meta & 0xFFFF));
          w.se[o] = x[q].e;
          w.sck[o] = bf == 255 ? w.wg_bp[lo[q]] : (bf == 0 ? kNoBinade : bf - 128);   // binade B for now
        }
      }
    }
  }
  __builtin_amdgcn_wave_barrier();
  // 3. per special: the ulps of the segment before it in its binade
#pragma unroll
  for (int q = 0; q < NHW; ++q) {
    WS &w = *ws[q];
    WTS(q, 1);
    bool bad = false;
    for (int o = lane; o < T[q]; o += 64) {
      const long long gap = (long long)w.sk[o] - (o > 0 ? w.sk[o - 1] : -1);
      const long long di = w.si[o] - (o > 0 ? w.si[o - 1] : 0);
      int du = 0, ck = -1;
      if (gap > 1) {
        const int B = w.sck[o];
        if (B < -17 || B > 22 || di < 0 || (di & ((1ll << (B + 17)) - 1)) != 0 || (di >> (B + 17)) >= (1ll << 24)) {
          bad = true;
        } else {
          du = (int)(di >> (B + 17));
          ck = B + 127;
        }
      } else if (di != 0) {
        bad = true;
      }
      w.sdu[o] = du;
      w.sck[o] = ck;
    }
    ok[q] = ok[q] && !__any(bad);
    if (!ok[q]) T[q] = 0;
  }
  __builtin_amdgcn_wave_barrier();
  // 4. the chains, 16 steps per unrolled block; entries past T are du 0, e 0 (no change)
  float s[NHW];
  bool bad[NHW];
  int Tm = 0;
#pragma unroll
  for (int q = 0; q < NHW; ++q) { s[q] = 0.0f; bad[q] = false; Tm = max(Tm, T[q]); WTS(q, 2); }
  for (int base = 0; base < Tm; base += 64) {
    const int o = base + lane;
    int du_l[NHW], ck_l[NHW];
    float e_l[NHW];
    uint32_t pre[NHW];
#pragma unroll
    for (int q = 0; q < NHW; ++q) {
      const bool in = o < T[q];
      du_l[q] = in ? ws[q]->sdu[o] : 0;
      ck_l[q] = in ? ws[q]->sck[o] : -1;
      e_l[q] = in ? ws[q]->se[o] : 0.0f;
      pre[q] = 0u;
    }
    const int cnt = min(64, Tm - base);
    for (int j0 = 0; j0 < cnt; j0 += 16) {
#pragma unroll
      for (int jj = 0; jj < 16; ++jj) {
        const int j = j0 + jj;
#pragma unroll
        for (int q = 0; q < NHW; ++q) {
          const uint32_t du = (uint32_t)__builtin_amdgcn_readlane(du_l[q], j);
          const float ev = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, e_l[q]), j));
          const uint32_t bits = __float_as_uint(s[q]);
          pre[q] = lane == j ? bits : pre[q];
          s[q] = __fadd_rn(__uint_as_float(bits + du), ev);
        }
      }
    }
    // the binade conditions of this block's steps: start in binade ck, no carry out of it
#pragma unroll
    for (int q = 0; q < NHW; ++q)
      if (ck_l[q] >= 0)
        bad[q] |= (int)(pre[q] >> 23) != ck_l[q] || (int)((pre[q] + (uint32_t)du_l[q]) >> 23) != ck_l[q];
  }
#pragma unroll
  for (int q = 0; q < NHW; ++q) {
    WTS(q, 3);
    bool good = ok[q] && !__any(bad[q]);
    // the trailing segment after the last special
    const long long k_last = T[q] > 0 ? ws[q]->sk[T[q] - 1] : -1, i_last = T[q] > 0 ? ws[q]->si[T[q] - 1] : 0;
    float sq = s[q];
    if (good && nfill - 1 - k_last > 0) good = advance(sq, blast_last[q], itot[q] - i_last);
    s_out[q] = sq;
    good_out[q] = good;
#ifdef BKV_EXPERIMENT_TS
    if (tsp[q] && lane == 0) tsp[q][4] = T[q];
#endif
  }
}


}  // namespace bkv
