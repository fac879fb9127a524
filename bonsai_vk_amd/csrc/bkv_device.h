// bkv_device.h - device building blocks shared by the split and fused decode kernels: the
// quantise-on-write append, the DPP-broadcast dot in the reference's order, the classification of
// softmax-sum steps and the exact binade arithmetic, the write-through cross-workgroup hand-off,
// and the q8_0/fp16 V accumulation.
#pragma once

#include "bkv_common.h"
#include "bkv_internal.h"

namespace bkv {

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
#ifdef BKV_EXPERIMENT_NODPP
  acc = fmaf(q, k, acc);
  return;
#endif
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
// qv[h][j] holds q16[h][16j + lane%16] in every DPP row. q: the group's first row, [4][hd] fp32.
__device__ __forceinline__ void load_q16_rows(const float *q, float (&qv)[kGqa][kHd / 16]) {
  const float *qg = q + (threadIdx.x & 15);
#pragma unroll
  for (int h = 0; h < kGqa; ++h)
#pragma unroll
    for (int j = 0; j < kHd / 16; ++j) qv[h][j] = round_f16(qg[h * kHd + 16 * j]);
#pragma unroll
  for (int h = 0; h < kGqa; ++h)
#pragma unroll
    for (int j = 0; j < kHd / 16; ++j) asm volatile("" : "+v"(qv[h][j]));
}

// Scores of one cached key against the group's 4 query heads, each one accumulation chain in
// ascending d (attn_vk.h:156-170). row: the key's LDS row - q8_0: 16 data uint4 then the scale
// uint4; fp16: 32 data uint4. The caller guarantees at least two VALU cycles between writing qv and
// this call (DPP source hazard).
template <int KF>
__device__ __forceinline__ void qk_row_dot(const uint4 *row, const float (&qv)[kGqa][kHd / 16],
                                           float (&acc)[kGqa]) {
#pragma unroll
  for (int h = 0; h < kGqa; ++h) acc[h] = 0.0f;
  if (KF == BKV_Q8_0) {
    const uint4 scl = row[16];
#pragma unroll
    for (int b = 0; b < kHd / 32; ++b) {
      const uint4 w0 = row[2 * b], w1 = row[2 * b + 1];
      float x0[16], x1[16];
      const uint32_t u0[4] = {w0.x, w0.y, w0.z, w0.w}, u1[4] = {w1.x, w1.y, w1.z, w1.w};
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        x0[i] = sbyte(u0[i >> 2], i & 3);
        x1[i] = sbyte(u1[i >> 2], i & 3);
      }
      const uint32_t sw = (b >> 1) == 0 ? scl.x : (b >> 1) == 1 ? scl.y : (b >> 1) == 2 ? scl.z : scl.w;
      const float sc = f16_to_f32((b & 1) ? (sw >> 16) : (sw & 0xFFFFu));
#pragma unroll
      for (int h = 0; h < kGqa; ++h) {
        float inner = 0.0f;
        Dot16<16>::run(inner, qv[h][2 * b], x0);
        Dot16<16>::run(inner, qv[h][2 * b + 1], x1);
        acc[h] = __fadd_rn(acc[h], __fmul_rn(sc, inner));
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < kHd / 16; ++j) {
      const uint4 w0 = row[2 * j], w1 = row[2 * j + 1];
      const uint32_t u[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
      float x[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) x[i] = f16_to_f32((u[i >> 1] >> ((i & 1) * 16)) & 0xFFFFu);
#pragma unroll
      for (int h = 0; h < kGqa; ++h) Dot16<16>::run(acc[h], qv[h][j], x);   // exact products
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


}  // namespace bkv
