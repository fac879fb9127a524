// bkv_prefill.hip - chunked prefill attention on the gfx950 matrix cores (bkv_attn_prefill_chunk).
//
// Query i of the chunk (position pos0 + i) attends causally to keys 0 .. pos0 + i, exactly the row
// bkv_attn_decode computes with nfill = pos0 + i + 1 (the reference's prefill is that decode row
// repeated, runtime_vk/attn_vk.h:261-311 per token; bonsai_forward.h:2752-2759). Rows are (query,
// head) pairs; the 4 query heads of one KV head share every K/V tile read.
//
// Work split: a workgroup owns 16 queries x 4 heads = 64 rows of one KV group and one contiguous
// range of 64-key tiles (a "split"); splits exist only to fill the chip when the chunk is short.
// Two passes over the same tiles:
//   stats  S^T = K . Q^T per tile on MFMA, masked causally; online (max, sum exp) per row,
//          written per split;
//   pv     the splits' statistics give the row max M and sum S; scores recomputed bit-identically,
//          p16 = f16(exp(s*scale - M) / S) (the reference rounds the normalised probability to
//          fp16 before PV, attn_vk.h:184-189), then out^T = V^T . P^T on MFMA;
//   merge  (more than one split) the normalised partial outputs are summed in split order, and the
//          gate applied.
//
// Exactness of the matrix-core operands: Q is rounded to fp16 as the reference does; a q8_0 K or V
// element d*b (fp16 scale d, int8 b) has up to 18 significant bits, so it enters the MFMA as the
// exact fp16 pair hi = f16(d*b), lo = d*b - hi (the rounding error of an fp16 product is an fp16
// number, computed by one fp16 fma), and fp16 x fp16 products are exact in the fp32 accumulator.
// What differs from the serial reference is only the order of the fp32 sums (dot products, the
// softmax sum and PV), hence a tolerance rather than bit-exact parity for prefill.

#include "bkv_device.h"
#include "bkv_exp.h"
#include "bkv_internal.h"
#include "bkv_pv8.h"

namespace bkv {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kPfNT = 256;      // 4 waves
constexpr int kPfRS = 144;      // LDS row stride in bytes of the P and V^T tiles (64 fp16 + pad)

__device__ __forceinline__ f4 mfma16(h8 a, h8 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ h2 as_h2(uint32_t w) { return __builtin_bit_cast(h2, w); }
__device__ __forceinline__ uint32_t as_u(h2 v) { return __builtin_bit_cast(uint32_t, v); }

// two signed bytes of w (already biased by 0x80 per byte), selected by SEL, as an exact fp16 pair:
// 0x64XX is the fp16 number 1024 + XX, so subtracting 1152 leaves the signed byte value.
template <uint32_t SEL>
__device__ __forceinline__ h2 bytes_h2(uint32_t wb) {
  const h2 x = as_h2(__builtin_amdgcn_perm(0x64646464u, wb, SEL));
  return x - h2{(_Float16)1152.0f, (_Float16)1152.0f};
}

// e / s correctly rounded to fp32, from rs = fp32(1/s) correctly rounded, without a division:
// q0 = e*rs is within 1.5 ulps of e/s; one correction q1 = q0 + (e - s*q0)*rs (the remainder exact
// by fma) brings it within one ulp, and a second is then the correctly rounded quotient (Markstein's
// theorem: y within half an ulp of 1/s, q within one ulp of e/s, r = e - s*q exact => RN(q + r*y)
// = RN(e/s)). Valid for 0 <= e <= s, s >= 1 (a softmax sum includes the maximum's e = 1): the
// remainders stay normal while the quotient is above 2^-60, and below that the quotient rounds to
// an fp16 zero whatever its last bits.
__device__ __forceinline__ float div_by_sum(float e, float s, float rs) {
  const float q0 = e * rs;
  const float q1 = __builtin_fmaf(__builtin_fmaf(-s, q0, e), rs, q0);
  float q2 = __builtin_fmaf(__builtin_fmaf(-s, q1, e), rs, q1);
  // the fp32 result itself: a conversion to fp16 of the fma would otherwise be folded into one
  // mixed-precision fma rounding once, straight to fp16 (a different result at fp16 ties)
  asm volatile("" : "+v"(q2));
  return q2;
}

// exact fp16 split of s*b: hi = f16(s*b) (rounded fp16 product), lo = the product's rounding error
__device__ __forceinline__ void split_prod(h2 b, h2 s, h2 &hi, h2 &lo) {
  hi = b * s;
  lo = __builtin_elementwise_fma(b, s, -hi);
}

// exp(x) for x <= 0 (or -inf) in fp32 to about 2 ulp: 2^(x log2 e) on the hardware exp2 with the
// rounding error of the product x*log2(e) carried as a first-order correction
__device__ __forceinline__ float fexp(float x) {
  x = fmaxf(x, -150.0f);
  constexpr float L = 0x1.715476p0f;          // log2(e) rounded to float
  constexpr float Llo = 1.925963033e-8f;      // log2(e) - L
  const float t = x * L;
  const float err = fmaf(x, L, -t) + x * Llo;
  const float y = __builtin_amdgcn_exp2f(t);
  return fmaf(y, err * 0.6931471806f, y);
}

struct PfGeo {
  int g, s, qb, q0, nqv, t0, t1;
  uint32_t kend;
};

// blockIdx -> (KV group, split, query block). Workgroups are dealt to the 8 XCDs round-robin; when
// the grid is a multiple of 8 the index is permuted so that one XCD runs consecutive query blocks
// of one (group, split), which read the same K/V tiles through that XCD's L2.
__device__ __forceinline__ PfGeo pf_geo(const PrefillArgs &a) {
  const int n = gridDim.x, b = blockIdx.x;
  const int i = (n & 7) == 0 ? (b & 7) * (n >> 3) + (b >> 3) : b;
  PfGeo p;
  p.qb = i % a.nqb;
  p.s = (i / a.nqb) % a.nsplit;
  p.g = i / (a.nqb * a.nsplit);
  p.q0 = p.qb * kPfQ;
  p.nqv = min(kPfQ, a.n_q - p.q0);
  p.kend = a.pos0 + (uint32_t)(p.q0 + p.nqv);
  const int nt = (int)((p.kend + kPfTile - 1) / kPfTile);
  p.t0 = (int)((int64_t)p.s * nt / a.nsplit);
  p.t1 = (int)((int64_t)(p.s + 1) * nt / a.nsplit);
  return p;
}

// Q fragments (MFMA B operand of S^T = K.Q^T): row-tile nt, k-step s, lane l holds Q[row 16nt +
// l%16][dims 64(l/16) + 8s .. + 8] in fp16 (rounded to nearest even)
__device__ __forceinline__ void load_q(const PrefillArgs &a, const PfGeo &p, int lane, h8 (&qf)[4][8]) {
  const int lr = lane & 15, lq = lane >> 4;
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    const int r = 16 * nt + lr;
    const int qi = min(p.q0 + (r >> 2), a.n_q - 1);
    const float *qp = a.q + ((size_t)qi * a.nh + (size_t)(p.g * kGqa + (r & 3))) * a.qs + 64 * lq;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const float4 x0 = *reinterpret_cast<const float4 *>(qp + 8 * s);
      const float4 x1 = *reinterpret_cast<const float4 *>(qp + 8 * s + 4);
      h8 h;
      h[0] = (_Float16)x0.x; h[1] = (_Float16)x0.y; h[2] = (_Float16)x0.z; h[3] = (_Float16)x0.w;
      h[4] = (_Float16)x1.x; h[5] = (_Float16)x1.y; h[6] = (_Float16)x1.z; h[7] = (_Float16)x1.w;
      qf[nt][s] = h;
    }
  }
}

// the raw K bytes one lane feeds to the MFMA for a tile: key kb + l%16, dims 64(l/16) .. + 64
template <int KF>
struct KRaw {
  uint4 d[KF ? 4 : 8];
  uint32_t sc;                  // q8_0: the scales of blocks 2(l/16), 2(l/16)+1
};

template <int KF, bool PG>
__device__ __forceinline__ void load_k(const LayerView &L, int nkv, int g, uint32_t key, int lq,
                                       KRaw<KF> &r) {
  const int64_t sl = slot_t<PG>(L, key);
  constexpr int RB = row_bytes(KF ? BKV_Q8_0 : BKV_F16);
  const uint4 *src = reinterpret_cast<const uint4 *>(L.kd + (sl * nkv + g) * RB + (RB / 4) * lq);
#pragma unroll
  for (int c = 0; c < (KF ? 4 : 8); ++c) r.d[c] = src[c];
  if constexpr (KF)
    r.sc = *reinterpret_cast<const uint32_t *>(L.ks + (sl * nkv + g) * kScaleRowBytes + 4 * lq);
}

// S^T tile (16 keys of this wave x 64 rows): acc[nt][i] = dot(K[key 4(l/16)+i], Q[row 16nt + l%16])
template <int KF>
__device__ __forceinline__ void qk_tile(const KRaw<KF> &r, const h8 (&qf)[4][8], f4 (&acc)[4]) {
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) acc[nt] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    if constexpr (KF) {
      const uint32_t w0 = r.d[s >> 1][(s & 1) * 2] ^ 0x80808080u;
      const uint32_t w1 = r.d[s >> 1][(s & 1) * 2 + 1] ^ 0x80808080u;
      const uint32_t sw = s < 4 ? (r.sc & 0xFFFFu) * 0x10001u : (r.sc >> 16) * 0x10001u;
      const h2 sc = as_h2(sw);
      h2 hi[4], lo[4];
      split_prod(bytes_h2<0x04010400u>(w0), sc, hi[0], lo[0]);
      split_prod(bytes_h2<0x04030402u>(w0), sc, hi[1], lo[1]);
      split_prod(bytes_h2<0x04010400u>(w1), sc, hi[2], lo[2]);
      split_prod(bytes_h2<0x04030402u>(w1), sc, hi[3], lo[3]);
      const h8 ah = {hi[0][0], hi[0][1], hi[1][0], hi[1][1], hi[2][0], hi[2][1], hi[3][0], hi[3][1]};
      const h8 al = {lo[0][0], lo[0][1], lo[1][0], lo[1][1], lo[2][0], lo[2][1], lo[3][0], lo[3][1]};
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        acc[nt] = mfma16(ah, qf[nt][s], acc[nt]);
        acc[nt] = mfma16(al, qf[nt][s], acc[nt]);
      }
    } else {
      const h8 ak = __builtin_bit_cast(h8, r.d[s]);
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) acc[nt] = mfma16(ak, qf[nt][s], acc[nt]);
    }
  }
}

// causal limit of the lane's rows: the last key row 16nt + l%16 may see (-1: no such query)
__device__ __forceinline__ void row_limits(const PrefillArgs &a, const PfGeo &p, int lr, int (&lim)[4]) {
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    const int r = 16 * nt + lr;
    lim[nt] = (r >> 2) < p.nqv ? (int)(a.pos0 + (uint32_t)(p.q0 + (r >> 2))) : -1;
  }
}

// ------------------------------------------------------------------ pass 1: row statistics
template <int KF, bool PG>
__global__ __launch_bounds__(kPfNT) void prefill_stats_kernel(PrefillArgs a) {
  const PfGeo p = pf_geo(a);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, lr = lane & 15, lq = lane >> 4;
  __shared__ float2 s_st[4][4][64];

  h8 qf[4][8];
  load_q(a, p, lane, qf);
  int lim[4];
  row_limits(a, p, lr, lim);
  float m[4], l[4];
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) { m[nt] = -3.0e38f; l[nt] = 0.f; }

  const uint32_t klast = p.kend - 1;
  KRaw<KF> cur, nxt;
  if (p.t0 < p.t1) load_k<KF, PG>(a.L, a.nkv, p.g, min((uint32_t)(p.t0 * kPfTile + 16 * w + lr), klast), lq, cur);
  for (int t = p.t0; t < p.t1; ++t) {
    const int tn = min(t + 1, p.t1 - 1);
    load_k<KF, PG>(a.L, a.nkv, p.g, min((uint32_t)(tn * kPfTile + 16 * w + lr), klast), lq, nxt);
    f4 acc[4];
    qk_tile<KF>(cur, qf, acc);
    const int kb = t * kPfTile + 16 * w + 4 * lq;
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      float v[4], mx = -INFINITY;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[i] = kb + i <= lim[nt] ? acc[nt][i] * a.scale : -INFINITY;
        mx = fmaxf(mx, v[i]);
      }
      const float mn = fmaxf(m[nt], mx);
      float sum = l[nt] * fexp(m[nt] - mn);
#pragma unroll
      for (int i = 0; i < 4; ++i) sum += fexp(v[i] - mn);
      m[nt] = mn;
      l[nt] = sum;
    }
    cur = nxt;
  }
  // the four lanes holding one row (l%16 equal), then the four waves
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) s_st[w][lq][16 * nt + lr] = make_float2(m[nt], l[nt]);
  __syncthreads();
  if (tid < 64) {
    float mm = -3.0e38f;
#pragma unroll
    for (int k = 0; k < 16; ++k) mm = fmaxf(mm, s_st[k >> 2][k & 3][tid].x);
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const float2 e = s_st[k >> 2][k & 3][tid];
      ss += e.y * fexp(e.x - mm);
    }
    if ((tid >> 2) < p.nqv) {
      const size_t row = (size_t)(p.q0 + (tid >> 2)) * a.nh + p.g * kGqa + (tid & 3);
      a.stats[(size_t)p.s * a.n_q * a.nh + row] = make_float2(mm, ss);
    }
  }
}

// ------------------------------------------------------------------ pass 2: probabilities and PV
template <int VF>
struct VRaw {
  uint4 a[VF ? 2 : 4], b[VF ? 2 : 4];   // keys 2kp, 2kp+1: dims 64w + 32h .. + 32
  uint32_t sa, sb;                       // q8_0: their scales (fp16 bits in the low half)
};

template <int VF, bool PG>
__device__ __forceinline__ void load_v(const LayerView &L, int nkv, int g, uint32_t ka, uint32_t kb,
                                       int w, int h, VRaw<VF> &r) {
  const int64_t sa = slot_t<PG>(L, ka), sb = slot_t<PG>(L, kb);
  constexpr int RB = row_bytes(VF ? BKV_Q8_0 : BKV_F16);
  constexpr int DB = VF ? 1 : 2;   // bytes per element
  const int off = (64 * w + 32 * h) * DB;
  const uint4 *pa = reinterpret_cast<const uint4 *>(L.vd + (sa * nkv + g) * RB + off);
  const uint4 *pb = reinterpret_cast<const uint4 *>(L.vd + (sb * nkv + g) * RB + off);
#pragma unroll
  for (int c = 0; c < (VF ? 2 : 4); ++c) { r.a[c] = pa[c]; r.b[c] = pb[c]; }
  if constexpr (VF) {
    const int blk = 2 * w + h;
    r.sa = *reinterpret_cast<const uint16_t *>(L.vs + (sa * nkv + g) * kScaleRowBytes + 2 * blk);
    r.sb = *reinterpret_cast<const uint16_t *>(L.vs + (sb * nkv + g) * kScaleRowBytes + 2 * blk);
  }
}

// V^T into the wave's LDS tiles: vt_hi/vt_lo[dim 0..63][key 0..63] (row stride kPfRS), the lane
// writing keys 2kp, 2kp+1 of dims 32h .. + 32
template <int VF>
__device__ __forceinline__ void put_vt(const VRaw<VF> &r, int kp, int h, char *vt_hi, char *vt_lo) {
  char *bh = vt_hi + (32 * h) * kPfRS + 4 * kp;
  if constexpr (VF) {
    char *bl = vt_lo + (32 * h) * kPfRS + 4 * kp;
    const h2 sc = as_h2((r.sa & 0xFFFFu) | (r.sb << 16));
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const uint32_t wa = r.a[c >> 2][c & 3] ^ 0x80808080u, wb = r.b[c >> 2][c & 3] ^ 0x80808080u;
      const uint32_t t0 = __builtin_amdgcn_perm(wb, wa, 0x05010400u);   // a0 b0 a1 b1
      const uint32_t t1 = __builtin_amdgcn_perm(wb, wa, 0x07030602u);   // a2 b2 a3 b3
      const h2 x[4] = {bytes_h2<0x04010400u>(t0), bytes_h2<0x04030402u>(t0),
                       bytes_h2<0x04010400u>(t1), bytes_h2<0x04030402u>(t1)};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        h2 hi, lo;
        split_prod(x[i], sc, hi, lo);
        *reinterpret_cast<uint32_t *>(bh + (4 * c + i) * kPfRS) = as_u(hi);
        *reinterpret_cast<uint32_t *>(bl + (4 * c + i) * kPfRS) = as_u(lo);
      }
    }
  } else {
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      const uint32_t wa = r.a[c >> 2][c & 3], wb = r.b[c >> 2][c & 3];
      *reinterpret_cast<uint32_t *>(bh + (2 * c) * kPfRS) = __builtin_amdgcn_perm(wb, wa, 0x05040100u);
      *reinterpret_cast<uint32_t *>(bh + (2 * c + 1) * kPfRS) = __builtin_amdgcn_perm(wb, wa, 0x07060302u);
    }
  }
}

template <int KF, int VF, bool PG>
__global__ __launch_bounds__(kPfNT) void prefill_pv_kernel(PrefillArgs a) {
  const PfGeo p = pf_geo(a);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, lr = lane & 15, lq = lane >> 4;
  const int kp = lane & 31, vh = lane >> 5;
  __shared__ __attribute__((aligned(16))) char s_p[2][64 * kPfRS];
  __shared__ __attribute__((aligned(16))) char s_vt[4][VF ? 2 : 1][64 * kPfRS];
  __shared__ float2 s_ms[64];

  // row max and 1/sum from the splits' statistics
  if (tid < 64) {
    float mm = -3.0e38f, ss = 0.f;
    if ((tid >> 2) < p.nqv) {
      const size_t row = (size_t)(p.q0 + (tid >> 2)) * a.nh + p.g * kGqa + (tid & 3);
      const size_t rs = (size_t)a.n_q * a.nh;
      for (int s = 0; s < a.nsplit; ++s) mm = fmaxf(mm, a.stats[s * rs + row].x);
      for (int s = 0; s < a.nsplit; ++s) {
        const float2 e = a.stats[s * rs + row];
        ss += e.y * fexp(e.x - mm);
      }
    }
    s_ms[tid] = make_float2(mm, ss > 0.f ? 1.0f / ss : 0.f);
  }
  h8 qf[4][8];
  load_q(a, p, lane, qf);
  int lim[4];
  row_limits(a, p, lr, lim);
  __syncthreads();
  float M[4], iS[4];
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    const float2 e = s_ms[16 * nt + lr];
    M[nt] = e.x;
    iS[nt] = e.y;
  }

  f4 o[4][4];   // [dim tile][row tile]: out^T[dim 64w + 16mt + 4(l/16) + i][row 16nt + l%16]
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) o[mt][nt] = f4{0.f, 0.f, 0.f, 0.f};

  char *vt_hi = s_vt[w][0];
  char *vt_lo = s_vt[w][VF ? 1 : 0];
  const uint32_t klast = p.kend - 1;
  KRaw<KF> kc, kn;
  VRaw<VF> vc, vn;
  auto vkeys = [&](int t, uint32_t &ka, uint32_t &kb) {
    ka = min((uint32_t)(t * kPfTile + 2 * kp), klast);
    kb = min((uint32_t)(t * kPfTile + 2 * kp + 1), klast);
  };
  if (p.t0 < p.t1) {
    load_k<KF, PG>(a.L, a.nkv, p.g, min((uint32_t)(p.t0 * kPfTile + 16 * w + lr), klast), lq, kc);
    uint32_t ka, kb;
    vkeys(p.t0, ka, kb);
    load_v<VF, PG>(a.L, a.nkv, p.g, ka, kb, w, vh, vc);
  }
  int buf = 0;
  for (int t = p.t0; t < p.t1; ++t) {
    const int tn = min(t + 1, p.t1 - 1);
    load_k<KF, PG>(a.L, a.nkv, p.g, min((uint32_t)(tn * kPfTile + 16 * w + lr), klast), lq, kn);
    {
      uint32_t ka, kb;
      vkeys(tn, ka, kb);
      load_v<VF, PG>(a.L, a.nkv, p.g, ka, kb, w, vh, vn);
    }
    f4 acc[4];
    qk_tile<KF>(kc, qf, acc);
    const int kb0 = t * kPfTile + 16 * w + 4 * lq;
    char *pb = s_p[buf];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      h2 pp[2];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float e = fexp(acc[nt][i] * a.scale - M[nt]) * iS[nt];
        pp[i >> 1][i & 1] = (_Float16)(kb0 + i <= lim[nt] ? e : 0.f);
      }
      *reinterpret_cast<uint2 *>(pb + (16 * nt + lr) * kPfRS + 2 * (16 * w + 4 * lq)) =
          make_uint2(as_u(pp[0]), as_u(pp[1]));
    }
    put_vt<VF>(vc, kp, vh, vt_hi, vt_lo);
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      h8 bp[4];
#pragma unroll
      for (int nt = 0; nt < 4; ++nt)
        bp[nt] = *reinterpret_cast<const h8 *>(pb + (16 * nt + lr) * kPfRS + 2 * (32 * ks + 8 * lq));
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const h8 ah = *reinterpret_cast<const h8 *>(vt_hi + (16 * mt + lr) * kPfRS + 2 * (32 * ks + 8 * lq));
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) o[mt][nt] = mfma16(ah, bp[nt], o[mt][nt]);
        if constexpr (VF) {
          const h8 al = *reinterpret_cast<const h8 *>(vt_lo + (16 * mt + lr) * kPfRS + 2 * (32 * ks + 8 * lq));
#pragma unroll
          for (int nt = 0; nt < 4; ++nt) o[mt][nt] = mfma16(al, bp[nt], o[mt][nt]);
        }
      }
    }
    buf ^= 1;
    kc = kn;
    vc = vn;
  }

  // rows' outputs: the final result (one split) or the split's normalised partial
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    const int r = 16 * nt + lr;
    if ((r >> 2) >= p.nqv) continue;
    const size_t row = (size_t)(p.q0 + (r >> 2)) * a.nh + p.g * kGqa + (r & 3);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const int d = 64 * w + 16 * mt + 4 * lq;
      const float4 v = make_float4(o[mt][nt][0], o[mt][nt][1], o[mt][nt][2], o[mt][nt][3]);
      if (a.nsplit > 1) {
        *reinterpret_cast<float4 *>(a.part + ((size_t)p.s * a.n_q * a.nh + row) * kHd + d) = v;
      } else {
        *reinterpret_cast<float4 *>(a.out + row * kHd + d) = v;
        if (a.gate) {
          const float4 gt = *reinterpret_cast<const float4 *>(a.gate + row * a.gs + d);
          float4 og;
          og.x = v.x * (1.0f / (1.0f + exp_cr(-gt.x)));
          og.y = v.y * (1.0f / (1.0f + exp_cr(-gt.y)));
          og.z = v.z * (1.0f / (1.0f + exp_cr(-gt.z)));
          og.w = v.w * (1.0f / (1.0f + exp_cr(-gt.w)));
          *reinterpret_cast<float4 *>(a.out_gated + row * kHd + d) = og;
        }
      }
    }
  }
}

// ------------------------------------------------------------------ merge of the splits + gate
__global__ __launch_bounds__(256) void prefill_merge_kernel(PrefillArgs a) {
  const size_t n4 = (size_t)a.n_q * a.nh * (kHd / 4);
  const size_t rs4 = n4;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (size_t)gridDim.x * 256) {
    const float4 *pp = reinterpret_cast<const float4 *>(a.part);
    float4 v = pp[i];
    for (int s = 1; s < a.nsplit; ++s) {
      const float4 x = pp[s * rs4 + i];
      v.x += x.x; v.y += x.y; v.z += x.z; v.w += x.w;
    }
    reinterpret_cast<float4 *>(a.out)[i] = v;
    if (a.gate) {
      const float4 gt = *reinterpret_cast<const float4 *>(a.gate + gate_index(4 * i, a.gs));
      float4 og;
      og.x = v.x * (1.0f / (1.0f + exp_cr(-gt.x)));
      og.y = v.y * (1.0f / (1.0f + exp_cr(-gt.y)));
      og.z = v.z * (1.0f / (1.0f + exp_cr(-gt.z)));
      og.w = v.w * (1.0f / (1.0f + exp_cr(-gt.w)));
      reinterpret_cast<float4 *>(a.out_gated)[i] = og;
    }
  }
}

hipError_t launch_prefill(const PrefillArgs &a, int kf, int vf, hipStream_t st) {
  const int grid = a.nkv * a.nqb * a.nsplit;
  const bool pg = a.L.page != 0;
  BKV_FMT_SWITCH(kf, vf, {
    if (pg) {
      hipLaunchKernelGGL((prefill_stats_kernel<KF_, true>), dim3(grid), dim3(kPfNT), 0, st, a);
      hipLaunchKernelGGL((prefill_pv_kernel<KF_, VF_, true>), dim3(grid), dim3(kPfNT), 0, st, a);
    } else {
      hipLaunchKernelGGL((prefill_stats_kernel<KF_, false>), dim3(grid), dim3(kPfNT), 0, st, a);
      hipLaunchKernelGGL((prefill_pv_kernel<KF_, VF_, false>), dim3(grid), dim3(kPfNT), 0, st, a);
    }
  });
  if (a.nsplit > 1) {
    const size_t n4 = (size_t)a.n_q * a.nh * (kHd / 4);
    const int blocks = (int)std::min<size_t>((n4 + 255) / 256, 2048);
    hipLaunchKernelGGL(prefill_merge_kernel, dim3(blocks), dim3(256), 0, st, a);
  }
  return hipGetLastError();
}

// ================================================================== exact prefill
// The default prefill: every (query, head) row reproduces the serial reference bit for bit up to
// the PV contraction. A workgroup owns 4 queries x 4 heads = 16 rows of one KV group and all of
// their keys, in up to three sweeps:
//   1  scores (q8_0 K: the correctly rounded inner sum of each block from the int8 matrix cores,
//      bkv_q8dot.h, then acc = acc + f16(scale)*inner in block order; fp16 K: the reference's serial
//      chain acc = acc + q16*k in ascending d, one exact fma per step on the fp32 matrix cores),
//      times the softmax scale, masked causally; the row max. Scores go to a scratch region
//      [key][row].
//   2  e = exp(v - max) correctly rounded, written back over the scores; one lane per row adds
//      them in key order (the reference's serial fp32 sum, attn_vk.h:175-189).
//   3  (fp16 V) p16 = f16(e / sum) (the correctly rounded fp32 quotient, from e * (1/sum) by two
//      remainder corrections, then round to nearest even), and out = sum p16 * v on the matrix
//      cores. q8_0 V: the sums go out instead, and prefill_pv64_kernel forms p16 and the PV for 64
//      rows at a time.
// Only the PV sum runs in another order than the reference (fp32 accumulation of exact products).

#ifdef BKV_EXPERIMENT_TS
#define PXTS(i) do { if (threadIdx.x == 0 && a.ts) a.ts[blockIdx.x * 16 + (i)] = (unsigned)wall_clock64(); } while (0)
#else
#define PXTS(i) do { } while (0)
#endif

// Workgroup barrier for LDS traffic only: every wave's LDS operations have completed, while its
// global loads (prefetches a step or more ahead) stay in flight. __syncthreads() also releases
// global memory, i.e. waits for every outstanding load and store of the wave first, which would
// void those prefetches. Used where the waves exchange data through LDS alone.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// scratch accesses (plain loads and stores: the scratch round trips are served largely by the
// memory-side cache, which non-temporal accesses bypass)
__device__ __forceinline__ void st_sc4(float *p, float4 v) { *reinterpret_cast<float4 *>(p) = v; }
__device__ __forceinline__ float4 ld_sc4(const float *p) { return *reinterpret_cast<const float4 *>(p); }

// ---------------------------------------------------------------- fp16 K scores on the matrix cores
// v_mfma_f32_16x16x1_4b_f32 computes, for 4 independent blocks b, D_b[i][j] += A_b[i] * B_b[j] with
// one rounding per element: A_b[i] comes from lane 16b + i, B_b[j] from lane 16b + j, and lane l
// holds D_b[4(l/16) + k][l%16] in accumulator register 4b + k. With K = 1 each step is exactly one
// fp32 fma per element (the product of two fp16 values is exact in fp32), so a chain of steps in
// ascending dimension is the reference's serial score, bit for bit. (q8_0 K: bkv_q8dot.h.)
typedef float fv16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ fv16 mfma_k1(float a, float b, fv16 c) {
  return __builtin_amdgcn_mfma_f32_16x16x1f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t word_of(const uint4 &v, int i) {
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

template <int KF, int VF, bool PG>
__global__ __launch_bounds__(256, 2) void prefill_exact_kernel(PrefillXArgs a) {
  const int n = gridDim.x, b = blockIdx.x;
  const int wi = (n & 7) == 0 ? (b & 7) * (n >> 3) + (b >> 3) : b;
  const int qb = wi % a.nqb, g = wi / a.nqb;
  const int q0 = a.q_base + qb * kPxQ;                   // first query (chunk index)
  const int nqv = min(kPxQ, a.q_base + a.n_q - q0);
  const uint32_t kend = a.pos0 + (uint32_t)(q0 + nqv);  // keys 0 .. kend-1
  const int ntile = (int)((kend + kPxTile - 1) / kPxTile);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  float *sc = a.sc + (size_t)wi * a.ld * kPxRows;
  // the causal limit of row r is pos0 + q0 + r/4 (rows of queries past the chunk see nothing)
  const int lim0 = (int)(a.pos0 + (uint32_t)q0);

  __shared__ float s_red[4][kPxRows];
  __shared__ float s_m[kPxRows], s_sum[kPxRows];
  __shared__ double s_t2[32];               // the exp table
  constexpr int ES = kPxRows + 1;          // LDS row stride (floats) of the exp tile
  constexpr int NT = kPxRows / 16;         // MFMA row tiles
  constexpr int PR = kPxRows / 4;          // probabilities per thread per 64-key tile
  constexpr int kBig2 = 2 * 256 * ES * 4, kBig3 = 2 * kPxRows * kPfRS + (VF ? 0 : 4 * 64 * kPfRS);
  __shared__ __attribute__((aligned(16))) char s_big[kBig2 > kBig3 ? kBig2 : kBig3];

  PXTS(0);
#ifdef BKV_EXPERIMENT_TS
  if (threadIdx.x == 0 && a.ts) a.ts[blockIdx.x * 16 + 8] = (unsigned)__smid();
#endif
  // ---------------------------------------------------------------- sweep 1: exact scores
  // the rows' q16 in LDS: s_q[r][d], row r = query q0 + r/4 (clamped into the chunk), head 4g + r%4
  if (tid < 32) s_t2[tid] = kExp2Tab[tid];
  if constexpr (KF) {
    // q8_0 K on the int8 matrix cores (bkv_q8dot.h): the digits of each of the workgroup's
    // queries' 4 q rows in LDS, their A operands in registers. A wave scores its 64 keys of a tile
    // as 4 key groups x 4 queries (one MFMA per block each) and transposes each key group's 4
    // queries so that lane l holds rows 4(l/16) + k: query l/16, heads 0..3. Each key group's K
    // bytes are requested a whole tile ahead (the rows come from HBM the first time any workgroup
    // of the XCD reads them; the workgroups run nearly in step).
    int8_t *s_lim = reinterpret_cast<int8_t *>(s_big);                    // [query][kLimBytes]
    int *s_lt = reinterpret_cast<int *>(s_big + kPxQ * kLimBytes);        // [query][head]
    static_assert(kPxQ * (kLimBytes + kGqa * 4) <= sizeof(s_big), "digits in the big LDS area");
    __shared__ unsigned s_wide;
    if (tid == 0) s_wide = 0u;
    __syncthreads();
    const int qlast = a.q_base + a.n_q - 1;
    auto qrows = [&](int jq) {                 // the 4 q rows of query jq (clamped into the chunk)
      return a.q + ((size_t)min(q0 + jq, qlast) * a.nh + g * kGqa) * a.qs;
    };
#pragma unroll 1
    for (int jq = 0; jq < kPxQ; ++jq)
      q8lim_build(qrows(jq), a.qs, s_lim + jq * kLimBytes, s_lt + jq * kGqa, &s_wide, tid, 256);
    __syncthreads();
    const bool wide = s_wide != 0u;
    long qa[kPxQ][8];
    int qt[kPxQ];                              // the exponent of head l/16 of each query
    {
      Q8Lim t;
#pragma unroll
      for (int jq = 0; jq < kPxQ; ++jq) {
        q8lim_load(s_lim + jq * kLimBytes, s_lt + jq * kGqa, t);
#pragma unroll
        for (int b = 0; b < 8; ++b) qa[jq][b] = t.a[b];
        qt[jq] = t.t;
      }
    }
    const int ql = lane >> 4, n16 = lane & 15;
    const bool qlive = ql < nqv;
    float mx[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    constexpr int RB = row_bytes(BKV_Q8_0);
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    struct KG { long b[8]; u32x4 s; };        // one key group's B operands and the lane key's scales
    // The loads are issued as inline asm, so that they stay where they are written (the compiler
    // would sink them to the end of the tile) and its wait counting leaves them alone: kg_wait<N>
    // waits until at most N vector memory operations issued after them are in flight, and names
    // the registers, so no read of them moves above it.
    auto load_kg = [&](uint32_t key0, int kg, KG &r) {
      const uint32_t key = min(key0 + (uint32_t)(16 * kg + n16), kend - 1);
      const int64_t ro = slot_t<PG>(a.L, key) * a.nkv + g;
      const uint8_t *src = a.L.kd + ro * RB + 8 * ql;
      const uint8_t *sp = a.L.ks + ro * kScaleRowBytes;
#define BKV_LD2(i) asm volatile("global_load_dwordx2 %0, %1, off offset:" #i "*32" : "=v"(r.b[i]) : "v"(src) : "memory")
      BKV_LD2(0); BKV_LD2(1); BKV_LD2(2); BKV_LD2(3); BKV_LD2(4); BKV_LD2(5); BKV_LD2(6); BKV_LD2(7);
#undef BKV_LD2
      asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(r.s) : "v"(sp) : "memory");
    };
    // the scores of key group kg of the tile at key0 (r[k]: row 4(l/16) + k), scaled and masked,
    // into the scratch and the row maxima
    auto emit = [&](uint32_t key0, int kg, const float (&r)[4]) {
      const uint32_t j = key0 + (uint32_t)(16 * kg + n16);
      const bool live = qlive && (int)j <= lim0 + ql;
      float v[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        v[k] = live ? r[k] * a.scale : -INFINITY;
        mx[k] = v[k] > mx[k] ? v[k] : mx[k];
      }
      st_sc4(sc + (size_t)j * kPxRows + 4 * ql, make_float4(v[0], v[1], v[2], v[3]));
    };
    if (!wide) {
      // a whole tile ahead. When key group kg is used, what was issued after its loads is the store
      // that followed them, the 3 later key groups' loads (9 each) and their stores: 31 operations
      // (27 to 30 in the first tile, whose loads went out back to back), so 27 are left in flight.
      KG kn[4];
      auto kg_wait = [](KG &r) {
        asm volatile("s_waitcnt vmcnt(27)"
                     : "+v"(r.b[0]), "+v"(r.b[1]), "+v"(r.b[2]), "+v"(r.b[3]), "+v"(r.b[4]), "+v"(r.b[5]),
                       "+v"(r.b[6]), "+v"(r.b[7]), "+v"(r.s)::"memory");
      };
#pragma unroll
      for (int kg = 0; kg < 4; ++kg) load_kg((uint32_t)((ntile - 1) * kPxTile + 64 * w), kg, kn[kg]);
      for (int t = ntile - 1; t >= 0; --t) {
        const uint32_t key0 = (uint32_t)(t * kPxTile + 64 * w);
#pragma unroll
        for (int kg = 0; kg < 4; ++kg) {
          KG &cur = kn[kg];
          kg_wait(cur);
          float r[4];
          const uint4 scl = make_uint4(cur.s.x, cur.s.y, cur.s.z, cur.s.w);
#pragma unroll
          for (int jq = 0; jq < kPxQ; ++jq) r[jq] = q8_score16r(cur.b, scl, qa[jq], qt[jq]);
          load_kg((uint32_t)(max(t - 1, 0) * kPxTile + 64 * w), kg, cur);
          transpose_rows4(r);
          emit(key0, kg, r);
        }
      }
      // every load has landed before its registers are free again
#pragma unroll
      for (int kg = 0; kg < 4; ++kg)
        asm volatile("s_waitcnt vmcnt(0)"
                     : "+v"(kn[kg].b[0]), "+v"(kn[kg].b[1]), "+v"(kn[kg].b[2]), "+v"(kn[kg].b[3]), "+v"(kn[kg].b[4]),
                       "+v"(kn[kg].b[5]), "+v"(kn[kg].b[6]), "+v"(kn[kg].b[7]), "+v"(kn[kg].s)::"memory");
    } else {
      // the wide path: lane = key 16 kg + l%16 against query l/16's 4 heads, fp64 inner sums
      for (int t = ntile - 1; t >= 0; --t) {
        const uint32_t key0 = (uint32_t)(t * kPxTile + 64 * w);
        for (int kg = 0; kg < 4; ++kg) {
          const uint32_t key = min(key0 + (uint32_t)(16 * kg + n16), kend - 1);
          const int64_t ro = slot_t<PG>(a.L, key) * a.nkv + g;
          float r[4];
          q8_score_key_slow(reinterpret_cast<const uint32_t *>(a.L.kd + ro * RB),
                            reinterpret_cast<const uint32_t *>(a.L.ks + ro * kScaleRowBytes), qrows(ql), a.qs, r);
          emit(key0, kg, r);
        }
      }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float m = row16_max(mx[k]);
      if ((lane & 15) == 0) s_red[w][4 * ql + k] = m;
    }
  } else {
    // fp16 K on the matrix cores: one chain of 256 steps per (row, key), acc = acc + q16*k in
    // ascending dimension (each product exact in fp32, each step one fma). Block b of the
    // instruction is key group b (keys 16b .. + 15 of a 64-key set), so one MFMA advances 64 keys x
    // 16 rows; a wave runs two sets (keys 64w .. of the two halves of a 512-key super tile) as two
    // independent chains, streaming each key's row 32 dimensions (64 B) at a time, one chunk ahead.
    // s_qh[d4][i] = q16 of row i, dims 4 d4 .. + 3 (the lanes of one row read the same float4).
    float4 *s_qh = reinterpret_cast<float4 *>(s_big);
    {
      const int qlast = a.q_base + a.n_q - 1;
      for (int i = tid; i < (kHd / 4) * kPxRows; i += 256) {
        const int r = i & 15, d4 = i >> 4;
        const int qi = min(q0 + (r >> 2), qlast);
        const float4 x = *reinterpret_cast<const float4 *>(a.q + ((size_t)qi * a.nh + g * kGqa + (r & 3)) * a.qs + 4 * d4);
        s_qh[i] = make_float4(round_f16(x.x), round_f16(x.y), round_f16(x.z), round_f16(x.w));
      }
    }
    __syncthreads();
    const int ql = lane >> 4;
    const bool qlive = ql < nqv;
    float mx[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    const int nsup = (int)((kend + 2 * kPxTile - 1) / (2 * kPxTile));
    constexpr int RB = row_bytes(BKV_F16);
    struct KChunk { uint4 d[2][4]; };          // [set][16 B]: dims 32c .. + 31 of the lane's key
    auto load_chunk = [&](int T, int c, KChunk &k) {
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        const uint32_t key = min((uint32_t)(T * 2 * kPxTile + st * kPxTile + 64 * w + lane), kend - 1);
        const uint4 *src = reinterpret_cast<const uint4 *>(a.L.kd + (slot_t<PG>(a.L, key) * a.nkv + g) * RB + 64 * c);
#pragma unroll
        for (int q = 0; q < 4; ++q) k.d[st][q] = src[q];
      }
    };
    auto chunk = [&](const KChunk &k, int c, fv16 (&d)[2]) {
#pragma unroll
      for (int i4 = 0; i4 < 8; ++i4) {
        const float4 q4 = s_qh[(8 * c + i4) * kPxRows + (lane & 15)];
        const float qa[4] = {q4.x, q4.y, q4.z, q4.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i = 4 * i4 + e;      // dimension within the chunk: 16-bit half i of the 64 B
#pragma unroll
          for (int st = 0; st < 2; ++st) {
            const uint32_t wv = word_of(k.d[st][i >> 3], (i >> 1) & 3);
            d[st] = mfma_k1(qa[e], f16_to_f32((i & 1) ? (wv >> 16) : (wv & 0xFFFFu)), d[st]);
          }
        }
      }
    };
    KChunk ka, kb;
    load_chunk(nsup - 1, 0, ka);
    // super tiles in descending key order (sweep 2 reads them ascending)
    for (int T = nsup - 1; T >= 0; --T) {
      fv16 d[2] = {fv16{}, fv16{}};
#pragma unroll
      for (int c = 0; c < kHd / 32; c += 2) {
        load_chunk(T, c + 1, kb);
        __builtin_amdgcn_sched_barrier(0);
        chunk(ka, c, d);
        __builtin_amdgcn_sched_barrier(0);
        if (c + 2 < kHd / 32) load_chunk(T, c + 2, ka);
        else load_chunk(max(T - 1, 0), 0, ka);
        __builtin_amdgcn_sched_barrier(0);
        chunk(kb, c + 1, d);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int st = 0; st < 2; ++st) {
#pragma unroll
        for (int bq = 0; bq < 4; ++bq) {
          const uint32_t j = (uint32_t)(T * 2 * kPxTile + st * kPxTile + 64 * w + 16 * bq + (lane & 15));
          const bool live = qlive && (int)j <= lim0 + ql;
          float v[4];
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            v[k] = live ? d[st][4 * bq + k] * a.scale : -INFINITY;
            mx[k] = v[k] > mx[k] ? v[k] : mx[k];
          }
          st_sc4(sc + (size_t)j * kPxRows + 4 * ql, make_float4(v[0], v[1], v[2], v[3]));
        }
      }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float m = row16_max(mx[k]);
      if ((lane & 15) == 0) s_red[w][4 * ql + k] = m;
    }
  }
  __syncthreads();
  if (tid < kPxRows) {
    float m = fmaxf(fmaxf(s_red[0][tid], s_red[1][tid]), fmaxf(s_red[2][tid], s_red[3][tid]));
    s_m[tid] = (tid >> 2) < nqv ? m : 0.f;
  }
  __syncthreads();

  PXTS(1);
  // ---------------------------------------------------------------- sweep 2: exp and serial sum
  // Waves 0..2 form e for 192 keys per step (one key per thread, its 16 rows) into an LDS tile
  // while wave 3 adds the previous step's e values of each row in key order (lane r: row r), so
  // the serial chains run beside the exps, and writes that tile over the scores (wave 3 reads no
  // global memory, so its stores never hold up a wait for the exp waves' score loads).
  constexpr int kEK = 192;                        // keys per step
  float *et = reinterpret_cast<float *>(s_big);   // [2][kEK][ES]
  const int nstep = (int)((kend + kEK - 1) / kEK + 1) & ~1;   // even: the exp waves run steps in pairs
  const uint32_t kscr = (uint32_t)(ntile * kPxTile);   // this workgroup's scratch keys
  float sum = 0.f;
  if (w < 3) {
    float mrow[kPxRows];
#pragma unroll
    for (int r = 0; r < kPxRows; ++r) mrow[r] = s_m[r];
    auto fetch = [&](int t, float4 (&v)[kPxRows / 4]) {
      const uint32_t j = min((uint32_t)(t * kEK + tid), kscr - 1);
      const float *src = sc + (size_t)j * kPxRows;
#pragma unroll
      for (int r4 = 0; r4 < kPxRows / 4; ++r4) v[r4] = ld_sc4(src + 4 * r4);
    };
    auto step = [&](int t, const float4 (&vc)[kPxRows / 4]) {
      const uint32_t j = (uint32_t)(t * kEK + tid);
      float *eb = et + (t & 1) * kEK * ES + tid * ES;
      const bool in = j < kscr;                    // keys past the scores: e = 0 (none are live)
      // all 16 exps first, then the LDS stores: independent exps interleave (their table reads in
      // flight together) instead of each waiting out an LDS round trip behind the stores before it
      float ev[kPxRows], xv[kPxRows];
      bool slow[kPxRows], any = false;
#pragma unroll
      for (int r4 = 0; r4 < kPxRows / 4; ++r4) {
        xv[4 * r4] = vc[r4].x - mrow[4 * r4];
        xv[4 * r4 + 1] = vc[r4].y - mrow[4 * r4 + 1];
        xv[4 * r4 + 2] = vc[r4].z - mrow[4 * r4 + 2];
        xv[4 * r4 + 3] = vc[r4].w - mrow[4 * r4 + 3];
      }
#pragma unroll
      for (int r = 0; r < kPxRows; ++r) {
        ev[r] = exp_t_fast(xv[r], s_t2, slow[r]);
        any = any || slow[r];
      }
      if (any) {
#pragma unroll
        for (int r = 0; r < kPxRows; ++r)
          if (slow[r]) ev[r] = exp_t_slow(xv[r]);
      }
#pragma unroll
      for (int r = 0; r < kPxRows; ++r) eb[r] = in ? ev[r] : 0.f;
      lds_barrier();
    };
    // two register sets: each step's scores are requested two steps ahead
    float4 va[kPxRows / 4], vb[kPxRows / 4];
    fetch(0, va);
    fetch(min(1, nstep - 1), vb);
    for (int t = 0; t < nstep; t += 2) {
      step(t, va);
      fetch(min(t + 2, nstep - 1), va);
      step(t + 1, vb);
      fetch(min(t + 3, nstep - 1), vb);
    }
    __syncthreads();
  } else {
    const int r = lane & 15;
    for (int t = 0; t <= nstep; ++t) {
      if (t > 0) {
        const float *tile = et + ((t - 1) & 1) * kEK * ES;
        if (lane < kPxRows) {
          const float *col = tile + r;
#pragma unroll 16
          for (int k = 0; k < kEK; ++k) sum = sum + col[k * ES];
        }
        // the tile over the scores: key k's 16 rows as 4 float4, within the region's ld keys
        float *dst = sc + (size_t)(t - 1) * kEK * kPxRows;
        const int kmax = (int)min((int64_t)kEK, a.ld - (int64_t)(t - 1) * kEK);
#pragma unroll
        for (int i = 0; i < kEK * kPxRows / 4 / 64; ++i) {
          const int f = lane + 64 * i, k = f >> 2, r4 = f & 3;
          const float *e4 = tile + k * ES + 4 * r4;
          if (k < kmax) st_sc4(dst + 4 * f, make_float4(e4[0], e4[1], e4[2], e4[3]));
        }
      }
      lds_barrier();
    }
    if (lane < kPxRows) s_sum[r] = (r >> 2) < nqv ? sum : 1.0f;
  }
  __syncthreads();

  PXTS(2);
  // ---------------------------------------------------------------- sweep 3: p16 and PV
  if constexpr (VF) {
    // q8_0 V: the exact sums go out, and prefill_pv64_kernel forms p16 and the PV for 64 rows at a
    // time (each V byte converted once per 64 rows instead of per 16)
    if (tid < kPxRows) a.sums[(size_t)wi * kPxRows + tid] = s_sum[tid];
    return;
  } else {
  const int lr = lane & 15, lq = lane >> 4, kp = lane & 31, vh = lane >> 5;
  char *s_p = s_big;                                              // [2][kPxRows][kPfRS]
  char *vt_hi = s_big + 2 * kPxRows * kPfRS + w * (VF ? 2 : 1) * 64 * kPfRS;
  char *vt_lo = vt_hi + (VF ? 64 * kPfRS : 0);
  f4 o[4][NT];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) o[mt][nt] = f4{0.f, 0.f, 0.f, 0.f};
  const int nt64 = (int)((kend + kPfTile - 1) / kPfTile);
  const int pk = tid >> 2, pr0 = PR * (tid & 3);   // this thread's probabilities: key pk, rows pr0..+PR
  float ssum[PR], srcp[PR];
#pragma unroll
  for (int i = 0; i < PR; ++i) {
    ssum[i] = s_sum[pr0 + i];
    srcp[i] = 1.0f / ssum[i];
  }
  float4 en[PR / 4];
  VRaw<VF> vrn;
  auto load_tile = [&](int t) {
    const float *src = sc + ((size_t)t * kPfTile + pk) * kPxRows + pr0;
#pragma unroll
    for (int i = 0; i < PR / 4; ++i) en[i] = ld_sc4(src + 4 * i);
    const uint32_t ka = min((uint32_t)(t * kPfTile + 2 * kp), kend - 1);
    const uint32_t kb = min((uint32_t)(t * kPfTile + 2 * kp + 1), kend - 1);
    load_v<VF, PG>(a.L, a.nkv, g, ka, kb, w, vh, vrn);
  };
  // tiles in descending key order (the PV sum's order is free): the last-written exp values first
  load_tile(nt64 - 1);
  for (int t = nt64 - 1; t >= 0; --t) {
    char *pb = s_p + (t & 1) * kPxRows * kPfRS;
    float ev[PR];
#pragma unroll
    for (int i = 0; i < PR / 4; ++i) {
      ev[4 * i] = en[i].x; ev[4 * i + 1] = en[i].y; ev[4 * i + 2] = en[i].z; ev[4 * i + 3] = en[i].w;
    }
    const VRaw<VF> vr = vrn;
    load_tile(max(t - 1, 0));   // in flight during this tile
#pragma unroll
    for (int i = 0; i < PR; ++i) {
      const _Float16 h = (_Float16)div_by_sum(ev[i], ssum[i], srcp[i]);
      *reinterpret_cast<_Float16 *>(pb + (pr0 + i) * kPfRS + 2 * pk) = h;
    }
    put_vt<VF>(vr, kp, vh, vt_hi, vt_lo);
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      h8 bp[NT];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
        bp[nt] = *reinterpret_cast<const h8 *>(pb + (16 * nt + lr) * kPfRS + 2 * (32 * ks + 8 * lq));
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const h8 ah = *reinterpret_cast<const h8 *>(vt_hi + (16 * mt + lr) * kPfRS + 2 * (32 * ks + 8 * lq));
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) o[mt][nt] = mfma16(ah, bp[nt], o[mt][nt]);
        if constexpr (VF) {
          const h8 al = *reinterpret_cast<const h8 *>(vt_lo + (16 * mt + lr) * kPfRS + 2 * (32 * ks + 8 * lq));
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) o[mt][nt] = mfma16(al, bp[nt], o[mt][nt]);
        }
      }
    }
  }
  PXTS(3);
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int r = 16 * nt + lr;
    if ((r >> 2) >= nqv) continue;
    const size_t row = (size_t)(q0 + (r >> 2)) * a.nh + g * kGqa + (r & 3);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const int d = 64 * w + 16 * mt + 4 * lq;
      const float4 v = make_float4(o[mt][nt][0], o[mt][nt][1], o[mt][nt][2], o[mt][nt][3]);
      *reinterpret_cast<float4 *>(a.out + row * kHd + d) = v;
      if (a.gate) {
        const float4 gt = *reinterpret_cast<const float4 *>(a.gate + row * a.gs + d);
        float4 og;
        og.x = v.x * (1.0f / (1.0f + exp_cr(-gt.x)));
        og.y = v.y * (1.0f / (1.0f + exp_cr(-gt.y)));
        og.z = v.z * (1.0f / (1.0f + exp_cr(-gt.z)));
        og.w = v.w * (1.0f / (1.0f + exp_cr(-gt.w)));
        *reinterpret_cast<float4 *>(a.out_gated + row * kHd + d) = og;
      }
    }
  }
  }
}

// ---------------------------------------------------------------- the exact prefill's PV, q8_0 V
// 16 queries (64 rows: query i, head h at row 4 i + h) of one KV group over one half of their key
// tiles: p16 = f16(e / sum) from the exact kernel's e scratch and sums (the reference's P16,
// attn_vk.h:190-200), out^T = V^T . P^T on v_mfma_f32_16x16x32_f16, wave w of 8 owning dims
// 32 w .. + 31 (one q8_0 block). Each 64-key tile of V goes into LDS by direct-to-LDS loads (one
// 1 KiB block of 4 keys per load, two per wave) in the blocked layout of bkv_pv8.h; lane l then reads
// A row i = l%16 of dimension tile mt (dim 32 w + 16 mt + i) over keys 8(l/16) .. + 7 of each 32-key
// half with one ds_read_b64_tr_b8, and the exact fp16 split of d*b (hi = f16(d*b), lo = d*b - hi)
// forms the operands, shared by the 64 rows. The two halves' partials are added in a fixed order by
// prefill_pv_merge_kernel.
template <bool PG>
__global__ __launch_bounds__(512, 1) void prefill_pv64_kernel(PrefillXArgs a) {
  constexpr int R = kGqa * kPvQ;                   // rows, kPvQ / kPxQ exact-kernel workgroups' worth
  constexpr int NTR = R / 16;                      // MFMA row tiles
  constexpr int RPW = R / 8;                       // rows per wave of the P tile
  static_assert(RPW % 4 == 0 && kPxRows % RPW == 0 || RPW % kPxRows == 0, "a wave's rows in whole float4s");
  const int n = gridDim.x, b = blockIdx.x;
  const int nqp = (a.n_q + kPvQ - 1) / kPvQ;
  const int wb = (n & 7) == 0 ? (b & 7) * (n >> 3) + (b >> 3) : b;
  const int qb = wb % nqp, sp = (wb / nqp) % kPvSplit, g = wb / (kPvSplit * nqp);
  const int q0 = a.q_base + kPvQ * qb;             // chunk index of the first query
  const int nqv = min(kPvQ, a.q_base + a.n_q - q0);
  const uint32_t kend = a.pos0 + (uint32_t)(q0 + nqv);
  const int ntl = (int)((kend + kPfTile - 1) / kPfTile);
  const int t0 = sp * ntl / kPvSplit, t1 = (sp + 1) * ntl / kPvSplit;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, lr = lane & 15, lq = lane >> 4;
  __shared__ __attribute__((aligned(16))) char s_p[2][R * kPfRS];   // P tiles [row][64 keys] fp16
  // this thread's probabilities: key pk of a tile, rows RPW w .. + RPW - 1 (of exact-kernel
  // workgroup xq, whose scratch holds their e up to its own last key kx); the wave's sums in scalar
  // registers
  const int pk = lane;
  const int xr = (R / kPxRows) * qb + RPW * w / kPxRows, roff = RPW * w % kPxRows;
  const int xq = min(xr, a.nqb - 1);
  const bool pv = kPxQ * xr < a.n_q;
  const uint32_t kx = a.pos0 + (uint32_t)min(a.q_base + kPxQ * xr + kPxQ, a.q_base + a.n_q);
  const size_t xw = (size_t)g * a.nqb + xq;
  const float *esrc = a.sc + xw * a.ld * kPxRows + roff;
  float ssum[RPW], srcp[RPW];
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    ssum[i] = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(
                                            __builtin_bit_cast(int, a.sums[xw * kPxRows + roff + i])));
    srcp[i] = 1.0f / ssum[i];
  }
  f4 o[2][NTR];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int nt = 0; nt < NTR; ++nt) o[mt][nt] = f4{0.f, 0.f, 0.f, 0.f};
  // V tiles: three LDS buffers (tile t in buffer t % 3), each 16 blocks of 4 keys (block i at 1024 i,
  // 16-byte chunk c of its row r at 64 (c ^ (i & 3)) + 16 r: the rows one transposed read takes
  // spread over the banks)
  __shared__ __attribute__((aligned(1024))) char s_v[3][16384];
  const uint32_t vbase = __builtin_amdgcn_readfirstlane(lds_addr(s_v));
  // the lane's read address in a tile buffer for key half ks (dim tile: XOR 64 (2 w + mt))
  uint32_t vrd[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const int j = lr >> 1, bl = 8 * ks + 2 * lq + (j >> 2);
    vrd[ks] = (uint32_t)(1024 * bl + 16 * (j & 3) + 8 * (lane & 1) + 64 * (bl & 3));
  }
  // (the loaded values are kept raw until the tile uses them: any arithmetic on them here would
  // make the wave wait for the loads at once)
  struct PvIn {
    float4 en[RPW / 4];                             // e of key pk, the thread's rows (valid if live)
    bool live;
    uint32_t vs;                                    // the block scale of key 32 (l%16 / 8) + 8 lq + l%8
  };
  // tiles past t1 (the loop runs whole groups of three) load tile t1 - 1 again and add nothing
  auto load_tile = [&](int tt, PvIn &in) {
    const int t = min(tt, t1 - 1);
    const uint32_t j = (uint32_t)(t * kPfTile + pk);
    const float *src = esrc + (size_t)min(j, kx - 1) * kPxRows;
#pragma unroll
    for (int i = 0; i < RPW / 4; ++i) in.en[i] = ld_sc4(src + 4 * i);
    in.live = pv && j < kx && tt < t1;
    // one scale load per lane: lane l%16 of each 16-lane row loads key (l%16 / 8, l%8)'s, and the row
    // shares them by DPP broadcasts in the tile
    const uint32_t skey = min((uint32_t)(t * kPfTile + 32 * (lr >> 3) + 8 * lq + (lr & 7)), kend - 1);
    in.vs = *reinterpret_cast<const uint16_t *>(a.L.vs + (slot_t<PG>(a.L, skey) * a.nkv + g) * kScaleRowBytes + 2 * w);
  };
  // the V rows of tile tt (clamped as above) into buffer tt % 3: wave w loads blocks 2 w, 2 w + 1
  // (keys 4 i + lane % 4, chunk (lane / 4) ^ (i % 4) at 16 lane)
  auto dma_tile = [&](int tt) {
    const int t = min(tt, t1 - 1);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int i = 2 * w + u;
      const uint32_t key = min((uint32_t)(t * kPfTile + 4 * i + (lane & 3)), kend - 1);
      const uint8_t *src = a.L.vd + (slot_t<PG>(a.L, key) * a.nkv + g) * kHd + 16 * ((lane >> 2) ^ (i & 3));
      asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src),
                   "s"(__builtin_amdgcn_readfirstlane(vbase + 16384u * (uint32_t)(tt % 3) + 1024u * i)) : "memory", "m0");
    }
  };
  auto tile = [&](int t, const PvIn &in) {
    char *pb = s_p[t & 1];
    float ev[RPW];
#pragma unroll
    for (int i = 0; i < RPW / 4; ++i) {
      ev[4 * i] = in.en[i].x; ev[4 * i + 1] = in.en[i].y; ev[4 * i + 2] = in.en[i].z; ev[4 * i + 3] = in.en[i].w;
    }
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
      const _Float16 h = (_Float16)div_by_sum(in.live ? ev[i] : 0.0f, ssum[i], srcp[i]);
      *reinterpret_cast<_Float16 *>(pb + (RPW * w + i) * kPfRS + 2 * pk) = h;
    }
    // the block scales of the lane's 16 keys: key (ks, c) from lane 8 ks + c of its row
    uint32_t vsk[16];
#define BKV_BC(i) vsk[i] = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)in.vs, 0x150 + (i), 0xF, 0xF, false)
    BKV_BC(0); BKV_BC(1); BKV_BC(2); BKV_BC(3); BKV_BC(4); BKV_BC(5); BKV_BC(6); BKV_BC(7);
    BKV_BC(8); BKV_BC(9); BKV_BC(10); BKV_BC(11); BKV_BC(12); BKV_BC(13); BKV_BC(14); BKV_BC(15);
#undef BKV_BC
    // this wave's V rows of tile t have landed when at most the loads issued after them are in
    // flight: tile t + 1's register loads (NL) and rows (2), tile t + 2's register loads (NL)
    constexpr int NL = RPW / 4 + 1;
    static_assert(2 * NL + 2 == 8 || 2 * NL + 2 == 12, "the wait count below");
    if constexpr (2 * NL + 2 == 8) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
    lds_barrier();                                  // the P tile and every wave's V rows of tile t
    dma_tile(t + 2);                                // (its buffer's last readers, tile t - 1, are done)
    const uint32_t vb = vbase + 16384u * (uint32_t)(t % 3);
    // the A operands (registers only): pair p of key half ks holds keys 2p, 2p+1
    h8 ah[2][2], al[2][2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const v2i_t bv = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
            (__attribute__((address_space(3))) v2i_t *)(uintptr_t)((vb + vrd[ks]) ^ (uint32_t)(64 * (2 * w + mt))));
        constexpr uint32_t kSel[4] = {0x0C010C00u, 0x0C030C02u, 0x0C050C04u, 0x0C070C06u};
        uint32_t hw[4], lw[4];
#pragma unroll
        for (int pp = 0; pp < 4; ++pp) {
          const uint32_t bw = __builtin_amdgcn_perm((uint32_t)bv.y, (uint32_t)bv.x, kSel[pp]) ^ 0x64806480u;
          const h2 x = as_h2(bw) - h2{(_Float16)1152.0f, (_Float16)1152.0f};
          h2 hi, lo;
          split_prod(x, as_h2(vsk[8 * ks + 2 * pp] | (vsk[8 * ks + 2 * pp + 1] << 16)), hi, lo);
          hw[pp] = as_u(hi);
          lw[pp] = as_u(lo);
        }
        ah[ks][mt] = __builtin_bit_cast(h8, make_uint4(hw[0], hw[1], hw[2], hw[3]));
        al[ks][mt] = __builtin_bit_cast(h8, make_uint4(lw[0], lw[1], lw[2], lw[3]));
      }
    }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
      for (int nt = 0; nt < NTR; ++nt) {
        const h8 bp = *reinterpret_cast<const h8 *>(pb + (16 * nt + lr) * kPfRS + 2 * (32 * ks + 8 * lq));
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          o[mt][nt] = mfma16(ah[ks][mt], bp, o[mt][nt]);
          o[mt][nt] = mfma16(al[ks][mt], bp, o[mt][nt]);
        }
      }
    }
  };
  // three register sets and V buffers, each tile's operands requested two tiles ahead (branch-free
  // groups of three, so that the compiler's wait counting keeps the two younger tiles' loads in
  // flight); the V rows of tile t + 2 go out once every wave has passed tile t's barrier
  if (t0 < t1) {
    PvIn in[3];
    load_tile(t0, in[0]);
    dma_tile(t0);
    load_tile(t0 + 1, in[1]);
    dma_tile(t0 + 1);
    for (int t = t0; t < t1; t += 3) {
#pragma unroll
      for (int u = 0; u < 3; ++u) {
        load_tile(t + u + 2, in[(u + 2) % 3]);
        __builtin_amdgcn_sched_barrier(0);
        tile(t + u, in[u]);
      }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the last rows landed before the LDS is released
  }
  // lane l holds out^T[dim 32 w + 16 mt + 4(l/16) + r][row 16 nt + l%16] in o[mt][nt][r]
  float *part = a.part + (size_t)sp * kPxSlice * a.nh * kHd;
#pragma unroll
  for (int nt = 0; nt < NTR; ++nt) {
    const int r = 16 * nt + lr;
    if ((r >> 2) >= nqv) continue;
    const size_t row = (size_t)(q0 - a.q_base + (r >> 2)) * a.nh + g * kGqa + (r & 3);
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
      *reinterpret_cast<float4 *>(part + row * kHd + 32 * w + 16 * mt + 4 * lq) =
          make_float4(o[mt][nt][0], o[mt][nt][1], o[mt][nt][2], o[mt][nt][3]);
  }
}

// out = partial of the first key half + partial of the second (in that order), and the gate
__global__ __launch_bounds__(256) void prefill_pv_merge_kernel(PrefillXArgs a) {
  const size_t n4 = (size_t)a.n_q * a.nh * (kHd / 4);
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n4) return;
  float4 v = reinterpret_cast<const float4 *>(a.part)[i];
#pragma unroll
  for (int s = 1; s < kPvSplit; ++s) {           // the key ranges in order
    const float4 y = reinterpret_cast<const float4 *>(a.part + (size_t)s * kPxSlice * a.nh * kHd)[i];
    v = make_float4(v.x + y.x, v.y + y.y, v.z + y.z, v.w + y.w);
  }
  const size_t row = i / (kHd / 4), d = 4 * (i % (kHd / 4));
  const size_t grow = (size_t)a.q_base * a.nh + row;             // row of the whole chunk
  *reinterpret_cast<float4 *>(a.out + grow * kHd + d) = v;
  if (a.gate) {
    const float4 gt = *reinterpret_cast<const float4 *>(a.gate + grow * a.gs + d);
    float4 og;
    og.x = v.x * (1.0f / (1.0f + exp_cr(-gt.x)));
    og.y = v.y * (1.0f / (1.0f + exp_cr(-gt.y)));
    og.z = v.z * (1.0f / (1.0f + exp_cr(-gt.z)));
    og.w = v.w * (1.0f / (1.0f + exp_cr(-gt.w)));
    *reinterpret_cast<float4 *>(a.out_gated + grow * kHd + d) = og;
  }
}

hipError_t launch_prefill_exact(const PrefillXArgs &a, int kf, int vf, hipStream_t st) {
  const int grid = a.nkv * a.nqb;
  const bool pg = a.L.page != 0;
  BKV_FMT_SWITCH(kf, vf, {
    if (pg) hipLaunchKernelGGL((prefill_exact_kernel<KF_, VF_, true>), dim3(grid), dim3(256), 0, st, a);
    else hipLaunchKernelGGL((prefill_exact_kernel<KF_, VF_, false>), dim3(grid), dim3(256), 0, st, a);
  });
  if (vf == BKV_Q8_0) {
    const int pgrid = a.nkv * kPvSplit * ((a.n_q + kPvQ - 1) / kPvQ);
    if (pg) hipLaunchKernelGGL(prefill_pv64_kernel<true>, dim3(pgrid), dim3(512), 0, st, a);
    else hipLaunchKernelGGL(prefill_pv64_kernel<false>, dim3(pgrid), dim3(512), 0, st, a);
    const size_t n4 = (size_t)a.n_q * a.nh * (kHd / 4);
    hipLaunchKernelGGL(prefill_pv_merge_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, st, a);
  }
  return hipGetLastError();
}

}  // namespace bkv
