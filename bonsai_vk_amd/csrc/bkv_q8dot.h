// bkv_q8dot.h - q8_0 K scores on the int8 matrix cores.
//
// The reference never quantises K (runtime_vk/shaders/attn_norm_rope2.comp:26-28), so the dot of a
// query row with a q8_0 K row has no reference order to follow. This build defines it as
//
//   score = ((0 + f16(s_0) * inner_0) + f16(s_1) * inner_1) + ... + f16(s_7) * inner_7
//   inner_b = the fp32 rounding (nearest even) of the EXACT sum of q16_d * int8_d over block b,
//
// every product and sum of the outer chain rounded to fp32 in block order. The inner sum has one
// rounding and no order: every product q16 * int8 is an integer multiple of 2^-24 below 2^23 in
// magnitude, so a block's exact sum is a multiple of 2^-24 below 2^28, which fp64 holds exactly
// (the CPU restatement sums it in fp64 in any order and rounds once).
//
// On the device the exact sum is an integer dot product. For head h let t be the smallest exponent
// of an fp16 ulp among the row's nonzero q16 values (all 256 dims); then Q_d = q16_d / 2^t is an
// integer, and when it fits four balanced base-256 digits, Q_d = sum_i c_i 256^i with c_i in
// [-128, 127] (the bytes of Q_d + 0x80808080, each minus 128). One v_mfma_i32_16x16x32_i8 per block
// and 16 keys then gives, for A row 4h + i (head h, digit i) and key column n, the exact integer
// o_i = sum_d c_i(d) * int8_d(n); x_b = o_0 + 256 o_1 + 65536 o_2 + 2^24 o_3 = sum_d Q_d int8_d exactly
// (combined in i32 pairs and one fp64 fma, every intermediate an integer below 2^53), and
// inner_b = fp32(x_b) * 2^t, one rounding. Because t is shared by the row's 8 blocks, the outer chain
// runs on the unscaled fp32(x_b) and the score is the chain's value times 2^t: every term of the
// scaled chain is 2^t times the unscaled one with the same rounding, as no value of either chain is
// subnormal (a nonzero term is at least 2^-24 * 2^-24, the smallest fp16 ulp times the smallest
// scale; every sum is a multiple of its terms' ulps) or overflows (|x_b| < 2^43, scales < 2^16,
// t <= 5). q16 rows whose digits do not fit (Q beyond 31 bits: an exponent spread of more than about
// 20 binades over the row, which needs |q| >= 2^-24 * 2^31 = 128 beside values near 2^-24) or that
// hold Inf / NaN take an fp64 VALU path per key with the same result.
#pragma once

#include "bkv_common.h"

namespace bkv {

typedef int v4i_t __attribute__((ext_vector_type(4)));

constexpr int kLimBytes = 8 * 16 * 32;   // digits in LDS: [block][row 4 h + i][32 dims] int8

// The A operands of one wave: lane l holds row l % 16 (head (l%16)/4, digit l % 4), dims
// 8 (l/16) .. + 7 of each block; t: the exponent of head l / 16 (the head whose scores lane l
// receives).
struct Q8Lim {
  long a[8];
  int t;
};

// Cooperative: the digits of the group's 4 q rows (fp32, row h at q + h * qs, in LDS or global
// memory; rounded to fp16 here as the reference's Q16 operand) into lim (kLimBytes, 4-byte aligned)
// and the rows' exponents into lt[h]. One wave per row: lane l takes dims 4 l .. 4 l + 3 (block l / 8).
// *wide (zeroed by the caller before a barrier) is set when a row's digits do not fit or a q16 is
// not finite. nt: threads taking part (a multiple of 64); tid: this thread's index among them.
__device__ __forceinline__ void q8lim_build(const float *q, int qs, int8_t *lim, int *lt, unsigned *wide, int tid,
                                            int nt) {
  const int lane = tid & 63, d0 = 4 * lane, b = lane >> 3;
  for (int h = tid >> 6; h < kGqa; h += nt >> 6) {    // (wave-uniform trip count)
    int mant[4], ue[4], neg[4];
    bool bad = false;
    int key = 127;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t bits = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)q[(size_t)h * qs + d0 + j]);
      const uint32_t ab = bits & 0x7FFFu;
      const int E = (int)(ab >> 10);
      bad = bad || E == 31;
      mant[j] = (int)(ab & 0x3FFu) | (E ? 0x400 : 0);
      ue[j] = max(E, 1) - 25;                      // the exponent of the value's ulp
      neg[j] = (int)(bits >> 15);
      if (mant[j] != 0) key = min(key, ue[j]);
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) key = min(key, __shfl_xor(key, o));
    const int t = key == 127 ? 0 : key;
    uint32_t V[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const long long m = mant[j] != 0 ? ((long long)mant[j] << (ue[j] - t)) : 0ll;   // shift <= 29
      const long long vv = (neg[j] ? -m : m) + 0x80808080ll;
      bad = bad || vv < 0 || vv > 0xFFFFFFFFll;
      V[j] = (uint32_t)vv ^ 0x80808080u;            // byte i: digit i as a two's complement int8
    }
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      uint32_t w = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) w |= ((V[j] >> (8 * d)) & 0xFFu) << (8 * j);
      *reinterpret_cast<uint32_t *>(lim + (b * 16 + 4 * h + d) * 32 + (d0 & 31)) = w;
    }
    if (lane == 0) lt[h] = t;
    if (__ballot(bad) != 0ull && lane == 0) atomicOr(wide, 1u);
  }
}

__device__ __forceinline__ void q8lim_load(const int8_t *lim, const int *lt, Q8Lim &L) {
  const int lane = threadIdx.x & 63, m = lane & 15, kq = lane >> 4;
#pragma unroll
  for (int b = 0; b < 8; ++b) L.a[b] = *reinterpret_cast<const long *>(lim + (b * 16 + m) * 32 + 8 * kq);
  L.t = lt[kq];
}

__device__ __forceinline__ float f16_half(uint32_t w, int hi) { return f16_to_f32(hi ? (w >> 16) : (w & 0xFFFFu)); }

// Scores of 16 keys from registers: bv[b] = the lane's 8 bytes of block b (dims 8 (l/16) .. + 7)
// of key l % 16, scl = that key's scale row; a, t: the A operands and the exponent (Q8Lim).
// Lane l receives the score of key l % 16 against head l / 16.
__device__ __forceinline__ float q8_score16r(const long (&bv)[8], const uint4 &scl, const long (&a)[8], int t) {
  v4i_t d[8];
#pragma unroll
  for (int b = 0; b < 8; ++b) d[b] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[b], bv[b], v4i_t{0, 0, 0, 0}, 0, 0, 0);
  const uint32_t sw[4] = {scl.x, scl.y, scl.z, scl.w};
  float acc = 0.0f;                            // the chain in units of 2^t
#pragma unroll
  for (int b = 0; b < 8; ++b) {
    const int lo = d[b][0] + (int)((uint32_t)d[b][1] << 8);
    const int hi = d[b][2] + (int)((uint32_t)d[b][3] << 8);
    const double x = __builtin_fma((double)hi, 65536.0, (double)lo);   // exact: an integer below 2^53
    acc = __fadd_rn(acc, __fmul_rn(f16_half(sw[b >> 1], b & 1), (float)x));
  }
  return __builtin_ldexpf(acc, t);
}

// Scores of 16 keys: row is the LDS row (16 data uint4, then the scale uint4) of key lane % 16;
// lane l receives the score of key l % 16 against head l / 16.
__device__ __forceinline__ float q8_score16(const uint4 *row, const Q8Lim &L) {
  const int kq = (threadIdx.x & 63) >> 4;
  const char *rb = reinterpret_cast<const char *>(row);
  long bv[8];
#pragma unroll
  for (int b = 0; b < 8; ++b) bv[b] = *reinterpret_cast<const long *>(rb + 32 * b + 8 * kq);
  return q8_score16r(bv, row[16], L.a, L.t);
}

// The wide path: one key's scores against the group's 4 heads (q, qs as for q8lim_build), each
// inner sum in fp64 (exact for finite operands; Inf / NaN as IEEE arithmetic gives them).
// data: the key's 256 bytes, sc: its 4 scale words.
__device__ __forceinline__ void q8_score_key_slow(const uint32_t *w, const uint32_t *sc, const float *q, int qs,
                                                  float (&acc)[kGqa]) {
#pragma unroll
  for (int h = 0; h < kGqa; ++h) acc[h] = 0.0f;
  for (int b = 0; b < 8; ++b) {
    const float s = f16_half(sc[b >> 1], b & 1);
#pragma unroll
    for (int h = 0; h < kGqa; ++h) {
      double x = 0.0;
      for (int e = 0; e < 32; ++e)
        x += (double)round_f16(q[(size_t)h * qs + 32 * b + e]) * (double)sbyte(w[8 * b + (e >> 2)], e & 3);
      acc[h] = __fadd_rn(acc[h], __fmul_rn(s, (float)x));
    }
  }
}
// the same for an LDS row (16 data uint4, then the scale uint4)
__device__ __forceinline__ void q8_score_key_slow(const uint4 *row, const float *q, int qs, float (&acc)[kGqa]) {
  const uint32_t *w = reinterpret_cast<const uint32_t *>(row);
  q8_score_key_slow(w, w + 64, q, qs, acc);
}

// r[c] (c = 0..3) holds, in lane (n, g) = (l % 16, l / 16), the value of item 16 c + n for head g;
// afterwards r[h] holds, in lane l, item l for head h (a 4 x 4 transpose of 16-lane rows by register)
__device__ __forceinline__ void transpose_rows4(float (&r)[4]) {
  const auto a02 = __builtin_amdgcn_permlane32_swap(__float_as_uint(r[0]), __float_as_uint(r[2]), false, false);
  const auto a13 = __builtin_amdgcn_permlane32_swap(__float_as_uint(r[1]), __float_as_uint(r[3]), false, false);
  const auto b01 = __builtin_amdgcn_permlane16_swap(a02[0], a13[0], false, false);
  const auto b23 = __builtin_amdgcn_permlane16_swap(a02[1], a13[1], false, false);
  r[0] = __uint_as_float(b01[0]);
  r[1] = __uint_as_float(b01[1]);
  r[2] = __uint_as_float(b23[0]);
  r[3] = __uint_as_float(b23[1]);
}

// Scores of the wave's 64 keys (key k's LDS row at rows + k * stride uint4) against the group's 4
// heads, one key per lane: four MFMA key groups, transposed.
__device__ __forceinline__ void q8_score64(const uint4 *rows, int stride, const Q8Lim &L, float (&acc)[kGqa]) {
  const int n = threadIdx.x & 15;
#pragma unroll
  for (int c = 0; c < 4; ++c) acc[c] = q8_score16(rows + (16 * c + n) * stride, L);
  transpose_rows4(acc);
}

}  // namespace bkv
