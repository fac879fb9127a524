// bkv_pv8.h - the speculative PV of a q8_0 V tile on the int8 matrix cores.
//
// out[h][d] = sum_k p_k,h * s_k,b(d) * v_k,d over a wave's keys, where p is an fp16 probability,
// s the key's fp16 scale of the 32-dim block b(d) and v its int8 byte (attn_vk.h:200-212 for the
// product; the order of the PV sum is not part of the contract). Every product x = p * s is exact in
// fp32 (two 11-bit significands). For head h the wave takes one power of two 2^sig(h) such that
// every x * 2^sig(h) < 2^30 (from the wave's largest p of the head and its largest scale) and
// rounds X = x * 2^sig to an integer Q < 2^30 (an error below 2^-31 of the largest product, far
// under the fp32 accumulation error of a serial sum). Q splits into four balanced base-256 digits
// c_i in [-128, 127] (the bytes of Q + 0x80808080, each minus 128), and one
// v_mfma_i32_16x16x32_i8 per 32 keys and 16 dims gives, for A row 4 h + i (head h, digit i) and
// dim column n, the exact integer o_i = sum_k c_i(k) * v_k,d. o_0 + 256 o_1 + 2^16 o_2 + 2^24 o_3 is
// exact in fp64; scaled by 2^-sig it is the head's sum over the keys, rounded once to fp32.
//
// The V rows sit in LDS (rows of kPv8Stride bytes, 256 data bytes each); the B operand of dim tile t
// (dims 16 t .. + 15) over 32 keys is one ds_read_b64_tr_b8: within each 16 lanes, lanes 2 j and
// 2 j + 1 point at dims 16 t .. + 7 and 16 t + 8 .. + 15 of key j of the lane group's 8 keys, and
// lane n then receives byte n of dim 16 t + n over those 8 keys.
#pragma once

#include "bkv_q8dot.h"

namespace bkv {

typedef int v2i_t __attribute__((ext_vector_type(2)));
// (vector types for rows that go into LDS: a copy of HIP's uint4 struct is a memcpy, which keeps
// an array of them in scratch memory)
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kPv8Stride = 272;          // LDS bytes per staged V row (256 + 16: 2-way bank spread)
constexpr int kPv8Rows = 32;             // keys per staging round (one MFMA k-extent)

// lane-constant byte selectors of the quad transpose in pv8_prep (lane % 4 = the A row's digit)
struct Pv8Sel {
  uint32_t k, s, x, y, lo, hi;
};

__device__ __forceinline__ Pv8Sel pv8_sel() {
  const int r = threadIdx.x & 3, p = r >> 1, q = r & 1, pp = 1 - p;
  Pv8Sel z;
  // v_perm_b32(S0, S1, sel): byte j of the result = byte sel_j of {S0:S1} (0..3: S1, 4..7: S0)
  z.k = (uint32_t)(4 + 2 * p) | (uint32_t)(5 + 2 * p) << 8 | (uint32_t)(2 * p) << 16 | (uint32_t)(2 * p + 1) << 24;
  z.s = (uint32_t)(4 + 2 * pp) | (uint32_t)(5 + 2 * pp) << 8 | (uint32_t)(2 * pp) << 16 | (uint32_t)(2 * pp + 1) << 24;
  // {K : R} -> positions q, 2 + q of K (bytes 4 + ..) and of R (bytes 0 + ..)
  z.x = (uint32_t)(4 + q) | (uint32_t)(6 + q) << 8 | (uint32_t)q << 16 | (uint32_t)(2 + q) << 24;
  z.y = (uint32_t)(5 - q) | (uint32_t)(7 - q) << 8 | (uint32_t)(1 - q) << 16 | (uint32_t)(3 - q) << 24;
  // {X : Z}: X holds the key pairs r, r ^ 2 and Z the pairs r ^ 1, r ^ 3 (two bytes each)
  const uint32_t X0 = 4, X2 = 6, Z0 = 0, Z2 = 2;
  uint32_t lo0, lo1, hi0, hi1;   // the first / second two-byte pair of each half
  switch (r) {
    case 0: lo0 = X0; lo1 = Z0; hi0 = X2; hi1 = Z2; break;
    case 1: lo0 = Z0; lo1 = X0; hi0 = Z2; hi1 = X2; break;
    case 2: lo0 = X2; lo1 = Z2; hi0 = X0; hi1 = Z0; break;
    default: lo0 = Z2; lo1 = X2; hi0 = Z0; hi1 = X0; break;
  }
  z.lo = lo0 | (lo0 + 1) << 8 | lo1 << 16 | (lo1 + 1) << 24;
  z.hi = hi0 | (hi0 + 1) << 8 | hi1 << 16 | (hi1 + 1) << 24;
  return z;
}

// The A operands of one round (32 keys) for the 8 blocks. Lane l: row l % 16 = (head h, digit
// i = l % 4), keys 8 (l / 16) .. + 7 of the round. The lane computes the digits of its quad's keys
// 2 i, 2 i + 1 (pa, pb: their p of head h times 2^sig(h); sa, sb: their scale rows, fp16 x 8) and
// the quad exchanges bytes so that every lane ends with digit i of all 8 keys.
// (B0, NB: blocks B0 .. B0 + NB - 1 only, into A[0 .. NB - 1])
template <int B0 = 0, int NB = 8>
__device__ __forceinline__ void pv8_prep(float pa, float pb, const uint4 &sa, const uint4 &sb, const Pv8Sel &z,
                                         long (&A)[NB]) {
  const uint32_t wa[4] = {sa.x, sa.y, sa.z, sa.w}, wb[4] = {sb.x, sb.y, sb.z, sb.w};
#pragma unroll
  for (int b = B0; b < B0 + NB; ++b) {
    // x = p * 2^sig * s (v_fma_mix_f32 with + 0: the product is exact), below 2^30; Q = x rounded
    // to an integer (half up: v_cvt_rpi_i32_f32)
    const int sh = 16 * (b & 1);
    const float xa = __builtin_fmaf(pa, (float)__builtin_bit_cast(_Float16, (uint16_t)(wa[b >> 1] >> sh)), 0.0f);
    const float xb = __builtin_fmaf(pb, (float)__builtin_bit_cast(_Float16, (uint16_t)(wb[b >> 1] >> sh)), 0.0f);
    int qa, qb;
    asm("v_cvt_rpi_i32_f32 %0, %1" : "=v"(qa) : "v"(xa));
    asm("v_cvt_rpi_i32_f32 %0, %1" : "=v"(qb) : "v"(xb));
    const uint32_t ua = (uint32_t)qa + 0x80808080u;
    const uint32_t ub = (uint32_t)qb + 0x80808080u;
    const uint32_t K = __builtin_amdgcn_perm(ua, ub, z.k);
    const uint32_t S = __builtin_amdgcn_perm(ua, ub, z.s);
    const uint32_t R = (uint32_t)__builtin_amdgcn_mov_dpp((int)S, 0x4E, 0xF, 0xF, false);   // quad_perm 2,3,0,1
    const uint32_t X = __builtin_amdgcn_perm(K, R, z.x);
    const uint32_t Y = __builtin_amdgcn_perm(K, R, z.y);
    const uint32_t Zv = (uint32_t)__builtin_amdgcn_mov_dpp((int)Y, 0xB1, 0xF, 0xF, false);  // quad_perm 1,0,3,2
    const uint32_t lo = __builtin_amdgcn_perm(X, Zv, z.lo) ^ 0x80808080u;
    const uint32_t hi = __builtin_amdgcn_perm(X, Zv, z.hi) ^ 0x80808080u;
    A[b - B0] = (long)((unsigned long)lo | ((unsigned long)hi << 32));
  }
}

// One round: acc[t] (+)= A[t / 2] x B(t) for the 16 dim tiles (FIRST: acc starts at zero); rows:
// LDS address of the round's first staged row (rows kPv8Stride bytes apart).
template <bool FIRST>
__device__ __forceinline__ void pv8_round(uint32_t rows, const long (&A)[8], v4i_t (&acc)[16]) {
  const int lane = threadIdx.x & 63;
  const uint32_t base = rows + (uint32_t)(((lane >> 4) * 8 + ((lane & 15) >> 1)) * kPv8Stride + 8 * (lane & 1));
#pragma unroll
  for (int t = 0; t < 16; ++t) {
    const v2i_t bv = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
        (__attribute__((address_space(3))) v2i_t *)(uintptr_t)(base + 16u * t));
    const long b = (long)((unsigned long)(uint32_t)bv.x | ((unsigned long)(uint32_t)bv.y << 32));
    acc[t] = __builtin_amdgcn_mfma_i32_16x16x32_i8(A[t >> 1], b, FIRST ? v4i_t{0, 0, 0, 0} : acc[t], 0, 0, 0);
  }
}

// ---------------------------------------------------------------- the blocked region layout
// A wave's 64 keys of V in one 17 KiB LDS region (a K tile's bytes, at a multiple of 1 KiB): block i
// (keys 4 i .. 4 i + 3) at 1024 i, its 16-byte chunk c of row r at 64 (c ^ (i & 3)) + 16 r (the XOR
// spreads the 32 rows one ds_read_b64_tr_b8 reads over the banks), then the 64 keys' scale rows
// (16 B each) at 16384. Direct-to-LDS loads fill it (one 1 KiB block per load), or the V registers.
constexpr int kPv8Region = 17408;
constexpr int kPv8Scales = 16384;

// direct-to-LDS loads of the region: rows(k) / scl(k): global addresses of key k's 256 data bytes
// and 16 scale bytes (k = 0 .. 63, the caller clamps keys past its range); 17 loads (inline asm: the
// caller waits for them with an explicit vmcnt)
template <typename RowF, typename SclF>
__device__ __forceinline__ void pv8_dma_region(uint32_t region, RowF rows, SclF scl) {
  const int lane = threadIdx.x & 63, r = lane & 3, sl = lane >> 2;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const uint8_t *src = rows(4 * i + r) + 16 * (sl ^ (i & 3));
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(region + 1024u * i)
                 : "memory", "m0");
  }
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(scl(lane)), "s"(region + (uint32_t)kPv8Scales)
               : "memory", "m0");
}

// the region from registers: vd[i] = chunk lane % 16 of key 4 i + lane / 16, vs[i] = that key's
// scale word (lane % 16) / 4
__device__ __forceinline__ void pv8_store_region(char *region, const u32x4 (&vd)[16], const uint32_t (&vs)[16]) {
  const int lane = threadIdx.x & 63, c = lane & 15, r = lane >> 4;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    *reinterpret_cast<u32x4 *>(region + 1024 * i + 64 * (c ^ (i & 3)) + 16 * r) = vd[i];
    if ((c & 3) == 0) *reinterpret_cast<uint32_t *>(region + kPv8Scales + 16 * (4 * i + r) + 4 * (c >> 2)) = vs[i];
  }
}

// One round over the region's keys 32 rd .. 32 rd + 31 (see pv8_round), dim tiles T0 .. T0 + NT - 1
// into acc[0 .. NT - 1] with A[i] the operand of block T0 / 2 + i
template <bool FIRST, int T0 = 0, int NT = 16>
__device__ __forceinline__ void pv8_round_region(uint32_t region, int rd, const long (&A)[NT / 2], v4i_t (&acc)[NT]) {
  const int lane = threadIdx.x & 63, j = (lane & 15) >> 1;
  const int b = 8 * rd + 2 * (lane >> 4) + (j >> 2);            // the block of the lane's key 8 (l/16) + j
  const uint32_t a0 = region + (uint32_t)(1024 * b + 16 * (j & 3) + 8 * (lane & 1) + 64 * (b & 3));
#pragma unroll
  for (int t = T0; t < T0 + NT; ++t) {
    const v2i_t bv = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
        (__attribute__((address_space(3))) v2i_t *)(uintptr_t)(a0 ^ (uint32_t)(64 * t)));
    const long bb = (long)((unsigned long)(uint32_t)bv.x | ((unsigned long)(uint32_t)bv.y << 32));
    acc[t - T0] = __builtin_amdgcn_mfma_i32_16x16x32_i8(A[(t - T0) >> 1], bb, FIRST ? v4i_t{0, 0, 0, 0} : acc[t - T0], 0, 0, 0);
  }
}

// The sums of tile t for the lane's head (lane / 16) and dim 16 t + lane % 16, scaled by 2^-sig.
__device__ __forceinline__ float pv8_value(const v4i_t &d, int nsig) {
  const int lo = d[0] + (int)((uint32_t)d[1] << 8);
  const int hi = d[2] + (int)((uint32_t)d[3] << 8);
  const double x = __builtin_fma((double)hi, 65536.0, (double)lo);   // exact: an integer below 2^53
  return (float)__builtin_ldexp(x, nsig);
}

// the exponent of an fp16 value's leading bit (subnormals and zero: -15, an upper bound)
__device__ __forceinline__ int f16_exp_bound(uint32_t bits) { return (int)((bits >> 10) & 0x1Fu) - 15; }

// the largest of the 8 fp16 values >= 0 of a scale row (as fp16 bits: their order is the values')
__device__ __forceinline__ uint32_t f16_row_max(const uint4 &r) {
  typedef unsigned short us2 __attribute__((ext_vector_type(2)));
  const us2 m = __builtin_elementwise_max(__builtin_elementwise_max(__builtin_bit_cast(us2, r.x), __builtin_bit_cast(us2, r.y)),
                                          __builtin_elementwise_max(__builtin_bit_cast(us2, r.z), __builtin_bit_cast(us2, r.w)));
  return max((uint32_t)m.x, (uint32_t)m.y);
}

}  // namespace bkv
