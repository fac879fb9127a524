// bkv_common.h - device helpers shared by the gfx950 KV-cache kernels: fp16 rounding, q8_0 block
// arithmetic, wave64 DPP reductions and cache addressing.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/bkv.h"

namespace bkv {

constexpr int kHd = 256;        // head_dim the kernels are specialised for
constexpr int kGqa = 4;         // query heads per KV head served from one K/V tile read
constexpr int kWave = 64;

// ------------------------------------------------------------------ fp16
// f32 -> binary16 bits, round to nearest even, with the reference packer's special cases
// (runtime_vk/shaders/f16_rne.glslh:24-55): any NaN -> sign|0x7E00. v_cvt_f16_f32 rounds to nearest
// even and keeps fp16 subnormals on gfx950, so only the NaN pattern needs the fix-up.
__device__ __forceinline__ uint32_t f32_to_f16_rne(float f) {
  const uint32_t hw = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
  const uint32_t x = __float_as_uint(f);
  const bool nan = (x & 0x7FFFFFFFu) > 0x7F800000u;
  return nan ? (((x >> 16) & 0x8000u) | 0x7E00u) : hw;
}

__device__ __forceinline__ float f16_to_f32(uint32_t h16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h16);
}

// value of f32 rounded through fp16 (RNE), as fp32
__device__ __forceinline__ float round_f16(float f) { return (float)(_Float16)f; }

// ------------------------------------------------------------------ q8_0 (attn_norm_rope2.comp:102-115)
__device__ __forceinline__ float q8_scale(float amax) { return amax > 1e-35f ? amax / 127.0f : 0.0f; }
__device__ __forceinline__ float q8_iscale(float amax) {
  const float d = q8_scale(amax);
  return d != 0.0f ? 1.0f / d : 0.0f;
}
template <bool RHAZ>
__device__ __forceinline__ uint32_t q8_byte(float x, float id) {
  const float t = x * id;
  float r = RHAZ ? roundf(t) : __builtin_rintf(t);
  r = (r != r) ? 0.0f : fminf(fmaxf(r, -127.0f), 127.0f);
  return (uint32_t)((int)r) & 0xFFu;
}

// sign-extended byte k (0..3) of a word, as float
__device__ __forceinline__ float sbyte(uint32_t w, int k) {
  return (float)(int)(int8_t)(uint8_t)(w >> (8 * k));
}

// ------------------------------------------------------------------ DPP reductions inside a row of 16
// quad_perm(1,0,3,2) = 0xB1, quad_perm(2,3,0,1) = 0x4E, row_half_mirror = 0x141, row_mirror = 0x140.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                               0xF, 0xF, false));
}
// sum over the 16 lanes of a DPP row; every lane of the row receives the total
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp<0xB1>(v);
  v += dpp<0x4E>(v);
  v += dpp<0x141>(v);
  v += dpp<0x140>(v);
  return v;
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp<0xB1>(v));
  v = fmaxf(v, dpp<0x4E>(v));
  v = fmaxf(v, dpp<0x141>(v));
  v = fmaxf(v, dpp<0x140>(v));
  return v;
}
// full-wave reductions (all 64 lanes receive the result)
__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
  v = row16_max(v);
  v = fmaxf(v, __shfl_xor(v, 16));
  v = fmaxf(v, __shfl_xor(v, 32));
  return v;
}

// ------------------------------------------------------------------ addressing
struct LayerView {
  const uint8_t *kd, *ks, *vd, *vs;   // this layer's arrays (scales may be null)
  const int32_t *bt;                  // this layer's block-table row, or null (contiguous)
  int page;                           // tokens per page (paged) or 0
  int64_t base;                       // key index 0 is position base (a window's first live key)
};

__device__ __forceinline__ int64_t slot_of(const LayerView &L, int64_t pos) {
  pos += L.base;
  if (L.page == 0) return pos;
  const int64_t pg = pos / L.page;
  return (int64_t)L.bt[pg] * L.page + (pos - pg * L.page);
}

// slot_of with the layout fixed at compile time (no branch between a row's index math and its
// loads); paged positions use 32-bit arithmetic (positions < 2^31)
template <bool PG>
__device__ __forceinline__ int64_t slot_t(const LayerView &L, int64_t pos) {
  if constexpr (!PG) {
    return pos + L.base;
  } else {
    const uint32_t p = (uint32_t)(pos + L.base), pg = p / (uint32_t)L.page;
    return (int64_t)L.bt[pg] * L.page + (int64_t)(p - pg * (uint32_t)L.page);
  }
}

// element oi = head*hd + d of an [nh][hd] output, in a gate array whose head rows are gs floats
// apart (hd: contiguous; 2*hd: the q/gate interleave of the engine's attn_q output)
__host__ __device__ __forceinline__ size_t gate_index(size_t oi, int gs) {
  return oi + (oi / kHd) * (size_t)(gs - kHd);
}

// bytes of one head row of the data array, per format
__host__ __device__ constexpr int row_bytes(int fmt) { return fmt == BKV_F16 ? kHd * 2 : kHd; }
// bytes of one head row of the scale array (q8_0 only)
constexpr int kScaleRowBytes = kHd / 32 * 2;   // 8 fp16 = 16 B

}  // namespace bkv

namespace bkv {

// exp of a float argument, correctly rounded to float: the value of (float)exp((double)x).
// Fast path: x = k ln2 + r (|r| <= ln2/2, ln2 split so that k*ln2_hi is exact), exp(r) by its
// Taylor polynomial to degree 11 in fp64 (truncation < 2^-50, rounding ~2^-52), scaled by 2^k and
// rounded once to float. When the fp64 value lies within 64 units of its last place of a float
// rounding boundary, or x is outside the float-normal range of the result, the library fp64 exp
// decides. Checked exhaustively on the host against (float)exp((double)x) for every float in
// [-104, 89]: no mismatch; 0.1% of those floats (nearly all outside (-87, 88)) take the library path.
__device__ __forceinline__ float exp_cr(float xf) {
  const double x = xf;
  if (!(x > -87.0 && x < 88.0)) return (float)exp(x);
  const double kd = rint(x * 0x1.71547652b82fep0);
  double r = fma(-kd, 0x1.62e42fee00000p-1, x);
  r = fma(-kd, 0x1.a39ef35793c76p-33, r);
  double p = 0x1.ae64567f544e4p-26;        // 1/11!
  p = fma(p, r, 0x1.27e4fb7789f5cp-22);    // 1/10!
  p = fma(p, r, 0x1.71de3a556c734p-19);
  p = fma(p, r, 0x1.a01a01a01a01ap-16);
  p = fma(p, r, 0x1.a01a01a01a01ap-13);
  p = fma(p, r, 0x1.6c16c16c16c17p-10);
  p = fma(p, r, 0x1.1111111111111p-7);
  p = fma(p, r, 0x1.5555555555555p-5);
  p = fma(p, r, 0x1.5555555555555p-3);
  p = fma(p, r, 0x1.0000000000000p-1);
  p = fma(p, r, 1.0);
  p = fma(p, r, 1.0);
  const double y = ldexp(p, (int)kd);
  const long long low = (long long)(__double_as_longlong(y) & 0x1FFFFFFFll) - 0x10000000ll;
  if (low >= -64 && low <= 64) return (float)exp(x);
  return (float)y;
}

// ------------------------------------------------------------------ workgroup scans (NT threads)
template <typename T>
__device__ __forceinline__ T wave_incl_scan(T v, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const T t = __shfl_up(v, o);
    if (lane >= o) v += t;
  }
  return v;
}
// exclusive prefix sum over the workgroup; *total receives the sum. sh: NT/64 scratch slots.
template <int NT, typename T>
__device__ __forceinline__ T block_excl_scan(T v, T *sh, T *total) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const T inc = wave_incl_scan(v, lane);
  if (lane == 63) sh[w] = inc;
  __syncthreads();
  T base = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < NT / 64; ++i) {
    if (i < w) base += sh[i];
    tot += sh[i];
  }
  __syncthreads();
  *total = tot;
  return base + inc - v;
}
template <int NT>
__device__ __forceinline__ float block_max(float v, float *sh) {
  v = wave_max(v);
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = sh[0];
#pragma unroll
  for (int i = 1; i < NT / 64; ++i) r = fmaxf(r, sh[i]);
  __syncthreads();
  return r;
}
template <int NT>
__device__ __forceinline__ double block_sum_f64(double v, double *sh) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  double r = 0.0;
#pragma unroll
  for (int i = 0; i < NT / 64; ++i) r += sh[i];
  __syncthreads();
  return r;
}

}  // namespace bkv

namespace bkv {
// K independent exclusive prefix sums over the workgroup at once; tot[k] receives the totals.
// sh: (NT/64)*K scratch slots.
template <int NT, int K, typename T>
__device__ __forceinline__ void block_excl_scan_k(const T (&v)[K], T (&ex)[K], T (&tot)[K], T *sh) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  T inc[K];
#pragma unroll
  for (int k = 0; k < K; ++k) inc[k] = wave_incl_scan(v[k], lane);
  if (lane == 63)
#pragma unroll
    for (int k = 0; k < K; ++k) sh[w * K + k] = inc[k];
  __syncthreads();
#pragma unroll
  for (int k = 0; k < K; ++k) {
    T base = 0, t = 0;
#pragma unroll
    for (int i = 0; i < NT / 64; ++i) {
      const T x = sh[i * K + k];
      if (i < w) base += x;
      t += x;
    }
    ex[k] = base + inc[k] - v[k];
    tot[k] = t;
  }
  __syncthreads();
}
}  // namespace bkv
