// bkv_norm_rope.hip - the reference's fused append front end (bkv_qk_norm_rope_append): per-head
// RMS norm, weight and rope of the projected Q and K, then K (and the raw V) quantised into the
// cache, Q returned as the fp32 rows the attention rounds to its fp16 operand.
//
// Arithmetic, in the reference's order (runtime_vk/attn_vk.h:102-122, the shader
// runtime_vk/shaders/attn_norm_rope2.comp:138-181):
//   ss = sum over d ascending of (x_d * x_d), each square rounded before it is added;
//   inv = 1 / sqrt(ss / hd + eps)  (correctly rounded division and square root);
//   n_d = (x_d * inv) * w_d;
//   inside the first nrot dims, pair p (p < nrot/2) with p + nrot/2: theta = base^(-2p/nrot) (the
//   exponent formed in fp32), a = pos * theta in fp32, y_p = lo*cos a - hi*sin a,
//   y_{p+nrot/2} = hi*cos a + lo*sin a, every product rounded; dims from nrot on pass through.
// pow, cos and sin are the correctly rounded fp32 values of the exact functions, formed as the
// fp64 library function rounded once to fp32 (the same contract as the softmax's exp). The
// reference's CPU mirror calls the C library's powf/cosf/sinf, which agree with these except where
// a C-library float result is not correctly rounded (one fp32 ulp).

#include "bkv_device.h"
#include "bkv_internal.h"

namespace bkv {

// one wave per row: grid (n_tok, nh + 2 nkv); rows [0, nh) are Q heads, [nh, nh + nkv) K heads,
// [nh + nkv, nh + 2 nkv) V heads
template <int KF, int VF>
__global__ __launch_bounds__(64) void norm_rope_append_kernel(NormRopeArgs a) {
  const int t = blockIdx.x, r = blockIdx.y, lane = threadIdx.x;
  const uint32_t pos = a.pos0 + (uint32_t)t;
  __shared__ __attribute__((aligned(16))) float s_x[kHd];
  __shared__ __attribute__((aligned(16))) float s_y[kHd];
  __shared__ float s_inv;
  const int64_t slot = slot_of(a.L, pos);
  if (r >= a.nh + a.nkv) {                 // V: raw into the cache
    const int h = r - a.nh - a.nkv;
    if (lane < 32) {
      uint8_t *dr = const_cast<uint8_t *>(a.L.vd) + (slot * a.nkv + h) * row_bytes(VF);
      uint8_t *sr = VF == BKV_Q8_0 ? const_cast<uint8_t *>(a.L.vs) + (slot * a.nkv + h) * kScaleRowBytes : nullptr;
      append_row<VF, false>(a.v_in + ((size_t)t * a.nkv + h) * kHd, dr, sr, lane);
    }
    return;
  }
  const bool is_q = r < a.nh;
  const int h = is_q ? r : r - a.nh;
  const float *x = is_q ? a.q_in + ((size_t)t * a.nh + h) * kHd : a.k_in + ((size_t)t * a.nkv + h) * kHd;
  const float *w = is_q ? a.qn_w : a.kn_w;
  const float4 xv = reinterpret_cast<const float4 *>(x)[lane];
  const float4 wv = reinterpret_cast<const float4 *>(w)[lane];
  // the squares, rounded, then one lane adds them in ascending d
  reinterpret_cast<float4 *>(s_y)[lane] = make_float4(xv.x * xv.x, xv.y * xv.y, xv.z * xv.z, xv.w * xv.w);
  __syncthreads();
  if (lane == 0) {
    float ss = 0.0f;
    for (int i = 0; i < kHd; ++i) ss = ss + s_y[i];
    s_inv = 1.0f / sqrtf(ss / (float)kHd + a.eps);
  }
  __syncthreads();
  const float inv = s_inv;
  const float4 n = make_float4((xv.x * inv) * wv.x, (xv.y * inv) * wv.y, (xv.z * inv) * wv.z, (xv.w * inv) * wv.w);
  reinterpret_cast<float4 *>(s_x)[lane] = n;
  reinterpret_cast<float4 *>(s_y)[lane] = n;
  __syncthreads();
  const int half = a.nrot / 2;
  for (int p = lane; p < half; p += 64) {
    const float ex = -2.0f * (float)p / (float)a.nrot;
    const float th = (float)pow((double)a.freq_base, (double)ex);
    const float ang = (float)pos * th;
    const float cs = (float)cos((double)ang), sn = (float)sin((double)ang);
    const float lo = s_x[p], hi = s_x[p + half];
    const float l1 = lo * cs, l2 = hi * sn, h1 = hi * cs, h2 = lo * sn;
    s_y[p] = l1 - l2;
    s_y[p + half] = h1 + h2;
  }
  __syncthreads();
  if (is_q) {
    reinterpret_cast<float4 *>(a.q_out + ((size_t)t * a.nh + h) * kHd)[lane] = reinterpret_cast<const float4 *>(s_y)[lane];
  } else if (lane < 32) {
    uint8_t *dr = const_cast<uint8_t *>(a.L.kd) + (slot * a.nkv + h) * row_bytes(KF);
    uint8_t *sr = KF == BKV_Q8_0 ? const_cast<uint8_t *>(a.L.ks) + (slot * a.nkv + h) * kScaleRowBytes : nullptr;
    append_row<KF, false>(s_y, dr, sr, lane);
  }
}

hipError_t launch_norm_rope_append(const NormRopeArgs &a, int kf, int vf, int n_tok, hipStream_t st) {
  BKV_FMT_SWITCH(kf, vf, hipLaunchKernelGGL((norm_rope_append_kernel<KF_, VF_>),
                                            dim3(n_tok, a.nh + 2 * a.nkv), dim3(64), 0, st, a));
  return hipGetLastError();
}

}  // namespace bkv
