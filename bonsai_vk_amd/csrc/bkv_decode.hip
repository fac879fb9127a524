// bkv_decode.hip - gfx950 kernels of the decode path: q8_0/fp16 append (quantise on write),
// split-K QK + partition statistics, global-softmax PV over LDS-staged probabilities, and the
// partition merge with the optional sigmoid gate.
//
// Per layer and decode token the work is three launches:
//   qk  grid (nch_qk, nkv): one workgroup per (key partition, KV head). Each K row is read once with
//       128-bit loads (16 lanes per q8_0 row, 32 per fp16 row), dequantised in registers and dotted
//       with the 4 query heads of the group. Scores go to the workspace, and each partition's
//       (max, sum exp) pair to the statistics array. The fused variant also appends the new token.
//   pv  grid (nch_pv, nkv): merges the statistics into the global max and sum of each head, forms
//       p = exp(s*scale - max)/sum rounded to fp16 exactly as the reference does before its PV
//       matmul, and accumulates p*V for the 4 heads from one V tile read.
//   red grid (nh): sums the partition partials and applies the gate.
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

template <int KF, int VF, bool RHAZ>
__global__ __launch_bounds__(64) void append_kernel(AppendArgs a) {
  const int t = blockIdx.x, g = blockIdx.y;
  append_token<KF, VF, RHAZ>(a, (int64_t)a.pos + t, t, g, threadIdx.x);
}

// ------------------------------------------------------------------ QK + partition statistics
template <int KF>
struct KRow {
  static constexpr int LPR = KF == BKV_Q8_0 ? 16 : 32;   // lanes per head row
  static constexpr int EPL = kHd / LPR;                  // elements per lane (16 or 8)
  static constexpr int KPW = kWave / LPR;                // rows per wave per step (4 or 2)
};

// partial dot of one lane's EPL elements of a K row with the 4 query heads
template <int KF>
__device__ __forceinline__ void k_partial(const uint4 w, float ksc, const float (&q)[kGqa][KRow<KF>::EPL],
                                          float (&part)[kGqa]) {
  const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int h = 0; h < kGqa; ++h) part[h] = 0.0f;
  if (KF == BKV_Q8_0) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float x = sbyte(ww[i >> 2], i & 3);
#pragma unroll
      for (int h = 0; h < kGqa; ++h) part[h] = fmaf(q[h][i], x, part[h]);
    }
#pragma unroll
    for (int h = 0; h < kGqa; ++h) part[h] *= ksc;
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float x = f16_to_f32((ww[i >> 1] >> ((i & 1) * 16)) & 0xFFFFu);
#pragma unroll
      for (int h = 0; h < kGqa; ++h) part[h] = fmaf(q[h][i], x, part[h]);
    }
  }
}

template <int KF, int VF, bool FUSE, bool RHAZ>
__global__ __launch_bounds__(256) void qk_kernel(QkArgs a) {
  using R = KRow<KF>;
  __shared__ float s_sc[kGqa][kMaxChunk];
  const int c = blockIdx.x, g = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane % R::LPR, kk = lane / R::LPR;
  const int64_t j0 = (int64_t)c * a.chunk;
  const int64_t j1 = min(j0 + (int64_t)a.chunk, (int64_t)a.nfill);
  const int n = (int)(j1 - j0);

  if (FUSE) {
    if (wave == 0 && (int64_t)a.ap.pos >= j0 && (int64_t)a.ap.pos < j1)
      append_token<KF, VF, RHAZ>(a.ap, a.ap.pos, 0, g, lane);
    __syncthreads();
  }

  // the lane's slice of the 4 query rows, rounded to fp16 (the reference's Q16 operand)
  float q[kGqa][R::EPL];
#pragma unroll
  for (int h = 0; h < kGqa; ++h) {
    const float4 *qp = reinterpret_cast<const float4 *>(a.q + (size_t)(g * kGqa + h) * kHd + sub * R::EPL);
#pragma unroll
    for (int i = 0; i < R::EPL / 4; ++i) {
      const float4 t = qp[i];
      q[h][4 * i] = round_f16(t.x); q[h][4 * i + 1] = round_f16(t.y);
      q[h][4 * i + 2] = round_f16(t.z); q[h][4 * i + 3] = round_f16(t.w);
    }
  }

  const LayerView &L = a.L;
  constexpr int RB = row_bytes(KF);
  for (int jb = wave * R::KPW; jb < n; jb += 4 * R::KPW) {
    const int jl = jb + kk;
    const bool valid = jl < n;
    const int64_t slot = slot_of(L, j0 + (valid ? jl : 0));
    const uint4 w = *reinterpret_cast<const uint4 *>(L.kd + (slot * a.nkv + g) * RB + sub * 16);
    float ksc = 1.0f;
    if (KF == BKV_Q8_0) {
      const uint32_t sw = *reinterpret_cast<const uint32_t *>(L.ks + (slot * a.nkv + g) * kScaleRowBytes +
                                                              (sub >> 2) * 4);
      ksc = f16_to_f32(((sub >> 1) & 1) ? (sw >> 16) : (sw & 0xFFFFu));
    }
    float part[kGqa];
    k_partial<KF>(w, ksc, q, part);
#pragma unroll
    for (int h = 0; h < kGqa; ++h) {
      float v = row16_sum(part[h]);
      if (R::LPR == 32) v += __shfl_xor(v, 16);
      part[h] = v;
    }
    if (valid && sub < kGqa) {
      const float v = sub == 0 ? part[0] : sub == 1 ? part[1] : sub == 2 ? part[2] : part[3];
      s_sc[sub][jl] = v;
    }
  }
  __syncthreads();

  // wave h: scores of head h to the workspace, and the partition's (max, sum exp)
  {
    const int h = wave;
    float *dst = a.score + (size_t)(g * kGqa + h) * a.ld + j0;
    float m = -INFINITY;
    for (int t = lane; t < n; t += kWave) {
      const float s = s_sc[h][t];
      dst[t] = s;
      m = fmaxf(m, s * a.scale);
    }
    m = wave_max(m);
    float l = 0.0f;
    for (int t = lane; t < n; t += kWave) l += expf(s_sc[h][t] * a.scale - m);
    l = wave_sum(l);
    if (lane == 0) a.stats[(size_t)(g * kGqa + h) * a.nch_qk + c] = make_float2(m, l);
  }
}

// ------------------------------------------------------------------ PV over globally normalised P16
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

template <int VF>
__global__ __launch_bounds__(256) void pv_kernel(PvArgs a) {
  using R = KRow<VF>;
  __shared__ float s_p[kGqa][kMaxChunk];
  __shared__ float s_red[4][kGqa][kHd];
  __shared__ float s_ms[kGqa][2];
  const int c = blockIdx.x, g = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int sub = lane % R::LPR, kk = lane / R::LPR;
  const int64_t j0 = (int64_t)c * a.chunk;
  const int64_t j1 = min(j0 + (int64_t)a.chunk, (int64_t)a.nfill);
  const int n = (int)(j1 - j0);

  // global max and sum of head (g*4 + wave) from the QK partition statistics
  {
    const float2 *st = a.stats + (size_t)(g * kGqa + wave) * a.nch_qk;
    float m = -INFINITY;
    for (int i = lane; i < a.nch_qk; i += kWave) m = fmaxf(m, st[i].x);
    m = wave_max(m);
    float l = 0.0f;
    for (int i = lane; i < a.nch_qk; i += kWave) {
      const float2 v = st[i];
      l += v.y * expf(v.x - m);
    }
    l = wave_sum(l);
    if (lane == 0) { s_ms[wave][0] = m; s_ms[wave][1] = l; }
  }
  __syncthreads();
  // p16 of every key of the partition (attn_vk.h:175-189 then the fp16 operand cast, :295-296)
  for (int t = tid; t < n; t += 256) {
#pragma unroll
    for (int h = 0; h < kGqa; ++h) {
      const float s = a.score[(size_t)(g * kGqa + h) * a.ld + j0 + t];
      const float e = expf(s * a.scale - s_ms[h][0]);
      s_p[h][t] = round_f16(e / s_ms[h][1]);
    }
  }
  __syncthreads();

  float acc[kGqa][R::EPL];
#pragma unroll
  for (int h = 0; h < kGqa; ++h)
#pragma unroll
    for (int i = 0; i < R::EPL; ++i) acc[h][i] = 0.0f;

  const LayerView &L = a.L;
  constexpr int RB = row_bytes(VF);
  for (int jb = wave * R::KPW; jb < n; jb += 4 * R::KPW) {
    const int jl = jb + kk;
    const bool valid = jl < n;
    const int64_t slot = slot_of(L, j0 + (valid ? jl : 0));
    const uint4 w = *reinterpret_cast<const uint4 *>(L.vd + (slot * a.nkv + g) * RB + sub * 16);
    float vsc = 1.0f;
    if (VF == BKV_Q8_0) {
      const uint32_t sw = *reinterpret_cast<const uint32_t *>(L.vs + (slot * a.nkv + g) * kScaleRowBytes +
                                                              (sub >> 2) * 4);
      vsc = f16_to_f32(((sub >> 1) & 1) ? (sw >> 16) : (sw & 0xFFFFu));
    }
    float p[kGqa];
#pragma unroll
    for (int h = 0; h < kGqa; ++h) p[h] = valid ? s_p[h][jl] : 0.0f;
    v_accum<VF>(w, vsc, p, acc);
  }
  // reduce the row groups of the wave (lanes sub, sub+LPR, ...)
#pragma unroll
  for (int h = 0; h < kGqa; ++h)
#pragma unroll
    for (int i = 0; i < R::EPL; ++i) {
      float v = acc[h][i];
      if (R::LPR == 16) v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 32);
      acc[h][i] = v;
    }
  if (kk == 0) {
#pragma unroll
    for (int h = 0; h < kGqa; ++h)
#pragma unroll
      for (int i = 0; i < R::EPL; ++i) s_red[wave][h][sub * R::EPL + i] = acc[h][i];
  }
  __syncthreads();
#pragma unroll
  for (int h = 0; h < kGqa; ++h) {
    const float v = s_red[0][h][tid] + s_red[1][h][tid] + s_red[2][h][tid] + s_red[3][h][tid];
    a.part[((size_t)c * a.nh + g * kGqa + h) * kHd + tid] = v;
  }
}

// ------------------------------------------------------------------ partition merge + gate
__global__ __launch_bounds__(256) void reduce_kernel(RedArgs a) {
  const int h = blockIdx.x, d = threadIdx.x;
  float acc = 0.0f;
  for (int c = 0; c < a.nch_pv; ++c) acc += a.part[((size_t)c * a.nh + h) * kHd + d];
  const size_t o = (size_t)h * kHd + d;
  a.out[o] = acc;
  if (a.gate) a.out_gated[o] = acc * (1.0f / (1.0f + expf(-a.gate[o])));
}

// ------------------------------------------------------------------ launchers
#define BKV_FMT_SWITCH(KF, VF, ...)                                                    \
  do {                                                                                \
    if ((KF) == BKV_Q8_0 && (VF) == BKV_Q8_0) { constexpr int KF_ = 1, VF_ = 1; __VA_ARGS__; } \
    else if ((KF) == BKV_Q8_0) { constexpr int KF_ = 1, VF_ = 0; __VA_ARGS__; }       \
    else if ((VF) == BKV_Q8_0) { constexpr int KF_ = 0, VF_ = 1; __VA_ARGS__; }       \
    else { constexpr int KF_ = 0, VF_ = 0; __VA_ARGS__; }                             \
  } while (0)

hipError_t launch_append(const AppendArgs &a, int kf, int vf, int n_tok, hipStream_t st) {
  BKV_FMT_SWITCH(kf, vf, hipLaunchKernelGGL((append_kernel<KF_, VF_, false>), dim3(n_tok, a.nkv),
                                            dim3(64), 0, st, a));
  return hipGetLastError();
}

hipError_t launch_decode(const QkArgs &qa, const PvArgs &pa, const RedArgs &ra, int kf, int vf,
                         bool fuse, hipStream_t st) {
  BKV_FMT_SWITCH(kf, vf, {
    if (fuse)
      hipLaunchKernelGGL((qk_kernel<KF_, VF_, true, false>), dim3(qa.nch_qk, qa.nkv), dim3(256), 0, st, qa);
    else
      hipLaunchKernelGGL((qk_kernel<KF_, VF_, false, false>), dim3(qa.nch_qk, qa.nkv), dim3(256), 0, st, qa);
    hipLaunchKernelGGL((pv_kernel<VF_>), dim3(pa.nch_pv, pa.nkv), dim3(256), 0, st, pa);
  });
  hipLaunchKernelGGL(reduce_kernel, dim3(ra.nh), dim3(256), 0, st, ra);
  return hipGetLastError();
}

}  // namespace bkv
