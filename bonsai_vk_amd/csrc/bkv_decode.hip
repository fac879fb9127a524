// bkv_decode.hip - gfx950 kernels of the decode path: q8_0/fp16 append (quantise on write), QK in
// the reference's accumulation order, the exact serial softmax sum, PV over fp16 probabilities and
// the partition merge with the optional sigmoid gate.
//
// Per layer and decode token the work is four launches:
//   qk    grid (nch_qk, nkv): K tile in LDS, one accumulation chain per (key, head); scores and
//         per-partition (max, sum exp). The fused variant appends the new token first.
//   e     grid (nch_e, nh): e_j = exp(s_j*scale - max) and its exact placement on the serial sum;
//         the last workgroup of each head walks the chunk records to the exact fp32 sum.
//   pv    grid (nch_pv, nkv): p16 = f16(e/sum), p16*V for the 4 heads of a group per V tile read.
//   merge grid (nh, 4): sums the PV partials, applies the gate.
#include "bkv_common.h"
#include "bkv_device.h"
#include "bkv_internal.h"
#include "bkv_q8dot.h"

namespace bkv {

template <int KF, int VF, bool RHAZ>
__global__ __launch_bounds__(64) void append_kernel(AppendArgs a) {
  const int t = blockIdx.x, g = blockIdx.y;
  append_token<KF, VF, RHAZ>(a, (int64_t)a.pos + t, t, g, threadIdx.x);
}

template <int KF>
struct QkTile {
  static constexpr int DPR = KF == BKV_Q8_0 ? 16 : 32;      // data uint4 per K row
  static constexpr int UPR = DPR + 1;                       // + scales / pad (bank spread)
  static constexpr int NT = KF == BKV_Q8_0 ? 256 : 128;     // threads = keys per workgroup
  static constexpr int KEYS = NT;
};

template <int KF, int VF, bool FUSE, bool RHAZ>
__global__ __launch_bounds__(QkTile<KF>::NT) void qk_kernel(QkArgs a) {
  using T = QkTile<KF>;
  constexpr int NT = T::NT;
  __shared__ uint4 tile[T::KEYS * T::UPR];
  __shared__ float red[NT / 64 + 1];
  const int c = blockIdx.x, g = blockIdx.y, tid = threadIdx.x;
  const int64_t j0 = (int64_t)c * T::KEYS;
  const int n = (int)min((int64_t)T::KEYS, (int64_t)a.nfill - j0);
  const LayerView &L = a.L;

  if (c == 0 && g == 0 && tid < a.nkv * kGqa) a.counters[tid * kCounterStride] = 0u;
  if (FUSE) {
    if (tid < 64 && (int64_t)a.ap.pos >= j0 && (int64_t)a.ap.pos < j0 + n)
      append_token<KF, VF, RHAZ>(a.ap, a.ap.pos, 0, g, tid);
    __syncthreads();
  }
  constexpr int RB = row_bytes(KF);
  stage_rows<NT, T::KEYS, T::DPR, T::UPR>(tile, L.kd, RB, L, a.nkv, g, j0, n);
  if (KF == BKV_Q8_0) stage_rows<NT, T::KEYS, 1, T::UPR>(tile + 16, L.ks, kScaleRowBytes, L, a.nkv, g, j0, n);
  const float *qg = a.q + (size_t)g * kGqa * a.qs;
  float acc[kGqa];
  if constexpr (KF == BKV_Q8_0) {
    // the int8 matrix cores on the q rows' digits (bkv_q8dot.h)
    __shared__ __attribute__((aligned(16))) int8_t s_lim[kLimBytes];
    __shared__ int s_lt[kGqa];
    __shared__ unsigned s_wide;
    if (tid == 0) s_wide = 0u;
    __syncthreads();
    q8lim_build(qg, a.qs, s_lim, s_lt, &s_wide, tid, NT);
    __syncthreads();                           // the digits and the K tile
    if (s_wide == 0u) {
      Q8Lim qlim;
      q8lim_load(s_lim, s_lt, qlim);
      q8_score64(tile + (tid & ~63) * T::UPR, T::UPR, qlim, acc);
    } else {
      q8_score_key_slow(tile + tid * T::UPR, qg, a.qs, acc);
    }
  } else {
    float qv[kGqa][kHd / 16];
    load_q16_rows(qg, qv, a.qs);
    __syncthreads();
    asm volatile("s_nop 4");      // DPP source registers written above: VALU-write -> DPP-read gap
    qk_row_dot<KF>(tile + tid * T::UPR, qv, acc);
  }

  // scores, and per head the partition's (max, sum exp) used to place each key on the running sum
  const bool valid = tid < n;
#pragma unroll
  for (int h = 0; h < kGqa; ++h) {
    float m = -INFINITY;
    if (valid) {
      a.score[(size_t)(g * kGqa + h) * a.ld + j0 + tid] = acc[h];
      m = acc[h] * a.scale;
    }
    m = block_max<NT>(m, red);
    float l = valid ? __expf(acc[h] * a.scale - m) : 0.0f;
    l = wave_sum(l);
    if ((tid & 63) == 0) red[tid >> 6] = l;
    __syncthreads();
    if (tid == 0) {
      float t = 0.0f;
      for (int i = 0; i < NT / 64; ++i) t += red[i];
      a.stats[(size_t)(g * kGqa + h) * a.nch + c] = make_float2(m, t);
    }
    __syncthreads();
  }
}

#ifdef BKV_EXPERIMENT_TS
#define TS(i) do { if (tid == 0) a.dbg[h * 8 + (i)] = wall_clock64(); } while (0)
#else
#define TS(i) do { } while (0)
#endif
__global__ __launch_bounds__(256) void e_kernel(EArgs a) {
  constexpr int NT = 256, EPT = kE2Chunk / NT;       // 4 keys per thread
  __shared__ double shd[NT / 64];
  __shared__ long long shl[NT / 64];
  __shared__ int shi[NT / 64];
  __shared__ float shf[NT / 64 + 1];
  __shared__ int s_bin[kE2Chunk];
  __shared__ unsigned s_last;
  // walker staging (structure of arrays)
  __shared__ long long w_ibase[kWalkBatch];
  __shared__ int w_blast[kWalkBatch], w_cnt[kWalkBatch], w_off[kWalkBatch + 1];
  __shared__ long long w_i[kWalkBatch * kMaxSpecial];
  __shared__ long long w_k[kWalkBatch * kMaxSpecial];
  __shared__ float w_e[kWalkBatch * kMaxSpecial];
  __shared__ int w_b[kWalkBatch * kMaxSpecial];
  __shared__ int w_du[kWalkBatch * kMaxSpecial];
  const int c = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
  const int64_t j0 = (int64_t)c * kE2Chunk;
  const int n = (int)min((int64_t)kE2Chunk, (int64_t)a.nfill - j0);
  const float2 *st = a.stats + (size_t)h * a.nch_qk;
#ifdef BKV_EXPERIMENT_TS
  if (tid == 0 && c == 0) a.dbg[h * 8 + 5] = wall_clock64();
#endif

  float m = -INFINITY;
  for (int i = tid; i < a.nch_qk; i += NT) m = fmaxf(m, st[i].x);
  m = block_max<NT>(m, shf);
  const int cq = (int)(j0 / a.qk_chunk);
  double p = 0.0;
  for (int i = tid; i < cq; i += NT) p += (double)st[i].y * exp((double)st[i].x - (double)m);
  p = block_sum_f64<NT>(p, shd);

  // e for this thread's EPT consecutive keys
  float e[EPT];
  double loc = 0.0;
#pragma unroll
  for (int i = 0; i < EPT; ++i) {
    const int t = EPT * tid + i;
    e[i] = 0.0f;
    if (t < n) {
      const float v = a.score[(size_t)h * a.ld + j0 + t] * a.scale;
      e[i] = exp_cr(v - m);
      st_agent(&a.e[(size_t)h * a.ld + j0 + t], e[i]);
    }
    loc += (double)e[i];
  }
  double tot_d;
  double ab = p + block_excl_scan<NT, double>(loc, shd, &tot_d);
  bool sp[EPT];
  long long inc = 0, incs[EPT];
  int nsp_t = 0;
#pragma unroll
  for (int i = 0; i < EPT; ++i) {
    const int t = EPT * tid + i;
    int bin = kNoBinade;
    long long d = 0;
    sp[i] = false;
    if (t < n) classify(ab, ab + (double)e[i], e[i], sp[i], bin, d);
    ab += (double)e[i];
    s_bin[t] = (t < n && !sp[i]) ? bin : kNoBinade;
    incs[i] = d;
    inc += d;
    nsp_t += sp[i] ? 1 : 0;
  }
  long long tot_l;
  long long ipre = block_excl_scan<NT, long long>(inc, shl, &tot_l);
  int nsp;
  int idx = block_excl_scan<NT, int>(nsp_t, shi, &nsp);
  __syncthreads();                       // s_bin complete
  Special *spec = a.spec + ((size_t)h * a.nch + c) * kMaxSpecial;
#pragma unroll
  for (int i = 0; i < EPT; ++i) {
    const int t = EPT * tid + i;
    if (t < n && sp[i]) {
      if (idx < kMaxSpecial) {
        Special x;
        x.ipre = ipre;
        x.e = e[i];
        // binade of the step just before this one: in this chunk (non-special or kNoBinade),
        // or 255 = "the previous chunk's last step" for the chunk's first key
        const int bprev = t > 0 ? s_bin[t - 1] : 127;
        x.meta = t | ((bprev == kNoBinade ? 0 : (bprev + 128)) << 16);
        st_spec(&spec[idx], x);
      }
      ++idx;
    }
    ipre += incs[i];
  }
  if (tid == 0) {
    ChunkRec r;
    r.tot = tot_l;
    r.nsp = nsp;
    r.blast = s_bin[n - 1];
    st_rec(&a.rec[(size_t)h * a.nch + c], r);
  }
  __builtin_amdgcn_s_waitcnt(0);      // this thread's write-through stores have completed
  __syncthreads();
  if (tid == 0) s_last = atomicAdd(&a.counters[h * kCounterStride], 1u) == (unsigned)(a.nch - 1) ? 1u : 0u;
  __syncthreads();
  if (!s_last) return;
  TS(0);

  // ---- the walk (last workgroup of head h). Every field of a special is resolved in parallel -
  // its global key index, the global increment prefix before it, the binade of the step before
  // it - so thread 0's serial chain only carries the running sum. Segments between specials hold
  // only non-special steps: their sum is exact integer arithmetic in units of 2^-40.
  float s = 0.0f;
  long long i_prev = 0, k_prev = -1, ibase_run = 0;
  int blast_prev = kNoBinade;      // blast of the chunk before the current batch
  bool ok = true;
  for (int cb = 0; cb < a.nch && ok; cb += kWalkBatch) {
    const int nb = min(kWalkBatch, a.nch - cb);
    long long tot = 0;
    int cnt = 0;
    if (tid < nb) {
      const ChunkRec r = ld_rec(&a.rec[(size_t)h * a.nch + cb + tid]);
      tot = r.tot;
      cnt = r.nsp;
      w_blast[tid] = r.blast;
    }
    long long tsum;
    const long long ib = ibase_run + block_excl_scan<NT, long long>(tid < nb ? tot : 0, shl, &tsum);
    int csum;
    const int off = block_excl_scan<NT, int>(tid < nb ? min(cnt, kMaxSpecial) : 0, shi, &csum);
    if (tid < nb) {
      w_ibase[tid] = ib;
      w_cnt[tid] = cnt;
      w_off[tid] = off;
    }
    if (tid == 0) w_off[nb] = csum;
    __syncthreads();
    TS(1);
    // one special per thread: its chunk by binary search over the offsets, then a single load
    for (int o = tid; o < csum; o += NT) {
      int lo = 0, hi = nb - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (w_off[mid] <= o) lo = mid; else hi = mid - 1;
      }
      const int cc = lo, j = o - w_off[cc];
      const Special x = ld_spec(&a.spec[((size_t)h * a.nch + cb + cc) * kMaxSpecial + j]);
      const int pos = x.meta & 0xFFFF, bf = (x.meta >> 16) & 0xFF;
      int bprev;
      if (bf == 255) bprev = cc > 0 ? w_blast[cc - 1] : blast_prev;
      else bprev = bf == 0 ? kNoBinade : bf - 128;
      w_i[o] = w_ibase[cc] + x.ipre;
      w_k[o] = (long long)(cb + cc) * kE2Chunk + pos;
      w_e[o] = x.e;
      w_b[o] = bprev;
    }
    __syncthreads();
    TS(2);
    // per special, in parallel: the segment before it as a whole number of ulps of its binade
    // (du < 0: empty segment), checked for divisibility; any overflowed chunk forces the fallback
    bool bad = false;
    for (int o = tid; o < csum; o += NT) {
      const long long di = w_i[o] - (o > 0 ? w_i[o - 1] : i_prev);
      const long long gap = w_k[o] - (o > 0 ? w_k[o - 1] : k_prev);
      int du = -1;
      if (gap > 1) {
        const int B = w_b[o];
        if (B < -17 || B > 22 || di < 0 || (di & ((1ll << (B + 17)) - 1)) != 0 || (di >> (B + 17)) >= (1ll << 24))
          bad = true;
        else
          du = (int)(di >> (B + 17));
      } else if (di != 0) {
        bad = true;
      }
      w_du[o] = du;
    }
    for (int cc = tid; cc < nb; cc += NT) bad |= w_cnt[cc] > kMaxSpecial;
    if (__syncthreads_or(bad)) ok = false;
    TS(6);
#ifdef BKV_EXPERIMENT_TS
    if (tid == 0) a.dbg[h * 8 + 7] = csum;
#endif
    if (tid < 64) {
      // the serial chain on wave 0: lane i holds special base+i; the chain itself is wave-uniform
      // (readlane), so it runs on the scalar unit except for the one fp32 add per special.
      const int lane = tid;
      bool good = ok;
      for (int base = 0; base < csum; base += 64) {
        const int o = base + lane;
        const int du_l = o < csum ? w_du[o] : -1, b_l = o < csum ? w_b[o] : 0;
        const float e_l = o < csum ? w_e[o] : 0.0f;
        const int cnt = min(64, csum - base);
        for (int i = 0; i < cnt; ++i) {
          const int du = __builtin_amdgcn_readlane(du_l, i);
          const int b = __builtin_amdgcn_readlane(b_l, i);
          const float ev = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, e_l), i));
          if (du >= 0) {
            const uint32_t bits = __float_as_uint(s);
            const uint32_t m = ((bits & 0x7FFFFFu) | 0x800000u) + (uint32_t)du;
            good = good && (int)(bits >> 23) == b + 127 && m < (1u << 24);
            s = __uint_as_float(((uint32_t)(b + 127) << 23) | (m & 0x7FFFFFu));
          }
          s = __fadd_rn(s, ev);
        }
      }
      if (tid == 0) s_last = good ? 1u : 0u;
    }
    __syncthreads();
    if (csum > 0) {                              // every thread carries the last special forward
      k_prev = w_k[csum - 1];
      i_prev = w_i[csum - 1];
    }
    TS(3);
    ok = s_last != 0;
    ibase_run += tsum;
    blast_prev = w_blast[nb - 1];
    __syncthreads();
  }
  if (tid == 0 && ok && (int64_t)a.nfill - 1 - k_prev > 0) {   // the trailing segment
    if (!advance(s, blast_prev, ibase_run - i_prev)) ok = false;
  }
  if (tid == 0) s_last = ok ? 1u : 0u;
  __syncthreads();
  if (!s_last) {
    // fallback: the serial loop itself, NT terms staged in LDS at a time
    float *stage = w_e;
    float ss = 0.0f;
    for (int64_t b0 = 0; b0 < a.nfill; b0 += NT) {
      const int nb = (int)min((int64_t)NT, (int64_t)a.nfill - b0);
      if (tid < nb) stage[tid] = ld_agent(&a.e[(size_t)h * a.ld + b0 + tid]);
      __syncthreads();
      if (tid == 0)
        for (int i = 0; i < nb; ++i) ss = __fadd_rn(ss, stage[i]);
      __syncthreads();
    }
    s = ss;
  }
  if (tid == 0) {
    a.sum[h] = s;
    a.status[h] = s_last ? 0u : 1u;
  }
  TS(4);
}

template <int VF>
__global__ __launch_bounds__(256) void pv_kernel(PvArgs a) {
  using R = KRow<VF>;
  __shared__ float s_p[kGqa][kPvMaxChunk];
  __shared__ float s_red[4][kGqa][kHd];
  const int c = blockIdx.x, g = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int sub = lane % R::LPR, kk = lane / R::LPR;
  const int64_t j0 = (int64_t)c * a.chunk;
  const int n = (int)min((int64_t)a.chunk, (int64_t)a.nfill - j0);

  float inv[kGqa];
#pragma unroll
  for (int h = 0; h < kGqa; ++h) inv[h] = a.sum[g * kGqa + h];
  for (int t = tid; t < n; t += 256) {
#pragma unroll
    for (int h = 0; h < kGqa; ++h) {
      const float e = a.e[(size_t)(g * kGqa + h) * a.ld + j0 + t];
      s_p[h][t] = round_f16(e / inv[h]);
    }
  }
  __syncthreads();

  float acc[kGqa][R::EPL];
#pragma unroll
  for (int h = 0; h < kGqa; ++h)
#pragma unroll
    for (int i = 0; i < R::EPL; ++i) acc[h][i] = 0.0f;

  const LayerView &L = a.L;
  constexpr int RB = row_bytes(VF), U = 4, STEP = 4 * R::KPW;   // keys per workgroup step
  for (int jb = wave * R::KPW; jb < n; jb += STEP * U) {
    uint4 w[U];
    uint32_t sw[U];
    int jl[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {                 // all U row loads in flight before any FMA
      jl[u] = jb + u * STEP + kk;
      const int64_t slot = slot_of(L, j0 + (jl[u] < n ? jl[u] : 0));
      w[u] = *reinterpret_cast<const uint4 *>(L.vd + (slot * a.nkv + g) * RB + sub * 16);
      if (VF == BKV_Q8_0)
        sw[u] = *reinterpret_cast<const uint32_t *>(L.vs + (slot * a.nkv + g) * kScaleRowBytes + (sub >> 2) * 4);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool valid = jl[u] < n;
      float vsc = 1.0f;
      if (VF == BKV_Q8_0) vsc = f16_to_f32(((sub >> 1) & 1) ? (sw[u] >> 16) : (sw[u] & 0xFFFFu));
      float p[kGqa];
#pragma unroll
      for (int h = 0; h < kGqa; ++h) p[h] = valid ? s_p[h][jl[u]] : 0.0f;
      v_accum<VF>(w[u], vsc, p, acc);
    }
  }
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
// gated = out * (1/(1 + exp(-gate))) (attn_vk.h:210-212)
__global__ __launch_bounds__(256) void merge_kernel(RedArgs a) {
  __shared__ float s[4][64];
  const int h = blockIdx.x, tid = threadIdx.x;
  const int d = blockIdx.y * 64 + (tid & 63), grp = tid >> 6;
  float acc = 0.0f;
  for (int c = grp; c < a.nch; c += 4) acc += a.part[((size_t)c * a.nh + h) * kHd + d];
  s[grp][tid & 63] = acc;
  __syncthreads();
  if (tid < 64) {
    const float v = (s[0][tid] + s[1][tid]) + (s[2][tid] + s[3][tid]);
    const size_t o = (size_t)h * kHd + d;
    a.out[o] = v;
    if (a.gate) a.out_gated[o] = v * (1.0f / (1.0f + exp_cr(-a.gate[gate_index(o, a.gs)])));
  }
}

// ------------------------------------------------------------------ launchers
hipError_t launch_append(const AppendArgs &a, int kf, int vf, int n_tok, hipStream_t st) {
  BKV_FMT_SWITCH(kf, vf, hipLaunchKernelGGL((append_kernel<KF_, VF_, false>), dim3(n_tok, a.nkv),
                                            dim3(64), 0, st, a));
  return hipGetLastError();
}

int qk_keys_per_wg(int kf) { return kf == BKV_Q8_0 ? QkTile<1>::KEYS : QkTile<0>::KEYS; }

hipError_t launch_decode(const QkArgs &qa, const EArgs &ea, const PvArgs &pa, const RedArgs &ra,
                         int kf, int vf, bool fuse, hipStream_t st) {
  BKV_FMT_SWITCH(kf, vf, {
    constexpr int NT = QkTile<KF_>::NT;
    if (fuse)
      hipLaunchKernelGGL((qk_kernel<KF_, VF_, true, false>), dim3(qa.nch, qa.nkv), dim3(NT), 0, st, qa);
    else
      hipLaunchKernelGGL((qk_kernel<KF_, VF_, false, false>), dim3(qa.nch, qa.nkv), dim3(NT), 0, st, qa);
    hipLaunchKernelGGL(e_kernel, dim3(ea.nch, ea.nh), dim3(256), 0, st, ea);
    hipLaunchKernelGGL((pv_kernel<VF_>), dim3(pa.nch, pa.nkv), dim3(256), 0, st, pa);
  });
  hipLaunchKernelGGL(merge_kernel, dim3(ra.nh, 4), dim3(256), 0, st, ra);
  return hipGetLastError();
}

// zero a workspace (bkv_workspace_init) and fill cache arrays (bkv_kv_fill_synthetic): kernels,
// not memsets, so that the calls can sit inside a captured graph
__global__ void workspace_init_kernel(unsigned *sync, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) sync[i] = 0u;
}

hipError_t launch_workspace_init(unsigned *sync, size_t nwords, hipStream_t st) {
  const int blocks = (int)std::min<size_t>(1024, (nwords + 255) / 256);
  hipLaunchKernelGGL(workspace_init_kernel, dim3(blocks > 0 ? blocks : 1), dim3(256), 0, st, sync, nwords);
  return hipGetLastError();
}

__global__ __launch_bounds__(256) void fill_words_kernel(unsigned *p, size_t n, unsigned value) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) p[i] = value;
}

hipError_t launch_fill_words(unsigned *p, size_t nwords, unsigned value, hipStream_t st) {
  if (nwords == 0) return hipSuccess;
  const int blocks = (int)std::min<size_t>(4096, (nwords + 255) / 256);
  hipLaunchKernelGGL(fill_words_kernel, dim3(blocks), dim3(256), 0, st, p, nwords, value);
  return hipGetLastError();
}

}  // namespace bkv
