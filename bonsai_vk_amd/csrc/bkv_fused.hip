// bkv_fused.hip - one launch per layer and decode token: append, QK in the reference's order, the
// exact serial softmax sum, PV over fp16 probabilities and the partition merge.
//
// Workgroup w serves KV group g = w % nkv and keys [wi*kpw, (wi+1)*kpw) with wi = w / nkv, in R
// passes of NT keys (one key per thread; NT = 192 for q8_0 K, 128 for fp16 K). The phases that need
// every workgroup of a group are joined by arrival counters: a workgroup counts itself in, the last
// one to arrive does the phase's group-wide step (global max; the walk to the exact sum; the final
// merge) and raises the phase flag, and every workgroup waits for the flag only after it has arrived
// itself. The grid is sized so that all workgroups are resident at once, so every wait is reached by
// its producers; each wait is also bounded and records an error word instead of hanging.
// While the walk runs, the other workgroups stage their first V pass into LDS.
#include <algorithm>
#include <cstdlib>
#include <cstring>

#include "bkv_common.h"
#include "bkv_device.h"
#include "bkv_internal.h"

namespace bkv {

constexpr unsigned kSpinLimit = 1u << 24;

// float <-> unsigned with the same order (for atomicMax); 0 orders below every float
__device__ __forceinline__ unsigned ordered_bits(float f) {
  const unsigned u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float from_ordered_bits(unsigned o) {
  return __uint_as_float((o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o);
}


// Arrival of workgroup idx of n at a phase. Counting is two-level to keep same-address atomics
// short: idx goes to sub-counter idx % 8, and the last arrival of each sub-group counts into the main
// counter. Each counter is reset by its last arrival, ready for the next call. Returns true (in every
// thread) for the overall last arrival.
constexpr int kSub = 8;
constexpr int kMergeBatch = 12;   // partials whose loads are in flight together in the merge
__device__ __forceinline__ bool arrive(unsigned *cnt, unsigned *sub, int idx, int n, unsigned *sh) {
  __builtin_amdgcn_s_waitcnt(0);           // this thread's write-through stores have completed
  __syncthreads();
  if (threadIdx.x == 0) {
    const int k = idx % kSub, members = (n - k + kSub - 1) / kSub, nsub = n < kSub ? n : kSub;
    unsigned last = 0u;
    if (atomicAdd(sub + k * kCounterStride, 1u) == (unsigned)(members - 1)) {
      st_agent(sub + k * kCounterStride, 0u);
      if (atomicAdd(cnt, 1u) == (unsigned)(nsub - 1)) {
        st_agent(cnt, 0u);
        last = 1u;
      }
    }
    *sh = last;
  }
  __syncthreads();
  return *sh != 0;
}
// the last arrival raises the phase flag after its own stores completed
__device__ __forceinline__ void publish(unsigned *flag, unsigned gen) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) st_agent(flag, gen);
}
__device__ __forceinline__ void wait_flag(const unsigned *flag, unsigned gen, unsigned *err) {
  if (threadIdx.x == 0) {
    unsigned spins = 0;
    while (ld_agent(flag) != gen) {
      __builtin_amdgcn_s_sleep(2);
      if (++spins > kSpinLimit) {
        atomicOr(err, 1u);
        break;
      }
    }
  }
  __syncthreads();
}

#ifdef BKV_EXPERIMENT_TS
// phase timestamps of workgroup (w) into the sync area's upper half: [w][16] u32
#define FTS(i) do { if (threadIdx.x == 0 && blockIdx.x < 768) (a.sync + 32768)[blockIdx.x * 16 + (i)] = (unsigned)wall_clock64(); } while (0)
#else
#define FTS(i) do { } while (0)
#endif
// threads (= keys per pass) of a fused workgroup: 192 for q8_0 K (3 per CU: 52 KB K tile),
// 128 for fp16 K (2 per CU: 67 KB)
template <int KF>
struct FusedCfg {
  static constexpr int NT = KF == BKV_Q8_0 ? 192 : 128;
  static constexpr int MINB = KF == BKV_Q8_0 ? 3 : 2;
};

// q8_0 V data rows [j0, j0+n) of group g into the LDS tile, 256 B per row (16 lanes read a row's
// 256 contiguous bytes: conflict-free), zero beyond n; the block scales stay in registers.
template <int NT>
__device__ __forceinline__ void load_v_tile(uint4 *tile, const LayerView &L, int nkv, int g, int64_t j0, int n) {
  stage_rows<NT, NT, 16, 16, 4>(tile, L.vd, row_bytes(BKV_Q8_0), L, nkv, g, j0, n);
}

template <int KF, int VF, bool FUSE>
__global__ __launch_bounds__(FusedCfg<KF>::NT, FusedCfg<KF>::MINB) void fused_kernel(FusedArgs a) {
  constexpr int NT = FusedCfg<KF>::NT, NW = NT / 64;
  constexpr int UPR = KF == BKV_Q8_0 ? 17 : 33;         // LDS uint4 per K row (data + scale / pad)
  constexpr int DPR = KF == BKV_Q8_0 ? 16 : 32;
  constexpr int RB = row_bytes(KF);
  using VR = KRow<VF>;
  constexpr int VIT = NT / (NW * VR::KPW);               // PV steps per sub-chunk per lane
  __shared__ uint4 tile[NT * UPR];
  static_assert(VF != BKV_Q8_0 || sizeof(tile) >= NT * 256 + kGqa * NT * 2, "V tile + fp16 p must fit");
  static_assert(sizeof(tile) >= kGqa * sizeof(WalkScratch), "walk scratch must fit the K tile");
  __shared__ float shf[NT / 64 + 1];
  __shared__ double shd[NT / 64];
  __shared__ long long shl[NT / 64];
  __shared__ int shi[NT / 64];
  __shared__ double shd4[NT / 64 * kGqa];
  __shared__ long long shl4[NT / 64 * kGqa];
  __shared__ int shi4[NT / 64 * kGqa];
  __shared__ unsigned s_flag;
  __shared__ float s_m[kGqa], s_sum[kGqa];
  __shared__ double s_p0[kGqa];

  const int w = blockIdx.x, nkv = a.nkv, g = w % nkv, wi = w / nkv, gg = a.gg, R = a.rsub;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t kbase = (int64_t)wi * a.kpw;
  const int64_t kend = min((int64_t)a.nfill, kbase + (int64_t)a.kpw);   // this workgroup's keys
  const LayerView &L = a.L;
  unsigned *sync = a.sync;
  // sync words, one 256 B line each: per group kGroupLines lines (3 counters, 3 flags, 8 + 8
  // sub-counters of phases A and B, kMergeSub of the merge), then the generation, the end-of-call
  // counter (+ 8 sub-counters) and the error word
  unsigned *gl = sync + (size_t)g * kGroupLines * kCounterStride;
  unsigned *cntA = gl, *cntB = gl + kCounterStride, *cntC = gl + 2 * kCounterStride;
  unsigned *flA = gl + 3 * kCounterStride, *flB = gl + 4 * kCounterStride, *flC = gl + 5 * kCounterStride;
  unsigned *subA = gl + 6 * kCounterStride, *subB = gl + 14 * kCounterStride, *subC = gl + 22 * kCounterStride;
  unsigned *top = sync + (size_t)nkv * kGroupLines * kCounterStride;
  unsigned *genp = top, *cntD = top + kCounterStride, *subD = top + 2 * kCounterStride;
  unsigned *err = top + 10 * kCounterStride;
  const unsigned gen = ld_agent(genp) + 1u;
  FTS(0);

  if (FUSE) {
    if (tid < 64 && (int64_t)a.ap.pos >= kbase && (int64_t)a.ap.pos < kend)
      append_token<KF, VF, false>(a.ap, a.ap.pos, 0, g, tid);
    __syncthreads();
  }

  // ---------------------------------------------------------------- QK
  float qv[kGqa][kHd / 16];
  load_q16_rows(a.q + (size_t)g * kGqa * a.qs, qv, a.qs);
  float sc[kRMax][kGqa];
  float mloc[kGqa];
#pragma unroll
  for (int h = 0; h < kGqa; ++h) mloc[h] = -INFINITY;
  __syncthreads();
  asm volatile("s_nop 4");
#pragma unroll
  for (int r = 0; r < kRMax; ++r) {
    if (r < R) {
      const int64_t j0 = kbase + (int64_t)r * NT;
      const int n = (int)max((int64_t)0, min((int64_t)NT, kend - j0));
      stage_rows<NT, NT, DPR, UPR>(tile, L.kd, RB, L, nkv, g, j0, n);
      if (KF == BKV_Q8_0) stage_rows<NT, NT, 1, UPR>(tile + 16, L.ks, kScaleRowBytes, L, nkv, g, j0, n);
      __syncthreads();
      float acc[kGqa];
      qk_row_dot<KF>(tile + tid * UPR, qv, acc);
#pragma unroll
      for (int h = 0; h < kGqa; ++h) {
        sc[r][h] = acc[h];
        if (tid < n) mloc[h] = fmaxf(mloc[h], acc[h] * a.scale);
      }
      __syncthreads();
    }
  }
  FTS(1);
  // the workgroup's (max, sum exp) per head
  float lsum[kGqa];
#pragma unroll
  for (int h = 0; h < kGqa; ++h) {
    mloc[h] = block_max<NT>(mloc[h], shf);
    float l = 0.0f;
#pragma unroll
    for (int r = 0; r < kRMax; ++r)
      if (r < R && kbase + (int64_t)r * NT + tid < kend) l += __expf(sc[r][h] * a.scale - mloc[h]);
    l = wave_sum(l);
    if (lane == 0) shf[wave] = l;
    __syncthreads();
    float t = 0.0f;
#pragma unroll
    for (int i = 0; i < NW; ++i) t += shf[i];
    lsum[h] = t;
    __syncthreads();
  }
  if (tid < kGqa) {
    float m = mloc[0], l = lsum[0];
#pragma unroll
    for (int h = 1; h < kGqa; ++h)
      if (tid == h) { m = mloc[h]; l = lsum[h]; }
    st_f2(&a.stats[(size_t)(g * kGqa + tid) * gg + wi], make_float2(m, l));
    atomicMax(&a.mxenc[(gen & 1u) * a.nh + g * kGqa + tid], ordered_bits(m));
  }
  // the other slot of the running max is the next call's: clear it (0 = empty)
  if (w == 0 && tid < a.nh) st_agent(&a.mxenc[((gen + 1u) & 1u) * a.nh + tid], 0u);

  // ---------------------------------------------------------------- phase A: global max
  FTS(2);
  if (arrive(cntA, subA, wi, gg, &s_flag)) publish(flA, gen);
  FTS(3);
  wait_flag(flA, gen, err);
  FTS(4);
  if (tid < kGqa) s_m[tid] = from_ordered_bits(ld_agent(&a.mxenc[(gen & 1u) * a.nh + g * kGqa + tid]));
  __syncthreads();
  // approximate fp64 position of this workgroup's first key on each head's running sum
#pragma unroll
  for (int h = 0; h < kGqa; ++h) {
    double p = 0.0;
    for (int i = tid; i < wi; i += NT) {
      const float2 st = ld_f2(&a.stats[(size_t)(g * kGqa + h) * gg + i]);
      p += (double)st.y * exp((double)st.x - (double)s_m[h]);
    }
    p = block_sum_f64<NT>(p, shd);
    if (tid == 0) s_p0[h] = p;
  }
  __syncthreads();

  // ---------------------------------------------------------------- e, classification, records
  // LDS reuse: the K tile is free now. s_bin[h][k] binade of key k (kNoBinade if special),
  // later s_pp[h][k] the fp16 probabilities.
  int *s_bin = reinterpret_cast<int *>(tile);
  float ev[kRMax][kGqa];
  long long itot[kGqa];
  int nspc[kGqa];
  double carry[kGqa];
#pragma unroll
  for (int h = 0; h < kGqa; ++h) { itot[h] = 0; nspc[h] = 0; carry[h] = s_p0[h]; }
  Special *spec_g = a.spec + (size_t)(g * kGqa) * gg * kMaxSpecial;
#pragma unroll
  for (int r = 0; r < kRMax; ++r) {
    if (r < R) {
      const int64_t j = kbase + (int64_t)r * NT + tid;
      const bool valid = j < kend;
      double ed[kGqa], ex[kGqa], td[kGqa];
#pragma unroll
      for (int h = 0; h < kGqa; ++h) {
        ev[r][h] = valid ? exp_cr(sc[r][h] * a.scale - s_m[h]) : 0.0f;
        if (valid) st_agent(&a.e[(size_t)(g * kGqa + h) * a.ld + j], ev[r][h]);
        ed[h] = (double)ev[r][h];
      }
      block_excl_scan_k<NT, kGqa, double>(ed, ex, td, shd4);
      bool sp[kGqa];
      long long inc[kGqa], ipre[kGqa], tl[kGqa];
      int isp[kGqa], idx[kGqa], tn[kGqa];
#pragma unroll
      for (int h = 0; h < kGqa; ++h) {
        sp[h] = false;
        int bin = kNoBinade;
        inc[h] = 0;
        if (valid) classify(carry[h] + ex[h], carry[h] + ex[h] + ed[h], ev[r][h], sp[h], bin, inc[h]);
        carry[h] += td[h];
        s_bin[h * kRMax * NT + r * NT + tid] = (valid && !sp[h]) ? bin : kNoBinade;
        isp[h] = (valid && sp[h]) ? 1 : 0;
      }
      block_excl_scan_k<NT, kGqa, long long>(inc, ipre, tl, shl4);
      block_excl_scan_k<NT, kGqa, int>(isp, idx, tn, shi4);     // its barriers publish s_bin too
#pragma unroll
      for (int h = 0; h < kGqa; ++h) {
        const long long ip = itot[h] + ipre[h];
        const int id = nspc[h] + idx[h];
        itot[h] += tl[h];
        nspc[h] += tn[h];
        if (valid && sp[h] && id < kMaxSpecial) {
          const int pos = r * NT + tid;
          const int bprev = pos > 0 ? s_bin[h * kRMax * NT + pos - 1] : 127;
          Special x;
          x.ipre = ip;
          x.e = ev[r][h];
          x.meta = pos | ((bprev == kNoBinade ? 0 : (bprev + 128)) << 16);
          st_spec(&spec_g[((size_t)h * gg + wi) * kMaxSpecial + id], x);
        }
      }
    }
  }
  if (tid < kGqa) {
    const int h = tid;
    const int64_t nk = max((int64_t)0, kend - kbase);
    ChunkRec rc;
    rc.tot = h == 0 ? itot[0] : h == 1 ? itot[1] : h == 2 ? itot[2] : itot[3];
    rc.nsp = h == 0 ? nspc[0] : h == 1 ? nspc[1] : h == 2 ? nspc[2] : nspc[3];
    rc.blast = nk > 0 ? s_bin[h * kRMax * NT + (int)nk - 1] : kNoBinade;
    st_rec(&a.rec[(size_t)(g * kGqa + h) * gg + wi], rc);
  }

  // ---------------------------------------------------------------- phase B: the exact sums
  FTS(5);
  if (arrive(cntB, subB, wi, gg, &s_flag)) {
    // wave w walks heads w, w+NW, ... interleaved; LDS scratch: the K tile, one WalkScratch per head
    constexpr int NHW = (kGqa + NW - 1) / NW;
    const ChunkRec *rp[NHW];
    const Special *spp[NHW];
    WalkScratch *wsp[NHW];
    unsigned *tsp[NHW];
    float sres[NHW];
    bool gres[NHW];
    int nhere = 0;
#pragma unroll
    for (int q = 0; q < NHW; ++q) {
      const int h = min(wave + q * NW, kGqa - 1), hh = g * kGqa + h;
      if (wave + q * NW < kGqa) nhere = q + 1;
      rp[q] = a.rec + (size_t)hh * gg;
      spp[q] = a.spec + (size_t)hh * gg * kMaxSpecial;
      wsp[q] = reinterpret_cast<WalkScratch *>(tile) + h;
#ifdef BKV_EXPERIMENT_TS
      tsp[q] = a.sync + 32768 + 768 * 16 + hh * 8;
#else
      tsp[q] = nullptr;
#endif
    }
    walk_heads<NHW>(rp, spp, nhere, gg, (int64_t)a.kpw, (int64_t)a.nfill, wsp, sres, gres, tsp);
#pragma unroll
    for (int q = 0; q < NHW; ++q) {
      if (q < nhere) {
        const int hh = g * kGqa + wave + q * NW;
        float s = sres[q];
        if (!gres[q]) {
          // fallback: the serial loop itself over the stored e of this head
          float ss = 0.0f;
          for (int64_t b0 = 0; b0 < (int64_t)a.nfill; b0 += 64) {
            const int nb = (int)min((int64_t)64, (int64_t)a.nfill - b0);
            const float x = lane < nb ? ld_agent(&a.e[(size_t)hh * a.ld + b0 + lane]) : 0.0f;
            for (int i = 0; i < nb; ++i) ss = __fadd_rn(ss, __shfl(x, i));
          }
          s = ss;
        }
        if (lane == 0) {
          st_agent(&a.sum[hh], s);
          st_agent(&a.status[hh], gres[q] ? 0u : 1u);
        }
      }
    }
    publish(flB, gen);
    __syncthreads();                       // walk scratch released
  }
  // q8_0 V pass 0 into the LDS tile and its block scales into registers, while the walk runs
  const int vsub = lane % VR::LPR, vkk = lane / VR::LPR;
  uint32_t vsw[VF == BKV_Q8_0 ? VIT : 1];
  if constexpr (VF == BKV_Q8_0) {
    const int n0 = (int)max((int64_t)0, min((int64_t)NT, kend - kbase));
    load_v_tile<NT>(tile, L, nkv, g, kbase, n0);
#pragma unroll
    for (int it = 0; it < VIT; ++it) {
      const int row = wave * VR::KPW + vkk + it * NW * VR::KPW;
      const int64_t slot = slot_of(L, row < n0 ? kbase + row : kbase);
      vsw[it] = *reinterpret_cast<const uint32_t *>(L.vs + (slot * nkv + g) * kScaleRowBytes + (vsub >> 2) * 4);
    }
  }
  FTS(6);
  wait_flag(flB, gen, err);
  FTS(7);
  if (tid < kGqa) s_sum[tid] = ld_agent(&a.sum[g * kGqa + tid]);
  __syncthreads();

  // ---------------------------------------------------------------- p16 and PV
  // p16 = f16_rne(e / sum) (attn_vk.h:188 and the fp16 operand cast, :295-296) in LDS after the V
  // rows; out += p16 * V over this workgroup's keys, 4 heads per V row read.
  float acc[kGqa][VR::EPL];
#pragma unroll
  for (int h = 0; h < kGqa; ++h)
#pragma unroll
    for (int i = 0; i < VR::EPL; ++i) acc[h][i] = 0.0f;
  _Float16 *s_p16 = reinterpret_cast<_Float16 *>(reinterpret_cast<char *>(tile) + (VF == BKV_Q8_0 ? NT * 256 : 0));
#pragma unroll
  for (int r = 0; r < kRMax; ++r) {
    if (r < R) {
      const int64_t j0 = kbase + (int64_t)r * NT;
      const int n = (int)max((int64_t)0, min((int64_t)NT, kend - j0));
      if (r > 0) {
        __syncthreads();                    // pass r-1 done with the tile
        if constexpr (VF == BKV_Q8_0) {
          load_v_tile<NT>(tile, L, nkv, g, j0, n);
#pragma unroll
          for (int it = 0; it < VIT; ++it) {
            const int row = wave * VR::KPW + vkk + it * NW * VR::KPW;
            const int64_t slot = slot_of(L, row < n ? j0 + row : j0);
            vsw[it] = *reinterpret_cast<const uint32_t *>(L.vs + (slot * nkv + g) * kScaleRowBytes + (vsub >> 2) * 4);
          }
        }
      }
      {
        // the 4 heads' probabilities of key tid side by side: one 8-byte LDS read per V row
        _Float16 pk[kGqa];
#pragma unroll
        for (int h = 0; h < kGqa; ++h) pk[h] = (_Float16)(tid < n ? ev[r][h] / s_sum[h] : 0.0f);
        uint2 pw;
        pw.x = (uint32_t)__builtin_bit_cast(uint16_t, pk[0]) | ((uint32_t)__builtin_bit_cast(uint16_t, pk[1]) << 16);
        pw.y = (uint32_t)__builtin_bit_cast(uint16_t, pk[2]) | ((uint32_t)__builtin_bit_cast(uint16_t, pk[3]) << 16);
        reinterpret_cast<uint2 *>(s_p16)[tid] = pw;
      }
      __syncthreads();
#pragma unroll VF == BKV_Q8_0 ? VIT : 4
      for (int it = 0; it < VIT; ++it) {
        const int row = wave * VR::KPW + vkk + it * NW * VR::KPW;
        const bool valid = row < n;
        uint4 wv;
        float vsc = 1.0f;
        if constexpr (VF == BKV_Q8_0) {
          wv = tile[row * 16 + vsub];       // zero beyond n
          const uint32_t sw = vsw[it];
          vsc = f16_to_f32(((vsub >> 1) & 1) ? (sw >> 16) : (sw & 0xFFFFu));
        } else {
          const int64_t slot = slot_of(L, valid ? j0 + row : j0);
          wv = *reinterpret_cast<const uint4 *>(L.vd + (slot * nkv + g) * row_bytes(VF) + vsub * 16);
          if (!valid) wv = make_uint4(0u, 0u, 0u, 0u);
        }
        const uint2 pw = reinterpret_cast<const uint2 *>(s_p16)[row];   // zero beyond n
        float p[kGqa];
        p[0] = f16_to_f32(pw.x & 0xFFFFu);
        p[1] = f16_to_f32(pw.x >> 16);
        p[2] = f16_to_f32(pw.y & 0xFFFFu);
        p[3] = f16_to_f32(pw.y >> 16);
        v_accum<VF>(wv, vsc, p, acc);
      }
    }
  }
#pragma unroll
  for (int h = 0; h < kGqa; ++h)
#pragma unroll
    for (int i = 0; i < VR::EPL; ++i) {
      float v = acc[h][i];
      if (VR::LPR == 16) v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 32);
      acc[h][i] = v;
    }
  __syncthreads();
  float *s_red = reinterpret_cast<float *>(tile);          // [NW waves][kGqa][kHd]
  if (vkk == 0) {
#pragma unroll
    for (int h = 0; h < kGqa; ++h)
#pragma unroll
      for (int i = 0; i < VR::EPL; ++i) s_red[(wave * kGqa + h) * kHd + vsub * VR::EPL + i] = acc[h][i];
  }
  __syncthreads();
  float *part_g = a.part + (size_t)g * gg * kGqa * kHd;
  constexpr int kPairs = kGqa * kHd / 2;                  // a partial is [kGqa][kHd] fp32
  constexpr int PIT = (kPairs + NT - 1) / NT;
  for (int i = 0; i < PIT; ++i) {
    const int pr = tid + i * NT;
    if (pr < kPairs) {
      float2 v = make_float2(0.0f, 0.0f);
#pragma unroll
      for (int wv = 0; wv < NW; ++wv) {
        v.x += s_red[wv * kGqa * kHd + 2 * pr];
        v.y += s_red[wv * kGqa * kHd + 2 * pr + 1];
      }
      st_f2(reinterpret_cast<float2 *>(part_g + (size_t)wi * kGqa * kHd) + pr, v);
    }
  }

  // ---------------------------------------------------------------- phase C: merge + gate
  // Two-level, no waiting: the last arrival of each sub-group (wi % kMergeSub) sums its members' partials
  // in member order into a sub-partial, and the last of those sums the sub-partials in order.
  // The loads are issued kMergeBatch partials at a time so their latencies overlap.
  {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    const int k = wi % kMergeSub, members = (gg - k + kMergeSub - 1) / kMergeSub;
    const int nsub = gg < kMergeSub ? gg : kMergeSub;
    if (tid == 0) s_flag = atomicAdd(subC + k * kCounterStride, 1u) == (unsigned)(members - 1) ? 1u : 0u;
    __syncthreads();
    if (s_flag) {
      if (tid == 0) st_agent(subC + k * kCounterStride, 0u);
      float2 acc2[PIT];
      // sum of cnt blocks src + (first + m*step) * kGqa*kHd, m = 0..cnt-1, in m order
      auto sum_blocks = [&](const float *src, int first, int step, int cnt) {
#pragma unroll
        for (int i = 0; i < PIT; ++i) acc2[i] = make_float2(0.0f, 0.0f);
        for (int m0 = 0; m0 < cnt; m0 += kMergeBatch) {
          float2 t[kMergeBatch][PIT];
#pragma unroll
          for (int u = 0; u < kMergeBatch; ++u)
#pragma unroll
            for (int i = 0; i < PIT; ++i) {
              const int pr = tid + i * NT;
              t[u][i] = (m0 + u < cnt && pr < kPairs)
                            ? ld_f2(reinterpret_cast<const float2 *>(src + (size_t)(first + (m0 + u) * step) * kGqa * kHd) + pr)
                            : make_float2(0.0f, 0.0f);
            }
#pragma unroll
          for (int u = 0; u < kMergeBatch; ++u)
#pragma unroll
            for (int i = 0; i < PIT; ++i)
              if (m0 + u < cnt) { acc2[i].x += t[u][i].x; acc2[i].y += t[u][i].y; }
        }
      };
      sum_blocks(part_g, k, kMergeSub, members);
      float2 *sp = reinterpret_cast<float2 *>(a.subpart + ((size_t)g * kMergeSub + k) * kGqa * kHd);
#pragma unroll
      for (int i = 0; i < PIT; ++i)
        if (tid + i * NT < kPairs) st_f2(sp + tid + i * NT, acc2[i]);
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      if (tid == 0) {
        s_flag = atomicAdd(cntC, 1u) == (unsigned)(nsub - 1) ? 1u : 0u;
        if (s_flag) st_agent(cntC, 0u);
      }
      __syncthreads();
      if (s_flag) {
        sum_blocks(a.subpart + (size_t)g * kMergeSub * kGqa * kHd, 0, 1, nsub);
#pragma unroll
        for (int i = 0; i < PIT; ++i) {
          const int pr = tid + i * NT;
          if (pr < kPairs) {
            const size_t oi = (size_t)g * kGqa * kHd + 2 * pr;   // out is [nh][kHd], head g*kGqa+h
            const float2 v = acc2[i];
            *reinterpret_cast<float2 *>(a.out + oi) = v;
            if (a.gate) {
              const float2 gt = *reinterpret_cast<const float2 *>(a.gate + gate_index(oi, a.gs));
              *reinterpret_cast<float2 *>(a.out_gated + oi) =
                  make_float2(v.x * (1.0f / (1.0f + exp_cr(-gt.x))), v.y * (1.0f / (1.0f + exp_cr(-gt.y))));
            }
          }
        }
      }
    }
    FTS(9);
  }
  FTS(10);
  // ---------------------------------------------------------------- end of call: next generation
  if (arrive(cntD, subD, blockIdx.x, gridDim.x, &s_flag) && tid == 0) st_agent(genp, gen);
}

__global__ void workspace_init_kernel(unsigned *sync, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) sync[i] = 0u;
}

hipError_t launch_workspace_init(unsigned *sync, int nwords, hipStream_t st) {
  const int blocks = (int)std::min<long long>(1024, ((long long)nwords + 255) / 256);
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

template <int KF, int VF, bool FUSE>
static int fused_capacity() {
  static int cap = -1;
  if (cap < 0) {
    int dev = 0, per = 0;
    hipDeviceProp_t pr;
    if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&pr, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, fused_kernel<KF, VF, FUSE>, FusedCfg<KF>::NT, 0) != hipSuccess)
      cap = 0;
    else
      cap = per * pr.multiProcessorCount;
  }
  return cap;
}

int fused_keys_per_pass(int kf) { return kf == BKV_Q8_0 ? FusedCfg<1>::NT : FusedCfg<0>::NT; }

int fused_max_workgroups(int kf, int vf) {
  BKV_FMT_SWITCH(kf, vf, { return fused_capacity<KF_, VF_, false>(); });
  return 0;
}

// The grid never exceeds what the occupancy query says is resident at once on the device, so on a
// device not held by other long-running kernels every workgroup is running and each wait is reached
// by its producers. A plain launch is the default (a cooperative launch costs ~18 us more per call on
// ROCm 7); BKV_FUSED_LAUNCH=cooperative asks the runtime to guarantee co-residency instead. Either
// way every wait is bounded and records an error word rather than hanging.
hipError_t launch_fused(const FusedArgs &a, int kf, int vf, bool fuse, hipStream_t st) {
  const char *ev = getenv("BKV_FUSED_LAUNCH");
  const bool cooperative = ev && strcmp(ev, "cooperative") == 0;
  const dim3 grid(a.gg * a.nkv);
  void *args[] = {const_cast<FusedArgs *>(&a)};
  hipError_t e = hipErrorInvalidValue;
  BKV_FMT_SWITCH(kf, vf, {
    const dim3 block(FusedCfg<KF_>::NT);
    const void *fn = fuse ? reinterpret_cast<const void *>(&fused_kernel<KF_, VF_, true>)
                          : reinterpret_cast<const void *>(&fused_kernel<KF_, VF_, false>);
    e = cooperative ? hipLaunchCooperativeKernel(fn, grid, block, args, 0, st)
                    : hipLaunchKernel(fn, grid, block, args, 0, st);
  });
  return e;
}

}  // namespace bkv
