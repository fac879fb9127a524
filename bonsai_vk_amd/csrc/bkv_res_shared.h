// bkv_res_shared.h - device pieces of the single-launch decode kernels (bkv_resident.hip,
// bkv_stream.hip): LDS-DMA K staging, tagged cross-workgroup hand-off words and bounded polls, DPP
// scans and the exact-sum walk over the group's chunk records.
#pragma once

#include <type_traits>

#include "bkv_common.h"
#include "bkv_device.h"
#include "bkv_internal.h"

namespace bkv {

constexpr unsigned kResSpin = 1u << 21;   // polls per wait (seconds) before the error word is set
constexpr int kUPR = 17;            // LDS uint4 per staged K row: 16 data + the q8_0 scale uint4
constexpr int kResNW = kResNT / 64;
constexpr int kResXBytes = 23040;    // LDS beside the K tiles (160 KiB in all)
constexpr int8_t kNoBin8 = -128;     // kNoBinade in the int8 binade map

#ifdef BKV_EXPERIMENT_TS
#define RTS(i) do { if (threadIdx.x == 0 && a.ts) a.ts[blockIdx.x * 16 + (i)] = (unsigned)wall_clock64(); } while (0)
#define RTSW(i, wv) do { if (threadIdx.x == 64 * (wv) && a.ts) a.ts[blockIdx.x * 16 + (i)] = (unsigned)wall_clock64(); } while (0)
#define RTSV(i) do { if ((threadIdx.x & 63) == 0 && a.tsw) a.tsw[(blockIdx.x * 8 + (threadIdx.x >> 6)) * 16 + (i)] = (unsigned)wall_clock64(); } while (0)
// the same slot with the shader clock (cycles, for the clock rate of a phase)
#define RTSC(i) do { if ((threadIdx.x & 63) == 0 && a.tsw) a.tsw[(blockIdx.x * 8 + (threadIdx.x >> 6)) * 16 + (i)] = (unsigned)__builtin_readcyclecounter(); } while (0)
#else
#define RTSC(i) do { } while (0)
#define RTSV(i) do { } while (0)
#define RTSW(i, wv) do { } while (0)
#define RTS(i) do { } while (0)
#endif

// every LDS access of this wave issued so far has completed, and the compiler keeps memory
// operations on their side of this point
__device__ __forceinline__ void wave_lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Arrive at a group barrier and wait until n workgroups have arrived. Waves below storing_waves
// first wait for their own stores (write-through stores complete at the device coherence point;
// the other waves have none this call needs, and their loads stay in flight), then one atomic per
// workgroup. The wait is bounded: a timeout sets the error word and lets the kernel finish.
__device__ __forceinline__ void group_barrier(unsigned *cnt, unsigned n, unsigned *err,
                                              int storing_waves = kResNT / 64) {
  if ((int)(threadIdx.x >> 6) < storing_waves) __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    atomicAdd(cnt, 1u);
    unsigned spins = 0;
    while (ld_agent(cnt) < n) {
      __builtin_amdgcn_s_sleep(1);
      if (++spins > kResSpin) {
        atomicOr(err, 1u);
        break;
      }
    }
  }
  __syncthreads();
}

// Chunk ch of the K rows of this wave's keys j0 .. j0+63 (rows >= n repeat row n-1) into
// kt[row * kUPR + col]: 16 uint4 per row (q8_0: the whole 256 B row; fp16: half a row), and for
// q8_0 the row's 16 B of block scales at column 16. Load i reads rows 4i..4i+3, 16 lanes per row.

// Cache slots of a workgroup's keys kb + k (0 <= k < nk). Paged: through an LDS copy of the block-
// table entries its keys span (lut[p - pf] for page p), so that no lookup is a global load (whose
// wait would also wait for every tile load in flight). The host takes this kernel only when a
// workgroup's keys span at most kResPgMax pages.
struct SlotMap {
  const LayerView *L;
  int64_t kb;
  const int *lut;
  uint32_t pf;
};
template <bool PG>
__device__ __forceinline__ int64_t slot_k(const SlotMap &m, int k) {
  if constexpr (!PG) {
    return m.kb + k + m.L->base;
  } else {
    const uint32_t pgs = (uint32_t)m.L->page, p = (uint32_t)(m.kb + k + m.L->base), pg = p / pgs;
    return (int64_t)m.lut[min(pg - m.pf, (uint32_t)kResPgMax - 1u)] * pgs + (int64_t)(p - pg * pgs);
  }
}

// k0: the first key (within the workgroup's range) of the n rows staged
template <int KF, bool PG>
__device__ __forceinline__ void stage_k_wave(uint4 *kt, const SlotMap &sm, int nkv, int g, int k0,
                                             int n, int ch) {
  // direct-to-LDS: load i writes the 64 consecutive tile slots 64 i .. 64 i + 63 (row = slot / kUPR,
  // column = slot % kUPR); column 16 is the q8_0 scale row (for fp16 K an unused copy of column 0).
  // Issued as inline asm, so the compiler neither waits for these loads nor counts them: the caller
  // waits with wait_vm<N>() before reading the tile, N = vector memory operations issued since.
  const int lane = threadIdx.x & 63;
  constexpr int RB = row_bytes(KF);
  const uint32_t base = __builtin_amdgcn_readfirstlane(lds_addr(kt));
  // q8_0 K: every slot first, so no lookup (an LDS read when paged) sits between the tile loads;
  // fp16 K, whose scores hold more registers, looks each one up in turn
  constexpr bool PRE = KF == BKV_Q8_0;
  uint32_t sls[PRE ? kUPR : 1];
  if constexpr (PRE)
#pragma unroll
    for (int i = 0; i < kUPR; ++i) sls[i] = (uint32_t)slot_k<PG>(sm, k0 + min((64 * i + lane) / kUPR, n - 1));
#pragma unroll
  for (int i = 0; i < kUPR; ++i) {
    const int slotx = 64 * i + lane, row = slotx / kUPR, col = slotx - row * kUPR;
    const int64_t sl = PRE ? (int64_t)sls[PRE ? i : 0] : slot_k<PG>(sm, k0 + min(row, n - 1));
    const uint8_t *src = (KF == BKV_Q8_0 && col == 16)
                             ? sm.L->ks + (sl * nkv + g) * kScaleRowBytes
                             : sm.L->kd + (sl * nkv + g) * RB + (ch * 16 + (col & 15)) * 16;
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off"
                 :: "v"(src), "s"(base + 1024u * i) : "memory", "m0");
  }
}
template <int N>
__device__ __forceinline__ void wait_vm() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory"); }

// ---------------------------------------------------------------- the walk (one wave, one head)
// walk_heads (bkv_device.h) for a group of at most 64 workgroups whose records the wave already
// holds (lane c: record of workgroup c, valid for c < gg).
// inclusive prefix sums over the wave by DPP row shifts and row broadcasts (no LDS round trips);
// lanes whose source lies outside the pattern read 0. 64-bit values move as two 32-bit halves.
template <int CTRL, int RM>
__device__ __forceinline__ long long dpp0_i64(long long v) {
  const int lo = __builtin_amdgcn_update_dpp(0, (int)v, CTRL, RM, 0xF, false);
  const int hi = __builtin_amdgcn_update_dpp(0, (int)(v >> 32), CTRL, RM, 0xF, false);
  return ((long long)hi << 32) | (long long)(unsigned)lo;
}
__device__ __forceinline__ long long wave_scan_i64(long long v) {
  v += dpp0_i64<0x111, 0xF>(v);
  v += dpp0_i64<0x112, 0xF>(v);
  v += dpp0_i64<0x114, 0xF>(v);
  v += dpp0_i64<0x118, 0xF>(v);
  v += dpp0_i64<0x142, 0xA>(v);
  v += dpp0_i64<0x143, 0xC>(v);
  return v;
}
__device__ __forceinline__ int wave_scan_i32(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);
  return v;
}
// REG: up to 64 specials resolved, segmented and chained in registers (one per lane); otherwise
// through the LDS scratch w.
template <typename WS, bool REG = true>
__device__ void walk_one(const ChunkRec &x, const Special *spec, int gg, int64_t kpw, int64_t nfill, WS &w,
                         float &s_out, bool &good_out, unsigned *tsw = nullptr) {
  const int lane = threadIdx.x & 63;
  constexpr int kWalkCap = WS::kCap;
  static_assert(WS::kWg <= 64, "one record per lane");
  bool ok = gg <= WS::kWg;
  // 1. prefix scans over the records
  const bool in = lane < gg;
  const long long tot = in ? x.tot : 0;
  const int cnt = in ? min(x.nsp, kMaxSpecial) : 0;
  const bool over = in && x.nsp > kMaxSpecial;
  const long long incl = wave_scan_i64(tot);
  const int oincl = wave_scan_i32(cnt);
  int bp = __shfl_up(in ? x.blast : kNoBinade, 1);
  if (lane == 0) bp = kNoBinade;
  if (in) {
    w.wg_ib[lane] = incl - tot;
    w.wg_off[lane] = oincl - cnt;
    w.wg_bp[lane] = bp;
  }
  const int T0 = __builtin_amdgcn_readlane(oincl, 63);
  if (lane == 0) w.wg_off[gg] = T0;
  const long long itot = ((long long)__builtin_amdgcn_readlane((int)(incl >> 32), 63) << 32) |
                         (long long)(unsigned)__builtin_amdgcn_readlane((int)incl, 63);
  const int blast_last = __builtin_amdgcn_readlane(in ? x.blast : kNoBinade, gg - 1);
  ok = ok && !__any(over) && T0 <= kWalkCap;
  const int T = ok ? T0 : 0;
  __builtin_amdgcn_wave_barrier();
  if (tsw && lane == 0) tsw[0] = (unsigned)wall_clock64();
  // the chain: per special, the sum's bits advance by du ulps and e is added in fp32; pre (lane j)
  // keeps the bits before step j. Blocks of 16 steps, then of 4 (entries past the live ones are
  // du 0, e 0: no change; n <= 64 and j stays a multiple of 4, so no index passes lane 63).
  auto chain = [&](float &s, int du_l, float e_l, int n, uint32_t &pre) {
    auto step = [&](int j) {
      const uint32_t du = (uint32_t)__builtin_amdgcn_readlane(du_l, j);
      const float ev = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, e_l), j));
      const uint32_t bits = __float_as_uint(s);
      pre = lane == j ? bits : pre;
      s = __fadd_rn(__uint_as_float(bits + du), ev);
    };
    int j0 = 0;
    for (; j0 + 16 <= n; j0 += 16) {
#pragma unroll
      for (int jj = 0; jj < 16; ++jj) step(j0 + jj);
    }
    for (; j0 < n; j0 += 4) {
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) step(j0 + jj);
    }
  };
  // the ulps of the segment before a special in its binade B (the sum's exponent field ck = B + 127
  // at both ends), from the gaps in key index and increment prefix to the previous special
  auto segment = [](long long gap, long long di, int B, int &du, int &ck) -> bool {
    du = 0;
    ck = -1;
    if (gap > 1) {
      if (B < -17 || B > 22 || di < 0 || (di & ((1ll << (B + 17)) - 1)) != 0 || (di >> (B + 17)) >= (1ll << 24))
        return true;
      du = (int)(di >> (B + 17));
      ck = B + 127;
      return false;
    }
    return di != 0;
  };
  auto resolve = [&](int o, long long &si, int &sk, float &se, int &sb) {
    int l = 0, hi = gg - 1;
    while (l < hi) {
      const int mid = (l + hi + 1) >> 1;
      if (w.wg_off[mid] <= o) l = mid; else hi = mid - 1;
    }
    const Special sx = ld_spec(&spec[(size_t)l * kMaxSpecial + (o - w.wg_off[l])]);
    const int bf = (sx.meta >> 16) & 0xFF;
    si = w.wg_ib[l] + sx.ipre;
    sk = (int)(l * kpw + (sx.meta & 0xFFFF));
    se = sx.e;
    sb = bf == 255 ? w.wg_bp[l] : (bf == 0 ? kNoBinade : bf - 128);
  };
  float s = 0.0f;
  bool good;
  long long k_last = -1, i_last = 0;
  if (REG && T <= 64) {
    // one special per lane: resolved, segmented and chained in registers
    long long si = 0;
    int sk = -1, sb = kNoBinade;
    float se = 0.0f;
    if (lane < T) resolve(lane, si, sk, se, sb);
    if (tsw && lane == 0) tsw[1] = (unsigned)wall_clock64();   // (instrumented builds: the wave's clocks)
    long long psi = ((long long)__shfl_up((int)(si >> 32), 1) << 32) | (long long)(unsigned)__shfl_up((int)si, 1);
    int psk = __shfl_up(sk, 1);
    if (lane == 0) {
      psi = 0;
      psk = -1;
    }
    int du = 0, ck = -1;
    const bool bad = lane < T && segment((long long)sk - psk, si - psi, sb, du, ck);
    ok = ok && !__any(bad);
    const int Tc = ok ? T : 0;
    if (tsw && lane == 0) tsw[2] = (unsigned)wall_clock64();
    const bool inn = lane < Tc;
    uint32_t pre = 0u;
    chain(s, inn ? du : 0, inn ? se : 0.0f, Tc, pre);
    const bool bad2 = inn && ck >= 0 && ((int)(pre >> 23) != ck || (int)((pre + (uint32_t)du) >> 23) != ck);
    good = ok && !__any(bad2);
    if (Tc > 0) {
      k_last = __builtin_amdgcn_readlane(sk, Tc - 1);
      i_last = ((long long)__builtin_amdgcn_readlane((int)(si >> 32), Tc - 1) << 32) |
               (long long)(unsigned)__builtin_amdgcn_readlane((int)si, Tc - 1);
    }
  } else {
    // 2. the specials, resolved to global key index, increment prefix and starting binade
    for (int o = lane; o < T; o += 64) resolve(o, w.si[o], w.sk[o], w.se[o], w.sck[o]);
    __builtin_amdgcn_wave_barrier();
    if (tsw && lane == 0) tsw[1] = (unsigned)wall_clock64();
    // 3. per special: the ulps of the segment before it in its binade
    bool bad = false;
    for (int o = lane; o < T; o += 64) {
      const long long gap = (long long)w.sk[o] - (o > 0 ? w.sk[o - 1] : -1);
      const long long di = w.si[o] - (o > 0 ? w.si[o - 1] : 0);
      int du, ck;
      bad = segment(gap, di, w.sck[o], du, ck) || bad;
      w.sdu[o] = du;
      w.sck[o] = ck;
    }
    ok = ok && !__any(bad);
    const int Tc = ok ? T : 0;
    __builtin_amdgcn_wave_barrier();
    if (tsw && lane == 0) tsw[2] = (unsigned)wall_clock64();
    // 4. the chain, 64 specials per block
    bool bad2 = false;
    for (int base = 0; base < Tc; base += 64) {
      const int o = base + lane;
      const bool inn = o < Tc;
      const int du_l = inn ? w.sdu[o] : 0, ck_l = inn ? w.sck[o] : -1;
      uint32_t pre = 0u;
      chain(s, du_l, inn ? w.se[o] : 0.0f, min(64, Tc - base), pre);
      if (ck_l >= 0) bad2 |= (int)(pre >> 23) != ck_l || (int)((pre + (uint32_t)du_l) >> 23) != ck_l;
    }
    good = ok && !__any(bad2);
    if (Tc > 0) {
      k_last = w.sk[Tc - 1];
      i_last = w.si[Tc - 1];
    }
  }
  if (tsw && lane == 0) { tsw[3] = (unsigned)wall_clock64(); tsw[4] = (unsigned)T; }
  if (good && nfill - 1 - k_last > 0) good = advance(s, blast_last, itot - i_last);
  s_out = s;
  good_out = good;
}

// ---------------------------------------------------------------- tagged hand-off words
// A per-workgroup value and its arrival in one 64-bit store: the two low bits carry the call's tag
// (1 or 2 by call parity; 0 = cleared). Every call clears the entries of workgroups it does not
// run, so an entry read during a call holds that call's tag, the previous call's tag, or 0.
__device__ __forceinline__ unsigned long long pack_stats(float m, float l, unsigned tag) {
  return ((unsigned long long)__float_as_uint(m) << 32) | ((__float_as_uint(l) & ~3u) | tag);
}
// record: tot (< 2^51) in w0 bits 2.., nsp in w1 bits 2..17, blast+128 (0: none) in bits 18..25
__device__ __forceinline__ void pack_rec(const ChunkRec &r, unsigned tag, unsigned long long &w0,
                                         unsigned long long &w1) {
  w0 = ((unsigned long long)r.tot << 2) | tag;
  const unsigned b = r.blast == kNoBinade ? 0u : (unsigned)(r.blast + 128);
  w1 = ((unsigned long long)(unsigned)r.nsp << 2) | ((unsigned long long)b << 18) | tag;
}
__device__ __forceinline__ ChunkRec unpack_rec(unsigned long long w0, unsigned long long w1) {
  ChunkRec r;
  r.tot = (long long)(w0 >> 2);
  r.nsp = (int)((w1 >> 2) & 0xFFFFu);
  const unsigned b = (unsigned)((w1 >> 18) & 0xFFu);
  r.blast = b == 0 ? kNoBinade : (int)b - 128;
  return r;
}
// wait until lanes < n of the wave see `tag` in the low bits of their word(s); bounded
__device__ __forceinline__ void poll_tagged(const unsigned long long *p, int stride, int words, int n,
                                            unsigned tag, unsigned long long (&v)[2], unsigned *err) {
  const int lane = threadIdx.x & 63;
  unsigned spins = 0;
  for (;;) {
    bool ok = true;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      if (i < words) {
        v[i] = lane < n ? ld_agent(p + (size_t)lane * stride + i) : (unsigned long long)tag;
        ok = ok && (unsigned)(v[i] & 3u) == tag;
      }
    }
    if (__all(ok)) return;
    __builtin_amdgcn_s_sleep(1);
    if (++spins > kResSpin) {
      if (lane == 0) atomicOr(err, 1u);
      return;
    }
  }
}

// ---------------------------------------------------------------- DPP scans
// A DPP move in which lanes whose source lies outside the pattern (or in a masked row) read 0.
template <int CTRL, int RM>
__device__ __forceinline__ int dpp0(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, RM, 0xF, false);
}
template <int CTRL, int RM>
__device__ __forceinline__ float dpp0(float v) {
  return __builtin_bit_cast(float, dpp0<CTRL, RM>(__builtin_bit_cast(int, v)));
}
template <int CTRL, int RM>
__device__ __forceinline__ double dpp0(double v) {
  const long long u = __builtin_bit_cast(long long, v);
  const int lo = dpp0<CTRL, RM>((int)u), hi = dpp0<CTRL, RM>((int)(u >> 32));
  return __builtin_bit_cast(double, ((long long)hi << 32) | (long long)(unsigned)lo);
}
template <int C, int RM>
struct DppCtl {
  static constexpr int c = C, rm = RM;
};
// inclusive prefix sum over the wave: row_shr 1, 2, 4, 8 inside each row of 16 lanes, then
// row_bcast 15 (rows 1, 3) and row_bcast 31 (rows 2, 3)
template <typename T>
__device__ __forceinline__ T wave_incl_scan_dpp(T v) {
  v += dpp0<0x111, 0xF>(v);
  v += dpp0<0x112, 0xF>(v);
  v += dpp0<0x114, 0xF>(v);
  v += dpp0<0x118, 0xF>(v);
  v += dpp0<0x142, 0xA>(v);
  v += dpp0<0x143, 0xC>(v);
  return v;
}
// fp16 K, half row CH (dims 128*CH .. 128*CH+127): acc = acc + q16_d * k_d in ascending d, exact
// products (attn_vk.h:156-170)
template <int CH>
__device__ __forceinline__ void qk_f16_half(const uint4 *row, const float (&qv)[kGqa][kHd / 16],
                                            float (&acc)[kGqa]) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint4 w0 = row[2 * j], w1 = row[2 * j + 1];
    const uint32_t u[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = f16_to_f32((u[i >> 1] >> ((i & 1) * 16)) & 0xFFFFu);
#pragma unroll
    for (int h = 0; h < kGqa; ++h) Dot16<16>::run(acc[h], qv[h][CH * 8 + j], x);
  }
}

// The 4 heads' scores of one fp16 K key per lane on the fp32 matrix cores, over dims D0 .. D0 +
// 16 NJ - 1 of its row (row: those dims' staged bytes, 16 B per 8 dims): v_mfma_f32_4x4x1f32 takes,
// for lane l and accumulator i, A from lane 4 (l / 4) + i and B from lane l, one exact fma per step
// (K = 1; the product of two fp16 values is exact in fp32), so with A = q16[l % 4][d] and B = the
// lane's key at d, accumulator i runs head i's chain acc = acc + q16 * k in ascending d: the
// reference's score, bit for bit (attn_vk.h:156-170). q16: the group's rounded q rows in LDS,
// [head][256] fp32.
typedef float fv4_t __attribute__((ext_vector_type(4)));
template <int D0, int NJ>
__device__ __forceinline__ void qk_f16_mfma(const uint4 *row, const float *q16, fv4_t &acc) {
  const float *qh = q16 + (threadIdx.x & 3) * kHd + D0;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const uint4 w0 = row[2 * j], w1 = row[2 * j + 1];
    const uint32_t u[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
    const float4 *q4 = reinterpret_cast<const float4 *>(qh + 16 * j);
    float qa[16];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float4 t = q4[c];
      qa[4 * c] = t.x; qa[4 * c + 1] = t.y; qa[4 * c + 2] = t.z; qa[4 * c + 3] = t.w;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i)
      acc = __builtin_amdgcn_mfma_f32_4x4x1f32(qa[i], f16_to_f32((u[i >> 1] >> ((i & 1) * 16)) & 0xFFFFu), acc, 0, 0, 0);
  }
}

// fp16 K in quarter rows: a wave's 64 keys, quarter Q (dims 64 Q .. + 63, 128 B per key) into LDS
// slot S of its tile region (kt: the region; slot S at 8 KiB S, key r at 128 r): 8 direct-to-LDS
// loads, load i taking keys 8 i .. 8 i + 7 (lane: key 8 i + lane / 8, 16-byte chunk lane % 8). As
// stage_k_wave: inline asm, the caller waits with wait_vm<N>().
template <bool PG>
__device__ __forceinline__ void stage_k16_quarter(uint4 *kt, const SlotMap &sm, int nkv, int g, int k0, int n, int Q,
                                                  int S) {
  const int lane = threadIdx.x & 63;
  const uint32_t base = __builtin_amdgcn_readfirstlane(lds_addr(kt) + 8192u * (uint32_t)S);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int64_t sl = slot_k<PG>(sm, k0 + min(8 * i + (lane >> 3), n - 1));
    const uint8_t *src = sm.L->kd + (sl * nkv + g) * row_bytes(BKV_F16) + 128 * Q + 16 * (lane & 7);
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" :: "v"(src), "s"(base + 1024u * i) : "memory", "m0");
  }
}

// one query head's score of one fp16 K key (the tail), half row CH: as qk_row_dot, with qt[j] =
// q16[h][16j + lane%16] for the head h of the lane's DPP row
template <int CH>
__device__ __forceinline__ void qk_f16_half1(const uint4 *row, const float (&qt)[kHd / 16], float &acc) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint4 w0 = row[2 * j], w1 = row[2 * j + 1];
    const uint32_t u[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = f16_to_f32((u[i >> 1] >> ((i & 1) * 16)) & 0xFFFFu);
    Dot16<16>::run(acc, qt[CH * 8 + j], x);
  }
}
// inclusive prefix sum inside each DPP row of 16 lanes
template <typename T>
__device__ __forceinline__ T row_incl_scan_dpp(T v) {
  v += dpp0<0x111, 0xF>(v);
  v += dpp0<0x112, 0xF>(v);
  v += dpp0<0x114, 0xF>(v);
  v += dpp0<0x118, 0xF>(v);
  return v;
}

// classify (bkv_device.h) without branches, the increment as an exact double
__device__ __forceinline__ void classify_d(double abefore, double aafter, float e, bool &special, int &bin,
                                           double &inc) {
  const int B = ilogb(aafter);
  const double lo = ldexp(1.0, B);
  const double t = ldexp((double)e, 23 - B);
  const bool ok = aafter >= 0x1p-17 && aafter < 0x1p22 && !(aafter > 2.0 * lo * (1.0 - kMargin)) &&
                  !(abefore < lo * (1.0 + kMargin)) && (t - floor(t) != 0.5);
  special = !ok;
  bin = ok ? B : kNoBinade;
  inc = ok ? ldexp(rint(t), B + 17) : 0.0;
}

// Across the workgroup's waves: sh[i * kGqa + h] holds wave i's total of head h. Lanes 0..kResNW-1
// scan those totals (DPP row shifts inside the first row of 16), and every lane takes its wave's
// exclusive prefix and the workgroup total by readlane, instead of each lane summing kResNW values.
__device__ __forceinline__ int rd_lane(int v, int l) { return __builtin_amdgcn_readlane(v, l); }
__device__ __forceinline__ float rd_lane(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ double rd_lane(double v, int l) {
  const long long u = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_readlane((int)u, l), hi = __builtin_amdgcn_readlane((int)(u >> 32), l);
  return __longlong_as_double(((long long)hi << 32) | (long long)(unsigned)lo);
}
template <typename T>
__device__ __forceinline__ void xwave_prefix(const T *sh, int h, int wave, T &before, T &total) {
  static_assert(kResNW <= 16, "one DPP row holds the wave totals");
  const int lane = threadIdx.x & 63;
  T x = lane < kResNW ? sh[lane * kGqa + h] : T(0);
  x += dpp0<0x111, 0xF>(x);
  x += dpp0<0x112, 0xF>(x);
  x += dpp0<0x114, 0xF>(x);
  if (kResNW > 8) x += dpp0<0x118, 0xF>(x);
  total = rd_lane(x, kResNW - 1);
  before = wave > 0 ? rd_lane(x, wave - 1) : T(0);
}

// the workgroup-wide max / sum of four values at once (every thread receives them)
// the wave's max (sum) in lane 63: DPP row reductions, then row_bcast 15 into rows 1, 3 and row_bcast
// 31 into rows 2, 3 (rows a broadcast does not write read the neutral element)
__device__ __forceinline__ float wave_max_l63(float v) {
  v = row16_max(v);
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp((int)0xFF800000u, __float_as_int(v), 0x142, 0xA, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp((int)0xFF800000u, __float_as_int(v), 0x143, 0xC, 0xF, false)));
  return v;
}
__device__ __forceinline__ float wave_sum_l63(float v) {
  v = row16_sum(v);
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xA, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x143, 0xC, 0xF, false));
  return v;
}
// qv[h][j] for a per-lane h, as masked bits (a select chain would be folded into an indexed
// access, which moves qv to private memory)
__device__ __forceinline__ float pick4h(const float (&qv)[kGqa][kHd / 16], int h, int j) {
  uint32_t b = 0u;
#pragma unroll
  for (int i = 0; i < kGqa; ++i) b |= __float_as_uint(qv[i][j]) & (0u - (uint32_t)(h == i));
  return __uint_as_float(b);
}

// v[i] by masks over the values (a select of the elements lets the compiler select their addresses
// instead, which keeps the array in scratch memory)
template <typename T>
__device__ __forceinline__ T pick4(const T (&v)[kGqa], int i) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8, "32- or 64-bit elements");
  using U = std::conditional_t<sizeof(T) == 4, uint32_t, uint64_t>;
  U b = 0;
#pragma unroll
  for (int j = 0; j < kGqa; ++j) b |= __builtin_bit_cast(U, v[j]) & (U(0) - (U)(i == j));
  return __builtin_bit_cast(T, b);
}

// PV over a wave's register-resident q8_0 V rows (slots s: key 32 s + 4 wave + vkk), probabilities
// from p[k] (4 fp16 per key). DELTA: the probabilities are p[k] - q[k] (exact in fp32), and a slot

}  // namespace bkv
