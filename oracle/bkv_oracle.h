/* bkv_oracle.h - CPU oracle of the KV-cache path. TEST INFRASTRUCTURE ONLY: it is the checker the
 * parity tests, smoke() and bench.py's cpu_baseline leg compare the HIP path against, and is never
 * linked into or called by the product library.
 *
 * It restates, in plain C and in the reference's exact operation order, the arithmetic of
 * hiyoing/bonsai-vk's KV path (paths relative to the reference root):
 *   fp16 pack/unpack ........ runtime_vk/f16_rne_host.h:27-53 (f32_to_f16_bits),
 *                             runtime_vk/ptq_decode.h:47-77 (f16_to_f32)
 *   q8_0 quantise-on-write .. runtime_vk/shaders/attn_norm_rope2.comp:102-115 (q8_scale/q8_iscale/
 *                             q8_byte), :184-217 (block absmax, data and scale words)
 *   fp16 K/V append ......... runtime_vk/shaders/attn_norm_rope2.comp:167-181
 *   score/softmax/P16/PV .... runtime_vk/attn_vk.h:156-212 and :261-311 (attn_forward<true>)
 *   fp64 ideal leg .......... runtime_vk/attn_vk.h:320-387 (attn_forward_ideal)
 *   q8_0 reconstruction ..... runtime_vk/bonsai_forward.h:1404-1488 (kv_dump)
 *   QK RMS norm + rope ...... runtime_vk/attn_vk.h:82-84, :102-122 (attn_rms_norm, attn_rope), with
 *                             runtime_vk/shaders/attn_norm_rope2.comp:138-181 (the fused append)
 *   arena layout ............ runtime_vk/kv_guard.h:94-150, runtime_vk/bonsai_forward.h:1940-1973
 *
 * Parity pins (what checks each function; see tests/test_oracle_*.py):
 *   bko_f16_to_f32 ... exhaustive over 2^16 patterns against numpy float16 (IEEE binary16).
 *   bko_f32_to_f16 ... every f32 exponent class, ties and carries against numpy's RNE cast, and the
 *                      reference's own packer compiled from its sources (oracle/_ref, when built).
 *   bko_q8_block ..... invariants (|q|<=127, max|q|==127 per live block, d_half = f16(amax/127),
 *                      dead blocks), brute force over tiny blocks, and the reference's dumped q8_0 V
 *                      (runs/kv_q8_0_v4.tsv) re-derived from the fp16 V of the same run.
 *   bko_attn_decode .. the reference's attn_score_row/attn_softmax_row/attn_pv_row/attn_gate_row
 *                      compiled from runtime_vk/attn_vk.h (bit-exact, fp16 cache), plus closed forms:
 *                      one key -> p = 1, identical keys -> uniform p, GQA-identical scores.
 *                      q8_0 K (no reference counterpart, this build's contract): each block's inner
 *                      sum against exact rational arithmetic (Python fractions) rounded once to fp32,
 *                      and against brute-force edge blocks (fp16 subnormal q, -128 bytes, max fp16).
 *   bko_attn_decode_ideal ... numpy float64 recomputation in tests.
 *   bko_norm_rope_row  in libm-float mode, the reference's attn_rms_norm + attn_rope compiled from
 *                      runtime_vk/attn_vk.h (bit-exact); closed forms: position 0 is the weighted
 *                      norm alone, dims past n_rot pass through, the rotation preserves each pair's
 *                      norm, a float64 recomputation to 1e-6.
 */
#ifndef BKV_ORACLE_H
#define BKV_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#include "../include/bkv.h"

#ifdef __cplusplus
extern "C" {
#endif

/* fp16 */
uint16_t bko_f32_to_f16(float f);
float bko_f16_to_f32(uint16_t h);
void bko_f32_to_f16_array(const float *x, uint16_t *h, size_t n);
void bko_f16_to_f32_array(const uint16_t *h, float *x, size_t n);

/* one q8_0 block of 32 values -> 32 bytes (int8 as uint8) + fp16 scale bits.
 * rhaz = 0: ties round half to even (the contract); rhaz = 1: half away from zero (ggml roundf). */
void bko_q8_block(const float *x, int rhaz, uint8_t *q, uint16_t *scale_bits);

/* number of exact .5 ties (x*id == k + 0.5) met while quantising one block (tie census) */
int bko_q8_block_ties(const float *x);

/* physical slot of logical position pos (desc pointers are HOST pointers here) */
int64_t bko_slot(const bkv_cache_desc *d, int layer, int64_t pos);

/* append n_tok tokens: k, v host fp32 [n_tok][nkv][hd] */
void bko_kv_append(const bkv_cache_desc *d, int layer, uint32_t pos, int n_tok,
                   const float *k, const float *v, int rhaz);

/* reconstruct one cached row (K if which == 0, V if which == 1) as fp32 [hd] */
void bko_load_row(const bkv_cache_desc *d, int which, int layer, int64_t pos, int head, float *out);

/* serial mirror of one decode step over positions [0, nfill).
 * q [nh][hd] fp32; gate may be NULL (then out_gated is not written).
 * dbg_score / dbg_prob (fp32 [nh][nfill]) and dbg_p16 (u16 [nh][nfill]) may be NULL.
 * nthreads > 1 runs the independent head rows on OpenMP threads (same numbers). */
void bko_attn_decode(const bkv_cache_desc *d, int layer, uint32_t nfill, const float *q,
                     const float *gate, float *out, float *out_gated, float *dbg_score,
                     float *dbg_prob, uint16_t *dbg_p16, int nthreads);

/* the same over a subset of head rows [h0, h1) (for bounded CPU-baseline samples) */
void bko_attn_decode_heads(const bkv_cache_desc *d, int layer, uint32_t nfill, const float *q,
                           const float *gate, float *out, float *out_gated, int h0, int h1);

/* fp64 ideal leg on the cached (already fp16/q8_0) K/V: round_bits bit0 = round Q to fp16,
 * bit1 = round P to fp16. out [nh][hd] double. */
void bko_attn_decode_ideal(const bkv_cache_desc *d, int layer, uint32_t nfill, const float *q,
                           int round_bits, double *out);

/* chunked prefill: row i = decode over [0, pos0+i] with q + i*nh*hd */
void bko_attn_prefill(const bkv_cache_desc *d, int layer, uint32_t pos0, int n_q, const float *q,
                      const float *gate, float *out, float *out_gated, int nthreads);

/* exp mode: 0 = correctly rounded (float)exp((double)x) (default), 1 = libm expf */
void bko_set_exp_mode(int mode);

/* Per-head RMS norm, weight and rope of one row (attn_vk.h:102-122, the shader's order
 * attn_norm_rope2.comp:138-165): ss = sum x*x ascending, inv = 1/sqrt(ss/hd + eps),
 * y = (x*inv)*w, then inside the first nrot dims the half-split rotation by
 * theta_p = base^(-2p/nrot) at angle pos*theta_p. libm_float = 0: pow/cos/sin are the correctly
 * rounded values (float)f((double)x), the contract the gfx950 kernel reproduces; 1: the C library's
 * powf/cosf/sinf, as the reference's CPU mirror calls them. */
void bko_norm_rope_row(int hd, int nrot, float eps, float freq_base, const float *x, const float *w,
                       uint32_t pos, int libm_float, float *y);
/* The fused append of n_tok tokens at pos0..: Q rows normed + roped into q_out [n_tok][nh][hd]
 * (fp32, the values the reference packs to Q16), K rows normed + roped and appended, V appended raw
 * (attn_norm_rope2.comp:138-217; attn_vk.h:266-281). */
void bko_norm_rope_append(const bkv_cache_desc *d, int layer, uint32_t pos0, int n_tok,
                          const float *q_in, const float *k_in, const float *v_in, const float *qn_w,
                          const float *kn_w, int nrot, float eps, float freq_base, int rhaz,
                          float *q_out);

/* seeded synthetic data: splitmix64 -> Box-Muller (double) -> float * sigma.
 * Element i of stream (seed, stream_id) is a pure function of (seed, stream_id, i). */
uint64_t bko_splitmix64(uint64_t x);
void bko_fill_normal(float *x, size_t n, uint64_t seed, uint64_t stream_id, float sigma);

/* K outlier channels: n_out distinct channels in [0, hd) for (seed, layer, kv head) */
void bko_outlier_channels(uint64_t seed, int layer, int head, int hd, int n_out, int *ch);

/* apply the outlier scaling in place to x [n_tok][nkv][hd] for one layer */
void bko_apply_outliers(float *x, int n_tok, int nkv, int hd, uint64_t seed, int layer,
                        int n_out, float factor);

/* wall-clock seconds (monotonic) */
double bko_now(void);

/* OpenMP thread count the library would use (omp_get_max_threads) */
int bko_max_threads(void);

#ifdef __cplusplus
}
#endif
#endif
