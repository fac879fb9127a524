/* bkv_oracle.c - CPU oracle of the KV-cache path (TEST INFRASTRUCTURE ONLY; see bkv_oracle.h).
 * Built with -O2 -ffp-contract=off and without -ffast-math: every float operation below rounds
 * exactly once, in the order written, as the reference's CPU mirror does. */
#include "bkv_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* exp used by the softmax and the gate. Mode 0 (default): the correctly rounded exp of the float
 * argument, formed as (float)exp((double)x) - the value both this oracle and the gfx950 kernels
 * compute. Mode 1: the C library's expf, as the reference's CPU mirror calls std::exp(float)
 * (runtime_vk/attn_vk.h:184,211); used to check the oracle against that mirror bit for bit. The two
 * differ only where the library's expf is not correctly rounded. */
static int g_exp_mode = 0;
void bko_set_exp_mode(int mode) { g_exp_mode = mode; }
static inline float oexp(float x) { return g_exp_mode ? expf(x) : (float)exp((double)x); }

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ------------------------------------------------------------------ fp16
 * f32 -> binary16, round to nearest even. Follows runtime_vk/f16_rne_host.h:27-53: Inf keeps its
 * sign, any NaN becomes the quiet pattern sign|0x7E00, an f32 subnormal becomes a signed zero (it is
 * below half of the smallest half subnormal), overflow goes to +-Inf, and a rounding carry may move
 * into the exponent. */
uint16_t bko_f32_to_f16(float f) {
  const uint32_t x = f2u(f);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const int32_t e = (int32_t)((x >> 23) & 0xFFu);
  const uint32_t m = x & 0x7FFFFFu;
  if (e == 0xFF) return (uint16_t)(sign | 0x7C00u | (m ? 0x0200u : 0u));
  if (e > 142) return (uint16_t)(sign | 0x7C00u);           /* |x| >= 2^16 -> Inf */
  if (e >= 113) {                                            /* half normal range */
    uint32_t h = sign | ((uint32_t)(e - 112) << 10) | (m >> 13);
    const uint32_t rest = m & 0x1FFFu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) ++h;
    return (uint16_t)h;
  }
  if (e == 0) return (uint16_t)sign;
  {                                                          /* half subnormal: 2^-24 steps */
    const uint32_t mant = m | 0x800000u;
    const uint32_t shift = (uint32_t)(126 - e);
    uint32_t k, half, rest;
    if (shift >= 25u) return (uint16_t)sign;
    half = 1u << (shift - 1u);
    rest = mant & ((1u << shift) - 1u);
    k = mant >> shift;
    if (rest > half || (rest == half && (k & 1u))) ++k;
    return (uint16_t)(sign | k);
  }
}

/* binary16 -> f32, exact; a NaN keeps its payload shifted into the f32 mantissa
 * (runtime_vk/ptq_decode.h:47-77). */
float bko_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t ex = (h >> 10) & 0x1Fu, man = h & 0x3FFu;
  if (ex == 0) {
    const float v = ldexpf((float)man, -24);
    return sign ? -v : v;
  }
  if (ex == 0x1F) return u2f(sign | 0x7F800000u | (man << 13));
  return u2f(sign | ((ex + 112u) << 23) | (man << 13));
}

void bko_f32_to_f16_array(const float *x, uint16_t *h, size_t n) {
  for (size_t i = 0; i < n; ++i) h[i] = bko_f32_to_f16(x[i]);
}
void bko_f16_to_f32_array(const uint16_t *h, float *x, size_t n) {
  for (size_t i = 0; i < n; ++i) x[i] = bko_f16_to_f32(h[i]);
}

/* ------------------------------------------------------------------ q8_0
 * runtime_vk/shaders/attn_norm_rope2.comp:102-115 and :184-217.
 *   amax = max |x| over the 32 values (order-free; a NaN element does not raise it)
 *   d    = amax > 1e-35f ? amax / 127.0f : 0           (correctly rounded division)
 *   id   = d != 0 ? 1.0f / d : 0                       (from the ROUNDED d, not 127/amax)
 *   q    = clamp(round(x * id), -127, 127), NaN -> 0   (round = RNE, or half-away with rhaz)
 *   stored scale = f16_rne(d)
 * The reference rounds with GLSL round(); which way its driver broke .5 ties is not recorded, so
 * the tie rule is a switch (RNE is the contract). */
static inline float q8_scale(float amax) { return amax > 1e-35f ? amax / 127.0f : 0.0f; }
static inline float q8_iscale(float amax) {
  const float dd = q8_scale(amax);
  return dd != 0.0f ? 1.0f / dd : 0.0f;
}
static inline uint8_t q8_byte(float x, float id, int rhaz) {
  const float t = x * id;
  float r = rhaz ? roundf(t) : rintf(t);
  int qi;
  if (r != r) r = 0.0f;
  if (r > 127.0f) r = 127.0f;
  if (r < -127.0f) r = -127.0f;
  qi = (int)r;
  return (uint8_t)(qi & 0xFF);
}

void bko_q8_block(const float *x, int rhaz, uint8_t *q, uint16_t *scale_bits) {
  float amax = 0.0f, id;
  int i;
  for (i = 0; i < 32; ++i) {
    const float a = fabsf(x[i]);
    if (a > amax) amax = a;
  }
  id = q8_iscale(amax);
  for (i = 0; i < 32; ++i) q[i] = q8_byte(x[i], id, rhaz);
  *scale_bits = bko_f32_to_f16(q8_scale(amax));
}

int bko_q8_block_ties(const float *x) {
  float amax = 0.0f, id;
  int i, n = 0;
  for (i = 0; i < 32; ++i) {
    const float a = fabsf(x[i]);
    if (a > amax) amax = a;
  }
  id = q8_iscale(amax);
  for (i = 0; i < 32; ++i) {
    const float t = x[i] * id;
    if (t - floorf(t) == 0.5f) ++n;
  }
  return n;
}

/* ------------------------------------------------------------------ layout
 * Words per slot of each array (runtime_vk/kv_guard.h:118-130): fp16 hd/2 words per head; q8_0 data
 * hd/4 words per head and hd/64 scale words per head. */
static inline int64_t words_data(int fmt, int hd) { return fmt == BKV_F16 ? hd / 2 : hd / 4; }

int64_t bko_slot(const bkv_cache_desc *d, int layer, int64_t pos) {
  if (d->page_tokens <= 0) return pos;
  {
    const int32_t *bt = d->block_table + (int64_t)layer * d->max_pages;
    return (int64_t)bt[pos / d->page_tokens] * d->page_tokens + pos % d->page_tokens;
  }
}

static inline uint32_t *arr(const bkv_cache_desc *d, int i, int layer) {
  void *base = i == 0 ? d->k_data : i == 1 ? d->k_scales : i == 2 ? d->v_data : d->v_scales;
  return (uint32_t *)((char *)base + (uint64_t)layer * d->layer_stride_bytes[i]);
}

/* write one head row x[hd] of tensor `which` (0 K, 1 V) into slot `slot` */
static void store_row(const bkv_cache_desc *d, int which, int layer, int64_t slot, int head,
                      const float *x, int rhaz) {
  const int fmt = which ? d->v_fmt : d->k_fmt, hd = d->hd, nkv = d->nkv;
  uint32_t *data = arr(d, which ? 2 : 0, layer);
  if (fmt == BKV_F16) {
    /* attn_norm_rope2.comp:167-181: word w = pack2_rne(x[2w], x[2w+1]) */
    uint32_t *row = data + (slot * nkv + head) * (hd / 2);
    for (int w = 0; w < hd / 2; ++w)
      row[w] = (uint32_t)bko_f32_to_f16(x[2 * w]) | ((uint32_t)bko_f32_to_f16(x[2 * w + 1]) << 16);
  } else {
    uint32_t *row = data + (slot * nkv + head) * (hd / 4);
    uint32_t *srow = arr(d, which ? 3 : 1, layer) + (slot * nkv + head) * (hd / 64);
    for (int b = 0; b < hd / 32; ++b) {
      uint8_t q[32];
      uint16_t s;
      bko_q8_block(x + 32 * b, rhaz, q, &s);
      for (int w = 0; w < 8; ++w)          /* element e -> byte e%4 of word e/4 */
        row[b * 8 + w] = (uint32_t)q[4 * w] | ((uint32_t)q[4 * w + 1] << 8) |
                         ((uint32_t)q[4 * w + 2] << 16) | ((uint32_t)q[4 * w + 3] << 24);
      if (b & 1) srow[b >> 1] = (srow[b >> 1] & 0xFFFFu) | ((uint32_t)s << 16);
      else       srow[b >> 1] = (srow[b >> 1] & 0xFFFF0000u) | (uint32_t)s;
    }
  }
}

void bko_kv_append(const bkv_cache_desc *d, int layer, uint32_t pos, int n_tok, const float *k,
                   const float *v, int rhaz) {
  for (int t = 0; t < n_tok; ++t) {
    const int64_t slot = bko_slot(d, layer, (int64_t)pos + t);
    for (int h = 0; h < d->nkv; ++h) {
      const size_t off = ((size_t)t * d->nkv + h) * d->hd;
      store_row(d, 0, layer, slot, h, k + off, rhaz);
      store_row(d, 1, layer, slot, h, v + off, rhaz);
    }
  }
}

/* q8_0 reconstruction = float(f16 scale) * float(sign-extended byte), formed in fp32 (exact: an
 * 11-bit significand times an 8-bit integer), runtime_vk/bonsai_forward.h:1470-1476. */
static inline float q8_elem(const uint32_t *row, const uint32_t *srow, int e) {
  const uint32_t w = row[e >> 2];
  const int b = (int)((w >> ((e & 3) * 8)) & 0xFFu);
  const int sb = b >= 128 ? b - 256 : b;
  const uint32_t sw = srow[(e / 32) >> 1];
  const float sc = bko_f16_to_f32((uint16_t)(((e / 32) & 1) ? (sw >> 16) : (sw & 0xFFFFu)));
  return sc * (float)sb;
}

void bko_load_row(const bkv_cache_desc *d, int which, int layer, int64_t pos, int head,
                  float *out) {
  const int fmt = which ? d->v_fmt : d->k_fmt, hd = d->hd, nkv = d->nkv;
  const int64_t slot = bko_slot(d, layer, pos);
  const uint32_t *data = arr(d, which ? 2 : 0, layer);
  if (fmt == BKV_F16) {
    const uint32_t *row = data + (slot * nkv + head) * (hd / 2);
    for (int w = 0; w < hd / 2; ++w) {
      out[2 * w] = bko_f16_to_f32((uint16_t)(row[w] & 0xFFFFu));
      out[2 * w + 1] = bko_f16_to_f32((uint16_t)(row[w] >> 16));
    }
  } else {
    const uint32_t *row = data + (slot * nkv + head) * (hd / 4);
    const uint32_t *srow = arr(d, which ? 3 : 1, layer) + (slot * nkv + head) * (hd / 64);
    for (int e = 0; e < hd; ++e) out[e] = q8_elem(row, srow, e);
  }
}

/* ------------------------------------------------------------------ decode (serial mirror)
 * One head row, exactly runtime_vk/attn_vk.h:156-212 in order:
 *   score_j = sum over d ascending of q16_d * k_d, as acc = acc + a*b (fp16 K: lo then hi half of
 *             each word); q8_0 K (this build's contract): per 32-block the correctly rounded exact
 *             sum of q16_d * int8_d, then acc = acc + f16(scale) * inner in block order
 *   v_j = score_j * scale; mx = max_j v_j from -INF; p_j = exp(v_j - mx); sum ascending; p_j /= sum
 *   p16_j = f16_rne(p_j); out_d = sum over j ascending of f16->f32(p16_j) * V_jd
 *   gated_d = out_d * (1 / (1 + exp(-gate_d)))
 * The mask the reference adds is all zero on this path (a masked slot is simply not attended). */
static void decode_row(const bkv_cache_desc *d, int layer, uint32_t nfill, const float *qrow,
                       const float *grow, float *orow, float *gout, float *dsc, float *dpr,
                       uint16_t *dp16, int head, float *s, float *pr, float *krow) {
  const int hd = d->hd, g = head / (d->nh / d->nkv);
  float q16[256];
  for (int i = 0; i < hd; ++i) q16[i] = bko_f16_to_f32(bko_f32_to_f16(qrow[i]));
  for (uint32_t j = 0; j < nfill; ++j) {
    const int64_t slot = bko_slot(d, layer, j);
    float acc = 0.0f;
    if (d->k_fmt == BKV_F16) {
      const uint32_t *row = arr(d, 0, layer) + (slot * d->nkv + g) * (hd / 2);
      for (int w = 0; w < hd / 2; ++w) {
        const float klo = bko_f16_to_f32((uint16_t)(row[w] & 0xFFFFu));
        const float khi = bko_f16_to_f32((uint16_t)(row[w] >> 16));
        acc = acc + q16[2 * w] * klo;
        acc = acc + q16[2 * w + 1] * khi;
      }
    } else {
      /* q8_0 K (no reference counterpart: the reference never compresses K). The block scale is
       * factored out of each 32-element block, and the block's inner sum q16_d * int8_d is the
       * fp32 rounding of its EXACT value: every product is a multiple of 2^-24 below 2^23, so the
       * fp64 sum below is exact in any order (below 2^28 in magnitude) and one cast rounds it.
       * Then acc = acc + f16(scale) * inner, in block order. */
      const uint32_t *row = arr(d, 0, layer) + (slot * d->nkv + g) * (hd / 4);
      const uint32_t *srow = arr(d, 1, layer) + (slot * d->nkv + g) * (hd / 64);
      for (int b = 0; b < hd / 32; ++b) {
        const uint32_t sw = srow[b >> 1];
        const float sc = bko_f16_to_f32((uint16_t)((b & 1) ? (sw >> 16) : (sw & 0xFFFFu)));
        double x = 0.0;
        for (int e = 32 * b; e < 32 * b + 32; ++e) {
          const uint32_t w = row[e >> 2];
          const int by = (int)((w >> ((e & 3) * 8)) & 0xFFu);
          x += (double)q16[e] * (double)(by >= 128 ? by - 256 : by);
        }
        const float inner = (float)x;
        const float t = sc * inner;
        acc = acc + t;
      }
    }    s[j] = acc;
  }
  {
    float mx = -INFINITY, sum = 0.0f;
    for (uint32_t j = 0; j < nfill; ++j) {
      const float v = s[j] * d->scale;
      if (v > mx) mx = v;
    }
    for (uint32_t j = 0; j < nfill; ++j) {
      const float v = s[j] * d->scale;
      pr[j] = oexp(v - mx);
      sum = sum + pr[j];
    }
    for (uint32_t j = 0; j < nfill; ++j) {
      const float p = pr[j] / sum;
      const uint16_t h = bko_f32_to_f16(p);
      if (dsc) dsc[j] = s[j];
      if (dpr) dpr[j] = p;
      if (dp16) dp16[j] = h;
      pr[j] = bko_f16_to_f32(h);
    }
  }
  for (int dd = 0; dd < hd; ++dd) orow[dd] = 0.0f;
  for (uint32_t j = 0; j < nfill; ++j) {
    bko_load_row(d, 1, layer, j, g, krow);       /* V row j, reconstructed exactly */
    for (int dd = 0; dd < hd; ++dd) orow[dd] = orow[dd] + pr[j] * krow[dd];
  }
  if (grow && gout)
    for (int dd = 0; dd < hd; ++dd) gout[dd] = orow[dd] * (1.0f / (1.0f + oexp(-grow[dd])));
}

static void decode_range(const bkv_cache_desc *d, int layer, uint32_t nfill, const float *q,
                         const float *gate, float *out, float *out_gated, float *dbg_score,
                         float *dbg_prob, uint16_t *dbg_p16, int h0, int h1, int nthreads) {
  const int hd = d->hd;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads > 0 ? nthreads : 1)
#endif
  for (int h = h0; h < h1; ++h) {
    float *s = (float *)malloc(sizeof(float) * (nfill ? nfill : 1));
    float *pr = (float *)malloc(sizeof(float) * (nfill ? nfill : 1));
    float krow[256];
    decode_row(d, layer, nfill, q + (size_t)h * hd, gate ? gate + (size_t)h * hd : NULL,
               out + (size_t)h * hd, out_gated ? out_gated + (size_t)h * hd : NULL,
               dbg_score ? dbg_score + (size_t)h * nfill : NULL,
               dbg_prob ? dbg_prob + (size_t)h * nfill : NULL,
               dbg_p16 ? dbg_p16 + (size_t)h * nfill : NULL, h, s, pr, krow);
    free(s);
    free(pr);
  }
  (void)nthreads;
}

void bko_attn_decode(const bkv_cache_desc *d, int layer, uint32_t nfill, const float *q,
                     const float *gate, float *out, float *out_gated, float *dbg_score,
                     float *dbg_prob, uint16_t *dbg_p16, int nthreads) {
  decode_range(d, layer, nfill, q, gate, out, out_gated, dbg_score, dbg_prob, dbg_p16, 0, d->nh,
               nthreads);
}

void bko_attn_decode_heads(const bkv_cache_desc *d, int layer, uint32_t nfill, const float *q,
                           const float *gate, float *out, float *out_gated, int h0, int h1) {
  decode_range(d, layer, nfill, q, gate, out, out_gated, NULL, NULL, NULL, h0, h1, 1);
}

/* fp64 leg (runtime_vk/attn_vk.h:320-387 semantics) on the cached K/V values. */
void bko_attn_decode_ideal(const bkv_cache_desc *d, int layer, uint32_t nfill, const float *q,
                           int round_bits, double *out) {
  const int hd = d->hd, gq = d->nh / d->nkv;
  double *s = (double *)malloc(sizeof(double) * (nfill ? nfill : 1));
  float row[256];
  for (int h = 0; h < d->nh; ++h) {
    const int g = h / gq;
    double qd[256], mx = -INFINITY, sum = 0.0;
    for (int i = 0; i < hd; ++i) {
      const float qi = q[(size_t)h * hd + i];
      qd[i] = (round_bits & 1) ? (double)bko_f16_to_f32(bko_f32_to_f16(qi)) : (double)qi;
    }
    for (uint32_t j = 0; j < nfill; ++j) {
      double acc = 0.0;
      bko_load_row(d, 0, layer, j, g, row);
      for (int i = 0; i < hd; ++i) acc += qd[i] * (double)row[i];
      s[j] = acc * (double)d->scale;
      if (s[j] > mx) mx = s[j];
    }
    for (uint32_t j = 0; j < nfill; ++j) { s[j] = exp(s[j] - mx); sum += s[j]; }
    for (int i = 0; i < hd; ++i) out[(size_t)h * hd + i] = 0.0;
    for (uint32_t j = 0; j < nfill; ++j) {
      double p = s[j] / sum;
      if (round_bits & 2) p = (double)bko_f16_to_f32(bko_f32_to_f16((float)p));
      bko_load_row(d, 1, layer, j, g, row);
      for (int i = 0; i < hd; ++i) out[(size_t)h * hd + i] += p * (double)row[i];
    }
  }
  free(s);
}

void bko_attn_prefill(const bkv_cache_desc *d, int layer, uint32_t pos0, int n_q, const float *q,
                      const float *gate, float *out, float *out_gated, int nthreads) {
  const size_t rs = (size_t)d->nh * d->hd;
  for (int i = 0; i < n_q; ++i)
    bko_attn_decode(d, layer, pos0 + (uint32_t)i + 1u, q + i * rs, gate ? gate + i * rs : NULL,
                    out + i * rs, out_gated ? out_gated + i * rs : NULL, NULL, NULL, NULL, nthreads);
}

/* ------------------------------------------------------------------ QK norm + rope
 * attn_rms_norm / attn_rope (runtime_vk/attn_vk.h:102-122) with rope_theta (:82-84): the squares are
 * rounded before they are added (the shader materialises them, attn_norm_rope2.comp:140-150), the
 * rotation reads the normed input for both partners and rounds each product. */
void bko_norm_rope_row(int hd, int nrot, float eps, float freq_base, const float *x, const float *w,
                       uint32_t pos, int libm_float, float *y) {
  float ss = 0.0f;
  for (int d = 0; d < hd; ++d) {
    const float sq = x[d] * x[d];
    ss = ss + sq;
  }
  const float inv = 1.0f / sqrtf(ss / (float)hd + eps);
  float n[256];
  for (int d = 0; d < hd; ++d) {
    const float t = x[d] * inv;
    n[d] = t * w[d];
  }
  const int half = nrot / 2;
  for (int p = 0; p < half; ++p) {
    const float ex = -2.0f * (float)p / (float)nrot;
    const float th = libm_float ? powf(freq_base, ex) : (float)pow((double)freq_base, (double)ex);
    const float a = (float)pos * th;
    const float cs = libm_float ? cosf(a) : (float)cos((double)a);
    const float sn = libm_float ? sinf(a) : (float)sin((double)a);
    const float lo = n[p], hi = n[p + half];
    const float l1 = lo * cs, l2 = hi * sn, h1 = hi * cs, h2 = lo * sn;
    y[p] = l1 - l2;
    y[p + half] = h1 + h2;
  }
  for (int d = nrot; d < hd; ++d) y[d] = n[d];
}

void bko_norm_rope_append(const bkv_cache_desc *d, int layer, uint32_t pos0, int n_tok,
                          const float *q_in, const float *k_in, const float *v_in, const float *qn_w,
                          const float *kn_w, int nrot, float eps, float freq_base, int rhaz,
                          float *q_out) {
  const size_t hd = (size_t)d->hd;
  float *kr = (float *)malloc(sizeof(float) * (size_t)n_tok * d->nkv * hd);
  for (int t = 0; t < n_tok; ++t) {
    for (int h = 0; h < d->nh; ++h) {
      const size_t o = ((size_t)t * d->nh + h) * hd;
      bko_norm_rope_row(d->hd, nrot, eps, freq_base, q_in + o, qn_w, pos0 + (uint32_t)t, 0, q_out + o);
    }
    for (int h = 0; h < d->nkv; ++h) {
      const size_t o = ((size_t)t * d->nkv + h) * hd;
      bko_norm_rope_row(d->hd, nrot, eps, freq_base, k_in + o, kn_w, pos0 + (uint32_t)t, 0, kr + o);
    }
  }
  bko_kv_append(d, layer, pos0, n_tok, kr, v_in, rhaz);
  free(kr);
}

/* ------------------------------------------------------------------ synthetic data
 * splitmix64 (Steele, Lea, Flood 2014): z = x + 0x9E3779B97F4A7C15, then two xor-shift-multiply
 * rounds and a final xor-shift. Counter-based use: value i of stream (seed, sid) is
 * splitmix64(seed ^ splitmix64(sid) + i * golden). */
uint64_t bko_splitmix64(uint64_t x) {
  uint64_t z = x + 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

static inline double unit_open(uint64_t r) {   /* (0, 1] */
  return ((double)(r >> 11) + 1.0) * (1.0 / 9007199254740992.0);
}

void bko_fill_normal(float *x, size_t n, uint64_t seed, uint64_t stream_id, float sigma) {
  const uint64_t base = seed ^ bko_splitmix64(stream_id + 0x1234567ull);
  for (size_t i = 0; i < n; i += 2) {
    /* Box-Muller: one pair of uniforms -> two independent normals */
    const uint64_t c = base + (uint64_t)(i / 2) * 2ull * 0x9E3779B97F4A7C15ull;
    const double u1 = unit_open(bko_splitmix64(c));
    const double u2 = unit_open(bko_splitmix64(c + 0x9E3779B97F4A7C15ull));
    const double r = sqrt(-2.0 * log(u1)), t = 6.283185307179586 * u2;
    x[i] = (float)(r * cos(t) * (double)sigma);
    if (i + 1 < n) x[i + 1] = (float)(r * sin(t) * (double)sigma);
  }
}

void bko_outlier_channels(uint64_t seed, int layer, int head, int hd, int n_out, int *ch) {
  uint64_t c = bko_splitmix64(seed * 0x100000001B3ull + (uint64_t)layer * 977u + (uint64_t)head);
  int k = 0;
  while (k < n_out) {
    int cand, dup = 0;
    c = bko_splitmix64(c);
    cand = (int)(c % (uint64_t)hd);
    for (int i = 0; i < k; ++i) dup |= ch[i] == cand;
    if (!dup) ch[k++] = cand;
  }
}

void bko_apply_outliers(float *x, int n_tok, int nkv, int hd, uint64_t seed, int layer, int n_out,
                        float factor) {
  int ch[64];
  if (n_out > 64) n_out = 64;
  for (int h = 0; h < nkv; ++h) {
    bko_outlier_channels(seed, layer, h, hd, n_out, ch);
    for (int t = 0; t < n_tok; ++t)
      for (int i = 0; i < n_out; ++i) x[((size_t)t * nkv + h) * hd + ch[i]] *= factor;
  }
}

double bko_now(void) {
  struct timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

int bko_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
