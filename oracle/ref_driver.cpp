// ref_driver.cpp - exposes the reference's own CPU mirror (hiyoing/bonsai-vk runtime_vk/attn_vk.h,
// f16_rne_host.h, ptq_decode.h, compiled from where they lie under the reference checkout) through a
// C ABI, so tests can check the oracle restatement against it. TEST INFRASTRUCTURE ONLY: built into
// oracle/_ref/ by oracle/Makefile, never linked into the product library.
#include <cstdint>
#include <vector>

#include "attn_vk.h"

extern "C" {

uint16_t ref_f32_to_f16_bits(float f) { return f32_to_f16_bits(f); }
float ref_f16_to_f32(uint16_t h) { return f16_to_f32(h); }

// One decode step of one head row through the reference's stage functions (attn_vk.h:156-212), in the
// order attn_forward<true> calls them (attn_vk.h:284-309): score row, softmax row, P16 rounding, PV
// row, gate row. q16 is [hd/2] packed words, kc/vc the fp16 arenas [cap][nkv][hd/2].
void ref_decode_row(int hd, int nh, int nkv, float scale, const uint32_t *q16, const uint32_t *kc,
                    const uint32_t *vc, int kv_head, int nfill, const float *gate, float *score,
                    float *prob, uint16_t *p16, float *pregate, float *gated) {
  AttnCfg c;
  c.hd = hd; c.nh = nh; c.nkv = nkv; c.scale = scale; c.cap = nfill; c.seq = 1;
  const int hw = c.hw();
  std::vector<float> s(nfill), p(nfill), pr(nfill), mask(nfill, 0.0f);
  attn_score_row(c, q16, kc, nkv * hw, kv_head, nfill, s.data());
  attn_softmax_row(c, s.data(), mask.data(), nfill, p.data());
  for (int j = 0; j < nfill; ++j) {
    score[j] = s[j];
    prob[j] = p[j];
    p16[j] = f32_to_f16_bits(p[j]);
    pr[j] = f32_to_f16_as_f32(p[j]);
  }
  attn_pv_row(c, pr.data(), vc, nkv * hw, kv_head, nfill, pregate);
  attn_gate_row(pregate, gate, hd, gated);
}

// The decode step of rows = n_layers * nh head rows through ref_decode_row, nthreads OpenMP threads
// over the rows (a CPU decode of every layer's heads, for timing the reference's own path): row r is
// layer r / nh, head r % nh of that layer; layer l's arenas start layer_words words past the previous
// layer's (0: every layer reads the same arenas). q16 [rows][hd/2], out [rows][hd].
void ref_decode_rows(int hd, int nh, int nkv, float scale, int n_layers, const uint32_t *q16,
                     const uint32_t *kc, const uint32_t *vc, size_t layer_words, int nfill,
                     const float *gate, float *out, int nthreads) {
  const int rows = n_layers * nh, hw = hd / 2;
#pragma omp parallel num_threads(nthreads)
  {
    std::vector<float> s(nfill), p(nfill), g(hd);
    std::vector<uint16_t> p16(nfill);
#pragma omp for schedule(dynamic, 1)
    for (int r = 0; r < rows; ++r) {
      const int l = r / nh, h = r % nh;
      ref_decode_row(hd, nh, nkv, scale, q16 + (size_t)r * hw, kc + (size_t)l * layer_words,
                     vc + (size_t)l * layer_words, h / (nh / nkv), nfill, gate + (size_t)r * hd,
                     s.data(), p.data(), p16.data(), out + (size_t)r * hd, g.data());
    }
  }
}

// One row through the reference's attn_rms_norm then attn_rope (attn_vk.h:102-122), as attn_forward
// calls them for a Q or K row (attn_vk.h:268-276), into a separate output (the alias-safe form).
void ref_norm_rope_row(int hd, int nrot, float eps, float freq_base, const float *x, const float *w,
                       int pos, float *y) {
  AttnCfg c;
  c.hd = hd; c.nrot = nrot; c.eps = eps; c.freq_base = freq_base;
  std::vector<float> n(hd);
  attn_rms_norm(c, x, w, n.data());
  attn_rope(c, n.data(), pos, y);
}

}  // extern "C"
