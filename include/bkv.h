/* bkv.h - C ABI of the MI355X (gfx950) KV-cache path: quantise-on-write KV append, the gather over
 * cached keys/values, and GQA softmax attention (decode and chunked prefill).
 *
 * Every entry point takes plain pointers and sizes. Device pointers are caller-owned memory
 * (hipMalloc or any allocator); the library never allocates on these paths. Calls are
 * stream-ordered: they enqueue work on `stream` and return without a host synchronisation. Calls on
 * one cache are thread-compatible, not thread-safe. No C++ exception crosses this boundary.
 *
 * Reference interfaces replaced (hiyoing/bonsai-vk, paths relative to its root):
 *  - bkv_kv_append        <- the K/V branch of shaders/attn_norm_rope2.comp:167-217, dispatched from
 *                            runtime_vk/bonsai_forward.h:609-612 (attn_block). K/V arrive post-RoPE.
 *  - bkv_attn_decode      <- the QK-softmax row kernel + PV(+gate) kernel pair dispatched at
 *                            runtime_vk/bonsai_forward.h:622-633 (attn_qk_softmax*.comp,
 *                            attn_pv{,_q8v,_q8v_gqa}.comp); CPU twin runtime_vk/attn_vk.h:156-212.
 *  - bkv_attn_prefill_chunk <- the prefill loop of one decode step per prompt token
 *                            (runtime_vk/bonsai_forward.h:2752-2759); same result per query row.
 *  - bkv_decode_step      <- the append + QK + PV sequence of one attention layer at one position
 *                            (runtime_vk/bonsai_forward.h:603-633), fused into fewer launches.
 *  - bkv_geom_check       <- KvGeom::check / compute (runtime_vk/kv_guard.h:94-150).
 */
#ifndef BKV_H
#define BKV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* hipStream_t without pulling in the HIP headers (same definition as hip_runtime_api.h). */
typedef struct ihipStream_t *hipStream_t;

/* ------------------------------------------------------------------ formats and errors */
enum bkv_fmt {
  BKV_F16  = 0,   /* [slot][nkv][hd/2] u32, element 2w in the low half of word w (RNE packed)  */
  BKV_Q8_0 = 1    /* data [slot][nkv][hd/4] u32 (element e = byte e%4 of word e/4, int8) plus   */
                  /* scales [slot][nkv][hd/64] u32 (fp16 scale of block 2i low, 2i+1 high)      */
};

enum bkv_err {
  BKV_OK          = 0,
  BKV_EINVAL      = -1,  /* a NULL pointer or a field out of range                             */
  BKV_ESHAPE      = -2,  /* geometry rule broken: hd%32, (hd/32) odd, nh%nkv, hd>256 ...         */
  BKV_ECAP        = -3,  /* position >= cap (the KvGuard REFUSE case), or nfill == 0            */
  BKV_EALIGN      = -4,  /* a device pointer not 16-byte aligned                                */
  BKV_EWORKSPACE  = -5,  /* workspace NULL or smaller than bkv_workspace_bytes()                */
  BKV_EHIP        = -6,  /* the HIP runtime reported an error on launch                         */
  BKV_EUNSUPPORTED = -7, /* a valid request this build does not implement                       */
  BKV_ETIMEOUT    = -8,  /* a decode kernel's bounded wait gave up (bkv_workspace_error)        */
  BKV_ESCRATCH    = -9   /* the call needs more than bkv_static_scratch_bytes() of workspace    */
};

/* bkv_workspace_bytes() op codes */
enum bkv_op { BKV_OP_DECODE = 0, BKV_OP_PREFILL = 1 };

/* ------------------------------------------------------------------ the cache descriptor
 * One descriptor covers the attention layers of one model. Per layer there are four arrays (K data,
 * K scales, V data, V scales); scales are NULL for an fp16 tensor. Layer l's array starts at
 * base + l * layer_stride_bytes[i]. Slot s of an array holds one position of all nkv heads, in the
 * per-format layout of enum bkv_fmt - the reference arena layout (runtime_vk/kv_guard.h:118-130,
 * runtime_vk/bonsai_forward.h:1940-1973) when page_tokens == 0.
 *
 * Contiguous (page_tokens == 0): position p lives in slot p, 0 <= p < cap.
 * Paged (page_tokens > 0): the pool has cap slots (cap % page_tokens == 0); position p lives in slot
 *   block_table[layer * max_pages + p / page_tokens] * page_tokens + p % page_tokens,
 *   and positions run up to max_pages * page_tokens. block_table is device memory.              */
typedef struct bkv_cache_desc {
  int32_t n_layers, nh, nkv, hd;   /* 8, 16, 4, 256 for the reference model                      */
  int32_t cap;                     /* slots per layer (contiguous) or pool slots (paged)          */
  int32_t k_fmt, v_fmt;            /* enum bkv_fmt                                                */
  int32_t page_tokens;             /* 0 = contiguous                                              */
  int32_t max_pages;               /* block-table row length (paged only)                         */
  float   scale;                   /* softmax scale applied to the raw dot, 1/sqrt(hd) = 0.0625   */
  void *k_data, *k_scales, *v_data, *v_scales;
  uint64_t layer_stride_bytes[4];  /* k_data, k_scales, v_data, v_scales                          */
  const int32_t *block_table;      /* [n_layers][max_pages] physical page ids, NULL if contiguous */
} bkv_cache_desc;

/* Validate a descriptor (no device access). Returns BKV_OK or the first rule broken. */
int bkv_geom_check(const bkv_cache_desc *d);

/* Bytes per slot per layer of each array, as KvGeom::compute derives them (kv_guard.h:118-130). */
uint64_t bkv_slot_bytes(const bkv_cache_desc *d, int which /* 0 k_data 1 k_scales 2 v_data 3 v_scales */);

/* Largest position count a call can attend over: cap, or max_pages * page_tokens when paged. */
int64_t bkv_max_positions(const bkv_cache_desc *d);

/* ------------------------------------------------------------------ the path
 * kv_append: write n_tok consecutive positions pos, pos+1, ... of `layer`.
 *   k, v: device fp32 [n_tok][nkv][hd] (post-RoPE K, raw V). fp16 tensors are RNE packed; q8_0
 *   tensors are quantised on write (per 32-block: d = amax/127 if amax > 1e-35 else 0,
 *   id = 1/d, q = clamp(rne(x*id), -127, 127), scale stored as RNE fp16 of d).                  */
int bkv_kv_append(const bkv_cache_desc *d, int layer, uint32_t pos, int n_tok,
                  const float *k, const float *v, hipStream_t stream);

/* attn_decode: one query token attending over positions [0, nfill) of `layer`.
 *   q: device fp32 [nh][hd], rounded RNE to fp16 before the dot (the reference's Q16 operand).
 *   out: device fp32 [nh][hd] attention result (the reference's PGATE).
 *   gate/out_gated: optional (both NULL or both set): out_gated = out * 1/(1+exp(-gate)).
 *   Semantics per head row: score = q16 . k, v = score*scale, p = exp(v - max)/sum, p rounded to
 *   fp16, out = sum_j p16_j * V_j (q8_0 V reconstructed as f16(scale)*int8).                   */
int bkv_attn_decode(const bkv_cache_desc *d, int layer, uint32_t nfill,
                    const float *q, const float *gate, float *out, float *out_gated,
                    void *workspace, size_t ws_bytes, hipStream_t stream);

/* decode_step: kv_append of one token at `pos` followed by attn_decode with nfill = pos+1, with the
 * append fused into the attention launch.                                                      */
int bkv_decode_step(const bkv_cache_desc *d, int layer, uint32_t pos,
                    const float *k, const float *v, const float *q, const float *gate,
                    float *out, float *out_gated, void *workspace, size_t ws_bytes,
                    hipStream_t stream);

/* attn_prefill_chunk: n_q query tokens at positions pos0 .. pos0+n_q-1 (already appended), each
 * attending causally over [0, pos0+i]. q: [n_q][nh][hd] fp32, out/out_gated/gate: [n_q][nh][hd].
 * Row i equals attn_decode(nfill = pos0+i+1) on the same cache (to the stated tolerance).       */
int bkv_attn_prefill_chunk(const bkv_cache_desc *d, int layer, uint32_t pos0, int n_q,
                           const float *q, const float *gate, float *out, float *out_gated,
                           void *workspace, size_t ws_bytes, hipStream_t stream);

/* Prepare a workspace for its first use: zeroes it (a small kernel on `stream`, no memset). Call
 * once after allocating it; the caller must not write into the workspace afterwards. */
int bkv_workspace_init(const bkv_cache_desc *d, void *workspace, size_t ws_bytes, hipStream_t stream);

/* Timing fixture: fill every slot of every layer's K data, K scales, V data and V scales with the
 * 32-bit word 0x3C003C00 (fp16 1.0 in both halves: fp16 K/V = 1.0, q8_0 bytes 0 / 60 with scale
 * 1.0), so that attention can be timed at any context without a prompt. Replaces kv_fill_synthetic
 * (runtime_vk/bonsai_forward.h:1355-1370), which fills the whole KV arena with that word. A kernel,
 * not a memset; stream-ordered. */
int bkv_kv_fill_synthetic(const bkv_cache_desc *d, hipStream_t stream);

/* The reference's fused append front end (attn_norm_rope2.comp:138-217, dispatched by attn_block at
 * runtime_vk/bonsai_forward.h:609-612; CPU mirror attn_vk.h:102-122, :266-281): for n_tok tokens at
 * positions pos0.., the projected Q and K rows get the per-head RMS norm (eps), the norm weight
 * (qn_w / kn_w, [hd]) and the half-split rope over the first nrot dims (freq_base); K is then
 * appended like bkv_kv_append, V (no norm, no rope) too, and the roped Q rows go to
 * q_out [n_tok][nh][hd] (fp32; bkv_attn_decode rounds them to the fp16 operand, as the reference's
 * Q16 pack does). pow / cos / sin are correctly rounded (the reference's mirror uses powf / cosf /
 * sinf, one fp32 ulp apart where those are not). q_out may alias q_in. */
int bkv_qk_norm_rope_append(const bkv_cache_desc *d, int layer, uint32_t pos0, int n_tok,
                            const float *q_in, const float *k_in, const float *v_in,
                            const float *qn_w, const float *kn_w, int nrot, float eps,
                            float freq_base, float *q_out, hipStream_t stream);

/* One chunk of a prompt for one layer: bkv_kv_append of the chunk's n_q tokens at pos0 .. pos0+n_q-1
 * (k, v: [n_q][nkv][hd] post-RoPE K and raw V), then bkv_attn_prefill_chunk over them. The chunked
 * form of the engine's prompt loop, which runs one decode step per prompt token
 * (runtime_vk/bonsai_forward.h:2752-2759); row i equals bkv_decode_step at pos0 + i. The workspace
 * is the prefill one (bkv_workspace_bytes(d, BKV_OP_PREFILL, ...)). Argument errors are reported
 * before anything is launched. */
int bkv_prefill_step(const bkv_cache_desc *d, int layer, uint32_t pos0, int n_q, const float *k,
                     const float *v, const float *q, const float *gate, float *out,
                     float *out_gated, void *workspace, size_t ws_bytes, hipStream_t stream);

/* Attention over the live window of keys [kstart, nfill) only: bkv_attn_decode as if the keys
 * before kstart did not exist. This is the reference's eviction of the farthest KV blocks, which
 * masks them out of the softmax with -INF in the additive score mask (runtime_vk/kv_guard.h:579-637
 * decides, runtime_vk/bonsai_forward.h the MASK window); a -INF key adds exactly +0 to the serial
 * sum and nothing to PV, so the window is the same computation. kstart < nfill; workspace sized for
 * nfill - kstart keys or more. */
int bkv_attn_decode_window(const bkv_cache_desc *d, int layer, uint32_t kstart, uint32_t nfill,
                           const float *q, const float *gate, float *out, float *out_gated,
                           void *workspace, size_t ws_bytes, hipStream_t stream);

/* Q and the gate straight from the engine's attn_q output, qg = [nh][2*hd] per query: head h's
 * hd query values, then its hd gate values (the per-head interleave that deint_qg splits,
 * runtime_vk/shaders/deint_qg.comp:1-45, before attn_qk_softmax and attn_pv_q8v read q and the gate,
 * attn_pv_q8v.comp:112). Same results as bkv_attn_decode / bkv_decode_step /
 * bkv_attn_prefill_chunk given the de-interleaved q and gate; out_gated may be NULL (then the gate
 * is not read). For the prefill, qg is [n_q][nh][2*hd]. */
int bkv_attn_decode_qg(const bkv_cache_desc *d, int layer, uint32_t nfill, const float *qg,
                       float *out, float *out_gated, void *workspace, size_t ws_bytes,
                       hipStream_t stream);
int bkv_decode_step_qg(const bkv_cache_desc *d, int layer, uint32_t pos, const float *k,
                       const float *v, const float *qg, float *out, float *out_gated,
                       void *workspace, size_t ws_bytes, hipStream_t stream);
int bkv_attn_prefill_chunk_qg(const bkv_cache_desc *d, int layer, uint32_t pos0, int n_q,
                              const float *qg, float *out, float *out_gated, void *workspace,
                              size_t ws_bytes, hipStream_t stream);

/* Whether a decode on this workspace gave up waiting (no counterpart in the reference, whose
 * Vulkan fences abort on a device loss; for callers that check their results). The single-launch
 * decode kernels synchronise their workgroups with bounded polls. A poll that runs out (the grid
 * was not co-resident, e.g. another kernel held CUs) sets an error word in the workspace, and that
 * call's output is not valid. This synchronises `stream`, returns BKV_ETIMEOUT if the error word
 * is set, else BKV_OK. After a timeout it re-initialises the whole workspace (ws_bytes bytes, as
 * bkv_workspace_init does; this clears the word), because the call that gave up left the
 * workspace's counters mid-protocol; later calls then run normally. */
int bkv_workspace_error(const bkv_cache_desc *d, void *workspace, size_t ws_bytes, hipStream_t stream);

/* Diagnostics: byte offset in the workspace of the error word bkv_workspace_error reads (out[0];
 * the stream and resident kernels share it). */
int bkv_error_words(const bkv_cache_desc *d, uint64_t out[1]);

/* Which decode implementation a call with nfill keys takes on the current device: 3 = the stream
 * single launch (q8_0 K and V, up to 528 keys per workgroup: the default where it applies), 2 = the
 * resident single launch (every format, up to 2048 keys per workgroup), 0 = the four-launch split
 * path (everything else); -1 = bad arguments. The environment variable BKV_DECODE = split |
 * resident | stream forces one where its plan fits (read on every call). BKV_COOP=1 (read once)
 * launches the stream kernel cooperatively: the runtime then refuses a grid that cannot be
 * co-resident, at about 18 us more per call. */
int bkv_decode_path(const bkv_cache_desc *d, uint32_t nfill);

/* Workspace needed by op (enum bkv_op) for contexts up to max_ctx positions (prefill: max_ctx is
 * pos0 + n_q, the chunk is bounded by BKV_PREFILL_MAX_Q). Returns 0 on a bad descriptor.      */
size_t bkv_workspace_bytes(const bkv_cache_desc *d, int op, uint32_t max_ctx);

/* Diagnostics (no counterpart in the reference; for parity tests and profiling): where a decode of
 * nfill keys keeps its intermediates inside the workspace. out[0] = row stride ld (floats),
 * out[1] = offset of the scores [nh][ld] fp32, out[2] = offset of e_j = exp(s_j*scale - max)
 * [nh][ld] fp32, out[3] = offset of the exact serial softmax sums [nh] fp32, out[4] = offset of the
 * walker status [nh] u32 (1 = the exact walk fell back to the serial loop), out[5] = workspace
 * bytes needed. Returns BKV_OK or an error for a bad descriptor. */
int bkv_debug_layout(const bkv_cache_desc *d, uint32_t nfill, uint64_t out[6]);

/* bkv_decode_step with no workspace argument and no allocation anywhere (no counterpart in the
 * reference; for callers that cannot allocate: code under HIP graph capture, serving loops or
 * harnesses that forbid hipMalloc). The workspace is a static device array of
 * bkv_static_scratch_bytes() (16 MiB) per GPU, part of the loaded library, zeroed by a small kernel
 * on `stream` at the first call on each GPU. Calls whose decode plan needs more than that return
 * BKV_ESCRATCH before launching anything (about 64K keys at nkv = 4; the exact need is
 * bkv_debug_layout's out[5]). Every call on one GPU shares that GPU's array: calls that overlap in
 * time on one GPU (two streams, two threads) race and give wrong results; serialise them. Other
 * errors and results are those of bkv_decode_step. */
int bkv_decode_step_static(const bkv_cache_desc *d, int layer, uint32_t pos,
                           const float *k, const float *v, const float *q, const float *gate,
                           float *out, float *out_gated, hipStream_t stream);
size_t bkv_static_scratch_bytes(void);

/* bkv_workspace_error for the static array of bkv_decode_step_static (no counterpart in the
 * reference; for the same callers): synchronises `stream`, returns BKV_ETIMEOUT if a static call
 * on the current GPU gave up waiting (its output is not valid) and then zeroes the array, so that
 * later static calls start from a clean workspace; BKV_OK otherwise (also when no static call has
 * run on this GPU). d: any descriptor of the calls (its nkv places the error word). */
int bkv_static_error(const bkv_cache_desc *d, hipStream_t stream);

/* Zeroes the current GPU's static array on `stream` (no counterpart in the reference): what
 * bkv_workspace_init is for a caller's workspace, e.g. after the decode path was switched with
 * BKV_DECODE. Stream-ordered; no allocation. */
int bkv_static_reset(hipStream_t stream);

/* Diagnostics (no counterpart in the reference; for tests): the device address of the current
 * GPU's static array in *out (NULL before the first static call or reset on this GPU). */
int bkv_static_debug_address(void **out);

/* Human-readable text of an enum bkv_err value (static storage). */
const char *bkv_strerror(int err);

/* Text of the last HIP error seen by this thread (empty if none). */
const char *bkv_last_hip_error(void);

/* Library version string. */
const char *bkv_version(void);

#define BKV_PREFILL_MAX_Q 4096

#ifdef __cplusplus
}
#endif
#endif /* BKV_H */
