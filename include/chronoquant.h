/*
 * chronoquant.h — C ABI of the MI355X (gfx950) ChronoQuant KV-cache hot path.
 *
 * The library is libchronoquant.so, built from the .hip sources in chronoquant_mlx_amd/csrc.
 * Every entry point:
 *   - returns an int status (CQ_OK == 0); no exception ever crosses the ABI;
 *   - takes caller-owned DEVICE pointers (the library never allocates device
 *     memory; scratch space is an explicit workspace argument);
 *   - is stream ordered and asynchronous (work is enqueued on `stream`, a
 *     hipStream_t passed as void*; NULL means the legacy default stream);
 *   - is re-entrant for distinct buffers and streams.  The library's global
 *     state is limited to per-device caches filled once (occupancy figures,
 *     the address of cq_decode_attn_noalloc's static scratch), that scratch
 *     itself, and the test hook cq_set_fold_poll_bound.
 *
 * Storage layout (identical to the reference's logical tensors; an outer
 * capacity dimension per (sequence, kv head) lets appends write in place):
 *   keyframes  fp16   [B][H][cap_keyframes][D]     I-frames (anchors)
 *   packed     uint32 [B][H][cap_pframes][W]       W = ceil(D/8); nibble i of word w
 *                                                  holds code(dim 8w+i) + 8, bits 4i..4i+3
 *   scales     fp16   [B][H][cap_pframes]          one scale per P-frame row
 * Opt-in dense rows (cq_component.packing = CQ_PACK_DENSE): a 2- or 3-bit
 * component's packed rows hold its codes at their own width instead, as a
 * little-endian bit stream: dim d's field code + 2^(bits-1) occupies stream
 * bits [bits*d, bits*d + bits) (bit k of the stream is bit k % 32 of word
 * k / 32), W = ceil(D * bits / 32) words per row, unused bits 0.  (With
 * bits = 4 this is exactly the INT4 layout.)  This library's format: the
 * reference has no counterpart (it names physical variable-bit packing as
 * what its INT4 lanes are not, README.md:57, patch.py:94-98).
 * Token t of a sequence is an I-frame iff t % stride == 0; otherwise it is
 * P-frame slot t - t/stride - 1 coded against anchor t/stride.
 * The active prefix of each array is exactly the reference's tensor
 * (cache.py:46-51, cache.py:63-85).
 */
#ifndef CHRONOQUANT_H
#define CHRONOQUANT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void *cq_stream_t; /* hipStream_t */

enum cq_status {
  CQ_OK = 0,
  CQ_ERR_ARG = 1,         /* null pointer or invalid scalar argument */
  CQ_ERR_SHAPE = 2,       /* head_dim / heads / lengths out of range */
  CQ_ERR_DTYPE = 3,       /* unsupported dtype code */
  CQ_ERR_ALIGN = 4,       /* pointer misaligned for the required vector width */
  CQ_ERR_CAPACITY = 5,    /* append or read beyond the cache capacity */
  CQ_ERR_WORKSPACE = 6,   /* workspace missing or smaller than required */
  CQ_ERR_UNSUPPORTED = 7, /* valid request the library does not implement */
  CQ_ERR_LAUNCH = 8,      /* kernel launch reported an error */
  CQ_ERR_SCRATCH = 9,     /* shape needs more than the static scratch holds */
  CQ_ERR_TIMEOUT = 10     /* an earlier decode's split wait ran out (cq_decode_status) */
};

enum cq_dtype { CQ_F16 = 0, CQ_BF16 = 1, CQ_F32 = 2 };

enum cq_component_id { CQ_KEYS = 0, CQ_VALUES = 1 };

/* One compressed component (keys or values) of a batch of sequences. */
typedef struct cq_component {
  uint16_t *keyframes;   /* fp16 [B][H][cap_keyframes][D] */
  uint32_t *packed;      /* [B][H][cap_pframes][W] */
  uint16_t *scales;      /* fp16 [B][H][cap_pframes] */
  int64_t cap_keyframes; /* rows reserved per (b, h) */
  int64_t cap_pframes;   /* rows reserved per (b, h) */
  int32_t stride;        /* I-frame period, >= 1 */
  int32_t delta_bits;    /* residual bits, 2..4 */
  float dead_zone;       /* dead-zone ratio, >= 0 */
  int32_t packing;       /* CQ_PACK_INT4 (codes in INT4 lanes, the reference's
                            layout) or CQ_PACK_DENSE (fields of delta_bits) */
} cq_component;

enum cq_packing { CQ_PACK_INT4 = 0, CQ_PACK_DENSE = 1 };

typedef struct cq_cache_desc {
  int32_t batch;      /* B */
  int32_t n_kv_heads; /* H */
  int32_t head_dim;   /* D, 1..256 */
  int32_t reserved;
  cq_component k;
  cq_component v;
} cq_cache_desc;

/* Residual quantisation of n_rows rows of head_dim values each.
 * Replaces ChronoQuantCodecMLX.quantize_delta (reference codec.py:23-65):
 * per row scale = absmax/(2^bits/2 - 1) with the dead-zone rescale, codes =
 * clip(round_half_even(delta/scale), -2^bits/2, 2^bits/2 - 1), computed with
 * the rounding of `dtype` after every operation; scales returned as fp16.
 * delta: [n_rows][head_dim] of `dtype`; codes: int8 [n_rows][head_dim];
 * scales: fp16 [n_rows]. */
int cq_quantize_delta(const void *delta, int32_t dtype, int64_t n_rows,
                      int32_t head_dim, int32_t delta_bits, float dead_zone,
                      int8_t *codes, uint16_t *scales, cq_stream_t stream);

/* INT4 packing. Replaces pack_int4_codes (reference kernels.py:34-54, MSL
 * kernels.py:9-22): nibble = clip(code + 8, 0, 15), 8 nibbles per uint32,
 * head_dim padded to a multiple of 8 with nibble 0.
 * codes: int8 [n_rows][head_dim]; packed: [n_rows][ceil(head_dim/8)]. */
int cq_pack_int4(const int8_t *codes, int64_t n_rows, int32_t head_dim,
                 uint32_t *packed, cq_stream_t stream);

/* Inverse of cq_pack_int4. Replaces unpack_int4_codes (reference
 * kernels.py:57-61): code = ((word >> 4i) & 15) - 8, truncated to head_dim. */
int cq_unpack_int4(const uint32_t *packed, int64_t n_rows, int32_t head_dim,
                   int8_t *codes, cq_stream_t stream);

/* Append n_new tokens per sequence to both components: I-frame every stride,
 * otherwise residual against the anchor, quantised and packed in place.
 * Replaces ChronoQuantCache._append_component / update_and_fetch (reference
 * cache.py:87-129, 198-215) fused with the codec and the pack kernel.
 * keys / values: element (b, h, s, d) at base + b*sb + h*sh + s*ss + d
 *   (strides in elements, [3] = {sb, sh, ss}; d is contiguous), of `dtype`.
 * Positions: token s of sequence b lands at position offsets[b] + s when
 *   `offsets` (device int32 [B]) is non-NULL, else at `offset` + s.
 * The caller guarantees the capacities hold the new rows. */
int cq_append(const cq_cache_desc *cache, const void *keys,
              const int64_t *key_strides, const void *values,
              const int64_t *value_strides, int32_t dtype, int64_t n_new,
              const int32_t *offsets, int64_t offset, cq_stream_t stream);

/* Full fp16 reconstruction of one component for positions [0, seq_len).
 * Replaces ChronoQuantCache._reconstruct_component (reference
 * cache.py:131-156): r = fp16(anchor + fp16(fp16(code) * scale)) for
 * P-frames, the anchor for I-frames.  out: fp16 [B][H][seq_len][D]. */
int cq_reconstruct(const cq_cache_desc *cache, int32_t component,
                   int64_t seq_len, uint16_t *out, cq_stream_t stream);

/* Bytes of workspace cq_decode_attn needs for this shape.  The workspace
 * must be zero-filled once before its first use.  Its first 1.75 MiB hold the
 * split counters (one per sequence x kv head x q-head chunk, at most 16384),
 * split-ready flags and split fold records, which every call returns to
 * zero, so one workspace can be reused — also by calls of other shapes and
 * by cq_prefill_attn — without clearing.  Calls that share a workspace must
 * be ordered on one stream.  The workspace must be 256-byte aligned. */
size_t cq_decode_workspace_size(int32_t batch, int32_t n_kv_heads,
                                int32_t n_q_heads, int32_t head_dim,
                                int64_t max_seq_len);

/* Fused dequant + GQA scaled-dot-product attention for one query token per
 * sequence over the compressed cache (split-K flash decode; the last
 * workgroup of each kv head merges the splits).  Replaces
 * chronoquant_sdpa_kernel (reference kernels.py:248-279, MSL :79-228) and the
 * fused branch of chronoquant_sdpa (attention.py:45-59), generalised to B>=1
 * and per-sequence lengths.
 * q: [B][n_q_heads][head_dim] of q_dtype; q' = q*scale is rounded to q_dtype
 *   as in attention.py:46.  q head j reads kv head j / (n_q_heads/H).
 * Lengths: seq_lens (device int32 [B]) when non-NULL, else seq_len for all.
 * out: [B][n_q_heads][head_dim] of out_dtype. */
int cq_decode_attn(const cq_cache_desc *cache, const void *q, int32_t q_dtype,
                   int32_t n_q_heads, float scale, const int32_t *seq_lens,
                   int64_t seq_len, int64_t max_seq_len, void *out,
                   int32_t out_dtype, void *workspace, size_t workspace_bytes,
                   cq_stream_t stream);

/* Bytes of the static device scratch cq_decode_attn_noalloc works in (one
 * array per GPU, held from the library's first use on that GPU until the
 * process ends). */
#define CQ_NOALLOC_SCRATCH_BYTES (32u << 20)

/* cq_decode_attn without the workspace argument: the split partials and
 * counters live in a static device array of CQ_NOALLOC_SCRATCH_BYTES per
 * GPU instead of caller memory, so the call allocates nothing (no
 * hipMalloc, no library allocation).  No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops that forbid allocation).
 * Same arguments, kernels and results as cq_decode_attn (bit-identical
 * outputs).  A shape whose workspace (cq_decode_workspace_size) exceeds
 * CQ_NOALLOC_SCRATCH_BYTES returns CQ_ERR_SCRATCH and launches nothing.
 * Every call on one GPU shares that GPU's scratch: calls that overlap in
 * time on one GPU (unordered streams, concurrent graph replays) race on it
 * and must not be issued.  The counters in it start at zero and every call
 * returns them to zero.  The first call on each GPU resolves the array's
 * device address (hipGetSymbolAddress) and must be made outside stream
 * capture. */
int cq_decode_attn_noalloc(const cq_cache_desc *cache, const void *q, int32_t q_dtype,
                           int32_t n_q_heads, float scale, const int32_t *seq_lens,
                           int64_t seq_len, int64_t max_seq_len, void *out,
                           int32_t out_dtype, cq_stream_t stream);

/* Split waits.  The decode kernels of one-generation grids (every workgroup
 * of the launch resident at once, which the split plans size for) let each
 * split wait, with a bounded poll, for the partials of the other splits of
 * its sequence.  Co-residency is what HIP launches of one resident
 * generation give on an idle device; it is not guaranteed when other kernels
 * occupy the CUs (for instance two decodes running at once on different
 * streams).  A wait that runs out of poll rounds folds what it has and sets
 * a sticky status word in the workspace.
 *
 * cq_decode_status synchronises `stream` and reads that word: CQ_OK when no
 * wait ran out since the last query, else CQ_ERR_TIMEOUT, after clearing the
 * workspace's split state (counters, flags, fold records and the word) so
 * that later calls are correct again.  The outputs of the calls since the
 * previous query are then unreliable.  workspace: a cq_decode_attn
 * workspace, or NULL for the current device's cq_decode_attn_noalloc
 * scratch.  Not callable under stream capture (it synchronises).  No
 * counterpart in the reference (whose Metal kernel has no split waits). */
int cq_decode_status(void *workspace, cq_stream_t stream);

/* Test hook: the poll rounds of every later split wait (rounds < 1 restores
 * the default, 2^20).  Returns the previous bound.  Process-wide; for tests
 * that force a wait to run out while every kernel still exits normally. */
int32_t cq_set_fold_poll_bound(int32_t rounds);

/* Same contract as cq_decode_attn but always runs the portable (VALU) decode
 * kernel, for any head_dim <= 256 and q dtype; the test suite uses it to
 * check the specialised kernels against a second GPU implementation. */
int cq_decode_attn_generic(const cq_cache_desc *cache, const void *q,
                           int32_t q_dtype, int32_t n_q_heads, float scale,
                           const int32_t *seq_lens, int64_t seq_len,
                           int64_t max_seq_len, void *out, int32_t out_dtype,
                           void *workspace, size_t workspace_bytes,
                           cq_stream_t stream);

/* Uncompressed fp16 split-K flash decode, the comparison baseline the
 * compressed path has to beat (no reference counterpart: it stands for the
 * host framework's own fp16 SDPA over a plain KVCache).
 * k, v: fp16 [B][H][cap_tokens][D]; same q / out / workspace contract. */
int cq_fp16_decode_attn(const uint16_t *k, const uint16_t *v,
                        int64_t cap_tokens, int32_t batch, int32_t n_kv_heads,
                        int32_t head_dim, const void *q, int32_t q_dtype,
                        int32_t n_q_heads, float scale, const int32_t *seq_lens,
                        int64_t seq_len, int64_t max_seq_len, void *out,
                        int32_t out_dtype, void *workspace,
                        size_t workspace_bytes, cq_stream_t stream);

/* Chunked-prefill attention over the compressed cache: the n_q query tokens
 * of every sequence are its last n_q cached tokens (positions seq_len - n_q
 * .. seq_len - 1, appended before the call), attending causally (query i
 * sees keys <= seq_len - n_q + i) or, with causal = 0, to all seq_len keys.
 * Replaces the reconstruct fallback of chronoquant_sdpa for q_len > 1 with
 * mask None or "causal" (reference attention.py:61-74 over cache.py:131-160):
 * K/V rebuilt as fp16(anchor + fp16(fp16(code) * scale)), q' = fp16(q *
 * fp16(scale)), fp16 scores, fp32 softmax, fp16 weights, fp16 output.
 * head_dim 128, n_q_heads / n_kv_heads dividing 256.  q_dtype CQ_F16 or
 * CQ_BF16 (bf16: q' = bf16(q * bf16(scale)) and fp32 scores, as the
 * reference's bf16 x fp16 promotion computes them; output bf16).
 * q, out: [B][n_q_heads][n_q][128] of q_dtype, 16-byte aligned.
 * workspace: caller-owned, zero-initialised device memory of at least
 * cq_prefill_workspace_size(...) bytes, 256-byte aligned, for the split-K
 * partials (the kernels leave its counter region zeroed again, so it is
 * reused without clearing; it may be the decode workspace when large
 * enough).  NULL: the key range is not split (slower, same result). */
int cq_prefill_attn(const cq_cache_desc *cache, const void *q, int32_t q_dtype,
                    int32_t n_q_heads, int64_t n_q, float scale, int32_t causal,
                    int64_t seq_len, void *out, void *workspace, size_t workspace_bytes,
                    cq_stream_t stream);

/* Workspace bytes cq_prefill_attn needs for this shape on the current device
 * (0: none; the key range is not split).  No counterpart in the reference
 * (its fallback materialises the scores instead). */
size_t cq_prefill_workspace_size(int32_t batch, int32_t n_kv_heads, int32_t n_q_heads,
                                 int64_t n_q, int64_t seq_len);

/* ---- Fused elementwise ops of the end-to-end decoder ------------------
 * No counterpart in the reference's own files: these are the roles of
 * mlx's mx.fast.rms_norm / mx.fast.rope and mlx_lm's SwiGLU inside the
 * mlx_lm Qwen models that the reference's end-to-end runs drive
 * (patch.py:91-104 fills those models' cache slots).  dtype: CQ_F16,
 * CQ_BF16 or CQ_F32 for every tensor argument except the fp32 rotary
 * tables; math in fp32, one rounding per stored value. */

/* y = W x for one input row (a Linear layer with M = 1: the decoder's
 * projections in a decode step).  W: [n][k] row-major (a torch Linear
 * weight), x: [k], y: [n]; dtype CQ_F16 or CQ_BF16, fp32 accumulation, one
 * rounding per output.  k % 8 == 0, W and x 16-byte aligned. */
int cq_gemv(const void *w, const void *x, void *y, int64_t n, int32_t k, int32_t dtype,
            cq_stream_t stream);

/* cq_gemv of an RMSNorm'd row: h = round(x + residual) (residual null: h =
 * x), y = W round(h * rsqrt(mean(h^2) + eps) * norm_w), the decoder's
 * "add + RMSNorm, then project" in one launch.  h_out (optional, requires
 * residual): h is written there.  k <= 8192; norm_w, residual, h_out
 * 16-byte aligned. */
int cq_gemv_rms_norm(const void *w, const void *x, const void *residual, const void *norm_w,
                     float eps, void *h_out, void *y, int64_t n, int32_t k, int32_t dtype,
                     cq_stream_t stream);

/* cq_gemv of the SwiGLU gate of a fused [gate | up] row of 2k elements:
 * y = W round(round(silu(gate)) * up) (cq_silu_mul's values). */
int cq_gemv_silu(const void *w, const void *gate_up, void *y, int64_t n, int32_t k,
                 int32_t dtype, cq_stream_t stream);

/* y[r] = x[r] * rsqrt(mean(x[r]^2) + eps) * w, rows of dim elements. */
int cq_rms_norm(const void *x, const void *w, void *y, int64_t rows, int32_t dim,
                float eps, int32_t dtype, cq_stream_t stream);

/* Residual add + RMSNorm: h_out = round(x + residual), y = RMSNorm(h_out)
 * with weight w (the transformer block's "h = x + attn; norm(h)"). */
int cq_add_rms_norm(const void *x, const void *residual, const void *w, void *h_out,
                    void *y, int64_t rows, int32_t dim, float eps, int32_t dtype,
                    cq_stream_t stream);

/* Split of a fused QKV projection into the attention layout with per-head
 * RMSNorm and rotary embedding.  qkv: [batch][seq][(n_q_heads + 2 *
 * n_kv_heads) * head_dim] (query heads, key heads, value heads).  Query and
 * key heads: RMSNorm with q_w / k_w ([head_dim], null for none; the
 * normalised value is rounded to dtype), then rotary embedding on
 * half-split dims (dims j, j + head_dim/2 rotate by the angle whose fp32
 * cos/sin are cos_t/sin_t[pos][j], tables [max_pos][head_dim/2]).  Value
 * heads are copied.  q_out [batch][n_q_heads][seq][head_dim], k_out/v_out
 * [batch][n_kv_heads][seq][head_dim].  positions: int64, element (b, l) at
 * positions[b * pos_bstride + l]; a position outside [0, max_pos) gives NaN
 * rows instead of a read outside the tables.  head_dim 128. */
int cq_qkv_norm_rope(const void *qkv, const void *q_w, const void *k_w, void *q_out,
                     void *k_out, void *v_out, const float *cos_t, const float *sin_t,
                     int64_t max_pos, const int64_t *positions, int64_t pos_bstride,
                     int32_t batch, int64_t seq, int32_t n_q_heads, int32_t n_kv_heads,
                     int32_t head_dim, float eps, int32_t dtype, cq_stream_t stream);

/* One decode token per sequence from the fused QKV projection straight into
 * the caches: cq_qkv_norm_rope's query and key rows, then cq_append of the
 * key and value rows, in one launch (no counterpart in the reference, where
 * the model's q/k norm, RoPE and cache.update_and_fetch (cache.py:198-215)
 * are separate steps).  qkv: [batch][(n_q_heads + 2 * n_kv_heads) * 128],
 * batch and n_kv_heads those of the cache, head_dim 128.  q_out:
 * [batch][n_q_heads][128] of dtype.  positions as for cq_qkv_norm_rope with
 * seq = 1 (the rotary position of sequence b at positions[b * pos_bstride]).
 * Cache position: offsets[b] (device int32 [batch]) when non-NULL, else
 * offset; with offsets the capacities cannot be checked on the host and
 * rows past them are dropped.  lengths (device int32 [batch], may be NULL)
 * receives position + 1 per sequence, the lengths the decode then reads.
 * Bit-identical to cq_qkv_norm_rope followed by cq_append. */
int cq_qkv_rope_append(const cq_cache_desc *cache, const void *qkv, const void *q_w,
                       const void *k_w, void *q_out, const float *cos_t, const float *sin_t,
                       int64_t max_pos, const int64_t *positions, int64_t pos_bstride,
                       int32_t n_q_heads, float eps, int32_t dtype, const int32_t *offsets,
                       int64_t offset, int32_t *lengths, cq_stream_t stream);

/* y[r][c] = silu(gu[r][c]) * gu[r][n + c]: the SwiGLU gate over rows of a
 * fused [gate | up] projection (2n wide); silu rounded to dtype first. */
int cq_silu_mul(const void *gu, void *y, int64_t rows, int64_t n, int32_t dtype,
                cq_stream_t stream);

/* Static description of a status code. */
const char *cq_status_string(int32_t status);

#ifdef __cplusplus
}
#endif

#endif /* CHRONOQUANT_H */
