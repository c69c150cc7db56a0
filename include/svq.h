/*
 * svq.h - C ABI of the gfx950 GGUF SoA dequantize + GEMV library (libsvq.so),
 * with the fused decode attention of the decoder layers around it.
 *
 * Weights use the structure-of-arrays layout that the reference builds at load
 * time (quantization.py:67-90, `pack_gguf_soa`): for an N x K matrix with
 * K % 32 == 0 there are N * K / 32 blocks of 32 weights, block b = row * (K/32)
 * + kb, and
 *   q[b * W .. b * W + W)  the block payload without its scale, W = 16 (Q4_0),
 *                          20 (Q5_0: uint32 LE high-bit mask, then 16 nibble
 *                          bytes) or 32 (Q8_0: int8);
 *   s[b]                   the fp16 bits of the block scale d.
 * Weight j of a block (App. of the reference layout, quantization.py:34-47):
 *   Q8_0: d * (int8)q[j]
 *   Q4_0: d * ((q[j % 16] >> 4 * (j / 16)) & 15) - 8)
 *   Q5_0: d * ((nibble(j) | ((qh >> j) & 1) << 4) - 16)
 *
 * Every pointer is a device pointer owned by the caller; the library never
 * allocates, frees or retains memory, never synchronizes and only enqueues
 * kernels on `stream` (a hipStream_t, NULL = the null stream), so every entry
 * point may be captured into a HIP graph.
 *
 * Return codes: 0 on success; a negative SVQ_E* code when an argument is
 * rejected (checked before any HIP call, so it needs no GPU); a positive
 * hipError_t when a HIP call fails. svq_last_error() describes the last
 * failure of the calling thread.
 */
#ifndef SVQ_H
#define SVQ_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SVQ_ABI_VERSION 3

/* Quantization codes: the reference's kernel codes (quantization.py:120). */
#define SVQ_Q4_0 4
#define SVQ_Q5_0 5
#define SVQ_Q8_0 8

/* Element types of dequantized or GEMV outputs. SVQ_F16 and SVQ_F32 are 0
   and 1, so a `y_is_fp32` / `out_is_fp32` flag passes as one of them. */
#define SVQ_F16 0
#define SVQ_F32 1
#define SVQ_BF16 2

#define SVQ_MAX_ROWS 8 /* largest M of svq_gemv */

#define SVQ_E_QTYPE (-1)   /* qtype is not 4, 5 or 8 */
#define SVQ_E_SHAPE (-2)   /* bad m, n, k (k % 32, sizes, ranges) */
#define SVQ_E_NULL (-3)    /* a required pointer is NULL */
#define SVQ_E_DTYPE (-4)   /* unsupported output element type */
#define SVQ_E_RANGE (-5)   /* a size exceeds the 32-bit offsets the kernels use */
#define SVQ_E_ALIGN (-6)   /* x / q / out not aligned for 16-byte accesses
                              (q: 4 bytes for Q5_0; s, bias: 2 bytes) */
#define SVQ_E_WORKSPACE (-7) /* workspace smaller than the call needs */
#define SVQ_E_FORMAT (-8)  /* malformed or truncated GGUF file */
#define SVQ_E_IO (-9)      /* a GGUF file cannot be opened, read or mapped */

/* Activations of svq_gemv_fused. */
#define SVQ_ACT_NONE 0
#define SVQ_ACT_GELU_TANH 1 /* F.gelu(..., approximate='tanh') */

#define SVQ_HEAD_DIM 128 /* head dimension of svq_decode_attention */
#define SVQ_MAX_GROUP 16 /* largest query heads per key/value head */

/* Version of this ABI (SVQ_ABI_VERSION). */
int svq_abi_version(void);

/* Message describing the last failed call on this thread ("" if none). */
const char *svq_last_error(void);

/*
 * y[m, n] = sum_k x[m, k] * W[n, k] + bias[n] for 1 <= m <= SVQ_MAX_ROWS.
 * Replaces `soa_gemv` (quantization.py:232-265) and the `_soa_gemv` Triton
 * kernel (quantization.py:171-229) it launches, and also covers the beam
 * widths 3..8 that the reference sends to `_soa_mm` (quantization.py:313-319).
 *   x     fp16 [m, k] row-major
 *   q, s  SoA payload and fp16 scale bits of the n x k matrix
 *   bias  fp16 [n] or NULL
 *   y     [m, n] row-major: fp16 with y_is_fp32 = 0 (SVQ_F16, as the
 *         reference stores), fp32 with y_is_fp32 = 1 (SVQ_F32); other values
 *         are rejected (SVQ_E_DTYPE). y may share no byte with x, q, s or bias.
 * Each block's integer dot product is accumulated in fp32 and multiplied by
 * its scale once (quantization.py:199, 215); bias is added in fp32 before the
 * final rounding.
 */
int svq_gemv(const void *x, const uint8_t *q, const uint16_t *s,
             const uint16_t *bias, void *y, int m, int n, int k, int qtype,
             int y_is_fp32, void *stream);

/*
 * svq_gemv with the decoder-layer ops around it fused in; y is fp16:
 *   y = residual + act(fp16(W . fp16(LayerNorm(x)) + bias))
 * Replaces the op sequences around the reference's quantized linears in a
 * decode step (runtime_8b.py:37, 53-54 and 110; runtime_1b.py:33, 46-47 and
 * 91): `input_layernorm` / `post_attention_layernorm` / `norm` before
 * `q/k/v_proj`, `c_fc` and `lm_head`, `F.gelu(approximate='tanh')` after
 * `c_fc`, and the residual `x + o_proj(...)`, `x + c_proj(...)`.
 *   ln_weight, ln_bias  fp16 [k] (16-byte aligned), or both NULL for no
 *             LayerNorm; ln_eps as torch.nn.LayerNorm's eps. Each x row is
 *             normalized with fp32 statistics and rounded to fp16 before the
 *             product, as the separate LayerNorm's fp16 output.
 *   activation  SVQ_ACT_NONE or SVQ_ACT_GELU_TANH, applied to the rounded
 *             product and rounded again
 *   residual  fp16 [m, n] added last (then rounded), or NULL; may be y itself
 *             (in place). Otherwise y may share no byte with any input (x,
 *             q, s, bias, LayerNorm parameters, residual): SVQ_E_SHAPE.
 * With a LayerNorm, x must fit the streaming kernels' LDS staging (m * k * 2
 * bytes plus offset sums within 156 KB), otherwise SVQ_E_SHAPE.
 */
int svq_gemv_fused(const void *x, const uint8_t *q, const uint16_t *s,
                   const uint16_t *bias, void *y, int m, int n, int k, int qtype,
                   const uint16_t *ln_weight, const uint16_t *ln_bias, float ln_eps,
                   const uint16_t *residual, int activation, void *stream);

/*
 * svq_gemv_fused without the LayerNorm, with a caller-provided workspace
 * that lets long rows (K > 8192 at m = 2..8) split K across workgroups: each
 * workgroup stages only a slice of x (at most 4608 columns) and writes fp32
 * partial sums to the workspace, and a second kernel adds the slices in a
 * fixed order and applies bias, activation and residual. Same results as
 * svq_gemv_fused within fp32 summation order; shapes that do not split, or a
 * workspace smaller than svq_gemv_split_workspace reports, run in one pass.
 * Replaces the same reference calls as svq_gemv / svq_gemv_fused
 * (quantization.py:232-265; runtime_8b.py:57 for c_proj with its residual).
 *   workspace  device memory, 16-byte aligned, or NULL; calls sharing one
 *              must not overlap (same stream, or ordered by events); it may
 *              share no byte with y or an input
 * y is fp16, with the overlap rules of svq_gemv_fused.
 */
int svq_gemv_split(const void *x, const uint8_t *q, const uint16_t *s,
                   const uint16_t *bias, void *y, int m, int n, int k, int qtype,
                   const uint16_t *residual, int activation, void *workspace,
                   int64_t workspace_bytes, void *stream);

/* Bytes of workspace svq_gemv_split uses for this shape (0: one pass), or a
   negative SVQ_E* code for an invalid shape. */
int64_t svq_gemv_split_workspace(int m, int n, int k, int qtype);

/* Bytes of the static scratch of svq_gemv_split_static (per GPU). */
#define SVQ_STATIC_SCRATCH_BYTES (4 << 20)

/*
 * svq_gemv_split without a workspace argument, for callers that cannot
 * allocate device memory: code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc. It has no counterpart in the reference
 * (whose soa_gemv, quantization.py:232-265, needs no scratch). The K split's
 * partial sums go to a static device array of SVQ_STATIC_SCRATCH_BYTES per
 * GPU, held until the process ends: a shape whose
 * svq_gemv_split_workspace(m, n, k, qtype) exceeds it is rejected
 * (SVQ_E_WORKSPACE); shapes that run in one pass use none. The call makes no
 * hipMalloc, hipFree or other allocating call. Every call on a GPU shares
 * that GPU's array, so calls that overlap on one GPU (streams without an
 * order between them) race. The first call on each device resolves the
 * array's device address (hipGetSymbolAddress, no allocation); make it
 * before capturing a graph that records the call. Arguments, checks and
 * results are those of svq_gemv_split.
 */
int svq_gemv_split_static(const void *x, const uint8_t *q, const uint16_t *s,
                          const uint16_t *bias, void *y, int m, int n, int k, int qtype,
                          const uint16_t *residual, int activation, void *stream);

/*
 * Diagnostic with no counterpart in the reference (whose launch tuple is the
 * per-(qtype, M) table SOA_GEMV_CONFIG, quantization.py:121-127): the launch
 * svq_gemv would make for this shape on the current device, as
 * plan[0..7] = {kernel (1 streaming, 2 chunked, 3 MFMA 16x16x32, 4 MFMA
 * 4x4x4), log2 lanes per row (MFMA: K splits), rows per lane group (MFMA
 * 16x16x32: 16-row tiles per wave; MFMA 4x4x4: rows per lane), waves per
 * workgroup, waves, workgroups, resident-wave capacity used for the choice
 * (MFMA: tile slots per workgroup), chunk units (chunked only)}.
 * Queries device attributes; launches nothing.
 */
int svq_gemv_plan(int m, int n, int k, int qtype, int32_t *plan);

/*
 * out[b * 32 + j] = weight j of block b, for b < nblocks, rounded from the
 * exact fp32 product to out_dtype: SVQ_F16 (0) or SVQ_F32 (1), i.e. an
 * out_is_fp32 flag, or SVQ_BF16 (2); round to nearest even. Replaces
 * `dequantize_soa` (quantization.py:93-105) on the GPU.
 */
int svq_dequant(const uint8_t *q, const uint16_t *s, void *out,
                int64_t nblocks, int qtype, int out_dtype, void *stream);

/*
 * Row gather + dequantize: out[i, :] = row ids[i] of the nrows x k matrix,
 * for i < nids (ids int64). Replaces the `index_select` + `dequantize_soa`
 * pair of `GGUFEmbedding.forward` (quantization.py:421-446). An id outside
 * [0, nrows) yields a row of NaN instead of a memory access.
 */
int svq_dequant_rows(const uint8_t *q, const uint16_t *s, const int64_t *ids,
                     int64_t nids, int64_t nrows, int k, void *out,
                     int qtype, int out_dtype, void *stream);

/*
 * Bytes of workspace svq_decode_attention needs for this shape (a negative
 * SVQ_E* code for an invalid one): the per-chunk partial results of the
 * attention, written and read within one call (no initialization needed).
 * Calls that share one workspace must not overlap (same stream, or ordered by
 * events).
 */
int64_t svq_decode_attention_workspace(int rows, int heads, int kv_heads, int span);

/*
 * Decode attention of one layer for one new token per row, fused with the
 * rotary embedding and the cache write. Replaces the decode branch of the
 * reference blocks: StarCoder2 (runtime_8b.py:38-55: `_rotate` of q and k,
 * `index_copy_` of k and v into slot `position`, `baddbmm` with the bias and
 * alpha = head_dim^-0.5, fp32 softmax, `bmm` with V) and GPTBigCode
 * multi-query (runtime_1b.py:30-45: no rotation, kv_heads = 1).
 *   qkv       fp16 [rows, qkv_stride]: q (heads x 128), then k and v
 *             (kv_heads x 128 each), as a fused q/k/v projection writes them
 *   cos, sin  fp16 [128] rotary tables of the position, or both NULL
 *   keys, values  fp16 [rows, kv_heads, capacity, 128] cache of this layer;
 *             slot *position of every (row, kv head) receives the new k / v
 *   position  device int64 scalar, 0 <= *position < span (a slot outside
 *             [0, span) is neither written nor attended)
 *   bias      fp16 [span] additive score bias (0 / -inf masks), or NULL
 *   window    > 0: slots j > *position or j <= *position - window are masked
 *             (-inf), the decode step's causal sliding window (runtime_8b.py:
 *             103-105), in addition to `bias`; <= 0: no such mask
 *   out       fp16 [rows, heads x 128]
 * Query head h attends key/value head h / (heads / kv_heads). Scores are
 * rounded to fp16 as the reference's fp16 baddbmm stores them; softmax and
 * the weighted sum run in fp32.
 */
int svq_decode_attention(const uint16_t *qkv, int64_t qkv_stride, const uint16_t *cos,
                         const uint16_t *sin, uint16_t *keys, uint16_t *values,
                         int64_t capacity, const int64_t *position, const uint16_t *bias,
                         int window, int span, uint16_t *out, int rows, int heads, int kv_heads,
                         int head_dim, float scale, void *workspace,
                         int64_t workspace_bytes, void *stream);

/*
 * Beam reorder of a decode cache, fused over rows: every row r whose parent
 * p = parents[r] differs from r takes the first `length` slots of every
 * (plane, head) of row p; rows may exchange caches (all sources are read
 * before any row is written). Replaces CachedDecoding.reorder
 * (runtime_shared.py:388-394), whose parents come from the host; here they
 * are a device array, so a beam step needs no host round trip.
 *   cache    fp16 [planes, rows, heads, capacity, head_dim] contiguous
 *            (16-byte aligned), e.g. every layer's keys at once
 *   parents  device int64 [rows]; a value outside [0, rows) leaves its row
 *            unchanged
 * rows <= SVQ_MAX_ROWS, head_dim == SVQ_HEAD_DIM, length <= capacity,
 * planes * heads <= 65535.
 */
int svq_cache_reorder(uint16_t *cache, int64_t planes, int rows, int heads, int64_t capacity,
                      int head_dim, int64_t length, const int64_t *parents, void *stream);

/*
 * Survivor selection of one beam-sampling step once the number of draws is
 * known (runtime_shared.py:233-262 without the finished-beam bookkeeping):
 *   1. draws = torch.multinomial(probs, draws) without replacement, as
 *      PyTorch computes it: the `draws` largest of probs / noise in
 *      descending order (ties: the smaller flat index first), over the
 *      candidate tokens only -- every other token must have probability 0;
 *   2. survivors = the drawn flat indices sorted by scores[pick] descending
 *      and stable, the first `beams` of them; when draws < beams the first
 *      survivor fills the rest, with running score -1e9;
 *   3. parents[b], tokens[b] = divmod(survivor b, vocab); running[b] =
 *      scores[survivor b];
 *   4. seen_out[b] = seen_in[parents[b]] with byte tokens[b] set to 1.
 *   probs, noise, scores  fp32 [beams * vocab] (noise: Exp(1) draws, > 0)
 *   candidates  int64 [beams, ncand]: token ids per beam, distinct per beam
 *   seen_in, seen_out  bool (one byte) [beams, seen_pitch], distinct buffers,
 *               16-byte aligned; seen_pitch >= vocab, a multiple of 16
 *   running, parents, tokens  [beams] outputs; tokens_copy: a second copy of
 *               tokens (e.g. the next step's input), or NULL
 *   compact     0: probs and scores are [beams * vocab]; 1: they are
 *               [beams, ncand] per candidate (svq_beam_candidates' outputs,
 *               ncand <= 64); noise is [beams * vocab] either way
 * beams <= 8, beams * ncand <= 1024, 1 <= draws <= min(2 * beams,
 * beams * ncand). Asynchronous on `stream`; exact (one fp32 division per
 * candidate, then comparisons and copies).
 */
int svq_beam_select(const float *probs, const float *noise, const float *scores,
                    const int64_t *candidates, int beams, int64_t vocab, int ncand, int draws,
                    const uint8_t *seen_in, uint8_t *seen_out, int64_t seen_pitch,
                    float *running, int64_t *parents, int64_t *tokens, int64_t *tokens_copy,
                    int compact, void *stream);

/*
 * Candidates of one beam-sampling step (runtime_shared.py:228-231), on each
 * beam row's kc largest warped log-probabilities instead of the whole
 * vocabulary: log_softmax of the fp16 logits in fp32, the repetition
 * penalty on seen tokens (v < 0 ? v * penalty : v / penalty), division by
 * the temperature (skipped at 1), top-k (every value below the k-th largest
 * becomes -inf), top-p over the kc values (softmax, sums from the smallest
 * up, removal where the sum <= 1 - top_p except the `keep` largest), plus
 * the beam's running score; then the softmax over all beams' candidates
 * jointly (the reference's softmax over the flattened [1, beams * vocab]
 * scores, whose other entries are -inf).
 *   logits      fp16 [beams, vocab]
 *   seen        bool [beams, seen_pitch]; seen_pitch >= vocab, a multiple of 16
 *   running     fp32 [beams]
 *   candidates  int64 [beams, kc] out: token ids, value descending, token ascending
 *   scores      fp32 [beams, kc] out: warped log-prob + running (-inf if removed)
 *   probs       fp32 [beams * kc] out: joint softmax of scores
 *   status      int64 [2 + beams] out: number of probs > 0, or -1 if any prob
 *               is NaN (torch.multinomial rejects such input); 1 if any row
 *               overflows (its kc-th largest value equals its k-th: the
 *               candidates may then miss tokens the reference keeps, and the
 *               caller must warp the whole vocabulary); then the flag per row
 *   workspace   svq_beam_candidates_workspace(beams, vocab, kc) bytes, 8-byte
 *               aligned, written and read within the call (no initialization)
 * beams <= 8, vocab <= 65536, 1 <= k <= kc <= min(64, vocab), keep <= kc.
 * Sums add in another order than torch's reductions: results agree with the
 * reference's to rounding. Asynchronous on `stream` (three kernels); calls
 * that share a workspace must not overlap. svq_beam_select with compact = 1
 * draws from these outputs.
 */
int svq_beam_candidates(const uint16_t *logits, const uint8_t *seen, int64_t seen_pitch,
                        const float *running, int beams, int vocab, int k, int kc, int keep,
                        float penalty, float temperature, double top_p, int64_t *candidates,
                        float *scores, float *probs, int64_t *status, void *workspace,
                        int64_t workspace_bytes, void *stream);

/* Bytes of workspace svq_beam_candidates needs (a negative SVQ_E* code for
 * an invalid shape). */
int64_t svq_beam_candidates_workspace(int beams, int vocab, int kc);

/*
 * GGUF container reader (host memory; no GPU needed). Replaces the PyPI
 * `gguf` GGUFReader the reference opens its checkpoints with
 * (gguf_support.py:101-121): GGUF versions 2 and 3, memory-mapped once,
 * every count, length and offset checked against the file before use.
 * writable_copy maps the file copy-on-write (the reference's mode "c"):
 * writes through the mapping stay private to the process.
 */
typedef struct svq_gguf svq_gguf;
int svq_gguf_open(const char *path, int writable_copy, svq_gguf **out);
void svq_gguf_close(svq_gguf *g);
int svq_gguf_version(const svq_gguf *g);
int64_t svq_gguf_alignment(const svq_gguf *g);

/* Metadata entries, in file order. For a string, value points at its bytes
 * (nbytes long, not NUL-terminated); for an array, at its first element, with
 * elem_type and count set (string elements keep their u64 length prefixes);
 * for a scalar, at its little-endian bytes. elem_type is -1 for non-arrays.
 * Pointers stay valid until svq_gguf_close. */
int64_t svq_gguf_kv_count(const svq_gguf *g);
int64_t svq_gguf_find_kv(const svq_gguf *g, const char *key); /* index or -1 */
int svq_gguf_kv(const svq_gguf *g, int64_t i, const char **key, int *type,
                const void **value, int64_t *nbytes, int *elem_type, int64_t *count);

/* Tensor infos, in file order: ggml type code, dims (dims[0] varies
 * fastest, unused dims 1), the byte offset of the data in the file and its
 * size. svq_gguf_find_tensor returns the first tensor of that name or -1. */
int64_t svq_gguf_tensor_count(const svq_gguf *g);
int64_t svq_gguf_find_tensor(const svq_gguf *g, const char *name);
int svq_gguf_tensor(const svq_gguf *g, int64_t i, const char **name, int *ggml_type,
                    int *n_dims, int64_t *dims, int64_t *data_offset, int64_t *nbytes);
const void *svq_gguf_tensor_data(const svq_gguf *g, int64_t i); /* NULL if out of range */

/*
 * AoS GGUF blocks -> the SoA arrays of `pack_gguf_soa` (quantization.py:67-90):
 * q[b * W ..] = block b without its 2 scale bytes, s[2b], s[2b + 1] = its fp16
 * scale bytes. Host memory; `threads` <= 0 uses the hardware threads.
 */
int svq_pack_soa(const uint8_t *aos, int64_t nblocks, int qtype, uint8_t *q, uint8_t *s,
                 int threads);

/*
 * Phase timeline of the streaming GEMV (libsvq_timeline.so only: the same
 * sources built with SVQ_TIMELINE; libsvq.so exports neither function). No
 * counterpart in the reference: profiling support for this library.
 *
 * svq_timeline_stamps: GEMV calls made after it (from any thread) write, for
 * every wave of the streaming MFMA kernel, 12 uint64 stamps of the 100 MHz
 * real-time clock to stamps[(linear workgroup * 4 + wave) * 12 ..]: entry,
 * x staged, first step done, first tile summed, end, the wave's tile count
 * (a count, not a time), x loads issued, work split known, and for a
 * LayerNorm staged from registers its mean known, variance known and
 * normalized x in LDS (else 0); the twelfth is unused. The buffer must hold
 * 48 uint64 per workgroup of the launch; NULL stops stamping.
 *
 * svq_timeline_read: a plain coalesced read of `bytes` (a multiple of 1024,
 * below 2^31) at p by `groups` workgroups of 4 waves, stamping entry and end
 * (stamps 0 and 4 of each wave) the same way; sink receives 256 uint32 per
 * workgroup.
 */
void svq_timeline_stamps(void *stamps);
int svq_timeline_read(const void *p, uint64_t bytes, int groups, void *sink, void *stamps,
                      void *stream);

#ifdef __cplusplus
}
#endif

#endif /* SVQ_H */
