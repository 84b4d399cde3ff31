/*
 * nmce.h -- C ABI of the MI355X (gfx950) vocabulary-parallel cross-entropy
 * library (libnmce.so).
 *
 * The library replaces the loss path of nano-megatron:
 *   nano_megatron/cross_entropy.py:16-85  (_VocabParallelCrossEntropy and
 *                                           vocab_parallel_cross_entropy)
 *   nano_megatron/model.py:169-192         (ParallelLMHead, fused variant)
 *
 * Conventions shared by every entry point:
 *   - All tensor pointers are device memory owned by the caller. Unless an
 *     entry point says otherwise the library never allocates, frees or
 *     synchronises; work is enqueued on `stream` (a hipStream_t, NULL = the
 *     legacy default stream).
 *   - A "row" is one token: the logits of row r start at logits + r*ld
 *     (elements) and hold `vocab_local` contiguous entries.
 *   - A shard covers global vocabulary ids [vocab_start, vocab_start+vocab_local).
 *     Targets are global ids (int64). A target outside the shard contributes
 *     nothing on that shard (the reference's target_mask, cross_entropy.py:28-36).
 *   - Return value: NMCE_OK (0), a negative NMCE_E* argument error, or a
 *     positive hipError_t reported by the launch.
 */
#ifndef NMCE_H
#define NMCE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element types of logits / gradients / hidden states / weights */
#define NMCE_F32 0
#define NMCE_BF16 1

/* status codes (negative: argument errors detected before any launch) */
#define NMCE_OK 0
#define NMCE_EINVAL_DTYPE (-1)
#define NMCE_EINVAL_SHAPE (-2)
#define NMCE_EINVAL_ALIGN (-3)
#define NMCE_EINVAL_PTR (-4)
#define NMCE_EINVAL_TP (-5)
#define NMCE_EINVAL_WORKSPACE (-6)
#define NMCE_EINVAL_SCRATCH (-7)

/* Rows covered by one int32 count of nmce_validate_targets. */
#define NMCE_VALIDATE_ROWS_PER_SLOT 1024

/* Human-readable text for a status code (static storage). */
const char* nmce_status_string(int status);

/* Library version, (major << 16) | minor. */
int nmce_version(void);

/*
 * Per-shard row statistics, one read pass over the shard's logits.
 * Replaces cross_entropy.py:21 (row max), :28-36 (masked target pick) and
 * :40-41 (exp-sum) for one vocabulary shard.
 *
 *   row_max[r]       = max_j x[r, j]                            (fp32)
 *   row_sumexp_m1[r] = sum_j exp(x[r, j] - row_max[r]) - 1      (fp32)
 *   target_logit[r]  = x[r, target[r]-vocab_start] if the target is in this
 *                      shard, else 0.0  (raw logit, not shifted)
 * The exp-sum is carried minus the maximum's own term (exactly 1), so that
 * for a confident token, whose other terms are all small, it keeps its
 * relative precision; the loss is formed from it with log1p, and a target
 * at the maximum gets the gradient -(sum - 1)/sum * g from it directly. For
 * fp32 logits the sum is accumulated with
 * the terms equal to 1 kept apart (relative error a few 2^-24); bf16 rows
 * accumulate the plain sum and subtract 1 per lane (absolute error a few
 * 2^-24), which keeps the bf16 pass within its memory-bound time.
 * A row whose shard holds only -inf gives row_max = -1e38 and
 * row_sumexp_m1 = -1 (an empty sum), which the combine gives no weight.
 * dtype: NMCE_F32 or NMCE_BF16 (math is fp32 either way).
 */
int nmce_ce_fwd_stats(const void* logits, int dtype, int64_t n_rows,
                      int64_t vocab_local, int64_t ld, const int64_t* target,
                      int64_t vocab_start, float* row_max, float* row_sumexp_m1,
                      float* target_logit, void* stream);

/*
 * Single-shard forward (TP=1): the statistics pass with the combine folded
 * in. Same results as nmce_ce_fwd_stats(vocab_start = 0) followed by
 * nmce_ce_combine(tp = 1), bit for bit, in one read pass and one launch.
 * Replaces cross_entropy.py:17-50 at world_size == 1.
 *   g_max[r], g_sumexp_m1[r], loss[r] as defined for nmce_ce_combine.
 */
int nmce_ce_fwd(const void* logits, int dtype, int64_t n_rows, int64_t vocab,
                int64_t ld, const int64_t* target, float* loss, float* g_max,
                float* g_sumexp_m1, void* stream);

/*
 * Cross-shard combine of per-shard statistics, done locally.
 * Replaces the three TP all-reduces and the loss line of cross_entropy.py
 * (:22-23 MAX, :37-38 SUM of the target logit, :42-43 SUM of exp-sums, :45).
 *
 * Shard k's statistic for row r sits at [k*shard_stride + r] of each input
 * (a [tp, ...] stack, e.g. the all-gathered [tp, 3, n_rows] buffer of a real
 * TP group with row_max = base, row_sumexp_m1 = base + n_rows, target_logit =
 * base + 2*n_rows and shard_stride = 3*n_rows).
 *
 *   g_max[r]       = max_k row_max[k, r]
 *   g_sumexp_m1[r] = sum_k (1 + row_sumexp_m1[k, r]) * exp(row_max[k, r] - g_max[r]) - 1
 *                    (formed without the cancellation: a shard at the maximum
 *                    adds its row_sumexp_m1, each further one its full sum)
 *   loss[r]        = log1p(g_sumexp_m1[r]) - (sum_k target_logit[k, r] - g_max[r])
 * Any of loss / g_max / g_sumexp_m1 may be NULL if not wanted.
 */
int nmce_ce_combine(const float* row_max, const float* row_sumexp_m1,
                    const float* target_logit, int tp, int64_t shard_stride,
                    int64_t n_rows, float* loss, float* g_max, float* g_sumexp_m1,
                    void* stream);

/*
 * Target validation (cross_entropy.py:79-81: every target must lie in
 * [0, vocab_total)). Writes nmce_validate_slots(n_rows) int32 counts of bad
 * targets, one per NMCE_VALIDATE_ROWS_PER_SLOT rows; every slot is written,
 * so the buffer needs no clearing. The caller raises if any count is nonzero.
 * bad_counts may be device memory or pinned host memory (hipHostMalloc,
 * which the device addresses at its host address): the Python host writes
 * the counts straight to the host that way, with no copy after the kernel.
 */
int64_t nmce_validate_slots(int64_t n_rows);
int nmce_validate_targets(const int64_t* target, int64_t n_rows,
                          int64_t vocab_total, int32_t* bad_counts,
                          void* stream);

/*
 * The same check (cross_entropy.py:79-81) in one workgroup, for a loss
 * kernel that follows on the same stream and must leave its inputs untouched
 * on a bad target (the reference raises before touching anything, :80-81):
 * the number of bad targets, saturated at INT32_MAX, goes to bad_count[0]
 * (for the host; device or pinned host memory) and to bad_flag[0] (device
 * memory, passed to nmce_ce_fwd_bwd as target_bad). Both are written
 * unconditionally, so neither needs clearing.
 */
int nmce_validate_targets_once(const int64_t* target, int64_t n_rows,
                               int64_t vocab_total, int32_t* bad_count,
                               int32_t* bad_flag, void* stream);

/*
 * Backward over one shard: grad = (softmax - onehot(target)) * grad_output.
 * Replaces cross_entropy.py:53-65 plus the autograd cast back to the logits
 * dtype (the .float() at :83).
 *
 *   grad[r, j] = (exp(x[r, j] - g_max[r]) / (1 + g_sumexp_m1[r])
 *                 - [j == target[r] - vocab_start]) * grad_output[r*gout_stride]
 * with the target column, when it holds the row maximum, formed as
 *   -g_sumexp_m1[r] / (1 + g_sumexp_m1[r]) * g,
 * the same value without the cancellation of softmax - 1 near 1 (a target
 * below the maximum has softmax <= 1/2, where the plain form is exact enough).
 * gout_stride = 0 broadcasts grad_output[0] to every row (the loss.mean()
 * case). grad may equal logits (in place, ld_grad == ld); otherwise the two
 * must not overlap. grad has the same dtype as logits.
 */
int nmce_ce_bwd(const void* logits, void* grad, int dtype, int64_t n_rows,
                int64_t vocab_local, int64_t ld, int64_t ld_grad,
                const int64_t* target, int64_t vocab_start, const float* g_max,
                const float* g_sumexp_m1, const float* grad_output,
                int64_t gout_stride, void* stream);

/*
 * nmce_ce_bwd with the upstream gradient divided by gout_div (> 0) per row:
 * grad_output[r*gout_stride] / gout_div replaces grad_output[r*gout_stride].
 * With gout_stride = 0 and gout_div = N this is the backward of
 * loss.mean() (cross_entropy.py:85) folded in: the scalar gradient of the
 * mean is read directly, and the per-token value is the same fp32 quotient
 * torch's MeanBackward forms, so the result is bit-identical to nmce_ce_bwd
 * on the expanded gradient. gout_div = 1 is nmce_ce_bwd.
 */
int nmce_ce_bwd_scaled(const void* logits, void* grad, int dtype, int64_t n_rows,
                       int64_t vocab_local, int64_t ld, int64_t ld_grad,
                       const int64_t* target, int64_t vocab_start, const float* g_max,
                       const float* g_sumexp_m1, const float* grad_output,
                       int64_t gout_stride, float gout_div, void* stream);

/*
 * nmce_ce_bwd_scaled with gout_stride = 0, after nmce_ce_fwd_bwd. `assumed`
 * (device, one float) is the upstream value that forward computed the
 * gradient for: when grad_output[0] equals it every workgroup returns at
 * once, leaving `grad` as written; otherwise this is nmce_ce_bwd_scaled
 * exactly (cross_entropy.py:53-65 with the mean of :85). grad_output[0] is
 * also written to `observed` (device, one float; may be NULL), which a
 * caller can pass as the next forward's grad_expected.
 */
int nmce_ce_bwd_scaled_unless(const void* logits, void* grad, int dtype, int64_t n_rows,
                              int64_t vocab_local, int64_t ld, int64_t ld_grad,
                              const int64_t* target, int64_t vocab_start, const float* g_max,
                              const float* g_sumexp_m1, const float* grad_output, float gout_div,
                              const float* assumed, float* observed, void* stream);

/*
 * One-pass forward and backward at TP = 1 (cross_entropy.py:17-65 with the
 * mean of :85, world_size == 1). Each row is read once and held on chip; the
 * kernel writes g_max, g_sumexp_m1 and loss, and the gradient for the
 * upstream value u of the mean (u / gout_div per token) into `grad`, where
 * u = grad_expected[0], or 1.0 when that is zero, subnormal, infinite or NaN;
 * u goes to grad_assumed[0]. Both are device pointers to one float. `grad`
 * is either a separate buffer or the logits themselves (grad == logits,
 * ld_grad == ld): the row's target logit is read before the row is
 * overwritten. Every output is bit-identical to nmce_ce_fwd followed by
 * nmce_ce_bwd_scaled with grad_output = {u} and gout_stride = 0.
 * The backward is then, for a separate buffer,
 * nmce_ce_bwd_scaled_unless(..., assumed = grad_assumed, ...), which
 * rewrites `grad` from the logits only when the real upstream value differs;
 * in place, nmce_ce_grad_rescale_unless.
 * Requirements: vocab a whole number of 16-byte vectors and at most
 * nmce_ce_fwd_bwd_max_vocab(dtype) (131072 bf16, 65536 fp32); logits, grad
 * and both row strides 16-byte aligned. No counterpart call in the reference,
 * whose forward likewise computes the softmax that its backward returns.
 * target_bad (may be NULL): the bad_flag of nmce_validate_targets_once,
 * enqueued before on the same stream. When it is nonzero the kernel writes
 * nothing at all, so logits that were to receive their gradient in place
 * are left as they were.
 */
int64_t nmce_ce_fwd_bwd_max_vocab(int dtype);
int nmce_ce_fwd_bwd(const void* logits, void* grad, int dtype, int64_t n_rows, int64_t vocab,
                    int64_t ld, int64_t ld_grad, const int64_t* target, float* loss, float* g_max,
                    float* g_sumexp_m1, const float* grad_expected, float* grad_assumed,
                    const int32_t* target_bad, float gout_div, void* stream);

/*
 * Backward after an in-place nmce_ce_fwd_bwd (grad == logits), whose
 * gradient was written for the upstream value assumed[0]: when
 * grad_output[0] equals it, every workgroup returns at once; otherwise every
 * entry of `grad` is multiplied by grad_output[0] / assumed[0] in fp32 and
 * rounded back to the gradient's dtype (cross_entropy.py:64: the gradient is
 * linear in grad_output). The logits are gone, so this cannot recompute; the
 * result is within four (fp32) or two (bf16) units in the last place of the
 * recomputed one, and equal to it when the ratio is a power of two.
 * grad_output[0] also goes to `observed` (may be NULL), the next forward's
 * grad_expected. Same layout requirements as nmce_ce_fwd_bwd.
 */
int nmce_ce_grad_rescale_unless(void* grad, int dtype, int64_t n_rows, int64_t vocab,
                                int64_t ld_grad, const float* grad_output, const float* assumed,
                                float* observed, void* stream);

/*
 * Measurement support (no counterpart in the reference): a plain copy of
 * `bytes` (multiple of 16, both pointers 16-byte aligned) with the loss
 * kernels' access pattern -- 16-byte non-temporal loads and stores. Its HBM
 * traffic is known exactly, so hardware byte counters (FETCH_SIZE,
 * WRITE_SIZE) read for it give the scale factors for the same counters read
 * on the loss kernels.
 */
int nmce_stream_copy(const void* src, void* dst, int64_t bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Fused LM head + cross entropy (bf16 only).
 *
 * Replaces ParallelLMHead.forward's projection logits = hidden @ weight.t()
 * (model.py:192, bf16 under autocast per model.py:255-257) followed by the
 * loss of cross_entropy.py:16-65, without storing the [n_rows, vocab_local]
 * logits. hidden is [n_rows, hidden_size] and weight (the vocabulary shard of
 * the tied embedding, tp_layers.py:108) is [vocab_local, hidden_size], both
 * row-major with row stride hidden_size, 16-byte aligned; hidden_size must be
 * a multiple of 64. Logits are accumulated in fp32 and not rounded to bf16.
 * --------------------------------------------------------------------------- */

/* Device workspace bytes needed by nmce_lmhead_ce_fwd_stats. */
int64_t nmce_lmhead_ce_fwd_workspace_bytes(int64_t n_rows, int64_t hidden_size,
                                           int64_t vocab_local);

/*
 * Per-shard statistics of the logits hidden @ weight^T, as nmce_ce_fwd_stats
 * computes them for a stored logit slab (cross_entropy.py:21, :28-36,
 * :40-41 on the shard [vocab_start, vocab_start + vocab_local)), the exp-sum
 * minus one accumulated with the terms equal to 1 kept apart. Combine the
 * shards with nmce_ce_combine (tp = 1 for a single shard).
 */
int nmce_lmhead_ce_fwd_stats(const void* hidden, const void* weight, int dtype, int64_t n_rows,
                             int64_t hidden_size, int64_t vocab_local, const int64_t* target,
                             int64_t vocab_start, float* row_max, float* row_sumexp_m1,
                             float* target_logit, void* workspace, int64_t workspace_bytes,
                             void* stream);

/*
 * nmce_lmhead_ce_fwd_stats without a workspace argument, for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). No counterpart in the reference.
 * The partial statistics go to a fixed 64 MiB device array inside the
 * library (one per GPU, held until the process ends), and the tokens are
 * processed in as many launches as it takes to fit them there; the results
 * are bit-identical to nmce_lmhead_ce_fwd_stats. The call allocates nothing.
 * Limit: 3 * ceil(vocab_local / 128) * 4 bytes per token must fit in 64 MiB
 * (vocab_local up to 715,827,840); beyond that it returns
 * NMCE_EINVAL_SCRATCH before launching anything. Every call on one GPU uses
 * the same array: calls that overlap on one GPU (different streams, or
 * threads) race and must be serialised by the caller.
 */
int nmce_lmhead_ce_fwd_stats_noalloc(const void* hidden, const void* weight, int dtype,
                                     int64_t n_rows, int64_t hidden_size, int64_t vocab_local,
                                     const int64_t* target, int64_t vocab_start, float* row_max,
                                     float* row_sumexp_m1, float* target_logit, void* stream);

/* Device workspace bytes needed by nmce_lmhead_ce_bwd for a vocabulary chunk
 * of vocab_chunk rows (<= 0: the whole shard in one chunk). */
int64_t nmce_lmhead_ce_bwd_workspace_bytes(int64_t n_rows, int64_t hidden_size,
                                           int64_t vocab_local, int64_t vocab_chunk);

/*
 * Backward workspace layout (all values in elements of int64), written to
 * layout[0 .. NMCE_LMHEAD_LAYOUT_FIELDS-1]:
 *   [0] total workspace bytes
 *   [1] ldt      tokens rounded up to 64 (row stride of X^T and dZ^T)
 *   [2] vpad     vocab_local rounded up to 256 (row stride of W^T)
 *   [3] chunk    vocabulary rows per chunk (multiple of 256)
 *   [4] n_chunks
 *   [5] byte offset of X^T   bf16 [hidden_size, ldt], zero beyond n_rows
 *   [6] byte offset of W^T   bf16 [hidden_size, vpad], zero beyond vocab_local
 *   [7] byte offset of dZ^T  bf16 [chunk, ldt] of the current chunk
 *   [8] byte offset of dZ    bf16 [n_rows, chunk] of the current chunk
 *   [9] byte offset of the fp32 [n_rows, hidden_size] accumulator of
 *       nmce_lmhead_ce_bwd (present when n_chunks > 1)
 */
#define NMCE_LMHEAD_LAYOUT_FIELDS 10
int nmce_lmhead_ce_bwd_layout(int64_t n_rows, int64_t hidden_size, int64_t vocab_local,
                              int64_t vocab_chunk, int64_t* layout);

/* Step 1 of a caller-driven backward: X^T and W^T into the workspace. */
int nmce_lmhead_ce_bwd_prepare(const void* hidden, const void* weight, int dtype, int64_t n_rows,
                               int64_t hidden_size, int64_t vocab_local, int64_t vocab_chunk,
                               void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Step 2, once per chunk c (rows [c*chunk, c*chunk + chunk) of the shard):
 * recompute that slice of the logits and write the logit gradient
 *   dZ[r, j] = (exp(z[r, j] - g_max[r]) / (1 + g_sumexp_m1[r])
 *               - [j == target[r] - vocab_start]) * grad_output[r*gout_stride]
 * (target column without cancellation, as in nmce_ce_bwd)
 * as bf16 into the workspace's dZ^T and dZ (zeros in their padding). The
 * caller then forms grad_weight rows = dZ^T_c X and grad_hidden += dZ_c W_c
 * (e.g. with a library GEMM on X^T and W^T) before the next chunk overwrites
 * them. This is the fused part of cross_entropy.py:53-65 + the matmul
 * backward of model.py:192.
 */
int nmce_lmhead_ce_bwd_dz(const void* hidden, const void* weight, int dtype, int64_t n_rows,
                          int64_t hidden_size, int64_t vocab_local, const int64_t* target,
                          int64_t vocab_start, const float* g_max, const float* g_sumexp_m1,
                          const float* grad_output, int64_t gout_stride, int64_t vocab_chunk,
                          int64_t chunk_index, void* workspace, int64_t workspace_bytes,
                          void* stream);

/*
 * Backward of the fused LM head + loss (cross_entropy.py:53-65 followed by
 * the matmul backward of model.py:192):
 *   dZ[r, j]        = (exp(z[r, j] - g_max[r]) / (1 + g_sumexp_m1[r])
 *                      - [j == target[r] - vocab_start]) * grad_output[r*gout_stride]
 *   grad_hidden     = dZ @ weight          [n_rows, hidden_size] bf16
 *   grad_weight     = dZ^T @ hidden        [vocab_local, hidden_size] bf16
 * with z = hidden @ weight^T recomputed chunk by chunk (vocab_chunk rows of
 * the shard at a time) and dZ rounded to bf16 before the two products, as the
 * reference's autocast matmul backward consumes a bf16 gradient. g_max and
 * g_sumexp_m1 are the combined statistics of the forward (nmce_ce_combine).
 * grad_hidden is this shard's contribution only (the TP all-reduce of the
 * input gradient, mappings.py:83-94, belongs to the caller).
 */
int nmce_lmhead_ce_bwd(const void* hidden, const void* weight, int dtype, int64_t n_rows,
                       int64_t hidden_size, int64_t vocab_local, const int64_t* target,
                       int64_t vocab_start, const float* g_max, const float* g_sumexp_m1,
                       const float* grad_output, int64_t gout_stride, void* grad_hidden,
                       void* grad_weight, int64_t vocab_chunk, void* workspace,
                       int64_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * One-pass fused LM head + loss: forward and backward in the forward, for
 * the upstream value the caller assumes (bf16 only; same operand layout as
 * above). The tokens go in chunks of token_chunk (rounded up to 256; <= 0:
 * all at once). Per chunk the statistics GEMM keeps its exponentials
 * P = exp(z - block max) in the workspace; once the chunk's statistics are
 * combined across the TP group, dZ follows from P by one factor per
 * (128-row block, token), in place, and the dX rows of the chunk and its
 * share of dW are formed by libnmce's GEMM, which reads dZ^T and the weight
 * as they lie and the chunk's hidden rows transposed (hidden_size x
 * token_chunk bf16). The one buffer that grows with both sizes is a chunk's
 * P, then dZ^T: bf16 [vocab_local, token_chunk], the size of the bf16 logits
 * when the chunk holds every token. The logits are computed once: 6 * n_rows * vocab_local *
 * hidden_size flops in all. vocab_local is at most 8388352 (65535 blocks of
 * 128 rows once padded to 256); a larger shard is NMCE_EINVAL_SHAPE.
 * Replaces model.py:192 followed by cross_entropy.py:17-65 and the matmul
 * backward of model.py:192; with a caller that assumes the right upstream
 * value, as the reference's forward computes the softmax its backward
 * returns (cross_entropy.py:48-49).
 * --------------------------------------------------------------------------- */

/*
 * Workspace layout (int64 values) written to layout[0 .. 11]:
 *   [0] total bytes  [1] chunk (tokens per chunk)  [2] n_chunks
 *   [3] ldt (chunk padded to 64)  [4] vpad (vocab_local padded to 256)
 *   [5] nb (ceil(vocab_local / 128))  [6..9] byte offsets of P^T
 *   (= dZ_c^T, [vpad, ldt]: the only buffer that grows with the vocabulary
 *   and the chunk; both backward products read it), the partial statistics,
 *   the fp32 dW accumulator (present when n_chunks > 1) and the fp32 partials
 *   of a chunk's dX product when it is split over K  [10] the number of K
 *   ranges of that product (1: not split; more when a chunk's dX has too few
 *   256x256 tiles to fill the current device's compute units)  [11] byte
 *   offset of the chunk's hidden rows transposed, X_c^T [hidden_size, ldt]
 *   bf16 (the dW product's second operand), which runs to the end.
 */
#define NMCE_LMHEAD_FUSED_LAYOUT_FIELDS 12
int nmce_lmhead_ce_fused_layout(int64_t n_rows, int64_t hidden_size, int64_t vocab_local,
                                int64_t token_chunk, int64_t* layout);

/* assumed[0] = hint[0], or 1.0 when hint[0] is zero, subnormal, infinite or
 * NaN (a gradient written for such a value could not be rescaled). Both are
 * device pointers to one float. */
int nmce_hint_assume(const float* hint, float* assumed, void* stream);

/*
 * Chunk c (tokens [c*chunk, min((c+1)*chunk, n_rows))): this shard's
 * statistics of those tokens, as nmce_lmhead_ce_fwd_stats computes them,
 * written at the tokens' positions of row_max / row_sumexp_m1 /
 * target_logit ([n_rows] each), and P of the chunk kept in the workspace.
 * Chunks run in order 0, 1, ..., each followed by its
 * nmce_lmhead_ce_fused_chunk_grads.
 */
int nmce_lmhead_ce_fused_chunk_stats(const void* hidden, const void* weight, int dtype,
                                     int64_t n_rows, int64_t hidden_size, int64_t vocab_local,
                                     const int64_t* target, int64_t vocab_start,
                                     int64_t token_chunk, int64_t chunk_index, float* row_max,
                                     float* row_sumexp_m1, float* target_logit, void* workspace,
                                     int64_t workspace_bytes, void* stream);

/*
 * Chunk c's gradients, given the combined statistics g_max / g_sumexp_m1 of
 * its tokens (nmce_ce_combine over the TP group) and this shard's
 * target_logit from nmce_lmhead_ce_fused_chunk_stats:
 *   dZ[t, v]          = (softmax - onehot) * grad_output[t*gout_stride] / gout_div
 *                       (target column as in nmce_ce_bwd), rounded to bf16
 *   grad_hidden rows  = dZ_c @ weight                 (this shard's share)
 *   grad_weight      += dZ_c^T @ hidden_c             (fp32 across chunks,
 *                       bf16 when the last chunk is done)
 * grad_hidden is [n_rows, hidden_size], grad_weight [vocab_local,
 * hidden_size], both bf16.
 */
int nmce_lmhead_ce_fused_chunk_grads(const void* hidden, const void* weight, int dtype,
                                     int64_t n_rows, int64_t hidden_size, int64_t vocab_local,
                                     const int64_t* target, int64_t vocab_start,
                                     int64_t token_chunk, int64_t chunk_index, const float* g_max,
                                     const float* g_sumexp_m1, const float* target_logit,
                                     const float* grad_output, int64_t gout_stride,
                                     float gout_div, void* grad_hidden, void* grad_weight,
                                     void* workspace, int64_t workspace_bytes, void* stream);

/*
 * The GEMM core of the fused path, exposed for testing and measurement (no
 * counterpart in the reference): c[i, j] = sum_l a[i, l] * b[j, l] for
 * i < m, j < n, l < k, with bf16 a [m, lda] and b [n, ldb], fp32
 * accumulation, and c [m, ldc] written as c_dtype (NMCE_BF16 or NMCE_F32).
 * k must be a multiple of 64; a and b 16-byte aligned, lda and ldb multiples
 * of 8.
 */
int nmce_gemm_nt_bf16(const void* a, int64_t lda, const void* b, int64_t ldb, int64_t m,
                      int64_t n, int64_t k, void* c, int c_dtype, int64_t ldc, void* stream);

/*
 * The same core with b MN-contiguous, as the fused backward products read
 * their operands (no counterpart in the reference; for tests):
 * c[i, j] = sum_l a(i, l) * b[l, j] with b [k, ldb], and a[i, l] ([m, lda],
 * K-contiguous) or, when a_mn, a[l, i] ([k, lda], MN-contiguous); bf16 c.
 * MN-contiguous operands need ld >= (columns rounded up to 8), 64 * ld < 2^31.
 * Bit-identical to nmce_gemm_nt_bf16 on the transposed operands.
 */
int nmce_gemm_mn_bf16(int a_mn, const void* a, int64_t lda, const void* b, int64_t ldb,
                      int64_t m, int64_t n, int64_t k, void* c, int64_t ldc, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NMCE_H */
