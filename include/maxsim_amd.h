/*
 * maxsim_amd.h -- C ABI of the MI355X (gfx950) MaxSim engine.
 *
 *   score(q, d) = sum_i max_j <q_i, d_j>        (fp32 accumulate, fp32 out)
 *
 * One entry point per operator of the reference's torch extension
 * (torch-ext/torch_binding.cpp:7-90, documented in torch-ext/torch_binding.h).
 * Every entry point:
 *   - takes raw DEVICE pointers, int64 sizes, a dtype tag and a HIP stream
 *     (pass a hipStream_t cast to void*; NULL = the null stream);
 *   - never allocates or frees memory; the only state kept between calls is
 *     per device and read-only to callers: cached device attributes (CU
 *     count, LDS limit, raised kernel LDS limits) and the address of the
 *     scratch array of maxsim_amd_packed_backward_typed_noalloc;
 *   - is asynchronous on `stream` (no host synchronisation);
 *   - returns MAXSIM_OK or an error code; maxsim_amd_last_error() then gives
 *     a message (thread-local, valid until the next call on that thread).
 *
 * Layout conventions (all arrays contiguous, row-major):
 *   embeddings : [rows, dim] of `dtype`; rows of one query / document are
 *                consecutive.
 *   offsets    : int32 CSR offsets, [n + 1], offsets[0] == 0.
 *   ids        : int32.
 *   argmax     : int32, one slot per (pair, query token); slots beyond a
 *                pair's real query length are written as 0.
 *   grads      : fp32 (the *_typed entry points can write the input dtype
 *                instead), shaped like the embeddings they belong to; every
 *                element is written (callers need not zero them).
 *
 * Semantics shared by all forward entry points (reference maxsim.cu:412-443,
 * tests/test_nan_inf.py): documents are scanned in ascending token order with
 * a strict `>` (first index wins ties); NaN similarities never win, so a
 * query token whose similarities are all NaN contributes -inf and argmax 0.
 * Pairs whose offsets / ids / lengths are invalid are not read; their score
 * is NaN and their argmax slots are 0.
 */
#ifndef MAXSIM_AMD_H_
#define MAXSIM_AMD_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  MAXSIM_FLOAT32 = 0,
  MAXSIM_FLOAT16 = 1,
  MAXSIM_BFLOAT16 = 2
} maxsim_dtype;

enum {
  MAXSIM_OK = 0,
  MAXSIM_ERR_INVALID = 1,     /* bad argument (null pointer, negative size...) */
  MAXSIM_ERR_UNSUPPORTED = 2, /* valid but outside what this build supports   */
  MAXSIM_ERR_LAUNCH = 3       /* the HIP runtime rejected a launch            */
};

/* Largest embedding dimension the kernels accept.  Dims up to 256 keep the
 * query blocks in registers (the fast paths); wider rows are streamed in
 * K-chunks by the forward and in slice chunks by the backward. */
#define MAXSIM_AMD_MAX_DIM 16384

int maxsim_amd_abi_version(void);
const char* maxsim_amd_last_error(void);

/* ---- Packed ragged pairs ------------------------------------------------ */

/* Replaces op `maxsim_forward` (torch_binding.h:21-27, maxsim.cu:819-922).
 * queries [total_q_tokens, dim], query_offsets [num_queries+1],
 * documents [total_d_tokens, dim], document_offsets [num_documents+1],
 * pair_query_ids / pair_document_ids [num_pairs] -> scores [num_pairs].
 * max_q_len > 0 bounds every query segment length (longer pairs are invalid). */
int maxsim_amd_forward(maxsim_dtype dtype, const void* queries,
                       int64_t total_q_tokens, const int32_t* query_offsets,
                       int64_t num_queries, const void* documents,
                       int64_t total_d_tokens, const int32_t* document_offsets,
                       int64_t num_documents, const int32_t* pair_query_ids,
                       const int32_t* pair_document_ids, int64_t num_pairs,
                       int64_t dim, int64_t max_q_len, float* scores,
                       void* stream);

/* Replaces op `maxsim_packed_forward_with_argmax` (torch_binding.h:101-108,
 * maxsim.cu:2039-2108).  As above plus argmax [num_pairs, max_q_len]. */
int maxsim_amd_packed_forward_with_argmax(
    maxsim_dtype dtype, const void* queries, int64_t total_q_tokens,
    const int32_t* query_offsets, int64_t num_queries, const void* documents,
    int64_t total_d_tokens, const int32_t* document_offsets,
    int64_t num_documents, const int32_t* pair_query_ids,
    const int32_t* pair_document_ids, int64_t num_pairs, int64_t dim,
    int64_t max_q_len, float* scores, int32_t* argmax, void* stream);

/* Bytes of device workspace that let maxsim_amd_packed_forward_with_argmax_ws
 * score the pairs document by document: R + 16384 + num_documents, where R
 * is 64 * (ceil(num_pairs / 4) + min(num_documents, num_pairs)) + 16 +
 * 8 * num_documents + 4 * num_pairs rounded up to a multiple of 16.  No
 * counterpart
 * in the reference, whose packed forward scores the pairs in the caller's
 * order. */
size_t maxsim_amd_packed_forward_workspace_size(int64_t num_documents, int64_t num_pairs);

/* Replaces ops `maxsim_packed_forward_with_argmax` (torch_binding.h:101-108,
 * maxsim.cu:2039-2108) and, with argmax NULL, `maxsim_forward`
 * (torch_binding.h:21-27), like the two entry points above, with a
 * workspace (device memory, 16-byte aligned, at least
 * maxsim_amd_packed_forward_workspace_size() bytes): the pairs are grouped by
 * document on the device and each document's rows are read from memory once
 * per four of its pairs rather than once per pair.  Taken for 16-bit inputs
 * of dim 64 or 128 with max_q_len <= 64, at most 16384 documents and at
 * least 4096 pairs; otherwise, or with a NULL, misaligned or smaller
 * workspace, this is the entry point without one.  Same results, bit for
 * bit, either way. */
int maxsim_amd_packed_forward_with_argmax_ws(
    maxsim_dtype dtype, const void* queries, int64_t total_q_tokens,
    const int32_t* query_offsets, int64_t num_queries, const void* documents,
    int64_t total_d_tokens, const int32_t* document_offsets,
    int64_t num_documents, const int32_t* pair_query_ids,
    const int32_t* pair_document_ids, int64_t num_pairs, int64_t dim,
    int64_t max_q_len, float* scores, int32_t* argmax, void* workspace,
    size_t workspace_bytes, void* stream);

/* Bytes of device workspace that let maxsim_amd_packed_backward group the
 * pairs by query and by document on the device and compute each gradient
 * row once, without floating-point atomics: 4 * (2 * num_queries + 1 +
 * 2 * num_documents + 1 + 2 * num_pairs).  No counterpart in the reference,
 * whose backward zero-fills the gradients and accumulates with atomics. */
size_t maxsim_amd_packed_backward_workspace_size(int64_t num_queries, int64_t num_documents,
                                                 int64_t num_pairs);

/* Replaces op `maxsim_packed_backward` (torch_binding.h:112-121,
 * maxsim.cu:2201-2286).  dscore [num_pairs] fp32, argmax [num_pairs,
 * max_q_len] -> dqueries [total_q_tokens, dim], ddocuments [total_d_tokens,
 * dim], both fp32.
 * With `workspace` (device memory, 4-byte aligned) of at least
 * maxsim_amd_packed_backward_workspace_size() bytes and max_q_len < 65536,
 * the gradients are computed per query and per document, each row written
 * once (rows before the first and after the last segment are zeroed); the
 * offsets must then be non-decreasing, since rows of overlapping segments
 * are owned twice.  NULL or a smaller workspace selects the zero-fill + fp32
 * atomics path. */
int maxsim_amd_packed_backward(
    maxsim_dtype dtype, const float* dscore, const void* queries,
    int64_t total_q_tokens, const int32_t* query_offsets, int64_t num_queries,
    const void* documents, int64_t total_d_tokens,
    const int32_t* document_offsets, int64_t num_documents,
    const int32_t* pair_query_ids, const int32_t* pair_document_ids,
    int64_t num_pairs, const int32_t* argmax, int64_t max_q_len, int64_t dim,
    float* dqueries, float* ddocuments, void* workspace, size_t workspace_bytes,
    void* stream);

/* maxsim_amd_packed_backward with the gradients written in `grad_dtype`:
 * MAXSIM_FLOAT32, or the input dtype, in which case each element is the
 * fp32 sum rounded to nearest even, as casting the fp32 gradients would
 * give (up to the fp32 summation order, which varies between runs for the
 * document gradient).  No counterpart in the reference: its autograd
 * Function (torch-ext/maxsim/__init__.py:445-454) returns fp32 gradients
 * and autograd casts them to the input dtype in a separate pass; writing the
 * input dtype directly removes that pass and halves the gradient writes.  A
 * 16-bit grad_dtype needs the grouped path (the workspace and
 * max_q_len < 65536) when num_pairs > 0; without it the call returns
 * MAXSIM_ERR_UNSUPPORTED before launching anything. */
int maxsim_amd_packed_backward_typed(
    maxsim_dtype dtype, maxsim_dtype grad_dtype, const float* dscore, const void* queries,
    int64_t total_q_tokens, const int32_t* query_offsets, int64_t num_queries,
    const void* documents, int64_t total_d_tokens,
    const int32_t* document_offsets, int64_t num_documents,
    const int32_t* pair_query_ids, const int32_t* pair_document_ids,
    int64_t num_pairs, const int32_t* argmax, int64_t max_q_len, int64_t dim,
    void* dqueries, void* ddocuments, void* workspace, size_t workspace_bytes,
    void* stream);

/* maxsim_amd_packed_backward_typed without a workspace argument and without
 * any allocation: the pair grouping lists live in a file-scope device array
 * of the library (16 MiB per device), so the call allocates nothing and its
 * kernels take that array's address.  The HIP runtime allocates the array
 * when it loads the library's code object on a device: every process that
 * loads the library holds 16 MiB on each device it uses, until it ends,
 * whether or not it calls this entry point.
 * No counterpart in the reference.  It is for callers that cannot allocate
 * device memory: code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc.  Limit: 2 * num_queries +
 * 2 * num_documents + 2 * num_pairs + 2 <= 4,194,304 (else
 * MAXSIM_ERR_UNSUPPORTED before anything is launched).  Every call on one
 * device shares that device's array: calls that overlap on one device (two
 * streams, two threads) race, so serialise them.  Same results as
 * maxsim_amd_packed_backward_typed with a workspace. */
int maxsim_amd_packed_backward_typed_noalloc(
    maxsim_dtype dtype, maxsim_dtype grad_dtype, const float* dscore, const void* queries,
    int64_t total_q_tokens, const int32_t* query_offsets, int64_t num_queries,
    const void* documents, int64_t total_d_tokens,
    const int32_t* document_offsets, int64_t num_documents,
    const int32_t* pair_query_ids, const int32_t* pair_document_ids,
    int64_t num_pairs, const int32_t* argmax, int64_t max_q_len, int64_t dim,
    void* dqueries, void* ddocuments, void* stream);

/* ---- Padded rerank ------------------------------------------------------ */

/* Replaces op `maxsim_padded_forward` (torch_binding.h:46-53,
 * maxsim.cu:924-1024).  queries [B*Lq_max, dim], query_lengths [B],
 * documents [B*C*Ld_max, dim], doc_lengths [B*C]; pair (b, c) scores query b
 * against document b*C + c -> scores [B*C]. */
int maxsim_amd_padded_forward(maxsim_dtype dtype, const void* queries,
                              const int32_t* query_lengths,
                              const void* documents,
                              const int32_t* doc_lengths, int64_t batch,
                              int64_t num_candidates, int64_t Lq_max,
                              int64_t Ld_max, int64_t dim, float* scores,
                              void* stream);

/* Replaces op `maxsim_padded_forward_with_argmax` (torch_binding.h:65-72,
 * maxsim.cu:1036-1116).  Adds argmax [B*C, Lq_max]. */
int maxsim_amd_padded_forward_with_argmax(
    maxsim_dtype dtype, const void* queries, const int32_t* query_lengths,
    const void* documents, const int32_t* doc_lengths, int64_t batch,
    int64_t num_candidates, int64_t Lq_max, int64_t Ld_max, int64_t dim,
    float* scores, int32_t* argmax, void* stream);

/* Replaces op `maxsim_padded_backward` (torch_binding.h:86-95,
 * maxsim.cu:1124-1210).  dscore [B*C] -> dqueries [B*Lq_max, dim],
 * ddocuments [B*C*Ld_max, dim] (padding rows get 0). */
int maxsim_amd_padded_backward(
    maxsim_dtype dtype, const float* dscore, const void* queries,
    const void* documents, const int32_t* query_lengths,
    const int32_t* doc_lengths, const int32_t* argmax, int64_t batch,
    int64_t num_candidates, int64_t Lq_max, int64_t Ld_max, int64_t dim,
    float* dqueries, float* ddocuments, void* stream);

/* maxsim_amd_padded_backward with the gradients written in `grad_dtype`:
 * MAXSIM_FLOAT32, or the input dtype, in which case each element is the fp32
 * sum rounded to nearest even -- bit for bit what casting the fp32
 * gradients would give.  No counterpart in the reference: its autograd
 * Function (torch-ext/maxsim/__init__.py:752-771) returns fp32 gradients
 * that autograd casts in a separate pass.  Every size the fp32 form accepts
 * is accepted. */
int maxsim_amd_padded_backward_typed(
    maxsim_dtype dtype, maxsim_dtype grad_dtype, const float* dscore, const void* queries,
    const void* documents, const int32_t* query_lengths,
    const int32_t* doc_lengths, const int32_t* argmax, int64_t batch,
    int64_t num_candidates, int64_t Lq_max, int64_t Ld_max, int64_t dim,
    void* dqueries, void* ddocuments, void* stream);

/* ---- Contrastive (all pairs) -------------------------------------------- */

/* Replaces op `maxsim_contrastive_forward` (torch_binding.h:133-135,
 * maxsim.cu:1718-1779).  queries [Nq, Lq, dim], documents [total_d_tokens,
 * dim], document_offsets [Nb+1] -> scores [Nq, Nb]. */
int maxsim_amd_contrastive_forward(maxsim_dtype dtype, const void* queries,
                                   int64_t num_queries, int64_t Lq,
                                   const void* documents,
                                   int64_t total_d_tokens,
                                   const int32_t* document_offsets,
                                   int64_t num_documents, int64_t dim,
                                   float* scores, void* stream);

/* Replaces op `maxsim_contrastive_forward_with_argmax` (torch_binding.h:
 * 144-147, maxsim.cu:1650-1716).  Adds argmax [Nq, Nb, Lq]. */
int maxsim_amd_contrastive_forward_with_argmax(
    maxsim_dtype dtype, const void* queries, int64_t num_queries, int64_t Lq,
    const void* documents, int64_t total_d_tokens,
    const int32_t* document_offsets, int64_t num_documents, int64_t dim,
    float* scores, int32_t* argmax, void* stream);

/* Bytes of device workspace that let maxsim_amd_contrastive_backward split
 * the dqueries gather by document range (one range per XCD, partial sums
 * added in a second pass).  0 for invalid sizes and for dim > 2048, where
 * the backward always takes the single-pass gather.  No counterpart in the
 * reference, whose backward accumulates with global atomics instead. */
size_t maxsim_amd_contrastive_backward_workspace_size(int64_t num_queries, int64_t Lq,
                                                      int64_t dim);

/* Replaces op `maxsim_contrastive_backward` (torch_binding.h:160-165,
 * maxsim.cu:1856-1920).  dscore [Nq, Nb], argmax [Nq, Nb, Lq] ->
 * dqueries [Nq, Lq, dim], ddocuments [total_d_tokens, dim].
 * `workspace` (device memory, 16-byte aligned for the vector path) of at
 * least maxsim_amd_contrastive_backward_workspace_size() bytes selects the
 * split dqueries pass; NULL or a smaller size selects the single-pass
 * gather.  Both give the same result up to fp32 summation order. */
int maxsim_amd_contrastive_backward(
    maxsim_dtype dtype, const float* dscore, const void* queries,
    int64_t num_queries, int64_t Lq, const void* documents,
    int64_t total_d_tokens, const int32_t* document_offsets,
    int64_t num_documents, const int32_t* argmax, int64_t dim,
    float* dqueries, float* ddocuments, void* workspace, size_t workspace_bytes,
    void* stream);

/* maxsim_amd_contrastive_backward with the gradients written in
 * `grad_dtype`: MAXSIM_FLOAT32, or the input dtype, in which case each
 * element is the fp32 sum rounded to nearest even -- bit for bit what
 * casting the fp32 gradients would give.  No counterpart in the reference:
 * its autograd Function (torch-ext/maxsim/__init__.py:947-953) returns the
 * fp32 gradients and autograd casts them to the input dtype in a separate
 * pass; writing the input dtype directly removes that pass and halves the
 * document-gradient write.  A 16-bit grad_dtype needs the document gradient
 * in a single pass over the entries (num_queries * (Lq + 1) up to 38,910 on
 * gfx950, whose workgroups may use 160 KB of LDS); beyond that the call returns MAXSIM_ERR_UNSUPPORTED before
 * launching anything, and the caller uses the fp32 form. */
int maxsim_amd_contrastive_backward_typed(
    maxsim_dtype dtype, maxsim_dtype grad_dtype, const float* dscore,
    const void* queries, int64_t num_queries, int64_t Lq,
    const void* documents, int64_t total_d_tokens,
    const int32_t* document_offsets, int64_t num_documents,
    const int32_t* argmax, int64_t dim, void* dqueries, void* ddocuments,
    void* workspace, size_t workspace_bytes, void* stream);

/* ---- Fused cross-entropy training loss ---------------------------------- */

/* Loss reductions, numbered as torch's (none, mean, sum). */
enum {
  MAXSIM_REDUCTION_NONE = 0,
  MAXSIM_REDUCTION_MEAN = 1,
  MAXSIM_REDUCTION_SUM = 2
};

/* Cross-entropy over the rows of contrastive scores: the loss of the
 * reference's training recipe, F.cross_entropy(scores / temperature,
 * targets) after score_contrastive_train (README.md:193-205; the reference
 * has no fused entry point, its users call torch).  scores [Nq, Nb] fp32
 * (the forward's output), targets [Nq] int32 in [0, Nb) or NULL for the
 * diagonal (target q = q, Nq <= Nb), inv_temperature = 1 / temperature.
 * Writes lse [Nq] = logsumexp_b(scores[q, b] * inv_temperature), which the
 * backward below needs, and loss: [Nq] per-row losses for
 * MAXSIM_REDUCTION_NONE, else one value (mean or sum over rows, added in a
 * fixed order).  An out-of-range target gives a NaN loss for its row. */
int maxsim_amd_cross_entropy_forward(const float* scores, int64_t num_queries,
                                     int64_t num_documents, const int32_t* targets,
                                     float inv_temperature, int reduction, float* lse,
                                     float* loss, void* stream);

/* The contrastive backward of that loss, fused: the gradient of
 * loss(score_contrastive(queries, documents)) with respect to queries and
 * documents, where each score gradient
 *   dscore[q, b] = w_q * (exp(scores[q, b] * inv_t - lse[q]) - [b == target_q]),
 *   w_q = inv_t * grad_loss[q or 0] * (1 / Nq for MAXSIM_REDUCTION_MEAN),
 * is computed inside the gradient kernels where they stage their weights:
 * there is no dscore tensor and no separate softmax pass.  grad_loss is the
 * upstream gradient of the loss ([Nq] for MAXSIM_REDUCTION_NONE, else one
 * value, on the device).  Every other argument, the workspace and the
 * gradient dtypes are those of maxsim_amd_contrastive_backward_typed.
 * No counterpart in the reference, whose users run torch's cross-entropy
 * and then maxsim_contrastive_backward on the resulting dscore. */
int maxsim_amd_contrastive_ce_backward_typed(
    maxsim_dtype dtype, maxsim_dtype grad_dtype, const float* scores, const float* lse,
    const int32_t* targets, const float* grad_loss, int reduction, float inv_temperature,
    const void* queries, int64_t num_queries, int64_t Lq, const void* documents,
    int64_t total_d_tokens, const int32_t* document_offsets, int64_t num_documents,
    const int32_t* argmax, int64_t dim, void* dqueries, void* ddocuments, void* workspace,
    size_t workspace_bytes, void* stream);

/* ---- Padded -> packed --------------------------------------------------- */

/* Replaces the boolean-mask gathers of `_pack_padded`
 * (torch-ext/maxsim/__init__.py:584-593; the whole helper is :516-620).
 * padded [num_segments * max_len, dim] holds num_segments segments of max_len
 * rows; segment s contributes its first lengths[s] rows (clamped to
 * [0, max_len]) to packed [packed_rows, dim] starting at row offsets[s].
 * The caller computes offsets (the exclusive prefix sum of the lengths) and
 * allocates packed; rows that would land at or beyond packed_rows are not
 * written.  Any dim > 0 is accepted (it is a copy). */
int maxsim_amd_pack_padded_rows(maxsim_dtype dtype, const void* padded, int64_t num_segments,
                                int64_t max_len, const int32_t* lengths,
                                const int32_t* offsets, int64_t dim, void* packed,
                                int64_t packed_rows, void* stream);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* MAXSIM_AMD_H_ */
