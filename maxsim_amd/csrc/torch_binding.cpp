// Thin torch binding over the C ABI (include/maxsim_amd.h).
//
// Registers the reference's nine operator schemas (torch-ext/torch_binding.cpp
// :7-90) under the `maxsim_amd` namespace for the CUDA dispatch key, which is
// the key PyTorch-ROCm uses for HIP devices.  Each op checks its tensors the
// way the reference host functions do (maxsim.cu:819-2286; TORCH_CHECK ->
// RuntimeError), makes inputs contiguous and int32, allocates the outputs
// with the caching allocator and calls the C ABI on the current HIP stream.
// The C ABI itself never allocates.
#include <ATen/ATen.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <torch/library.h>

#include <optional>
#include <tuple>
#include <vector>

#include "../../include/maxsim_amd.h"

namespace {

using at::Tensor;

maxsim_dtype to_dtype(const Tensor& t) {
  switch (t.scalar_type()) {
    case at::kFloat: return MAXSIM_FLOAT32;
    case at::kHalf: return MAXSIM_FLOAT16;
    case at::kBFloat16: return MAXSIM_BFLOAT16;
    default:
      TORCH_CHECK(false,
                  "queries/documents dtype must be float32, float16, or bfloat16; got ",
                  t.scalar_type());
  }
  return MAXSIM_FLOAT32;
}

void check_status(int rc) {
  TORCH_CHECK(rc == MAXSIM_OK, "maxsim_amd: ", maxsim_amd_last_error());
}

void* current_stream(const Tensor& t) {
  return reinterpret_cast<void*>(
      c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(t.device().index()).stream());
}

Tensor as_i32(const Tensor& t) {
  TORCH_CHECK(t.scalar_type() == at::kInt || t.scalar_type() == at::kLong,
              "index tensors must be int32 or int64; got ", t.scalar_type());
  return t.contiguous().to(at::kInt);
}

void check_embeddings(const Tensor& q, const Tensor& d) {
  TORCH_CHECK(q.device().is_cuda(), "queries must be a HIP (torch 'cuda') tensor");
  TORCH_CHECK(d.device() == q.device(),
              "documents must be on the same device as queries");
  TORCH_CHECK(q.scalar_type() == d.scalar_type(),
              "queries and documents must have the same dtype");
}

void check_on(const Tensor& t, const Tensor& q, const char* name) {
  TORCH_CHECK(t.device() == q.device(), name,
              " must be on the same device as queries");
}

at::TensorOptions f32_opts(const Tensor& q) {
  return at::TensorOptions().dtype(at::kFloat).device(q.device());
}
at::TensorOptions i32_opts(const Tensor& q) {
  return at::TensorOptions().dtype(at::kInt).device(q.device());
}

// ---- packed ---------------------------------------------------------------

// max_q_len < 0: validate offsets and ids on the host and infer the maximum
// query segment length (reference maxsim.cu:851-890, same messages).
int64_t host_validate_packed(const Tensor& qoff, int64_t total_q, const Tensor& doff,
                             int64_t total_d, const Tensor& qids, const Tensor& dids) {
  auto check_offsets = [](const Tensor& off, int64_t total, const char* name) {
    auto c = off.to(at::kCPU).to(at::kLong).contiguous();
    const int64_t* p = c.data_ptr<int64_t>();
    const int64_t n = c.numel();
    TORCH_CHECK(n >= 2, name, " must have length >= 2");
    TORCH_CHECK(p[0] == 0, name, "[0] must equal 0, got ", p[0]);
    TORCH_CHECK(p[n - 1] == total, name, "[-1] (", p[n - 1],
                ") must equal total token count (", total, ")");
    int64_t m = 0;
    for (int64_t i = 0; i + 1 < n; ++i) {
      const int64_t diff = p[i + 1] - p[i];
      TORCH_CHECK(diff > 0, "empty segment in ", name, " at index ", i);
      m = std::max(m, diff);
    }
    return std::make_pair(m, n - 1);
  };
  auto check_ids = [](const Tensor& ids, int64_t upper, const char* name) {
    auto c = ids.to(at::kCPU).to(at::kLong).contiguous();
    const int64_t* p = c.data_ptr<int64_t>();
    for (int64_t i = 0; i < c.numel(); ++i)
      TORCH_CHECK(p[i] >= 0 && p[i] < upper, name, "[", i, "] = ", p[i],
                  " out of range [0, ", upper, ")");
  };
  auto [mql, nq] = check_offsets(qoff, total_q, "query_offsets");
  auto [unused, nd] = check_offsets(doff, total_d, "document_offsets");
  (void)unused;
  check_ids(qids, nq, "pair_query_ids");
  check_ids(dids, nd, "pair_document_ids");
  return mql;
}

struct Packed {
  Tensor q, qoff, d, doff, qids, dids;
  int64_t mql;
};

Packed prep_packed(Tensor queries, Tensor query_offsets, Tensor documents,
                   Tensor document_offsets, Tensor pair_query_ids,
                   Tensor pair_document_ids, int64_t max_q_len) {
  check_embeddings(queries, documents);
  TORCH_CHECK(queries.dim() == 2 && documents.dim() == 2,
              "queries/documents must be 2-D [tokens, dim]");
  TORCH_CHECK(queries.size(1) == documents.size(1),
              "queries.dim must match documents.dim");
  check_on(query_offsets, queries, "query_offsets");
  check_on(document_offsets, queries, "document_offsets");
  check_on(pair_query_ids, queries, "pair_query_ids");
  check_on(pair_document_ids, queries, "pair_document_ids");
  TORCH_CHECK(pair_query_ids.dim() == 1 && pair_query_ids.sizes() == pair_document_ids.sizes(),
              "pair_query_ids and pair_document_ids must be 1-D with the same shape");
  Packed p;
  p.q = queries.contiguous();
  p.d = documents.contiguous();
  p.qoff = as_i32(query_offsets);
  p.doff = as_i32(document_offsets);
  p.qids = as_i32(pair_query_ids);
  p.dids = as_i32(pair_document_ids);
  if (max_q_len < 0) {
    p.mql = host_validate_packed(p.qoff, p.q.size(0), p.doff, p.d.size(0), p.qids, p.dids);
  } else {
    TORCH_CHECK(max_q_len > 0, "max_q_len must be > 0; got ", max_q_len);
    p.mql = max_q_len;
  }
  return p;
}

// Device workspace (bytes) of maxsim_amd_packed_forward_with_argmax_ws.
Tensor packed_forward_workspace(const Packed& p, int64_t np) {
  const size_t bytes = maxsim_amd_packed_forward_workspace_size(p.doff.numel() - 1, np);
  return at::empty({(int64_t)bytes}, p.q.options().dtype(at::kByte));
}

Tensor maxsim_forward(Tensor queries, Tensor query_offsets, Tensor documents,
                      Tensor document_offsets, Tensor pair_query_ids,
                      Tensor pair_document_ids, int64_t max_q_len) {
  Packed p = prep_packed(queries, query_offsets, documents, document_offsets,
                         pair_query_ids, pair_document_ids, max_q_len);
  const int64_t np = p.qids.numel();
  Tensor scores = at::empty({np}, f32_opts(p.q));
  if (np == 0) return scores;
  c10::hip::HIPGuardMasqueradingAsCUDA guard(p.q.device());
  // workspace for scoring the pairs document by document (see
  // maxsim_amd_packed_forward_workspace_size)
  Tensor ws = packed_forward_workspace(p, np);
  check_status(maxsim_amd_packed_forward_with_argmax_ws(
      to_dtype(p.q), p.q.data_ptr(), p.q.size(0), p.qoff.data_ptr<int32_t>(),
      p.qoff.numel() - 1, p.d.data_ptr(), p.d.size(0), p.doff.data_ptr<int32_t>(),
      p.doff.numel() - 1, p.qids.data_ptr<int32_t>(), p.dids.data_ptr<int32_t>(), np,
      p.q.size(1), p.mql, scores.data_ptr<float>(), nullptr, ws.data_ptr(),
      (size_t)ws.numel(), current_stream(p.q)));
  return scores;
}

std::tuple<Tensor, Tensor> maxsim_packed_forward_with_argmax(
    Tensor queries, Tensor query_offsets, Tensor documents, Tensor document_offsets,
    Tensor pair_query_ids, Tensor pair_document_ids, int64_t max_q_len) {
  TORCH_CHECK(max_q_len > 0, "max_q_len must be > 0");
  Packed p = prep_packed(queries, query_offsets, documents, document_offsets,
                         pair_query_ids, pair_document_ids, max_q_len);
  const int64_t np = p.qids.numel();
  Tensor scores = at::empty({np}, f32_opts(p.q));
  Tensor argmax = at::empty({np, p.mql}, i32_opts(p.q));
  if (np == 0) return {scores, argmax};
  c10::hip::HIPGuardMasqueradingAsCUDA guard(p.q.device());
  Tensor ws = packed_forward_workspace(p, np);
  check_status(maxsim_amd_packed_forward_with_argmax_ws(
      to_dtype(p.q), p.q.data_ptr(), p.q.size(0), p.qoff.data_ptr<int32_t>(),
      p.qoff.numel() - 1, p.d.data_ptr(), p.d.size(0), p.doff.data_ptr<int32_t>(),
      p.doff.numel() - 1, p.qids.data_ptr<int32_t>(), p.dids.data_ptr<int32_t>(), np,
      p.q.size(1), p.mql, scores.data_ptr<float>(), argmax.data_ptr<int32_t>(),
      ws.data_ptr(), (size_t)ws.numel(), current_stream(p.q)));
  return {scores, argmax};
}

// grads_in_input_dtype: gradients in the inputs' dtype (the typed entry
// point rounds each fp32 sum to nearest even, like a cast); where that path is
// unsupported, compute in fp32 and cast.
std::tuple<Tensor, Tensor> packed_backward_impl(
    Tensor dscore, Tensor queries, Tensor query_offsets, Tensor documents,
    Tensor document_offsets, Tensor pair_query_ids, Tensor pair_document_ids,
    Tensor argmax, int64_t max_q_len, bool grads_in_input_dtype) {
  TORCH_CHECK(max_q_len > 0, "max_q_len must be > 0");
  Packed p = prep_packed(queries, query_offsets, documents, document_offsets,
                         pair_query_ids, pair_document_ids, max_q_len);
  TORCH_CHECK(dscore.scalar_type() == at::kFloat, "dscore must be float32");
  TORCH_CHECK(argmax.scalar_type() == at::kInt, "argmax must be int32");
  check_on(dscore, p.q, "dscore");
  check_on(argmax, p.q, "argmax");
  const int64_t np = p.qids.numel();
  TORCH_CHECK(dscore.numel() == np, "dscore must have num_pairs elements");
  TORCH_CHECK(argmax.numel() == np * p.mql, "argmax must be [num_pairs, max_q_len]");
  Tensor g = dscore.contiguous();
  Tensor am = argmax.contiguous();
  c10::hip::HIPGuardMasqueradingAsCUDA guard(p.q.device());
  // workspace for grouping the pairs by query and document on the device
  // (see maxsim_amd_packed_backward_workspace_size)
  const size_t ws_bytes =
      maxsim_amd_packed_backward_workspace_size(p.qoff.numel() - 1, p.doff.numel() - 1, np);
  Tensor ws = at::empty({(int64_t)((ws_bytes + 3) / 4)},
                        p.q.options().dtype(at::kInt));
  const maxsim_dtype dt = to_dtype(p.q);
  auto run = [&](maxsim_dtype grad_dt, const at::TensorOptions& opts) {
    Tensor dq = at::empty({p.q.size(0), p.q.size(1)}, opts);
    Tensor dd = at::empty({p.d.size(0), p.d.size(1)}, opts);
    const int rc = maxsim_amd_packed_backward_typed(
        dt, grad_dt, g.data_ptr<float>(), p.q.data_ptr(), p.q.size(0),
        p.qoff.data_ptr<int32_t>(), p.qoff.numel() - 1, p.d.data_ptr(), p.d.size(0),
        p.doff.data_ptr<int32_t>(), p.doff.numel() - 1, p.qids.data_ptr<int32_t>(),
        p.dids.data_ptr<int32_t>(), np, am.data_ptr<int32_t>(), p.mql, p.q.size(1),
        dq.data_ptr(), dd.data_ptr(), ws.data_ptr(), ws_bytes, current_stream(p.q));
    return std::make_tuple(rc, dq, dd);
  };
  if (grads_in_input_dtype && dt != MAXSIM_FLOAT32) {
    auto [rc, dq, dd] = run(dt, p.q.options());
    if (rc == MAXSIM_OK) return {dq, dd};
    // ERR_UNSUPPORTED is returned before any launch; fall through to fp32
    TORCH_CHECK(rc == MAXSIM_ERR_UNSUPPORTED, "maxsim_amd: ", maxsim_amd_last_error());
  }
  auto [rc, dq, dd] = run(MAXSIM_FLOAT32, f32_opts(p.q));
  check_status(rc);
  if (grads_in_input_dtype && dt != MAXSIM_FLOAT32)
    return {dq.to(p.q.scalar_type()), dd.to(p.q.scalar_type())};
  return {dq, dd};
}

std::tuple<Tensor, Tensor> maxsim_packed_backward(
    Tensor dscore, Tensor queries, Tensor query_offsets, Tensor documents,
    Tensor document_offsets, Tensor pair_query_ids, Tensor pair_document_ids,
    Tensor argmax, int64_t max_q_len) {
  return packed_backward_impl(dscore, queries, query_offsets, documents, document_offsets,
                              pair_query_ids, pair_document_ids, argmax, max_q_len, false);
}

// Not one of the reference's operators: the autograd Function's backward,
// with gradients in the inputs' dtype.
std::tuple<Tensor, Tensor> maxsim_packed_backward_typed(
    Tensor dscore, Tensor queries, Tensor query_offsets, Tensor documents,
    Tensor document_offsets, Tensor pair_query_ids, Tensor pair_document_ids,
    Tensor argmax, int64_t max_q_len) {
  return packed_backward_impl(dscore, queries, query_offsets, documents, document_offsets,
                              pair_query_ids, pair_document_ids, argmax, max_q_len, true);
}

// ---- padded ---------------------------------------------------------------

struct Padded {
  Tensor q, d, qlen, dlen;
  int64_t B, C;
};

Padded prep_padded(Tensor queries, Tensor query_lengths, Tensor documents,
                   Tensor doc_lengths, int64_t Lq_max, int64_t Ld_max,
                   int64_t num_candidates) {
  check_embeddings(queries, documents);
  TORCH_CHECK(queries.dim() == 2 && documents.dim() == 2,
              "queries/documents must be 2-D [rows, dim]");
  TORCH_CHECK(queries.size(1) == documents.size(1),
              "queries.dim must match documents.dim");
  TORCH_CHECK(Lq_max > 0 && Ld_max > 0 && num_candidates > 0,
              "Lq_max, Ld_max and num_candidates must be > 0");
  check_on(query_lengths, queries, "query_lengths");
  check_on(doc_lengths, queries, "doc_lengths");
  Padded p;
  p.q = queries.contiguous();
  p.d = documents.contiguous();
  TORCH_CHECK(p.q.size(0) % Lq_max == 0, "queries rows must be a multiple of Lq_max");
  TORCH_CHECK(p.d.size(0) % Ld_max == 0, "documents rows must be a multiple of Ld_max");
  p.B = p.q.size(0) / Lq_max;
  p.C = num_candidates;
  TORCH_CHECK(p.d.size(0) / Ld_max == p.B * p.C,
              "documents rows must equal B * num_candidates * Ld_max");
  p.qlen = as_i32(query_lengths);
  p.dlen = as_i32(doc_lengths);
  TORCH_CHECK(p.qlen.numel() == p.B, "query_lengths must have B elements");
  TORCH_CHECK(p.dlen.numel() == p.B * p.C, "doc_lengths must have B * C elements");
  return p;
}

Tensor maxsim_padded_forward(Tensor queries, Tensor query_lengths, Tensor documents,
                             Tensor doc_lengths, int64_t Lq_max, int64_t Ld_max,
                             int64_t num_candidates) {
  Padded p = prep_padded(queries, query_lengths, documents, doc_lengths, Lq_max,
                         Ld_max, num_candidates);
  Tensor scores = at::empty({p.B * p.C}, f32_opts(p.q));
  if (p.B * p.C == 0) return scores;
  c10::hip::HIPGuardMasqueradingAsCUDA guard(p.q.device());
  check_status(maxsim_amd_padded_forward(
      to_dtype(p.q), p.q.data_ptr(), p.qlen.data_ptr<int32_t>(), p.d.data_ptr(),
      p.dlen.data_ptr<int32_t>(), p.B, p.C, Lq_max, Ld_max, p.q.size(1),
      scores.data_ptr<float>(), current_stream(p.q)));
  return scores;
}

std::tuple<Tensor, Tensor> maxsim_padded_forward_with_argmax(
    Tensor queries, Tensor query_lengths, Tensor documents, Tensor doc_lengths,
    int64_t Lq_max, int64_t Ld_max, int64_t num_candidates) {
  Padded p = prep_padded(queries, query_lengths, documents, doc_lengths, Lq_max,
                         Ld_max, num_candidates);
  Tensor scores = at::empty({p.B * p.C}, f32_opts(p.q));
  Tensor argmax = at::empty({p.B * p.C, Lq_max}, i32_opts(p.q));
  if (p.B * p.C == 0) return {scores, argmax};
  c10::hip::HIPGuardMasqueradingAsCUDA guard(p.q.device());
  check_status(maxsim_amd_padded_forward_with_argmax(
      to_dtype(p.q), p.q.data_ptr(), p.qlen.data_ptr<int32_t>(), p.d.data_ptr(),
      p.dlen.data_ptr<int32_t>(), p.B, p.C, Lq_max, Ld_max, p.q.size(1),
      scores.data_ptr<float>(), argmax.data_ptr<int32_t>(), current_stream(p.q)));
  return {scores, argmax};
}

// grads_in_input_dtype: gradients written in the inputs' dtype by the typed
// entry point (rounded to nearest even, the bits of a cast of the fp32 ones).
std::tuple<Tensor, Tensor> padded_backward_impl(
    Tensor dscore, Tensor queries, Tensor documents, Tensor query_lengths,
    Tensor doc_lengths, Tensor argmax, int64_t Lq_max, int64_t Ld_max,
    int64_t num_candidates, bool grads_in_input_dtype) {
  Padded p = prep_padded(queries, query_lengths, documents, doc_lengths, Lq_max,
                         Ld_max, num_candidates);
  TORCH_CHECK(dscore.scalar_type() == at::kFloat, "dscore must be float32");
  TORCH_CHECK(argmax.scalar_type() == at::kInt, "argmax must be int32");
  check_on(dscore, p.q, "dscore");
  check_on(argmax, p.q, "argmax");
  TORCH_CHECK(argmax.numel() == p.B * p.C * Lq_max, "argmax must be [B*C, Lq_max]");
  TORCH_CHECK(dscore.numel() == p.B * p.C, "dscore must have B*C elements");
  Tensor g = dscore.contiguous();
  Tensor am = argmax.contiguous();
  const maxsim_dtype dt = to_dtype(p.q);
  const bool typed = grads_in_input_dtype && dt != MAXSIM_FLOAT32;
  const at::TensorOptions opts = typed ? p.q.options() : f32_opts(p.q);
  Tensor dq = at::empty({p.q.size(0), p.q.size(1)}, opts);
  Tensor dd = at::empty({p.d.size(0), p.d.size(1)}, opts);
  c10::hip::HIPGuardMasqueradingAsCUDA guard(p.q.device());
  check_status(maxsim_amd_padded_backward_typed(
      dt, typed ? dt : MAXSIM_FLOAT32, g.data_ptr<float>(), p.q.data_ptr(), p.d.data_ptr(),
      p.qlen.data_ptr<int32_t>(), p.dlen.data_ptr<int32_t>(), am.data_ptr<int32_t>(),
      p.B, p.C, Lq_max, Ld_max, p.q.size(1), dq.data_ptr(), dd.data_ptr(),
      current_stream(p.q)));
  return {dq, dd};
}

std::tuple<Tensor, Tensor> maxsim_padded_backward(
    Tensor dscore, Tensor queries, Tensor documents, Tensor query_lengths,
    Tensor doc_lengths, Tensor argmax, int64_t Lq_max, int64_t Ld_max,
    int64_t num_candidates) {
  return padded_backward_impl(dscore, queries, documents, query_lengths, doc_lengths, argmax,
                              Lq_max, Ld_max, num_candidates, false);
}

std::tuple<Tensor, Tensor> maxsim_padded_backward_typed(
    Tensor dscore, Tensor queries, Tensor documents, Tensor query_lengths,
    Tensor doc_lengths, Tensor argmax, int64_t Lq_max, int64_t Ld_max,
    int64_t num_candidates) {
  return padded_backward_impl(dscore, queries, documents, query_lengths, doc_lengths, argmax,
                              Lq_max, Ld_max, num_candidates, true);
}

// ---- contrastive ----------------------------------------------------------

struct Contrastive {
  Tensor q, d, off;
};

Contrastive prep_contrastive(Tensor queries, Tensor documents, Tensor document_offsets) {
  check_embeddings(queries, documents);
  TORCH_CHECK(queries.dim() == 3, "queries must be [Nq, Lq, D]");
  TORCH_CHECK(documents.dim() == 2, "documents must be [total_d_tokens, D]");
  TORCH_CHECK(document_offsets.dim() == 1, "document_offsets must be 1-D");
  TORCH_CHECK(queries.size(2) == documents.size(1),
              "queries.D must match documents.D");
  check_on(document_offsets, queries, "document_offsets");
  TORCH_CHECK(document_offsets.numel() >= 1, "document_offsets must have at least 1 element");
  TORCH_CHECK(queries.size(1) > 0, "Lq must be > 0");
  TORCH_CHECK(queries.size(2) > 0, "dim must be > 0");
  Contrastive c;
  c.q = queries.contiguous();
  c.d = documents.contiguous();
  c.off = as_i32(document_offsets);
  return c;
}

Tensor maxsim_contrastive_forward(Tensor queries, Tensor documents,
                                  Tensor document_offsets) {
  Contrastive c = prep_contrastive(queries, documents, document_offsets);
  const int64_t Nq = c.q.size(0), Lq = c.q.size(1), Nb = c.off.numel() - 1;
  Tensor scores = at::empty({Nq, Nb}, f32_opts(c.q));
  if (Nq * Nb == 0) return scores;
  c10::hip::HIPGuardMasqueradingAsCUDA guard(c.q.device());
  check_status(maxsim_amd_contrastive_forward(
      to_dtype(c.q), c.q.data_ptr(), Nq, Lq, c.d.data_ptr(), c.d.size(0),
      c.off.data_ptr<int32_t>(), Nb, c.q.size(2), scores.data_ptr<float>(),
      current_stream(c.q)));
  return scores;
}

std::tuple<Tensor, Tensor> maxsim_contrastive_forward_with_argmax(
    Tensor queries, Tensor documents, Tensor document_offsets) {
  Contrastive c = prep_contrastive(queries, documents, document_offsets);
  const int64_t Nq = c.q.size(0), Lq = c.q.size(1), Nb = c.off.numel() - 1;
  Tensor scores = at::empty({Nq, Nb}, f32_opts(c.q));
  Tensor argmax = at::empty({Nq, Nb, Lq}, i32_opts(c.q));
  if (Nq * Nb == 0) return {scores, argmax};
  c10::hip::HIPGuardMasqueradingAsCUDA guard(c.q.device());
  check_status(maxsim_amd_contrastive_forward_with_argmax(
      to_dtype(c.q), c.q.data_ptr(), Nq, Lq, c.d.data_ptr(), c.d.size(0),
      c.off.data_ptr<int32_t>(), Nb, c.q.size(2), scores.data_ptr<float>(),
      argmax.data_ptr<int32_t>(), current_stream(c.q)));
  return {scores, argmax};
}

// The fused cross-entropy's saved state: the score gradients are computed
// from these inside the backward kernels instead of being read from dscore.
struct CeSpec {
  Tensor scores, lse, targets, grad_loss;  // targets undefined: the diagonal
  int64_t reduction;
  double inv_t;
};

// grads_in_input_dtype: write the gradients in the inputs' dtype (the C ABI's
// typed entry point, rounding to nearest even like a cast); when the shapes
// need the fp32 path, compute in fp32 and cast.  With `ce` the score
// gradients come from the fused cross-entropy and `dscore` is unused.
std::tuple<Tensor, Tensor> contrastive_backward_impl(
    Tensor dscore, Tensor queries, Tensor documents, Tensor document_offsets,
    Tensor argmax, bool grads_in_input_dtype, const CeSpec* ce = nullptr) {
  Contrastive c = prep_contrastive(queries, documents, document_offsets);
  const int64_t Nq = c.q.size(0), Lq = c.q.size(1), Nb = c.off.numel() - 1;
  TORCH_CHECK(argmax.scalar_type() == at::kInt, "argmax must be int32");
  check_on(argmax, c.q, "argmax");
  TORCH_CHECK(argmax.numel() == Nq * Nb * Lq, "argmax must be [Nq, Nb, Lq]");
  Tensor g;
  if (!ce) {
    TORCH_CHECK(dscore.scalar_type() == at::kFloat, "dscore must be float32");
    check_on(dscore, c.q, "dscore");
    TORCH_CHECK(dscore.numel() == Nq * Nb, "dscore must be [Nq, Nb]");
    g = dscore.contiguous();
  } else {
    TORCH_CHECK(ce->scores.numel() == Nq * Nb, "scores must be [Nq, Nb]");
    TORCH_CHECK(ce->lse.numel() == Nq, "lse must be [Nq]");
  }
  Tensor am = argmax.contiguous();
  c10::hip::HIPGuardMasqueradingAsCUDA guard(c.q.device());
  // With at least one document per XCD range and enough triples to fill the
  // chip, gather dq by range into a workspace of partial sums (see
  // maxsim_amd_contrastive_backward_workspace_size).  Below 2^20 (query
  // token, document) triples the single-pass walk is faster: one launch
  // fewer and no partial sums (C2-sized batches: 25 against 31 us).
  Tensor ws;
  size_t ws_bytes = 0;
  if (Nb >= 8 && Nq * Lq * Nb >= ((int64_t)1 << 20)) {
    ws_bytes = maxsim_amd_contrastive_backward_workspace_size(Nq, Lq, c.q.size(2));
    if (ws_bytes > 0)
      ws = at::empty({(int64_t)(ws_bytes / sizeof(float))}, f32_opts(c.q));
  }
  const maxsim_dtype dt = to_dtype(c.q);
  auto run = [&](maxsim_dtype grad_dt, const at::TensorOptions& opts) {
    Tensor dq = at::empty({Nq, Lq, c.q.size(2)}, opts);
    Tensor dd = at::empty({c.d.size(0), c.d.size(1)}, opts);
    void* wsp = ws.defined() ? ws.data_ptr() : nullptr;
    const size_t wsb = ws.defined() ? ws_bytes : 0;
    const int rc =
        ce ? maxsim_amd_contrastive_ce_backward_typed(
                 dt, grad_dt, ce->scores.data_ptr<float>(), ce->lse.data_ptr<float>(),
                 ce->targets.defined() ? ce->targets.data_ptr<int32_t>() : nullptr,
                 ce->grad_loss.data_ptr<float>(), (int)ce->reduction, (float)ce->inv_t,
                 c.q.data_ptr(), Nq, Lq, c.d.data_ptr(), c.d.size(0), c.off.data_ptr<int32_t>(),
                 Nb, am.data_ptr<int32_t>(), c.q.size(2), dq.data_ptr(), dd.data_ptr(), wsp, wsb,
                 current_stream(c.q))
           : maxsim_amd_contrastive_backward_typed(
                 dt, grad_dt, g.data_ptr<float>(), c.q.data_ptr(), Nq, Lq, c.d.data_ptr(),
                 c.d.size(0), c.off.data_ptr<int32_t>(), Nb, am.data_ptr<int32_t>(),
                 c.q.size(2), dq.data_ptr(), dd.data_ptr(), wsp, wsb, current_stream(c.q));
    return std::make_tuple(rc, dq, dd);
  };
  if (grads_in_input_dtype && dt != MAXSIM_FLOAT32) {
    auto [rc, dq, dd] = run(dt, c.q.options());
    if (rc == MAXSIM_OK) return {dq, dd};
    // ERR_UNSUPPORTED is returned before any launch; fall through to fp32
    TORCH_CHECK(rc == MAXSIM_ERR_UNSUPPORTED, "maxsim_amd: ", maxsim_amd_last_error());
  }
  auto [rc, dq, dd] = run(MAXSIM_FLOAT32, f32_opts(c.q));
  check_status(rc);
  if (grads_in_input_dtype && dt != MAXSIM_FLOAT32)
    return {dq.to(c.q.scalar_type()), dd.to(c.q.scalar_type())};
  return {dq, dd};
}

std::tuple<Tensor, Tensor> maxsim_contrastive_backward(
    Tensor dscore, Tensor queries, Tensor documents, Tensor document_offsets,
    Tensor argmax) {
  return contrastive_backward_impl(dscore, queries, documents, document_offsets, argmax, false);
}

// Not one of the reference's operators: the autograd Function's backward,
// with gradients in the inputs' dtype.
std::tuple<Tensor, Tensor> maxsim_contrastive_backward_typed(
    Tensor dscore, Tensor queries, Tensor documents, Tensor document_offsets,
    Tensor argmax) {
  return contrastive_backward_impl(dscore, queries, documents, document_offsets, argmax, true);
}

// ---- fused cross-entropy ----------------------------------------------------

Tensor ce_targets(const std::optional<Tensor>& targets, const Tensor& scores) {
  if (!targets.has_value()) return Tensor();
  check_on(*targets, scores, "targets");
  TORCH_CHECK(targets->dim() == 1 && targets->size(0) == scores.size(0),
              "targets must be [Nq] (one class index per query row)");
  return as_i32(*targets);
}

// Not one of the reference's operators: the loss of the reference's
// training recipe, F.cross_entropy(scores * inv_temperature, targets)
// (README.md:193-205), with the row log-sum-exp the fused backward needs.
// reduction: 0 none ([Nq] loss), 1 mean, 2 sum (0-dim loss).
std::tuple<Tensor, Tensor> maxsim_cross_entropy_forward(Tensor scores,
                                                        std::optional<Tensor> targets,
                                                        double inv_temperature,
                                                        int64_t reduction) {
  TORCH_CHECK(scores.device().is_cuda(), "scores must be a HIP (torch 'cuda') tensor");
  TORCH_CHECK(scores.dim() == 2 && scores.scalar_type() == at::kFloat,
              "scores must be float32 [Nq, Nb]");
  Tensor s = scores.contiguous();
  const int64_t nq = s.size(0), nb = s.size(1);
  Tensor t = ce_targets(targets, s);
  Tensor lse = at::empty({nq}, f32_opts(s));
  Tensor loss = reduction == MAXSIM_REDUCTION_NONE ? at::empty({nq}, f32_opts(s))
                                                   : at::empty({}, f32_opts(s));
  c10::hip::HIPGuardMasqueradingAsCUDA guard(s.device());
  check_status(maxsim_amd_cross_entropy_forward(
      s.data_ptr<float>(), nq, nb, t.defined() ? t.data_ptr<int32_t>() : nullptr,
      (float)inv_temperature, (int)reduction, lse.data_ptr<float>(), loss.data_ptr<float>(),
      current_stream(s)));
  return {lse, loss};
}

// Not one of the reference's operators: the fused backward of that loss
// through the contrastive scores, gradients in the inputs' dtype.
std::tuple<Tensor, Tensor> maxsim_contrastive_cross_entropy_backward(
    Tensor grad_loss, Tensor scores, Tensor lse, std::optional<Tensor> targets,
    double inv_temperature, int64_t reduction, Tensor queries, Tensor documents,
    Tensor document_offsets, Tensor argmax) {
  check_on(scores, queries, "scores");
  check_on(lse, queries, "lse");
  check_on(grad_loss, queries, "grad_loss");
  TORCH_CHECK(scores.scalar_type() == at::kFloat && lse.scalar_type() == at::kFloat &&
                  grad_loss.scalar_type() == at::kFloat,
              "scores, lse and grad_loss must be float32");
  CeSpec ce;
  ce.scores = scores.contiguous();
  ce.lse = lse.contiguous();
  ce.targets = ce_targets(targets, ce.scores);
  ce.grad_loss = grad_loss.contiguous();
  ce.reduction = reduction;
  ce.inv_t = inv_temperature;
  TORCH_CHECK(ce.grad_loss.numel() ==
                  (reduction == MAXSIM_REDUCTION_NONE ? ce.scores.size(0) : 1),
              "grad_loss must hold one value per row for reduction none, else one value");
  return contrastive_backward_impl(Tensor(), queries, documents, document_offsets, argmax, true,
                                   &ce);
}

// ---- padded -> packed -------------------------------------------------------

// Not one of the reference's operators: the device copy behind _pack_padded
// (torch-ext/maxsim/__init__.py:584-593).  padded [segments * max_len, dim],
// lengths and offsets [segments] (offsets: exclusive prefix sum of the
// lengths) -> packed [packed_rows, dim].
Tensor maxsim_pack_padded_rows(Tensor padded, Tensor lengths, Tensor offsets, int64_t max_len,
                               int64_t packed_rows) {
  TORCH_CHECK(padded.device().is_cuda(), "padded must be a HIP (torch 'cuda') tensor");
  TORCH_CHECK(padded.dim() == 2, "padded must be 2-D [segments * max_len, dim]");
  TORCH_CHECK(max_len >= 0 && packed_rows >= 0, "max_len and packed_rows must be >= 0");
  check_on(lengths, padded, "lengths");
  check_on(offsets, padded, "offsets");
  Tensor p = padded.contiguous();
  Tensor len = as_i32(lengths);
  Tensor off = as_i32(offsets);
  const int64_t nseg = len.numel();
  TORCH_CHECK(off.numel() >= nseg, "offsets must have one entry per segment");
  TORCH_CHECK(p.size(0) == nseg * max_len, "padded must have segments * max_len rows");
  Tensor out = at::empty({packed_rows, p.size(1)}, p.options());
  if (nseg == 0 || packed_rows == 0 || max_len == 0) return out;
  c10::hip::HIPGuardMasqueradingAsCUDA guard(p.device());
  check_status(maxsim_amd_pack_padded_rows(to_dtype(p), p.data_ptr(), nseg, max_len,
                                           len.data_ptr<int32_t>(), off.data_ptr<int32_t>(),
                                           p.size(1), out.data_ptr(), packed_rows,
                                           current_stream(p)));
  return out;
}

}  // namespace

TORCH_LIBRARY(maxsim_amd, m) {
  m.def("maxsim_forward(Tensor queries, Tensor query_offsets, Tensor documents, "
        "Tensor document_offsets, Tensor pair_query_ids, Tensor pair_document_ids, "
        "int max_q_len) -> Tensor");
  m.def("maxsim_padded_forward(Tensor queries, Tensor query_lengths, Tensor documents, "
        "Tensor doc_lengths, int Lq_max, int Ld_max, int num_candidates) -> Tensor");
  m.def("maxsim_padded_forward_with_argmax(Tensor queries, Tensor query_lengths, "
        "Tensor documents, Tensor doc_lengths, int Lq_max, int Ld_max, "
        "int num_candidates) -> (Tensor, Tensor)");
  m.def("maxsim_padded_backward(Tensor dscore, Tensor queries, Tensor documents, "
        "Tensor query_lengths, Tensor doc_lengths, Tensor argmax, int Lq_max, "
        "int Ld_max, int num_candidates) -> (Tensor, Tensor)");
  m.def("maxsim_packed_forward_with_argmax(Tensor queries, Tensor query_offsets, "
        "Tensor documents, Tensor document_offsets, Tensor pair_query_ids, "
        "Tensor pair_document_ids, int max_q_len) -> (Tensor, Tensor)");
  m.def("maxsim_packed_backward(Tensor dscore, Tensor queries, Tensor query_offsets, "
        "Tensor documents, Tensor document_offsets, Tensor pair_query_ids, "
        "Tensor pair_document_ids, Tensor argmax, int max_q_len) -> (Tensor, Tensor)");
  m.def("maxsim_contrastive_forward(Tensor queries, Tensor documents, "
        "Tensor document_offsets) -> Tensor");
  m.def("maxsim_contrastive_forward_with_argmax(Tensor queries, Tensor documents, "
        "Tensor document_offsets) -> (Tensor, Tensor)");
  m.def("maxsim_contrastive_backward(Tensor dscore, Tensor queries, Tensor documents, "
        "Tensor document_offsets, Tensor argmax) -> (Tensor, Tensor)");
  // not in the reference: gradients in the inputs' dtype (used by autograd)
  m.def("maxsim_packed_backward_typed(Tensor dscore, Tensor queries, Tensor query_offsets, "
        "Tensor documents, Tensor document_offsets, Tensor pair_query_ids, "
        "Tensor pair_document_ids, Tensor argmax, int max_q_len) -> (Tensor, Tensor)");
  m.def("maxsim_padded_backward_typed(Tensor dscore, Tensor queries, Tensor documents, "
        "Tensor query_lengths, Tensor doc_lengths, Tensor argmax, int Lq_max, "
        "int Ld_max, int num_candidates) -> (Tensor, Tensor)");
  m.def("maxsim_pack_padded_rows(Tensor padded, Tensor lengths, Tensor offsets, int max_len, "
        "int packed_rows) -> Tensor");
  m.def("maxsim_contrastive_backward_typed(Tensor dscore, Tensor queries, Tensor documents, "
        "Tensor document_offsets, Tensor argmax) -> (Tensor, Tensor)");
  m.def("maxsim_cross_entropy_forward(Tensor scores, Tensor? targets, float inv_temperature, "
        "int reduction) -> (Tensor, Tensor)");
  m.def("maxsim_contrastive_cross_entropy_backward(Tensor grad_loss, Tensor scores, "
        "Tensor lse, Tensor? targets, float inv_temperature, int reduction, Tensor queries, "
        "Tensor documents, Tensor document_offsets, Tensor argmax) -> (Tensor, Tensor)");
}

TORCH_LIBRARY_IMPL(maxsim_amd, CUDA, m) {
  m.impl("maxsim_forward", &maxsim_forward);
  m.impl("maxsim_padded_forward", &maxsim_padded_forward);
  m.impl("maxsim_padded_forward_with_argmax", &maxsim_padded_forward_with_argmax);
  m.impl("maxsim_padded_backward", &maxsim_padded_backward);
  m.impl("maxsim_padded_backward_typed", &maxsim_padded_backward_typed);
  m.impl("maxsim_packed_forward_with_argmax", &maxsim_packed_forward_with_argmax);
  m.impl("maxsim_packed_backward", &maxsim_packed_backward);
  m.impl("maxsim_packed_backward_typed", &maxsim_packed_backward_typed);
  m.impl("maxsim_contrastive_forward", &maxsim_contrastive_forward);
  m.impl("maxsim_contrastive_forward_with_argmax",
         &maxsim_contrastive_forward_with_argmax);
  m.impl("maxsim_contrastive_backward", &maxsim_contrastive_backward);
  m.impl("maxsim_contrastive_backward_typed", &maxsim_contrastive_backward_typed);
  m.impl("maxsim_pack_padded_rows", &maxsim_pack_padded_rows);
  m.impl("maxsim_cross_entropy_forward", &maxsim_cross_entropy_forward);
  m.impl("maxsim_contrastive_cross_entropy_backward",
         &maxsim_contrastive_cross_entropy_backward);
}
