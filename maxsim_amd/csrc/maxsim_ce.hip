// Cross-entropy over contrastive scores, the forward half of the fused
// training loss (maxsim_amd_cross_entropy_forward).
//
// The reference's training recipe is score_contrastive_train followed by
// F.cross_entropy(scores / temperature, targets) (README.md:193-205).  Here
// the loss is computed from the scores the forward kernel wrote: one wave per
// query row takes the row's log-sum-exp of scores * inv_t (max, then the sum
// of exp(v - max), both reduced across the wave in a fixed butterfly order),
// and writes it for the backward, which recomputes each softmax entry inside
// the gradient kernels (maxsim_bwd.hip, CeGrad) instead of reading a dscore
// tensor.  The mean or sum over rows is one workgroup adding the row losses
// in a fixed order, so the loss is bitwise reproducible.
//
// NaN and infinities follow the arithmetic: a NaN score makes its row's
// log-sum-exp NaN (exp(NaN) is NaN), a row of -inf scores gives NaN, as
// log_softmax does.
#include <cmath>

#include "maxsim_common.h"
#include "maxsim_host.h"

namespace maxsim {

constexpr int kCeThreads = 256;

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// One wave per query row: lse[q] = log sum_b exp(s[q, b] * inv_t); with
// per_row set, loss[q] = lse[q] - s[q, target_q] * inv_t.
__global__ __launch_bounds__(kCeThreads) void ce_lse_kernel(const float* __restrict__ s,
                                                            int64_t nq, int64_t nb,
                                                            const int32_t* __restrict__ targets,
                                                            float inv_t, float* __restrict__ lse,
                                                            float* __restrict__ loss, int per_row) {
  const int lane = threadIdx.x & 63;
  const int64_t q = (int64_t)blockIdx.x * (kCeThreads / 64) + (threadIdx.x >> 6);
  if (q >= nq) return;
  const float* row = s + q * nb;
  float m = -INFINITY;
  bool nan = false;
  for (int64_t b = lane; b < nb; b += 64) {
    const float v = row[b] * inv_t;
    nan |= v != v;
    m = fmaxf(m, v);
  }
  m = wave_max(m);
  float sum = 0.0f;
  for (int64_t b = lane; b < nb; b += 64) sum += expf(row[b] * inv_t - m);
  sum = wave_sum(sum);
  const bool any_nan = __any(nan);
  const float l = any_nan ? NAN : m + logf(sum);
  if (lane == 0) {
    lse[q] = l;
    if (per_row) {
      const int64_t t = targets ? (int64_t)targets[q] : q;
      loss[q] = (t >= 0 && t < nb) ? l - row[t] * inv_t : NAN;
    }
  }
}

// loss[0] = scale * sum_q (lse[q] - s[q, target_q] * inv_t): each thread adds
// a strided share of the rows in order, then a fixed tree over the threads.
__global__ __launch_bounds__(kCeThreads) void ce_reduce_kernel(const float* __restrict__ s,
                                                               int64_t nq, int64_t nb,
                                                               const int32_t* __restrict__ targets,
                                                               float inv_t,
                                                               const float* __restrict__ lse,
                                                               float scale,
                                                               float* __restrict__ loss) {
  __shared__ float part[kCeThreads];
  float acc = 0.0f;
  for (int64_t q = threadIdx.x; q < nq; q += kCeThreads) {
    const int64_t t = targets ? (int64_t)targets[q] : q;
    acc += (t >= 0 && t < nb) ? lse[q] - s[q * nb + t] * inv_t : NAN;
  }
  part[threadIdx.x] = acc;
  __syncthreads();
  for (int w = kCeThreads / 2; w >= 1; w >>= 1) {
    if ((int)threadIdx.x < w) part[threadIdx.x] += part[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) loss[0] = part[0] * scale;
}

}  // namespace maxsim

using namespace maxsim;

extern "C" {

int maxsim_amd_cross_entropy_forward(const float* scores, int64_t num_queries,
                                     int64_t num_documents, const int32_t* targets,
                                     float inv_temperature, int reduction, float* lse,
                                     float* loss, void* stream) {
  clear_error();
  if (num_queries < 0 || num_documents < 0) return fail(MAXSIM_ERR_INVALID, "negative size");
  if (reduction < MAXSIM_REDUCTION_NONE || reduction > MAXSIM_REDUCTION_SUM)
    return fail(MAXSIM_ERR_INVALID, "unknown reduction %d", reduction);
  if (!(inv_temperature > 0.0f) || !(inv_temperature < INFINITY))
    return fail(MAXSIM_ERR_INVALID, "inv_temperature must be finite and > 0");
  if (num_documents == 0 && num_queries > 0)
    return fail(MAXSIM_ERR_INVALID, "cross-entropy needs at least one document per row");
  if (!targets && num_queries > num_documents)
    return fail(MAXSIM_ERR_INVALID,
                "diagonal targets (targets == NULL) need num_queries <= num_documents");
  if (!loss || (num_queries > 0 && (!scores || !lse)))
    return fail(MAXSIM_ERR_INVALID, "null pointer argument");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int per_row = reduction == MAXSIM_REDUCTION_NONE ? 1 : 0;
  if (num_queries > 0) {
    const int64_t blocks = (num_queries + kCeThreads / 64 - 1) / (kCeThreads / 64);
    if (blocks > (int64_t)UINT32_MAX / kCeThreads)
      return fail(MAXSIM_ERR_UNSUPPORTED, "too many rows for one launch");
    hipLaunchKernelGGL(ce_lse_kernel, dim3((unsigned)blocks), dim3(kCeThreads), 0, st, scores,
                       num_queries, num_documents, targets, inv_temperature, lse, loss, per_row);
    if (int e = check_launch("ce_lse_kernel")) return e;
  }
  if (!per_row) {
    // mean over zero rows is NaN (0 / 0), as torch gives
    const float scale = reduction == MAXSIM_REDUCTION_MEAN
                            ? (num_queries > 0 ? 1.0f / (float)num_queries : NAN)
                            : 1.0f;
    hipLaunchKernelGGL(ce_reduce_kernel, dim3(1), dim3(kCeThreads), 0, st, scores, num_queries,
                       num_documents, targets, inv_temperature, lse, scale, loss);
    return check_launch("ce_reduce_kernel");
  }
  return MAXSIM_OK;
}

}  // extern "C"
