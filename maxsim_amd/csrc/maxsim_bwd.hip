// MaxSim backward kernels for gfx950 and the backward C-ABI entry points.
//
// Given the int32 argmax saved by the forward, the gradient is pure routing
// (reference maxsim.cu:564-613, 1788-1830, 2122-2169):
//     g = dscore[pair], j = argmax[pair, i]
//     dq[query token i]  += g * d[doc token j]
//     dd[doc token j]    += g * q[query token i]
//
// Contrastive and padded layouts are done owner-computes, with no global
// atomics:
//   * dq: a thread owns (query token, 8-element slice) and gathers the
//     winning document row of every document the token was scored against,
//     accumulating in fp32 registers.  Contrastive batches with a workspace
//     split the documents into one range per XCD (so each XCD's L2 serves the
//     gathers of its range) and add the eight partial sums in a second pass.
//   * dd (contrastive): one workgroup per (document, part of the embedding
//     dimension) buckets the document's argmax entries by target row in LDS
//     (counting sort) and sums g * q over each row's bucket in registers; the
//     dimension split keeps each XCD's slice of Q small enough for its L2.
//     A row's bucket is summed in bucket order, which follows the order of
//     the LDS atomics that filled it, so dd can differ between runs in the
//     last bits (dq and padded dd are bitwise reproducible).
//   * dd (padded): one wave per (query, candidate) document writes the
//     document's rows once (zeros) and adds its <= Lq contributions in query
//     token order.
// Packed pairs can share queries and documents arbitrarily; there dq and dd
// are zero-filled and accumulated with hardware fp32 global atomics.
#include "maxsim_common.h"
#include "maxsim_host.h"

#include <algorithm>
#include <mutex>
#include <type_traits>

namespace maxsim {

// 8 consecutive elements of a row as fp32 (elements at k >= dim read 0).
template <typename T>
__device__ __forceinline__ void load8f(const typename T::storage* row, int k0,
                                       int dim, bool vec, float out[8]) {
  if constexpr (T::bytes == 4) {
    if (vec) {
      const float4 a = *reinterpret_cast<const float4*>(row + k0);
      const float4 b = *reinterpret_cast<const float4*>(row + k0 + 4);
      out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
      out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) out[e] = (k0 + e < dim) ? row[k0 + e] : 0.0f;
    }
  } else {
    uint16_t v[8];
    if (vec) {
      const uint4 w = *reinterpret_cast<const uint4*>(row + k0);
      const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[2 * e] = (uint16_t)(ws[e] & 0xffffu);
        v[2 * e + 1] = (uint16_t)(ws[e] >> 16);
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = (k0 + e < dim) ? row[k0 + e] : (uint16_t)0;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if constexpr (__is_same(T, BF16)) {
        out[e] = __uint_as_float((uint32_t)v[e] << 16);
      } else {
        out[e] = (float)__builtin_bit_cast(_Float16, v[e]);
      }
    }
  }
}

// Element e (0..7) of a raw fragment as fp32.
__device__ __forceinline__ float frag_elem(const Frag<BF16>& f, int e) {
  const uint32_t w = (e >> 1) == 0 ? f.v.x : (e >> 1) == 1 ? f.v.y : (e >> 1) == 2 ? f.v.z : f.v.w;
  return __uint_as_float((e & 1) ? (w & 0xffff0000u) : (w << 16));
}
__device__ __forceinline__ float frag_elem(const Frag<F16>& f, int e) {
  const uint32_t w = (e >> 1) == 0 ? f.v.x : (e >> 1) == 1 ? f.v.y : (e >> 1) == 2 ? f.v.z : f.v.w;
  return (float)__builtin_bit_cast(_Float16, (uint16_t)((e & 1) ? (w >> 16) : (w & 0xffffu)));
}
__device__ __forceinline__ float frag_elem(const Frag<F32>& f, int e) {
  const uint4 h = e < 4 ? f.lo : f.hi;
  const int x = e & 3;
  return __uint_as_float(x == 0 ? h.x : x == 1 ? h.y : x == 2 ? h.z : h.w);
}

__device__ __forceinline__ void store8f(float* row, int k0, int dim, bool vec,
                                        const float v[8]) {
  if (vec) {
    *reinterpret_cast<float4*>(row + k0) = make_float4(v[0], v[1], v[2], v[3]);
    *reinterpret_cast<float4*>(row + k0 + 4) = make_float4(v[4], v[5], v[6], v[7]);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (k0 + e < dim) row[k0 + e] = v[e];
  }
}

// fp32 -> 16-bit gradient element, round to nearest even: torch's
// float -> bfloat16 rule (NaN becomes the quiet NaN 0x7FC0) and the
// hardware float -> half conversion under the default rounding mode, so a
// gradient written here equals the fp32 gradient cast by torch.  For bf16
// the hardware conversion (v_cvt_pk_bf16_f32 on gfx950) gives the rule's
// bits for every non-NaN float (all 2^32 patterns compared on the device)
// but keeps a NaN's sign and payload bits, so NaNs are replaced.
template <typename O>
__device__ __forceinline__ uint16_t to_out16(float f) {
  if constexpr (__is_same(O, BF16)) {
    return f != f ? (uint16_t)0x7fc0 : __builtin_bit_cast(uint16_t, (__bf16)f);
  } else {
    return __builtin_bit_cast(uint16_t, (_Float16)f);
  }
}

// Two 16-bit gradient elements in one word (a in the low half), bf16 in one
// paired conversion.
template <typename O>
__device__ __forceinline__ uint32_t pack_out16(float a, float b) {
  if constexpr (__is_same(O, BF16)) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    uint32_t w = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
    if (a != a) w = (w & 0xffff0000u) | 0x7fc0u;
    if (b != b) w = (w & 0x0000ffffu) | 0x7fc00000u;
    return w;
  } else {
    return (uint32_t)to_out16<O>(a) | ((uint32_t)to_out16<O>(b) << 16);
  }
}

// Element `off` of a gradient buffer of output type O.
template <typename O>
__device__ __forceinline__ void* out_at(void* base, int64_t off) {
  return static_cast<char*>(base) + off * O::bytes;
}

// Non-temporal 16-byte stores, for output rows that nothing re-reads while
// the kernel runs: their lines are marked for early eviction and leave L2 to
// the gathered rows.  A wave's stores should cover whole lines (consecutive
// lanes, consecutive 16-byte pieces): partial lines written this way cost
// far more than cached ones.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void store16_nt(void* p, u32x4_t v) {
  __builtin_nontemporal_store(v, static_cast<u32x4_t*>(p));
}

// 8 gradient elements in the output type O, 16-byte aligned (vec rows), as
// non-temporal stores.
template <typename O>
__device__ __forceinline__ void store8_nt(void* row_v, int k0, const float v[8]) {
  if constexpr (O::bytes == 4) {
    float* row = static_cast<float*>(row_v) + k0;
    store16_nt(row, u32x4_t{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                            __float_as_uint(v[3])});
    store16_nt(row + 4, u32x4_t{__float_as_uint(v[4]), __float_as_uint(v[5]),
                                __float_as_uint(v[6]), __float_as_uint(v[7])});
  } else {
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      w[e] = pack_out16<O>(v[2 * e], v[2 * e + 1]);
    store16_nt(static_cast<uint16_t*>(row_v) + k0, u32x4_t{w[0], w[1], w[2], w[3]});
  }
}

// 8 gradient elements in the output type O (F32, BF16 or F16).  With vec the
// row is 16-byte aligned and holds all 8 (dim % 8 == 0).
template <typename O>
__device__ __forceinline__ void store8(void* row_v, int k0, int dim, bool vec, const float v[8]) {
  if constexpr (O::bytes == 4) {
    store8f(static_cast<float*>(row_v), k0, dim, vec, v);
  } else {
    uint16_t* row = static_cast<uint16_t*>(row_v);
    if (vec) {
      uint32_t w[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        w[e] = pack_out16<O>(v[2 * e], v[2 * e + 1]);
      *reinterpret_cast<uint4*>(row + k0) = make_uint4(w[0], w[1], w[2], w[3]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (k0 + e < dim) row[k0 + e] = to_out16<O>(v[e]);
    }
  }
}

// ---------------------------------------------------------------------------
// Fill (used instead of hipMemsetAsync so the entry points stay capturable).
// ---------------------------------------------------------------------------
// E is float or uint16_t (zero bits are +0 in every dtype).
template <typename E>
__global__ __launch_bounds__(256) void fill_zero_kernel(E* p, int64_t n, bool vec) {
  constexpr int kPer = 16 / sizeof(E);
  const int64_t nv = vec ? n / kPer : 0;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nv; i += stride)
    reinterpret_cast<uint4*>(p)[i] = make_uint4(0u, 0u, 0u, 0u);
  for (int64_t i = nv * kPer + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    p[i] = E(0);
}

// ---------------------------------------------------------------------------
// dq gather, contrastive and padded layouts.
// Thread = (query row r, 8-element slice s).  For contrastive, query q has
// rows q*Lq .. and is scored against every document b; for padded, query b
// has rows b*Lq_max .. and candidates p = b*C + c.
// ---------------------------------------------------------------------------
// Upstream gradient of the contrastive score (query q, document b).  With
// `scores` null it is dscore[q * nb + b].  Otherwise the scores are the
// logits of a cross-entropy over each query's row (the fused loss of
// maxsim_amd_contrastive_ce_backward_typed): the gradient is
//   w_q * (exp(s[q, b] * inv_t - lse_q) - [b == target_q]),
//   w_q = scale * inv_t * grad_loss[per_row ? q : 0],
// computed where the kernels stage their weights, so no dscore tensor is
// written or read.
struct CeGrad {
  const float* scores = nullptr;
  const float* lse = nullptr;
  const int32_t* targets = nullptr;  // null: target_q = q (diagonal positives)
  const float* grad_loss = nullptr;
  int per_row = 0;
  float inv_t = 1.0f;
  float scale = 1.0f;
};

__device__ __forceinline__ float score_grad(const float* dscore, const CeGrad& ce, int64_t q,
                                            int64_t b, int64_t nb) {
  if (!ce.scores) return dscore[q * nb + b];
  const float p = expf(ce.scores[q * nb + b] * ce.inv_t - ce.lse[q]);
  const int64_t t = ce.targets ? (int64_t)ce.targets[q] : q;
  const float w = ce.scale * ce.inv_t * ce.grad_loss[ce.per_row ? q : 0];
  return w * (p - (b == t ? 1.0f : 0.0f));
}

struct DqArgs {
  CeGrad ce;
  const float* dscore;
  const void* q;  // unused by the gather itself (kept for symmetry)
  const void* d;
  const int32_t* argmax;
  void* dq;       // fp32, or the input's 16-bit type
  int dim;
  int nslices;
  int64_t rows;   // total query rows (Nq*Lq or B*Lq_max)
  int lq;         // rows per query (Lq or Lq_max); argmax row stride
  // contrastive
  const int32_t* doff;
  int64_t nb;
  int64_t total_d;
  // padded
  const int32_t* qlen;
  const int32_t* dlen;
  int64_t ncand;
  int ld_max;
  int padded;
  int csplit = 1;  // padded: lanes sharing one (row, slice), each over a candidate range
};

template <typename T, typename O>
__global__ __launch_bounds__(256) void dq_gather_kernel(DqArgs a, bool vec) {
  using S = typename T::storage;
  // padded with csplit > 1: csplit adjacent lanes (a power of two) share one
  // (row, slice); lane cs walks candidates [cs * per, (cs + 1) * per) and the
  // partial sums are added in cs order before the first lane stores
  const int64_t gid0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int cs = (int)(gid0 & (a.csplit - 1));
  const int64_t gid = gid0 / a.csplit;
  const int64_t row = gid / a.nslices;
  if (row >= a.rows) return;
  const int sl = (int)(gid - row * a.nslices);
  const int k0 = sl * 8;
  const int64_t qidx = row / a.lq;
  const int i = (int)(row - qidx * a.lq);
  const S* __restrict__ D = static_cast<const S*>(a.d);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};

  // Documents are processed U at a time: all index loads of a batch
  // are issued first, then all row loads, so each thread keeps several
  // gathers in flight.  Invalid entries read a clamped row and get weight 0.
  constexpr int U = 8;
  if (!a.padded) {
    const int32_t* am = a.argmax + qidx * a.nb * a.lq + i;
    for (int64_t b0 = 0; b0 < a.nb; b0 += U) {
      int64_t src[U];
      float w[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t b = b0 + u;
        src[u] = 0;
        w[u] = 0.0f;
        if (b < a.nb) {
          const int64_t s = a.doff[b], e = a.doff[b + 1];
          const int j = am[b * a.lq];
          if (s >= 0 && e > s && e <= a.total_d && j >= 0 && j < e - s) {
            src[u] = s + j;
            w[u] = 1.0f;
          }
        }
      }
      float v[U][8];
#pragma unroll
      for (int u = 0; u < U; ++u)
        load8f<T>(D + src[u] * (int64_t)a.dim, k0, a.dim, vec, v[u]);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t b = min(b0 + u, a.nb - 1);
        const float gb = (w[u] != 0.0f) ? score_grad(a.dscore, a.ce, qidx, b, a.nb) : 0.0f;
#pragma unroll
        for (int e2 = 0; e2 < 8; ++e2)
          acc[e2] = (w[u] != 0.0f) ? fmaf(gb, v[u][e2], acc[e2]) : acc[e2];
      }
    }
  } else {
    const int lqb = a.qlen[qidx];
    const int64_t per = (a.ncand + a.csplit - 1) / a.csplit;
    const int64_t c_lo = cs * per;
    const int64_t c_hi = min(a.ncand, c_lo + per);
    if (i < lqb && lqb <= a.lq) {
      for (int64_t c0 = c_lo; c0 < c_hi; c0 += U) {
        int64_t src[U];
        float w[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int64_t c = c0 + u;
          src[u] = 0;
          w[u] = 0.0f;
          if (c < c_hi) {
            const int64_t p = qidx * a.ncand + c;
            const int ld = a.dlen[p];
            const int j = a.argmax[p * a.lq + i];
            if (ld >= 1 && ld <= a.ld_max && j >= 0 && j < ld) {
              src[u] = p * a.ld_max + j;
              w[u] = 1.0f;
            }
          }
        }
        float v[U][8];
#pragma unroll
        for (int u = 0; u < U; ++u)
          load8f<T>(D + src[u] * (int64_t)a.dim, k0, a.dim, vec, v[u]);
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int64_t p = qidx * a.ncand + min(c0 + u, a.ncand - 1);
          const float gb = (w[u] != 0.0f) ? a.dscore[p] : 0.0f;
#pragma unroll
          for (int e2 = 0; e2 < 8; ++e2)
            acc[e2] = (w[u] != 0.0f) ? fmaf(gb, v[u][e2], acc[e2]) : acc[e2];
        }
      }
    }
    if (a.csplit > 1) {
      // every lane of a group is live here (a group shares its row)
      const int lead = (threadIdx.x & 63) & ~(a.csplit - 1);
      float tot[8];
#pragma unroll
      for (int e2 = 0; e2 < 8; ++e2) tot[e2] = acc[e2];
      for (int k = 1; k < a.csplit; ++k) {
#pragma unroll
        for (int e2 = 0; e2 < 8; ++e2) tot[e2] += __shfl(acc[e2], lead + k, 64);
      }
      if (cs != 0) return;
#pragma unroll
      for (int e2 = 0; e2 < 8; ++e2) acc[e2] = tot[e2];
    }
  }
  store8<O>(out_at<O>(a.dq, row * a.dim), k0, a.dim, vec, acc);
}

// ---------------------------------------------------------------------------
// dq, contrastive, split by document range.
//
// gfx950 dispatches workgroup w to XCD w % 8, and each XCD has its own L2.
// Range r = w % kXcds of the documents is therefore gathered only by the
// workgroups of one XCD, so each XCD's L2 serves 1/8 of D instead of all of
// it.  A thread owns (query row, 8-element slice, range) and writes its fp32
// partial sum to ws[range]; dq_reduce_kernel (or dd_bucket_kernel's fused
// share) adds the kXcds parts in range order, so dq is bitwise reproducible.
//
// The workgroup's rows and a chunk of the range's documents form a table of
// (source row, weight) pairs, built in LDS by one coalesced pass over the
// argmax, offsets and dscore; the gather loop then reads only the table and
// D, U winning rows in flight per lane, with no dependent index loads
// between batches.  Documents are added in order, one FMA each (weight 0 for
// an invalid entry).
// ---------------------------------------------------------------------------
constexpr int kDqBatch = 4;
constexpr int kDqSplitMaxDim = 2048;  // 8 * 256 slices: one row per workgroup at most
constexpr int kDqTable = 2048;  // (row, document) pairs staged per chunk

template <typename T, int U>
__global__ __launch_bounds__(256) void dq_split_kernel(DqArgs a, bool vec, float* ws,
                                                       int rows_per_group) {
  using S = typename T::storage;
  __shared__ int32_t t_src[kDqTable];  // [document in chunk][row in group]
  __shared__ float t_w[kDqTable];
  const int r = blockIdx.x % kXcds;
  const int64_t row0 = (int64_t)(blockIdx.x / kXcds) * rows_per_group;
  const int rpg = rows_per_group;
  const int chunk = kDqTable / rpg;
  const int tid = threadIdx.x;
  const int local = tid / a.nslices;
  const int64_t row = row0 + local;
  const bool active = local < rpg && row < a.rows;
  const int sl = tid - local * a.nslices;
  const int k0 = sl * 8;
  const int64_t b_lo = a.nb * r / kXcds;
  const int64_t b_hi = a.nb * (r + 1) / kXcds;
  const S* __restrict__ D = static_cast<const S*>(a.d);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int64_t c0 = b_lo; c0 < b_hi; c0 += chunk) {
    const int nc = (int)min((int64_t)chunk, b_hi - c0);
    __syncthreads();  // the previous chunk's table is consumed
    // consecutive threads take consecutive rows of one document: the argmax
    // reads of a query's tokens are contiguous
    for (int e = tid; e < nc * rpg; e += 256) {
      const int bl = e / rpg;
      const int lr = e - bl * rpg;
      const int64_t rw = row0 + lr;
      int32_t src = 0;
      float w = 0.0f;
      if (rw < a.rows) {
        const int64_t qidx = rw / a.lq;
        const int i = (int)(rw - qidx * a.lq);
        const int64_t b = c0 + bl;
        const int64_t s0 = a.doff[b], s1 = a.doff[b + 1];
        const int j = a.argmax[(qidx * a.nb + b) * a.lq + i];
        if (s0 >= 0 && s1 > s0 && s1 <= a.total_d && j >= 0 && j < s1 - s0) {
          src = (int32_t)(s0 + j);
          w = score_grad(a.dscore, a.ce, qidx, b, a.nb);
        }
      }
      t_src[e] = src;
      t_w[e] = w;
    }
    __syncthreads();
    if (active) {
      // full batches unmasked; the last one repeats its last document past
      // the chunk end and does not add it
      auto batch = [&](int bl, auto masked) {
        constexpr bool MASKED = decltype(masked)::value;
        float wt[U];
        Frag<T> v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int e = (MASKED ? min(bl + u, nc - 1) : bl + u) * rpg + local;
          wt[u] = t_w[e];
          v[u] = load_frag<T>(D + (int64_t)t_src[e] * a.dim, k0, a.dim, vec);
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int e2 = 0; e2 < 8; ++e2) {
            const float t = fmaf(wt[u], frag_elem(v[u], e2), acc[e2]);
            acc[e2] = (!MASKED || bl + u < nc) ? t : acc[e2];
          }
      };
      int bl = 0;
      for (; bl + U <= nc; bl += U) batch(bl, std::false_type{});
      if (bl < nc) batch(bl, std::true_type{});
    }
  }
  if (active) store8f(ws + (int64_t)r * a.rows * a.dim + row * a.dim, k0, a.dim, vec, acc);
}

// ---------------------------------------------------------------------------
// dq, contrastive, one pass over the documents in order (document walk).
//
// Thread = (query row, 8-element slice); a workgroup holds R rows.  Every
// workgroup walks all documents in the same order, kWalkTable / R documents
// per stage: the stage's table of (byte offset of the winning document row,
// weight) per (row, document) is built in LDS from argmax, offsets and
// dscore, then each lane gathers its row's winning rows, eight in flight
// (two 16-byte LDS reads fetch eight offsets, two more eight weights), and
// adds them in document order in fp32 registers.  A launch's workgroups are
// resident together and advance at the same rate, so at any moment the
// workgroups of one XCD gather from the same few documents, which its L2
// holds; D is streamed through each L2 once.  dq is written once in the
// output type O: no partial sums, no workspace, no second pass, and the
// order of the additions (documents ascending, one fmaf each) is the one
// dq_gather_kernel uses, so the two agree bit for bit.
//
// OFF32: D is smaller than 2 GiB, so the table holds 32-bit byte offsets
// (invalid entries -1) and a gather address is one add.  Otherwise the table
// holds row indices and the address is computed in 64 bits.
// ---------------------------------------------------------------------------
constexpr int kWalkTable = 2048;   // (row, document) entries per stage
constexpr int kWalkMaxRows = 32;   // rows per workgroup at most
constexpr int kWalkPad = 4;        // table row stride = docs per stage + 4 (ints)
constexpr int kWalkTableInts = kWalkTable + kWalkPad * kWalkMaxRows;

template <typename T, bool VEC, bool OFF32, typename O>
__global__ __launch_bounds__(256) void dq_walk_kernel(DqArgs a, int rows_per_group) {
  using S = typename T::storage;
  __shared__ __align__(16) int32_t t_src[kWalkTableInts];
  __shared__ __align__(16) float t_w[kWalkTableInts];
  const int R = rows_per_group;
  const int dps = kWalkTable / R;  // documents per stage, a multiple of 8
  const int stride = dps + kWalkPad;
  const int tid = threadIdx.x;
  const int64_t row0 = (int64_t)blockIdx.x * R;
  const int lr = tid / a.nslices;
  const int sl = tid - lr * a.nslices;
  const int64_t row = row0 + lr;
  const bool active = lr < R && row < a.rows;
  const int k0 = sl * 8;
  const uint32_t row_bytes = (uint32_t)a.dim * (uint32_t)sizeof(S);
  const char* __restrict__ Db = static_cast<const char*>(a.d);
  const S* __restrict__ D = static_cast<const S*>(a.d);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  const int tab = lr * stride;  // this lane's table row

  const uint32_t k0b = (uint32_t)k0 * (uint32_t)sizeof(S);
  auto gather = [&](int32_t src) -> Frag<T> {
    if constexpr (OFF32 && VEC) {
      // uniform base + one 32-bit offset per lane (the saddr form)
      const uint4* p = reinterpret_cast<const uint4*>(Db + ((uint32_t)src + k0b));
      Frag<T> f;
      if constexpr (T::bytes == 2) {
        f.v = p[0];
      } else {
        f.lo = p[0];
        f.hi = p[1];
      }
      return f;
    } else if constexpr (OFF32) {
      return load_frag<T>(reinterpret_cast<const S*>(Db + (uint32_t)src), k0, a.dim, VEC);
    } else {
      return load_frag<T>(D + (int64_t)src * a.dim, k0, a.dim, VEC);
    }
  };
  auto add = [&](const Frag<T>& v, float w) {
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = fmaf(w, frag_elem(v, e), acc[e]);
  };

  for (int64_t b0 = 0; b0 < a.nb; b0 += dps) {
    const int nd = (int)min((int64_t)dps, a.nb - b0);
    __syncthreads();  // the previous stage's table is consumed
    // consecutive threads take consecutive rows of one document: the argmax
    // reads of a query's tokens are contiguous
    for (int e = tid; e < R * dps; e += 256) {
      const int d = e / R;
      const int r = e - d * R;
      const int64_t rw = row0 + r;
      int32_t src = -1;
      float w = 0.0f;
      if (d < nd && rw < a.rows) {
        const int64_t qidx = rw / a.lq;
        const int i = (int)(rw - qidx * a.lq);
        const int64_t b = b0 + d;
        const int64_t s0 = a.doff[b], s1 = a.doff[b + 1];
        const int j = a.argmax[(qidx * a.nb + b) * a.lq + i];
        if (s0 >= 0 && s1 > s0 && s1 <= a.total_d && j >= 0 && j < s1 - s0) {
          src = OFF32 ? (int32_t)((uint32_t)(s0 + j) * row_bytes) : (int32_t)(s0 + j);
          w = score_grad(a.dscore, a.ce, qidx, b, a.nb);
        }
      }
      t_src[r * stride + d] = src;
      t_w[r * stride + d] = w;
    }
    __syncthreads();
    if (!active) continue;
    int d = 0;
    // eight documents per step; a step holding an invalid entry (or past
    // the stage's end) takes the masked form, which skips such entries
    for (; d < nd; d += 8) {
      // tab and d are multiples of 4: 16-byte LDS reads
      const int4* sp = static_cast<const int4*>(__builtin_assume_aligned(&t_src[tab + d], 16));
      const float4* wp = static_cast<const float4*>(__builtin_assume_aligned(&t_w[tab + d], 16));
      const int4 s_lo = sp[0], s_hi = sp[1];
      const float4 w_lo = wp[0], w_hi = wp[1];
      const int32_t s[8] = {s_lo.x, s_lo.y, s_lo.z, s_lo.w, s_hi.x, s_hi.y, s_hi.z, s_hi.w};
      const float w[8] = {w_lo.x, w_lo.y, w_lo.z, w_lo.w, w_hi.x, w_hi.y, w_hi.z, w_hi.w};
      int32_t smin = s[0];
#pragma unroll
      for (int u = 1; u < 8; ++u) smin = min(smin, s[u]);
      if (__all(smin >= 0) && d + 8 <= nd) {
        Frag<T> v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = gather(s[u]);
#pragma unroll
        for (int u = 0; u < 8; ++u) add(v[u], w[u]);
      } else {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          if (d + u < nd && s[u] >= 0) add(gather(s[u]), w[u]);
        }
      }
    }
  }
  if (active) store8<O>(out_at<O>(a.dq, row * a.dim), k0, a.dim, VEC, acc);
}

// ---------------------------------------------------------------------------
// dq, contrastive, one document range per XCD, all of an XCD's workgroups
// resident at once (dq_range_kernel).
//
// Random 16-byte gathers run at about 30 TB/s from L2 but 7-8 TB/s once
// they miss it (the MALL helps little for them), so the gather's working
// set must fit an XCD's 4 MB L2.  Documents are split into kXcds ranges,
// range r gathered only by the workgroups of XCD r (workgroup w runs on XCD
// w % 8), and the launch is one round (1024 workgroups of 128 rows at C5,
// four per CU), every workgroup walking its range's documents in order: the
// workgroups of an XCD then gather from the same few documents at any
// moment, and D is fetched from HBM about once.
//
// A wave holds 8 * 64 / NSL rows (NSL lanes per row, one 8-element slice
// each); a lane owns kRangeItems consecutive rows of one query (Lq % 8 ==
// 0).  Each stage of a workgroup first copies its rows' argmax for a chunk
// of documents into LDS with direct global->LDS loads (document-major, 32
// KB), and the chunk's weights and offsets with ordinary loads, so the walk
// waits on no HBM latency: per document a lane reads its rows' winners with
// two 16-byte LDS reads and issues eight gathers whose addresses are one
// multiply-add each.  The partial sums of range r go to ws[r];
// dq_reduce_kernel, or dd_bucket_kernel's fused share, adds the kXcds parts
// in range order.
// ---------------------------------------------------------------------------
constexpr int kRangeItems = 8;
constexpr int kRangeTableInts = 8192;              // argmax entries staged per stage (32 KB)
constexpr int kRangeMaxQueries = 2048 / 8 + 1;     // queries one workgroup's rows can touch

// Four waves per SIMD (<= 128 VGPRs) keep the launch one round at C5.
template <typename T, int NSL>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4)))
void dq_range_kernel(DqArgs a, float* __restrict__ ws) {
  using S = typename T::storage;
  constexpr int RPW = (64 / NSL) * kRangeItems;    // rows per wave
  constexpr int RW = 4 * RPW;                      // rows per workgroup
  constexpr int DC = kRangeTableInts / RW;         // documents per stage
  constexpr int QW = RW / 8 + 1;                   // queries per workgroup, at most
  __shared__ __align__(16) int32_t t_j[kRangeTableInts];  // [document][row]
  __shared__ float t_g[DC * QW];                          // [document][query]
  __shared__ int32_t t_off[DC + 1];
  const int r = blockIdx.x % kXcds;
  const int64_t row0 = (int64_t)(blockIdx.x / kXcds) * RW;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int sub = lane / NSL;
  const int sl = lane - sub * NSL;
  const int lr0 = wave * RPW + sub * kRangeItems;  // this lane's first row in the workgroup
  const int64_t row_base = row0 + lr0;
  const bool rows_ok = row_base < a.rows;          // all 8 rows valid: rows % 8 == 0
  const int64_t q_first = row0 / a.lq;
  const int q_lane = rows_ok ? (int)(row_base / a.lq - q_first) : 0;
  const int64_t b_lo = a.nb * r / kXcds;
  const int64_t b_hi = a.nb * (r + 1) / kXcds;
  const uint32_t row_bytes = (uint32_t)a.dim * (uint32_t)sizeof(S);
  const uint32_t k0b = (uint32_t)sl * 8u * (uint32_t)sizeof(S);
  const char* __restrict__ Db = static_cast<const char*>(a.d);
  const uint32_t lds_j = __builtin_amdgcn_readfirstlane(lds_addr(t_j));
  float acc[kRangeItems][8];
#pragma unroll
  for (int u = 0; u < kRangeItems; ++u)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[u][e] = 0.0f;

  for (int64_t c0 = b_lo; c0 < b_hi; c0 += DC) {
    const int nd = (int)min((int64_t)DC, b_hi - c0);
    __syncthreads();  // the previous stage's tables are consumed
    // argmax of the stage: LDS byte o holds document o / (4 RW), row
    // (o % (4 RW)) / 4 of the workgroup; a lane's 16 bytes are 4 consecutive
    // rows of one (query, document).  Entries past the stage's documents or
    // the last row are read from the start of argmax and never used.
    constexpr int kInstrs = kRangeTableInts * 4 / 1024;  // 1 KB per wave instruction
    for (int k = wave; k < kInstrs; k += 4) {
      const int o = k * 1024 + lane * 16;
      const int d = o / (RW * 4);
      const int64_t rw = row0 + (o - d * RW * 4) / 4;
      uint32_t src = 0;
      if (d < nd && rw < a.rows) {
        const int64_t q = rw / a.lq;
        src = (uint32_t)(((q * a.nb + c0 + d) * a.lq + (rw - q * a.lq)) * 4);
      }
      lds_dma16(a.argmax, src, lds_j + (uint32_t)k * 1024u);
    }
    for (int x = tid; x < nd * QW; x += 256) {
      const int d = x / QW;
      const int64_t q = q_first + (x - d * QW);
      t_g[x] = q < a.rows / a.lq ? score_grad(a.dscore, a.ce, q, c0 + d, a.nb) : 0.0f;
    }
    for (int x = tid; x <= nd; x += 256) t_off[x] = a.doff[c0 + x];
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's copies landed
    __syncthreads();
    if (!rows_ok) continue;
    for (int d = 0; d < nd; ++d) {
      const int4* jp = static_cast<const int4*>(__builtin_assume_aligned(&t_j[d * RW + lr0], 16));
      const int4 jlo = jp[0], jhi = jp[1];
      const int j[kRangeItems] = {jlo.x, jlo.y, jlo.z, jlo.w, jhi.x, jhi.y, jhi.z, jhi.w};
      const float g = t_g[d * QW + q_lane];
      const int s0 = __builtin_amdgcn_readfirstlane(t_off[d]);
      const int s1 = __builtin_amdgcn_readfirstlane(t_off[d + 1]);
      const bool doc_ok = s0 >= 0 && s1 > s0 && (int64_t)s1 <= a.total_d;
      const uint32_t len = doc_ok ? (uint32_t)(s1 - s0) : 0u;
      // every index is clamped into the document (an invalid document reads
      // row 0 of D), so each address is one min and one 24-bit multiply-add
      // (document lengths and row sizes are below 2^24)
      // (readfirstlane keeps the bound a scalar, so the clamp is one v_min)
      const uint32_t last = __builtin_amdgcn_readfirstlane(doc_ok ? len - 1u : 0u);
      const uint32_t base =
          __builtin_amdgcn_readfirstlane(doc_ok ? (uint32_t)s0 * row_bytes : 0u) + k0b;
      uint32_t jmax = (uint32_t)j[0];
#pragma unroll
      for (int u = 1; u < kRangeItems; ++u) jmax = max(jmax, (uint32_t)j[u]);
      // An out-of-range argmax (every entry of an invalid document) is
      // skipped, as the reference's guard does: the rare step that holds one
      // zeroes that fragment and its weight, so the additions below are the
      // same instructions either way.
      const bool all_ok = __all(jmax < len);
      Frag<T> v[kRangeItems];
      float w[kRangeItems];
#pragma unroll
      for (int u = 0; u < kRangeItems; ++u) {
        const uint32_t ju = min((uint32_t)j[u], last);
        const uint4* p = reinterpret_cast<const uint4*>(Db + (__umul24(ju, row_bytes) + base));
        if constexpr (T::bytes == 2) {
          v[u].v = p[0];
        } else {
          v[u].lo = p[0];
          v[u].hi = p[1];
        }
        w[u] = g;
      }
      if (!all_ok) {
#pragma unroll
        for (int u = 0; u < kRangeItems; ++u) {
          if ((uint32_t)j[u] >= len) {
            v[u] = zero_frag<T>();
            w[u] = 0.0f;
          }
        }
      }
#pragma unroll
      for (int u = 0; u < kRangeItems; ++u)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[u][e] = fmaf(w[u], frag_elem(v[u], e), acc[u][e]);
    }
  }
  if (rows_ok) {
#pragma unroll
    for (int u = 0; u < kRangeItems; ++u)
      store8f(ws + (int64_t)r * a.rows * a.dim + (row_base + u) * a.dim, sl * 8, a.dim, true,
              acc[u]);
  }
}

// dq[x] = sum over the kXcds partial buffers of x, in range order, written
// in the output type O (4 consecutive elements when vec).
template <typename O>
__device__ __forceinline__ void dq_reduce_unit(const float* __restrict__ ws,
                                               void* __restrict__ dq, int64_t n, bool vec,
                                               int64_t x) {
  if (vec) {
    // the partial sums are read once: non-temporal loads leave L2 to the
    // rows dD gathers when the reduce runs inside its launch (C5 fp32
    // backward 241 -> 232 us)
    const f32x4_t s0 = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(ws) + x);
    float4 s = make_float4(s0.x, s0.y, s0.z, s0.w);
#pragma unroll
    for (int r = 1; r < kXcds; ++r) {
      const f32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(ws + r * n) + x);
      s.x += v.x; s.y += v.y; s.z += v.z; s.w += v.w;
    }
    if constexpr (O::bytes == 4) {
      reinterpret_cast<float4*>(dq)[x] = s;
    } else {
      reinterpret_cast<uint2*>(dq)[x] =
          make_uint2(pack_out16<O>(s.x, s.y),
                     pack_out16<O>(s.z, s.w));
    }
  } else {
    float s = ws[x];
#pragma unroll
    for (int r = 1; r < kXcds; ++r) s += ws[r * n + x];
    if constexpr (O::bytes == 4)
      static_cast<float*>(dq)[x] = s;
    else
      static_cast<uint16_t*>(dq)[x] = to_out16<O>(s);
  }
}

// dq[x] = sum over the kXcds partial buffers, in range order, written in
// the output type O.
template <typename O>
__global__ __launch_bounds__(256) void dq_reduce_kernel(const float* __restrict__ ws,
                                                        void* __restrict__ dq,
                                                        int64_t n, bool vec) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t t0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t n4 = vec ? n / 4 : 0;
  for (int64_t x = t0; x < n4; x += stride) dq_reduce_unit<O>(ws, dq, n, true, x);
  for (int64_t x = n4 * 4 + t0; x < n; x += stride) dq_reduce_unit<O>(ws, dq, n, false, x);
}

// ---------------------------------------------------------------------------
// dd, contrastive: one workgroup per (document, part of the dimension), LDS
// counting sort.
//
// Document b receives one entry per (query q, token i): row argmax[q, b, i].
// The workgroup buckets those entries by target row in LDS (histogram,
// exclusive scan, scatter of entry ids), then groups of `group` lanes each
// own one row at a time and sum g[q, b] * q_row over the row's bucket in fp32
// registers, writing the gradient row once.  No floating-point atomics; every
// row of the document is written (zeros for rows no entry points at).
// Documents longer than `rows_per_pass` rows and entry sets larger than
// `entries_per_pass` are processed in passes (later entry passes add to the
// rows already written).
//
// Every document gathers rows from all of Q, so Q should stay in L2.  The
// embedding dimension is split into `parts` (1, 2, 4 or 8) slice ranges, part
// p handled only by XCDs [p * 8 / parts, (p + 1) * 8 / parts) (workgroup w
// runs on XCD w % 8): each XCD then gathers from 1 / parts of Q.  The
// bucketing is repeated per part; its argmax reads are the cheaper side.
// Batches of few documents also take more parts, to fill the chip.
// ---------------------------------------------------------------------------
struct DdArgs {
  CeGrad ce;
  const float* dscore;
  const void* q;
  const int32_t* argmax;
  const int32_t* doff;
  void* dd;              // fp32, or the input's 16-bit type (one entry pass only)
  int64_t nq;
  int64_t nb;
  int64_t total_d;
  int lq;
  int dim;
  int nslices;
  int rows_per_pass;     // R: rows bucketed per pass (LDS: 2 * (R + 1) ints)
  int entries_per_pass;  // E: entry ids held per pass (LDS: E ints)
  int parts;             // dimension parts (1, 2, 4 or 8; divides kXcds)
  int part_slices;       // 8-element slices per part (last part may hold fewer)
  int group;             // lanes per row: power of two, <= 16, part_slices <= NS * group
  // dd_bucket_kernel only: places per round of the deal (0: place b takes
  // document b), and the shift that turns a document's rows into its key
  int deal_places;
  int deal_shift;
  // dd_bucket_kernel only: when dq_ws is set, each workgroup also adds its
  // share of the kXcds dQ partial sums once its document is done (the work
  // of dq_reduce_kernel, in the same order), so the memory-bound reduce
  // overlaps the other workgroups' gathers instead of taking a launch.
  const float* dq_ws;
  void* dq_out;          // [dq_n] in the output type O
  int64_t dq_n;
  int dq_vec;            // dq_n % 4 == 0, dq_ws and dq_out 16-byte aligned
};

constexpr int kDdThreads = 512;
constexpr int kDdWaves = kDdThreads / 64;
constexpr int kDealKeys = 64;  // document keys of the dD deal: rows >> deal_shift, clamped
constexpr int kDdMaxGroup = 16;
constexpr int kDdBatch = 8;      // bucket entries gathered per step
constexpr int kDdBlock = 32;     // bucket entries per block sum
constexpr int kDdSortBatch = 8;  // argmax loads in flight per thread while sorting

// x / d for 0 <= x < 2^24, d >= 1, from a float reciprocal: x is exact in
// fp32 and the rounded product is within one of the quotient (exact for
// d <= 2), so one remainder check gives the exact result.  Avoids the
// branchy software integer division in the per-entry loops.
__device__ __forceinline__ int div_small(int x, int d, float inv_d) {
  int q = (int)((float)x * inv_d);
  const int r = x - q * d;
  q += (r >= d) ? 1 : 0;
  q -= (r < 0) ? 1 : 0;
  return q;
}

// Entries are processed in passes of whole queries when Lq <= E (qc queries
// x Lq tokens), else in chunks of one query's tokens; pass-local entry x is
// (query q0 + x / ic, token i0 + x % ic) with ic the tokens per query in the
// pass, so its Q row is q0 * Lq + i0 + x in both cases.  The bucket holds
// x | (x / ic) << 16 (x < 2^16), and the pass's dscore values are staged in
// LDS, so the summation needs no division and no per-entry global index.
// The gradient is written in the output type O; a 16-bit O requires a single
// entry pass (the host checks), since later passes add to the rows in fp32.
// Rows before the first and after the last document are zeroed by part 0 of
// the first and the last document.
template <typename T, bool VEC, int NS, typename O>
__global__ __launch_bounds__(kDdThreads) void dd_contrastive_kernel(DdArgs a) {
  using S = typename T::storage;
  extern __shared__ int lds_i[];
  const int R = a.rows_per_pass;
  const int E = a.entries_per_pass;
  int* start = lds_i;                 // [R + 1]
  int* cursor = start + (R + 1);      // [R + 1]
  int* ids = cursor + (R + 1);        // [E]
  float* gst = reinterpret_cast<float*>(ids + E);  // [queries per pass]

  // workgroup w -> XCD x = w % 8; part = x / (8 / parts); document
  // b = (w / 8) * (8 / parts) + x % (8 / parts)
  const int xcd = blockIdx.x % kXcds;
  const int per_part = kXcds / a.parts;
  const int part = xcd / per_part;
  const int64_t b = (int64_t)(blockIdx.x / kXcds) * per_part + xcd % per_part;
  if (b >= a.nb) return;
  if (part == 0 && (b == 0 || b == a.nb - 1)) {
    const int64_t head = min(max((int64_t)a.doff[0], (int64_t)0), a.total_d);
    const int64_t tail = min(max((int64_t)a.doff[a.nb], head), a.total_d);
    auto zero_rows = [&](int64_t lo, int64_t hi) {
      for (int64_t x = lo * a.dim + threadIdx.x; x < hi * a.dim; x += kDdThreads) {
        if constexpr (O::bytes == 4)
          static_cast<float*>(a.dd)[x] = 0.0f;
        else
          static_cast<uint16_t*>(a.dd)[x] = 0;
      }
    };
    if (b == 0) zero_rows(0, head);
    if (b == a.nb - 1) zero_rows(tail, a.total_d);
  }
  const int64_t d0 = a.doff[b], d1 = a.doff[b + 1];
  if (d0 < 0 || d1 <= d0 || d1 > a.total_d) return;
  const int ld = (int)(d1 - d0);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int G = a.group;
  const int ngroups = kDdThreads / G;
  const int grp = tid / G;
  const int gl = tid - grp * G;
  const int sl_lo = part * a.part_slices;
  const int sl_hi = min(sl_lo + a.part_slices, a.nslices);
  const S* __restrict__ Q = static_cast<const S*>(a.q);
  const int32_t* am_b = a.argmax + b * a.lq;   // entry (q, i) at am_b[q*nb*lq + i]
  const int64_t am_qstride = a.nb * a.lq;
  const int tok_chunk = min(a.lq, E);
  const int64_t qpp = (a.lq <= E) ? E / a.lq : 1;

  for (int r0 = 0; r0 < ld; r0 += R) {
    const int nrows = min(R, ld - r0);
    for (int64_t q0 = 0; q0 < a.nq; q0 += qpp) {
      for (int i0 = 0; i0 < a.lq; i0 += tok_chunk) {
        const int qc = (int)min(qpp, a.nq - q0);
        const int ic = min(tok_chunk, a.lq - i0);
        const int ne = qc * ic;
        const float inv_ic = 1.0f / (float)ic;
        const bool first = (q0 == 0 && i0 == 0);
        const int32_t* am_p = am_b + q0 * am_qstride + i0;
        const S* Qp = Q + (q0 * a.lq + i0) * (int64_t)a.dim;
        for (int x = tid; x <= nrows; x += kDdThreads) start[x] = 0;
        for (int x = tid; x < qc; x += kDdThreads)
          gst[x] = score_grad(a.dscore, a.ce, q0 + x, b, a.nb);
        __syncthreads();
        // Entry x's target row, relative to the row pass (out of range: not
        // in this pass or invalid).  Both sort phases read the argmax
        // kDdSortBatch entries per thread at a time, so that many loads are in
        // flight before the first LDS atomic waits on one.  Loads past ne read
        // entry ne - 1 and are dropped: an unconditional load keeps the
        // compiler from waiting on each one at a branch join.
        auto load_targets = [&](int x0, int (&jj)[kDdSortBatch], int (&pk)[kDdSortBatch]) {
#pragma unroll
          for (int k = 0; k < kDdSortBatch; ++k) {
            const int x = min(x0 + k * kDdThreads, ne - 1);
            const int ql = div_small(x, ic, inv_ic);
            jj[k] = am_p[ql * am_qstride + (x - ql * ic)] - r0;
            pk[k] = x | (ql << 16);
          }
#pragma unroll
          for (int k = 0; k < kDdSortBatch; ++k)
            if (x0 + k * kDdThreads >= ne) jj[k] = -1;
        };
        // 1. histogram of target rows
        for (int x0 = tid; x0 < ne; x0 += kDdThreads * kDdSortBatch) {
          int jj[kDdSortBatch], pk[kDdSortBatch];
          load_targets(x0, jj, pk);
#pragma unroll
          for (int k = 0; k < kDdSortBatch; ++k)
            if (jj[k] >= 0 && jj[k] < nrows) atomicAdd(&start[jj[k] + 1], 1);
        }
        __syncthreads();
        // 2. inclusive scan of start[1..nrows] by wave 0 (lane owns a run)
        if (tid < 64) {
          const int per = (nrows + 63) / 64;
          const int lo = 1 + lane * per;
          const int hi = min(lo + per, nrows + 1);
          int run = 0;
          for (int x = lo; x < hi; ++x) run += start[x];
          int incl = run;
#pragma unroll
          for (int off = 1; off < 64; off <<= 1) {
            const int v = __shfl_up(incl, off);
            if (lane >= off) incl += v;
          }
          int acc = incl - run;
          for (int x = lo; x < hi; ++x) {
            acc += start[x];
            start[x] = acc;
          }
        }
        __syncthreads();
        for (int x = tid; x < nrows; x += kDdThreads) cursor[x] = start[x];
        __syncthreads();
        // 3. scatter packed entry ids into their row buckets
        for (int x0 = tid; x0 < ne; x0 += kDdThreads * kDdSortBatch) {
          int jj[kDdSortBatch], pk[kDdSortBatch];
          load_targets(x0, jj, pk);
#pragma unroll
          for (int k = 0; k < kDdSortBatch; ++k)
            if (jj[k] >= 0 && jj[k] < nrows) ids[atomicAdd(&cursor[jj[k]], 1)] = pk[k];
        }
        __syncthreads();
        // 4. per-row fp32 sums, one group of G lanes per row; a row wider
        // than NS * G slices (dims above 256 per part) is summed in chunks
        for (int rr = grp; rr < nrows; rr += ngroups)
        for (int sc = sl_lo; sc < sl_hi; sc += NS * G) {
          float acc[NS][8];
          void* dst = out_at<O>(a.dd, (d0 + r0 + rr) * (int64_t)a.dim);
#pragma unroll
          for (int u = 0; u < NS; ++u) {
            const int sl = sc + gl + u * G;
            if (O::bytes == 4 && sl < sl_hi && !first) {
              load8f<F32>(static_cast<const float*>(dst), sl * 8, a.dim, VEC, acc[u]);
            } else {
#pragma unroll
              for (int k = 0; k < 8; ++k) acc[u][k] = 0.0f;
            }
          }
          const int s_end = start[rr + 1];
          // Blocked summation: entries are added into a block sum, and every
          // kDdBlock entries the block is added to the row sum.  A bucket can
          // hold every entry of the batch (one-row documents, duplicated
          // rows); plain sequential fp32 summation of n terms drifts like
          // eps * n, blocking brings that to about eps * (kDdBlock + n / kDdBlock).
          for (int s0 = start[rr]; s0 < s_end; s0 += kDdBlock) {
            const int s1 = min(s0 + kDdBlock, s_end);
            float blk[NS][8];
#pragma unroll
            for (int u = 0; u < NS; ++u)
#pragma unroll
              for (int e2 = 0; e2 < 8; ++e2) blk[u][e2] = 0.0f;
            // kDdBatch entries per step keep that many row loads in flight per
            // lane.  Full steps are unmasked; the last step of a block repeats
            // its first entry past the block end and does not add it.
            auto batch = [&](int s, auto masked) {
              constexpr bool MASKED = decltype(masked)::value;
              const S* row[kDdBatch];
              float gx[kDdBatch];
              bool ok[kDdBatch];
#pragma unroll
              for (int k = 0; k < kDdBatch; ++k) {
                ok[k] = !MASKED || s + k < s1;
                const uint32_t v = (uint32_t)ids[ok[k] ? s + k : s];
                row[k] = Qp + (int64_t)(v & 0xffffu) * a.dim;
                gx[k] = gst[v >> 16];
              }
#pragma unroll
              for (int u = 0; u < NS; ++u) {
                const int sl = sc + gl + u * G;
                if (sl < sl_hi) {
                  // raw 16-byte fragments, widened to fp32 inside the FMAs
                  Frag<T> v[kDdBatch];
#pragma unroll
                  for (int k = 0; k < kDdBatch; ++k)
                    v[k] = load_frag<T>(row[k], sl * 8, a.dim, VEC);
#pragma unroll
                  for (int k = 0; k < kDdBatch; ++k) {
#pragma unroll
                    for (int e2 = 0; e2 < 8; ++e2) {
                      const float t = fmaf(gx[k], frag_elem(v[k], e2), blk[u][e2]);
                      blk[u][e2] = (!MASKED || ok[k]) ? t : blk[u][e2];
                    }
                  }
                }
              }
            };
            int s = s0;
            for (; s + kDdBatch <= s1; s += kDdBatch) batch(s, std::false_type{});
            if (s < s1) batch(s, std::true_type{});
#pragma unroll
            for (int u = 0; u < NS; ++u)
#pragma unroll
              for (int e2 = 0; e2 < 8; ++e2) acc[u][e2] += blk[u][e2];
          }
#pragma unroll
          for (int u = 0; u < NS; ++u) {
            const int sl = sc + gl + u * G;
            if (sl < sl_hi) store8<O>(dst, sl * 8, a.dim, VEC, acc[u]);
          }
        }
        __syncthreads();
      }
    }
  }
}

// ---------------------------------------------------------------------------
// dd, contrastive, the common case (dd_bucket_kernel): rows of 16-byte
// fragments, dim <= 256 per part with an even number of 8-element slices,
// every (query, token) entry of a document in one LDS pass, Q below 2 GiB.
// Same counting sort and blocked row sums as dd_contrastive_kernel, with
// less work per entry:
//   * the document's argmax entries stay in registers between the
//     histogram and the scatter (one read of argmax instead of two), and
//     the (query, token) of an entry needs no division: a thread's entries
//     are x = tid + 512 k, so when Lq divides 512 the token is fixed and the
//     query advances by 512 / Lq;
//   * Q rows are addressed as one 32-bit offset from a uniform base (one
//     24-bit multiply-add per entry), and eight entries (eight 16-byte
//     loads) are in flight per lane;
//   * the groups of a wave run in lockstep, so a wave's time per round of
//     rows is its largest bucket: rows are visited in decreasing bucket
//     size (a counting sort of the rows by size class), so that the rows
//     of a round have about the same size (documents of at least
//     kBkOrderMin entries; below that the sort costs more than it saves).
// ---------------------------------------------------------------------------
// (a & 0xffff) * (b & 0xffff) + c in one VALU instruction (the compiler
// selects an AND and a 24-bit multiply-add for the same expression).
__device__ __forceinline__ uint32_t mad_u16(uint32_t a, uint32_t b, uint32_t c) {
  uint32_t r;
  asm("v_mad_u32_u16 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(b), "v"(c));
  return r;
}

constexpr int kBkBatch = 8;            // bucket entries gathered per step
constexpr int kBkMaxEntriesPerThread = 32;
constexpr int kBkClasses = 256;        // row size classes: ceil(entries / 4), capped
constexpr int kBkOrderMin = 4096;      // entries per document from which rows are ordered

template <typename T, int NS, typename O>
__device__ __forceinline__ void dd_bucket_document(DdArgs a) {
  using S = typename T::storage;
  extern __shared__ int lds_i[];
  const int R = a.rows_per_pass;
  const int E = a.entries_per_pass;
  // The staged score gradients come first, at LDS byte 0, so that an
  // entry id (row x | (query * 4) << 16) holds its weight's LDS address.
  float* gst = reinterpret_cast<float*>(lds_i);  // [Nq]
  int* start = lds_i + a.nq;          // [R + 1]
  int* cursor = start + (R + 1);      // [R + 1]
  int* ids = cursor + (R + 1);        // [E]

  const int xcd = blockIdx.x % kXcds;
  const int per_part = kXcds / a.parts;
  const int part = xcd / per_part;
  // place p of the grid (its workgroups: one per part)
  const int64_t p = (int64_t)(blockIdx.x / kXcds) * per_part + xcd % per_part;
  if (p >= a.nb) return;
  if (part == 0 && (p == 0 || p == a.nb - 1)) {
    const int64_t head = min(max((int64_t)a.doff[0], (int64_t)0), a.total_d);
    const int64_t tail = min(max((int64_t)a.doff[a.nb], head), a.total_d);
    auto zero_rows = [&](int64_t lo, int64_t hi) {
      for (int64_t x = lo * a.dim + threadIdx.x; x < hi * a.dim; x += kDdThreads) {
        if constexpr (O::bytes == 4)
          static_cast<float*>(a.dd)[x] = 0.0f;
        else
          static_cast<uint16_t*>(a.dd)[x] = 0;
      }
    };
    if (p == 0) zero_rows(0, head);
    if (p == a.nb - 1) zero_rows(tail, a.total_d);
  }
  // The document of place p.  A workgroup's time follows its document's
  // rows, and the workgroups of places p and p + deal_places run on one CU
  // (workgroups w and w + CUs share a CU when the grid is dealt round-robin
  // over the CUs) and share its VALU.  So the documents are ranked by rows,
  // longest first (every workgroup ranks them all itself, one thread per
  // document, the same ranks everywhere), and dealt so that the two places
  // of a CU take ranks that add up to the same total: with n2 = nb - P
  // places in the second round (P = deal_places), the P - n2 longest
  // documents take the CUs with one place, and the others pair rank
  // P - n2 + c with rank nb - 1 - c.  More than two rounds: longest first.
  int64_t b = p, d0, d1;
  if (a.deal_places > 0) {
    // scratch from LDS byte 0 (the staged gradients and bucket arrays, not
    // yet written); the pick in the last three ints of the cursor array,
    // which the first pass writes two barriers after it is read
    using Rank = RankScratch<kDdWaves, kDealKeys>;
    const Rank rs(lds_i);
    int* pick = ids - 3;                          // document, its first and end row
    static_assert(Rank::kBytes <= (2 * (1024 + 1) - 3) * (int)sizeof(int),
                  "ranking scratch ends before the pick");
    rs.clear();
    if (threadIdx.x == 0) pick[0] = -1;
    const bool own = threadIdx.x < a.nb;
    int key = 0, s0 = 0, e0 = 0;
    if (own) {
      s0 = a.doff[threadIdx.x];
      e0 = a.doff[threadIdx.x + 1];
      if (s0 >= 0 && e0 > s0 && (int64_t)e0 <= a.total_d)
        key = min((e0 - s0) >> a.deal_shift, kDealKeys - 1);
    }
    const int r = rs.rank(own, key);
    const int P = a.deal_places, nb = (int)a.nb, q = (int)p;
    int want = q;  // a permutation of [0, nb) for any P
    if (nb > P && nb <= 2 * P) {
      const int n2 = nb - P;
      want = q >= P ? nb - 1 - (q - P) : (q >= n2 ? q - n2 : P - n2 + q);
    }
    // the ranks are a permutation of [0, nb): exactly one thread matches
    // (were none to, the place would keep its own document)
    if (r == want) {
      pick[0] = (int)threadIdx.x;
      pick[1] = s0;
      pick[2] = e0;
    }
    __syncthreads();
    const int got = __builtin_amdgcn_readfirstlane(pick[0]);
    if (got >= 0) {
      b = got;
      d0 = __builtin_amdgcn_readfirstlane(pick[1]);
      d1 = __builtin_amdgcn_readfirstlane(pick[2]);
    } else {
      d0 = a.doff[b];
      d1 = a.doff[b + 1];
    }
  } else {
    d0 = a.doff[b];
    d1 = a.doff[b + 1];
  }
  if (d0 < 0 || d1 <= d0 || d1 > a.total_d) return;
  const int ld = (int)(d1 - d0);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int G = a.group;               // lanes per row; each lane owns NS slices
  const int ngroups = kDdThreads / G;
  const int grp = tid / G;
  const int gl = tid - grp * G;
  const int sl_lo = part * a.part_slices;
  const int sl_hi = min(sl_lo + a.part_slices, a.nslices);
  const int ne = (int)(a.nq * a.lq);   // every entry in one pass (host checks)
  const int32_t* am_b = a.argmax + b * a.lq;
  // The argmax is below 2^31 bytes (host checks), so the 32-bit byte
  // offsets below cannot wrap.
  const int am_qstride = (int)(a.nb * a.lq);
  const MAXSIM_GLOBAL char* Qb = uniform_gptr(static_cast<const char*>(a.q));
  const uint32_t row_bytes = (uint32_t)a.dim * (uint32_t)sizeof(S);
  // this lane's NS consecutive slices of a row, from sc (the host makes a
  // part exactly NS * G slices)
  const int sc = sl_lo + NS * gl;
  const uint32_t k0b = (uint32_t)sc * 8u * (uint32_t)sizeof(S);
  (void)sl_hi;
  // A thread's entries are x = tid + 512 k.  Lq divides 512 (host checks),
  // so every one of them has token tid % Lq and the query advances by
  // 512 / Lq: the argmax of entry k is one uniform base plus a 32-bit offset
  // that grows by a fixed step.
  const int q_t = tid / a.lq;
  const int i_t = tid - q_t * a.lq;
  const int q_step = kDdThreads / a.lq;
  const MAXSIM_GLOBAL char* amB = uniform_gptr(reinterpret_cast<const char*>(am_b));
  const uint32_t off_t = (uint32_t)(q_t * am_qstride + i_t) * 4u;
  const uint32_t off_step = (uint32_t)(q_step * am_qstride) * 4u;
  const uint32_t off_last = (uint32_t)((a.nq - 1) * am_qstride + (a.lq - 1)) * 4u;
  for (int x = tid; x < a.nq; x += kDdThreads) gst[x] = score_grad(a.dscore, a.ce, x, b, a.nb);

  // entries of this thread with a valid query: k < nk
  const int nk_t = min((int)((a.nq - q_t + q_step - 1) / q_step), kBkMaxEntriesPerThread);
  for (int r0 = 0; r0 < ld; r0 += R) {
    const int nrows = min(R, ld - r0);
    // Opaque per pass: otherwise the compiler hoists every entry's validity
    // mask and packed id out of the pass loop (64 SGPRs, 32 VGPRs, spills).
    int nk = nk_t, qt = q_t, xt = tid;
    uint32_t offt = off_t;
    __asm__ __volatile__("" : "+v"(nk), "+v"(qt), "+v"(xt), "+v"(offt));
    for (int x = tid; x <= nrows; x += kDdThreads) start[x] = 0;
    __syncthreads();
    // 1. read this thread's entries (all issued before the first atomic;
    // entries past the last query re-read the last entry and are dropped)
    // and histogram their target rows
    int jj[kBkMaxEntriesPerThread];
#pragma unroll
    for (int k = 0; k < kBkMaxEntriesPerThread; ++k) {
      const uint32_t off = min(offt + (uint32_t)k * off_step, off_last);
      const int v = *reinterpret_cast<const MAXSIM_GLOBAL int*>(amB + off);
      jj[k] = k < nk ? v - r0 : -1;
    }
#pragma unroll
    for (int k = 0; k < kBkMaxEntriesPerThread; ++k)
      if (jj[k] >= 0 && jj[k] < nrows) atomicAdd(&start[jj[k] + 1], 1);
    __syncthreads();
    // 2. inclusive scan of start[1..nrows] by wave 0 (a lane owns a run)
    if (tid < 64) {
      const int per = (nrows + 63) / 64;
      const int lo = 1 + lane * per;
      const int hi = min(lo + per, nrows + 1);
      int run = 0;
      for (int x = lo; x < hi; ++x) run += start[x];
      int incl = run;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int v = __shfl_up(incl, off);
        if (lane >= off) incl += v;
      }
      int acc = incl - run;
      for (int x = lo; x < hi; ++x) {
        acc += start[x];
        start[x] = acc;
      }
    }
    __syncthreads();
    for (int x = tid; x < nrows; x += kDdThreads) cursor[x] = start[x];
    __syncthreads();
    // 3. scatter packed entry ids (x | (query * 4) << 16: x < 2^14 and
    // query < 2^14, host checks) from the registers
#pragma unroll
    for (int k = 0; k < kBkMaxEntriesPerThread; ++k) {
      if (jj[k] >= 0 && jj[k] < nrows) {
        const uint32_t x = (uint32_t)(xt + k * kDdThreads);
        ids[atomicAdd(&cursor[jj[k]], 1)] = (int)(x | ((uint32_t)(qt + k * q_step) << 18));
      }
    }
    __syncthreads();
    // 4. row order: decreasing size class ceil(n / 4) (counting sort; the
    // class table and the order use the cursor array, free after the
    // scatter: kBkClasses ints, then nrows 16-bit row ids).  Small entry
    // sets keep the natural order.
    const bool ordered = ne >= kBkOrderMin;
    int* chist = cursor;
    uint16_t* order = reinterpret_cast<uint16_t*>(cursor + kBkClasses);
    auto row_class = [&](int x) {
      return kBkClasses - 1 - min((start[x + 1] - start[x] + 3) >> 2, kBkClasses - 1);
    };
    if (ordered) {
      for (int x = tid; x < kBkClasses; x += kDdThreads) chist[x] = 0;
      __syncthreads();
      for (int x = tid; x < nrows; x += kDdThreads) atomicAdd(&chist[row_class(x)], 1);
      __syncthreads();
      if (tid < 64) {
        constexpr int per = kBkClasses / 64;
        int c[per];
        int run = 0;
#pragma unroll
        for (int k = 0; k < per; ++k) {
          c[k] = chist[lane * per + k];
          run += c[k];
        }
        int incl = run;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
          const int v = __shfl_up(incl, off);
          if (lane >= off) incl += v;
        }
        int acc = incl - run;
#pragma unroll
        for (int k = 0; k < per; ++k) {
          chist[lane * per + k] = acc;
          acc += c[k];
        }
      }
      __syncthreads();
      for (int x = tid; x < nrows; x += kDdThreads)
        order[atomicAdd(&chist[row_class(x)], 1)] = (uint16_t)x;
      __syncthreads();
    }
    // 5. per-row fp32 sums: a group of G lanes per row, NS slices per lane
    for (int ix = grp; ix < nrows; ix += ngroups) {
      const int rr = ordered ? (int)order[ix] : ix;
      float acc[NS][8];
#pragma unroll
      for (int u = 0; u < NS; ++u)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[u][e] = 0.0f;
      void* dst = out_at<O>(a.dd, (d0 + r0 + rr) * (int64_t)a.dim);
      const int s_beg = start[rr], s_end = start[rr + 1];
      // the fma sums of the entries [s0, s0 + kDdBlock) into sum
      auto block = [&](int s0, float (&sum)[NS][8]) __attribute__((always_inline)) {
        const int s1 = min(s0 + kDdBlock, s_end);
        // KB entries from s (KB = 8, or 4 for a short tail)
        auto batch = [&](int s, auto masked, auto kb) {
          constexpr bool MASKED = decltype(masked)::value;
          constexpr int KB = decltype(kb)::value;
          uint32_t off[KB];
          float gx[KB];
          bool ok[KB];
#pragma unroll
          for (int k = 0; k < KB; ++k) {
            ok[k] = !MASKED || s + k < s1;
            const uint32_t v = (uint32_t)ids[ok[k] ? s + k : s];
            off[k] = mad_u16(v, row_bytes, k0b);
            gx[k] = *reinterpret_cast<const float*>(reinterpret_cast<const char*>(gst) + (v >> 16));
          }
          Frag<T> f[KB][NS];
#pragma unroll
          for (int k = 0; k < KB; ++k)
#pragma unroll
            for (int u = 0; u < NS; ++u) {
              const uint32_t o = off[k] + (uint32_t)u * 8u * (uint32_t)sizeof(S);
              if constexpr (T::bytes == 2) {
                f[k][u].v = load16(Qb, o);
              } else {
                f[k][u].lo = load16(Qb, o);
                f[k][u].hi = load16(Qb, o + 16u);
              }
            }
          // past the bucket's end (the last step of a block) an entry
          // repeats the step's first one; its fragment and weight are zeroed
          // (fmaf(0, 0, x) == x exactly), which is cheaper than selecting
          // each of its sums
          if constexpr (MASKED) {
#pragma unroll
            for (int k = 0; k < KB; ++k) {
              if (!ok[k]) {
                gx[k] = 0.0f;
#pragma unroll
                for (int u = 0; u < NS; ++u) f[k][u] = zero_frag<T>();
              }
            }
          }
#pragma unroll
          for (int k = 0; k < KB; ++k)
#pragma unroll
            for (int u = 0; u < NS; ++u)
#pragma unroll
              for (int e = 0; e < 8; ++e)
                sum[u][e] = fmaf(gx[k], frag_elem(f[k][u], e), sum[u][e]);
        };
        using B8 = std::integral_constant<int, kBkBatch>;
        using B4 = std::integral_constant<int, kBkBatch / 2>;
        int s = s0;
        for (; s + kBkBatch <= s1; s += kBkBatch) batch(s, std::false_type{}, B8{});
        if (s1 - s > kBkBatch / 2)
          batch(s, std::true_type{}, B8{});
        else if (s < s1)
          batch(s, std::true_type{}, B4{});
      };
      // The first block sums straight into the row sum; adding +0 then gives
      // the bits of 0 + block (a chain from +0 ends at -0 only when a
      // negative product rounds to zero, which this turns into +0).
      if (s_beg < s_end) {
        block(s_beg, acc);
#pragma unroll
        for (int u = 0; u < NS; ++u)
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[u][e] += 0.0f;
      }
      for (int s0 = s_beg + kDdBlock; s0 < s_end; s0 += kDdBlock) {
        float blk[NS][8];
#pragma unroll
        for (int u = 0; u < NS; ++u)
#pragma unroll
          for (int e = 0; e < 8; ++e) blk[u][e] = 0.0f;
        block(s0, blk);
#pragma unroll
        for (int u = 0; u < NS; ++u)
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[u][e] += blk[u][e];
      }
#pragma unroll
      for (int u = 0; u < NS; ++u) store8<O>(dst, (sc + u) * 8, a.dim, true, acc[u]);
    }
    __syncthreads();
  }
}

// One document (and dimension part) per workgroup and, when the dQ reduce
// is fused in, the workgroup's contiguous share of the reduce units (every
// workgroup takes one, including those with no valid document).  The share
// comes after the document for 16-bit gradients and before it for fp32 ones
// (C5: 240 -> 233 us and 259 -> 253 us, against 240 -> 236 and 259 -> 258
// the other way round; the dQ bits are the same either way).
template <typename T, int NS, typename O>
__global__ __launch_bounds__(kDdThreads) void dd_bucket_kernel(DdArgs a) {
  auto reduce_share = [&]() {
    const bool vec = a.dq_vec != 0;
    const int64_t units = vec ? a.dq_n / 4 : a.dq_n;
    const int64_t per = (units + gridDim.x - 1) / gridDim.x;
    const int64_t lo = (int64_t)blockIdx.x * per;
    const int64_t hi = min(lo + per, units);
    for (int64_t x = lo + threadIdx.x; x < hi; x += kDdThreads)
      dq_reduce_unit<O>(a.dq_ws, a.dq_out, a.dq_n, vec, x);
  };
  constexpr bool kReduceFirst = O::bytes == 4;
  if (kReduceFirst && a.dq_ws) reduce_share();
  dd_bucket_document<T, NS, O>(a);
  if (!kReduceFirst && a.dq_ws) reduce_share();
}

// ---------------------------------------------------------------------------
// dd, padded: a candidate's rows are split over nsplit waves (one candidate
// alone is too little work per wave when B*C is small); each wave writes its
// rows, zeros included, and adds its tokens in token order, so the result is
// deterministic and does not depend on the split.
// ---------------------------------------------------------------------------
struct PaddedDdArgs {
  const float* dscore;
  const void* q;
  const int32_t* argmax;
  const int32_t* qlen;
  const int32_t* dlen;
  void* dd;  // fp32, or the 16-bit output type O
  int64_t npairs;
  int64_t ncand;
  int lq_max;
  int ld_max;
  int dim;
  int pair;    // 16-bit O: dim even, q and dd 4-byte aligned (32-bit accesses)
  int am_lds;  // argmax ints per wave staged in LDS (0: none)
  int nsplit;  // waves per candidate, each owning rows_per_split rows
  int rows_per_split;
  int vec_rows;  // 64 % (dim / 8) == 0, q and dd 16-byte aligned: whole rows per lane group
};

// Element x of query row qrow as fp32.
template <typename T>
__device__ __forceinline__ float elem_f32(const typename T::storage* qrow, int x) {
  if constexpr (T::bytes == 4) {
    return qrow[x];
  } else if constexpr (__is_same(T, BF16)) {
    return __uint_as_float((uint32_t)qrow[x] << 16);
  } else {
    return (float)__builtin_bit_cast(_Float16, qrow[x]);
  }
}

// 16-bit O: each row of the candidate is written once.  For row r the wave
// ballots the query tokens whose argmax is r (64 tokens at a time) and sums
// g * q_t over them in token order, from zero, with the same fmaf sequence as
// the fp32 path below, then rounds: the bits are those of the fp32 gradient
// cast to O.  Rows no token points at, padding rows and the rows of an
// invalid candidate are zero.
//
// Each lane owns 4 elements of a row: with a.pair, elements 2*lane, +1 and
// 128 + 2*lane, +1 (32-bit loads and stores), else lane + 64*i.  The argmax
// of the first 256 tokens is kept in registers and the rest, when a.am_lds
// is set, in this wave's am_lds slice, so the row loop reads no global memory
// for it; otherwise tokens past 256 are read again for every row.
constexpr int kDdAmRegs = 4;
constexpr int kDdAmLdsMax = 4096;  // ints per wave: 64 KB for the 4 waves

template <typename T, typename O>
__device__ __forceinline__ void dd_padded_rows16(const PaddedDdArgs& a, int64_t p, int64_t b,
                                                 int r0, int r1, int lane, int32_t* am_lds) {
  using S = typename T::storage;
  uint16_t* base = static_cast<uint16_t*>(a.dd) + p * a.ld_max * (int64_t)a.dim;
  const int lqb = a.qlen[b];
  const int ld = a.dlen[p];
  const bool ok = lqb >= 1 && lqb <= a.lq_max && ld >= 1 && ld <= a.ld_max;
  const float g = a.dscore[p];
  const S* __restrict__ Q = static_cast<const S*>(a.q);
  const int32_t* am = a.argmax + p * a.lq_max;
  int amv[kDdAmRegs];
#pragma unroll
  for (int c = 0; c < kDdAmRegs; ++c) {
    const int t = 64 * c + lane;
    amv[c] = ok && t < lqb ? am[t] : -1;
  }
  if (a.am_lds) {
    if (ok)
      for (int t = 64 * kDdAmRegs + lane; t < lqb; t += 64) am_lds[t - 64 * kDdAmRegs] = am[t];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  // a lane covers 4 columns of each 256-column block; wider rows take
  // several blocks
  for (int cb = 0; cb < a.dim; cb += 256) {
  int xs[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    xs[i] = cb + (a.pair ? 128 * (i >> 1) + 2 * lane + (i & 1) : lane + 64 * i);
  for (int r = r0; r < r1; ++r) {
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (ok && r < ld) {
      for (int c0 = 0; c0 < lqb; c0 += 64) {
        const int t = c0 + lane;
        int j = -1;
        if (c0 < 64 * kDdAmRegs) {
#pragma unroll
          for (int c = 0; c < kDdAmRegs; ++c)
            if (c0 == 64 * c) j = amv[c];
        } else if (t < lqb) {
          j = a.am_lds ? am_lds[t - 64 * kDdAmRegs] : am[t];
        }
        uint64_t hits = __ballot(j == r);
        while (hits) {
          const int tok = c0 + __builtin_ctzll(hits);
          hits &= hits - 1;
          const S* qrow = Q + (b * a.lq_max + tok) * (int64_t)a.dim;
          if (a.pair) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              const int x = xs[2 * h];
              if (x < a.dim) {
                float v0, v1;
                if constexpr (T::bytes == 4) {
                  v0 = qrow[x];
                  v1 = qrow[x + 1];
                } else {
                  const uint32_t w = *reinterpret_cast<const uint32_t*>(qrow + x);
                  v0 = elem_f32<T>(reinterpret_cast<const S*>(&w), 0);
                  v1 = elem_f32<T>(reinterpret_cast<const S*>(&w), 1);
                }
                acc[2 * h] = fmaf(g, v0, acc[2 * h]);
                acc[2 * h + 1] = fmaf(g, v1, acc[2 * h + 1]);
              }
            }
          } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (xs[i] < a.dim) acc[i] = fmaf(g, elem_f32<T>(qrow, xs[i]), acc[i]);
          }
        }
      }
    }
    uint16_t* row = base + (int64_t)r * a.dim;
    if (a.pair) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int x = xs[2 * h];
        if (x < a.dim)
          *reinterpret_cast<uint32_t*>(row + x) =
              pack_out16<O>(acc[2 * h], acc[2 * h + 1]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (xs[i] < a.dim) row[xs[i]] = to_out16<O>(acc[i]);
    }
  }
  }
}

// a.vec_rows (either output type): each lane owns 8 elements of one row, so
// a wave covers 64 / (dim / 8) rows per step and writes each row once (16
// bytes per lane for 16-bit O, 32 for fp32), zeros included.  For each token
// landing in the step's rows (in token order) only the lanes of its row add
// it, so every element sees the fmaf sequence of the scalar fp32 path below.
template <typename T, typename O>
__device__ __forceinline__ void dd_padded_rows_vec(const PaddedDdArgs& a, int64_t p, int64_t b,
                                                   int r0, int r1, int lane, int32_t* am_lds) {
  using S = typename T::storage;
  const int64_t base = p * a.ld_max * (int64_t)a.dim;
  const int lqb = a.qlen[b];
  const int ld = a.dlen[p];
  const bool ok = lqb >= 1 && lqb <= a.lq_max && ld >= 1 && ld <= a.ld_max;
  const float g = a.dscore[p];
  const S* __restrict__ Q = static_cast<const S*>(a.q);
  const int32_t* am = a.argmax + p * a.lq_max;
  int amv[kDdAmRegs];
#pragma unroll
  for (int c = 0; c < kDdAmRegs; ++c) {
    const int t = 64 * c + lane;
    amv[c] = ok && t < lqb ? am[t] : -1;
  }
  if (a.am_lds) {
    if (ok)
      for (int t = 64 * kDdAmRegs + lane; t < lqb; t += 64) am_lds[t - 64 * kDdAmRegs] = am[t];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  const int L = a.dim >> 3;  // lanes per row
  const int rpi = 64 / L;    // rows per step
  const int sub = lane / L;
  const int e0 = (lane - sub * L) * 8;
  const int rmax = min(r1, ld);  // rows that can receive tokens
  for (int rb = r0; rb < r1; rb += rpi) {
    const int r = rb + sub;
    float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    if (ok && rb < rmax) {
      const int rhi = min(rb + rpi, rmax);
      for (int c0 = 0; c0 < lqb; c0 += 64) {
        const int t = c0 + lane;
        int j = -1;
        if (c0 < 64 * kDdAmRegs) {
#pragma unroll
          for (int c = 0; c < kDdAmRegs; ++c)
            if (c0 == 64 * c) j = amv[c];
        } else if (t < lqb) {
          j = a.am_lds ? am_lds[t - 64 * kDdAmRegs] : am[t];
        }
        uint64_t hits = __ballot(j >= rb && j < rhi);
        while (hits) {
          const int tl = __builtin_ctzll(hits);
          hits &= hits - 1;
          const int jt = __builtin_amdgcn_readlane(j, tl);
          if (r == jt) {
            const S* src = Q + (b * a.lq_max + c0 + tl) * (int64_t)a.dim + e0;
            float qv[8];
            if constexpr (T::bytes == 4) {
              const float4 w0 = reinterpret_cast<const float4*>(src)[0];
              const float4 w1 = reinterpret_cast<const float4*>(src)[1];
              qv[0] = w0.x; qv[1] = w0.y; qv[2] = w0.z; qv[3] = w0.w;
              qv[4] = w1.x; qv[5] = w1.y; qv[6] = w1.z; qv[7] = w1.w;
            } else {
              const uint4 w = *reinterpret_cast<const uint4*>(src);
              const S* v = reinterpret_cast<const S*>(&w);
#pragma unroll
              for (int e = 0; e < 8; ++e) qv[e] = elem_f32<T>(v, e);
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[e] = fmaf(g, qv[e], acc[e]);
          }
        }
      }
    }
    if (r < r1) {
      const int64_t at = base + (int64_t)r * a.dim + e0;
      if constexpr (O::bytes == 4) {
        float4* dst = reinterpret_cast<float4*>(static_cast<float*>(a.dd) + at);
        dst[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
        dst[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
      } else {
        uint4 o;
        o.x = pack_out16<O>(acc[0], acc[1]);
        o.y = pack_out16<O>(acc[2], acc[3]);
        o.z = pack_out16<O>(acc[4], acc[5]);
        o.w = pack_out16<O>(acc[6], acc[7]);
        *reinterpret_cast<uint4*>(static_cast<uint16_t*>(a.dd) + at) = o;
      }
    }
  }
}

template <typename T, typename O>
__global__ __launch_bounds__(256) void dd_padded_kernel(PaddedDdArgs a) {
  using S = typename T::storage;
  const int lane = threadIdx.x & 63;
  const int64_t w = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t p = w / a.nsplit;
  if (p >= a.npairs) return;
  const int64_t b = p / a.ncand;
  // this wave's rows of candidate p
  const int r0 = (int)(w - p * a.nsplit) * a.rows_per_split;
  const int r1 = min(a.ld_max, r0 + a.rows_per_split);
  if (r0 >= r1) return;
  extern __shared__ int32_t dd_am_lds[];
  int32_t* am_lds = dd_am_lds + (threadIdx.x >> 6) * a.am_lds;
  if (a.vec_rows) {
    dd_padded_rows_vec<T, O>(a, p, b, r0, r1, lane, am_lds);
    return;
  }
  if constexpr (O::bytes != 4) {
    dd_padded_rows16<T, O>(a, p, b, r0, r1, lane, am_lds);
    return;
  }
  float* base = static_cast<float*>(a.dd) + p * a.ld_max * (int64_t)a.dim;
  // zeroed with the lane mapping of the adds below, so each element's zero and
  // its adds come from one lane in program order
  for (int r = r0; r < r1; ++r)
    for (int x = lane; x < a.dim; x += 64) base[(int64_t)r * a.dim + x] = 0.0f;
  const int lqb = a.qlen[b];
  const int ld = a.dlen[p];
  if (lqb < 1 || lqb > a.lq_max || ld < 1 || ld > a.ld_max) return;
  const float g = a.dscore[p];
  const S* __restrict__ Q = static_cast<const S*>(a.q);
  // argmax 64 tokens at a time, one per lane; the tokens that land in this
  // wave's rows are then added in token order
  for (int c0 = 0; c0 < lqb; c0 += 64) {
    const int jl = c0 + lane < lqb ? a.argmax[p * a.lq_max + c0 + lane] : -1;
    uint64_t hits = __ballot(jl >= r0 && jl < r1 && jl < ld);
    while (hits) {
      const int t = __builtin_ctzll(hits);
      hits &= hits - 1;
      const int j = __builtin_amdgcn_readlane(jl, t);
      const S* qrow = Q + (b * a.lq_max + c0 + t) * (int64_t)a.dim;
      float* drow = base + (int64_t)j * a.dim;
      for (int x = lane; x < a.dim; x += 64) drow[x] = fmaf(g, elem_f32<T>(qrow, x), drow[x]);
    }
  }
}

// ---------------------------------------------------------------------------
// Packed: zero-filled outputs + fp32 global atomics.  Wave per pair; lanes
// split as (token group, 8-element slice).
// ---------------------------------------------------------------------------
struct PackedBwdArgs {
  const float* dscore;
  const void* q;
  const void* d;
  const int32_t* qoff;
  const int32_t* doff;
  const int32_t* qids;
  const int32_t* dids;
  const int32_t* argmax;
  void* dq;  // fp32, or the 16-bit output type of the grouped kernels
  void* dd;
  int64_t nq;
  int64_t nd;
  int64_t total_q;
  int64_t total_d;
  int64_t npairs;
  int slots;
  int dim;
  int nslices;
  int lanes_per_tok;
};

template <typename T>
__global__ __launch_bounds__(256) void packed_bwd_kernel(PackedBwdArgs a,
                                                         bool vec) {
  using S = typename T::storage;
  const int lane = threadIdx.x & 63;
  const int64_t p = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (p >= a.npairs) return;
  const int64_t qi = a.qids[p], di = a.dids[p];
  if (qi < 0 || qi >= a.nq || di < 0 || di >= a.nd) return;
  const int64_t qs = a.qoff[qi], qe = a.qoff[qi + 1];
  const int64_t ds = a.doff[di], de = a.doff[di + 1];
  if (qs < 0 || qe <= qs || qe > a.total_q || qe - qs > a.slots) return;
  if (ds < 0 || de <= ds || de > a.total_d) return;
  const int lq = (int)(qe - qs);
  const int ld = (int)(de - ds);
  const float g = a.dscore[p];
  const S* __restrict__ Q = static_cast<const S*>(a.q);
  const S* __restrict__ D = static_cast<const S*>(a.d);
  const int lpt = a.lanes_per_tok;
  const int tg = lane / lpt;
  const int tl = lane - tg * lpt;
  const int ntg = 64 / lpt;
  for (int i = tg; i < lq; i += ntg) {
    const int j = a.argmax[p * a.slots + i];
    if (j < 0 || j >= ld) continue;
    for (int sl = tl; sl < a.nslices; sl += lpt) {
      float qv[8], dv[8];
      load8f<T>(Q + (qs + i) * (int64_t)a.dim, sl * 8, a.dim, vec, qv);
      load8f<T>(D + (ds + j) * (int64_t)a.dim, sl * 8, a.dim, vec, dv);
      float* dqr = static_cast<float*>(a.dq) + (qs + i) * (int64_t)a.dim + sl * 8;
      float* ddr = static_cast<float*>(a.dd) + (ds + j) * (int64_t)a.dim + sl * 8;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        if (sl * 8 + u < a.dim) {
          atomicAdd(dqr + u, g * dv[u]);
          atomicAdd(ddr + u, g * qv[u]);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Packed, owner-computes (used when the caller provides a workspace).
//
// The pairs are grouped by query and by document on the device with a
// counting sort (count, scan, scatter of pair ids; integer atomics only).
// One workgroup per query then gathers its dq rows over the query's pairs,
// and one workgroup per document accumulates its dd rows in LDS, a chunk of
// rows at a time, and writes every row once: no zero-fill pass and no
// floating-point atomics in global memory.  Rows of the outputs that lie in
// no valid query / document segment are not written.
//
// Workspace (int32): qstart[nq + 1] qcur[nq] dstart[nd + 1] dcur[nd]
//                    qlist[P] dlist[P]
// ---------------------------------------------------------------------------
struct PackedGroups {
  int32_t* qstart;
  int32_t* qcur;
  int32_t* dstart;
  int32_t* dcur;
  int32_t* qlist;
  int32_t* dlist;
};

// Pair p is routed only if its ids and both segments are valid (the rule of
// packed_bwd_kernel).
__device__ __forceinline__ bool packed_pair_ok(const PackedBwdArgs& a, int64_t p, int64_t& qi,
                                               int64_t& di) {
  qi = a.qids[p];
  di = a.dids[p];
  if (qi < 0 || qi >= a.nq || di < 0 || di >= a.nd) return false;
  const int64_t qs = a.qoff[qi], qe = a.qoff[qi + 1];
  const int64_t ds = a.doff[di], de = a.doff[di + 1];
  if (qs < 0 || qe <= qs || qe > a.total_q || qe - qs > a.slots) return false;
  if (ds < 0 || de <= ds || de > a.total_d) return false;
  return true;
}

__global__ __launch_bounds__(256) void pair_count_kernel(PackedBwdArgs a, PackedGroups g) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; p < a.npairs; p += stride) {
    int64_t qi, di;
    if (!packed_pair_ok(a, p, qi, di)) continue;
    atomicAdd(&g.qstart[qi + 1], 1);
    atomicAdd(&g.dstart[di + 1], 1);
  }
}

// Workgroup 0 turns qstart[0..nq] (qstart[0] = 0, qstart[x + 1] = count of
// group x) into group starts by an inclusive scan, workgroup 1 does dstart;
// the cursors start at the group starts.
constexpr int kScanThreads = 1024;
constexpr int kScanPer = 16;  // values per thread held in registers (16,384 groups)
__global__ __launch_bounds__(kScanThreads) void group_scan_kernel(PackedGroups g, int64_t nq,
                                                                  int64_t nd) {
  __shared__ int wave_tot[kScanThreads / 64];
  int32_t* v = blockIdx.x == 0 ? g.qstart : g.dstart;
  int32_t* cur = blockIdx.x == 0 ? g.qcur : g.dcur;
  const int64_t n = (blockIdx.x == 0 ? nq : nd) + 1;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t per = (n + kScanThreads - 1) / kScanThreads;
  const int64_t lo = min((int64_t)tid * per, n), hi = min(lo + per, n);
  // a run of at most kScanPer values is loaded once, all loads in flight
  // together (a loop of dependent round trips took most of the kernel)
  int vals[kScanPer];
  const bool short_run = per <= kScanPer;
  int run = 0;
  if (short_run) {
#pragma unroll
    for (int e = 0; e < kScanPer; ++e) vals[e] = lo + e < hi ? v[lo + e] : 0;
#pragma unroll
    for (int e = 0; e < kScanPer; ++e) run += vals[e];
  } else {
    for (int64_t x = lo; x < hi; ++x) run += v[x];
  }
  int incl = run;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int t = __shfl_up(incl, off);
    if (lane >= off) incl += t;
  }
  if (lane == 63) wave_tot[wave] = incl;
  __syncthreads();
  if (wave == 0) {
    int w = lane < kScanThreads / 64 ? wave_tot[lane] : 0;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int t = __shfl_up(w, off);
      if (lane >= off) w += t;
    }
    if (lane < kScanThreads / 64) wave_tot[lane] = w;  // inclusive over waves
  }
  __syncthreads();
  int acc = incl - run + (wave > 0 ? wave_tot[wave - 1] : 0);
  if (short_run) {
#pragma unroll
    for (int e = 0; e < kScanPer; ++e) {
      const int64_t x = lo + e;
      if (x < hi) {
        acc += vals[e];
        v[x] = acc;
        if (x < n - 1) cur[x] = acc;
      }
    }
  } else {
    for (int64_t x = lo; x < hi; ++x) {
      acc += v[x];
      v[x] = acc;
      if (x < n - 1) cur[x] = acc;
    }
  }
}

__global__ __launch_bounds__(256) void pair_scatter_kernel(PackedBwdArgs a, PackedGroups g) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; p < a.npairs; p += stride) {
    int64_t qi, di;
    if (!packed_pair_ok(a, p, qi, di)) continue;
    g.qlist[atomicAdd(&g.qcur[qi], 1)] = (int32_t)p;
    g.dlist[atomicAdd(&g.dcur[di], 1)] = (int32_t)p;
  }
}

constexpr int kGroupThreads = 256;
constexpr int kPairStage = 256;  // pairs staged in LDS at a time

// Before the grouped packed backward, one launch: zero the grouping's
// counters (groups[0..n_groups)) and the rows of dq and dd before the first
// and after the last segment, which no per-segment workgroup owns (element
// type E: float, or 16-bit).  Against a fill and two zero_outside_kernel
// launches, two launches fewer.
template <typename E>
__global__ __launch_bounds__(256) void packed_init_kernel(int32_t* groups, int64_t n_groups,
                                                          E* dq, const int32_t* qoff, int64_t nq,
                                                          int64_t total_q, E* dd,
                                                          const int32_t* doff, int64_t nd,
                                                          int64_t total_d, int dim) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t t0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (int64_t x = t0; x < n_groups; x += stride) groups[x] = 0;
  auto outside = [&](E* out, const int32_t* off, int64_t nseg, int64_t total) {
    if (total <= 0) return;
    const int64_t head = min(max((int64_t)off[0], (int64_t)0), total);
    const int64_t tail = min(max((int64_t)off[nseg], head), total);
    const int64_t n_head = head * dim, n_tail = (total - tail) * dim;
    for (int64_t x = t0; x < n_head + n_tail; x += stride)
      out[x < n_head ? x : tail * dim + (x - n_head)] = E(0);
  };
  outside(dq, qoff, nq, total_q);
  outside(dd, doff, nd, total_d);
}

// dq: workgroup = (query qi, block of its tokens); thread = (token row,
// 8-element slice).
template <typename T, bool VEC, typename O>
__global__ __launch_bounds__(kGroupThreads) void dq_packed_kernel(PackedBwdArgs a,
                                                                  PackedGroups g) {
  using S = typename T::storage;
  __shared__ int64_t st_ds[kPairStage];
  __shared__ int32_t st_ld[kPairStage];
  __shared__ int32_t st_p[kPairStage];
  __shared__ float st_g[kPairStage];
  const int64_t qi = blockIdx.x;
  const int64_t qs = a.qoff[qi], qe = a.qoff[qi + 1];
  if (qs < 0 || qe <= qs || qe > a.total_q) return;
  const int lq = (int)(qe - qs);
  const int tid = threadIdx.x;
  // a row of more than kGroupThreads slices (dims above 2048) is covered in
  // rounds of kGroupThreads slices, one row per workgroup
  const int ns = min(a.nslices, kGroupThreads);
  const int rows_per_pass = kGroupThreads / ns;
  // token block of this workgroup (grid.y covers max_q_len)
  const int i0 = blockIdx.y * rows_per_pass;
  if (i0 >= lq) return;
  const int local = tid / ns;
  const int k_lo = g.qstart[qi], k_hi = g.qstart[qi + 1];
  const bool seg_ok = lq <= a.slots;
  const S* __restrict__ D = static_cast<const S*>(a.d);
  for (int sl = tid - local * ns; sl - (tid - local * ns) < a.nslices; sl += ns) {
    const bool active = local < rows_per_pass && sl < a.nslices;
    const int k0 = sl * 8;
    const int i = i0 + local;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int c0 = k_lo; seg_ok && c0 < k_hi; c0 += kPairStage) {
      const int nc = min(kPairStage, k_hi - c0);
      __syncthreads();
      if (tid < nc) {
        const int p = g.qlist[c0 + tid];
        const int64_t di = a.dids[p];
        const int64_t ds = a.doff[di];
        st_ds[tid] = ds;
        st_ld[tid] = (int)(a.doff[di + 1] - ds);
        st_p[tid] = p;
        st_g[tid] = a.dscore[p];
      }
      __syncthreads();
      if (!active || i >= lq) continue;
      constexpr int U = 4;
      for (int k = 0; k < nc; k += U) {
        const S* src[U];
        float w[U];
        bool ok[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int kk = min(k + u, nc - 1);
          const int j = a.argmax[(int64_t)st_p[kk] * a.slots + i];
          ok[u] = (k + u < nc) && j >= 0 && j < st_ld[kk];
          src[u] = D + (st_ds[kk] + (ok[u] ? j : 0)) * (int64_t)a.dim;
          w[u] = st_g[kk];
        }
        Frag<T> v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = load_frag<T>(src[u], k0, a.dim, VEC);
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float t = fmaf(w[u], frag_elem(v[u], e), acc[e]);
            acc[e] = ok[u] ? t : acc[e];
          }
      }
    }
    if (active && i < lq) store8<O>(out_at<O>(a.dq, (qs + i) * (int64_t)a.dim), k0, a.dim, VEC, acc);
  }
}

// dd: workgroup = document di.  The document's entries -- (pair k of its
// group, token i < Lq of that pair's query), target row argmax[p_k, i] -- are
// bucketed by target row in LDS (histogram, scan, scatter: a counting sort);
// then groups of G lanes each own one row at a time, sum g_k * q_row over the
// row's bucket in fp32 registers (blocked sums, as in the contrastive dd) and
// write the row once, zeros for rows no entry points at.  Entries are taken
// in stages of nc pairs x tc tokens (nc * tc <= kPkEntries), documents longer
// than kPkRows rows in row passes; later stages add to the rows written.
// With a 16-bit output type O, documents that need more than one stage are
// left to dd_packed_multi_kernel (a 16-bit row cannot hold the partial sum a
// later stage would add to), so every row written here is written once.
constexpr int kPkRows = 1024;     // rows bucketed per pass
constexpr int kPkEntries = 2048;  // entries per stage (bucket ids held in LDS)

// True when a document with n_pairs pairs needs more than one stage of
// entries in dd_packed_kernel.
__device__ __forceinline__ bool dd_packed_multi_stage(const PackedBwdArgs& a, int n_pairs) {
  const int tc = min(a.slots, kPkEntries);
  return a.slots > tc || n_pairs > min(kPairStage, kPkEntries / tc);
}

// Waves per SIMD the register allocation leaves room for.  With 16-bit rows
// (half the write bytes) the kernel waits on each workgroup's chain of
// dependent loads, and five workgroups per CU (96 VGPRs, a few spills in the
// batch-of-8 path) beat four at 106 VGPRs: C4 typed backward 179.6 -> 170.3
// us.  fp32 rows are bound by their writes, and the same bound cost 10 us
// there (294.5 -> 304.6 us), so they keep the compiler's allocation, as do
// unaligned rows (element loads: 148 VGPRs, whose cap would spill 47).
template <bool VEC, int NS, typename O>
constexpr int kPkMinWaves = (VEC && NS == 1 && O::bytes == 2) ? 5 : 1;

template <typename T, bool VEC, int NS, typename O>
__global__ __launch_bounds__(kGroupThreads, (kPkMinWaves<VEC, NS, O>)) void dd_packed_kernel(
    PackedBwdArgs a, PackedGroups g, int G) {
  using S = typename T::storage;
  __shared__ int start[kPkRows + 1];
  __shared__ int cursor[kPkRows + 1];
  __shared__ int ids[kPkEntries];
  __shared__ int64_t st_qs[kPairStage];
  __shared__ int32_t st_lq[kPairStage];
  __shared__ int32_t st_p[kPairStage];
  __shared__ float st_g[kPairStage];
  __shared__ int n_full;  // rows with entries in this stage
  const int64_t di = blockIdx.x;
  const int64_t ds = a.doff[di], de = a.doff[di + 1];
  if (ds < 0 || de <= ds || de > a.total_d) return;
  const int ld = (int)(de - ds);
  const int tid = threadIdx.x, lane = tid & 63;
  const int grp = tid / G, gl = tid - grp * G;
  const int ngroups = kGroupThreads / G;
  const int k_lo = g.dstart[di], k_hi = g.dstart[di + 1];
  if constexpr (O::bytes != 4) {
    if (dd_packed_multi_stage(a, k_hi - k_lo)) return;
  }
  const int dim = a.dim;
  const int tc = min(a.slots, kPkEntries);               // tokens per stage
  const int stage_pairs = min(kPairStage, kPkEntries / tc);
  const float inv_tc = 1.0f / (float)tc;
  const S* __restrict__ Q = static_cast<const S*>(a.q);
  const int sl_hi = a.nslices;

  for (int r0 = 0; r0 < ld; r0 += kPkRows) {
    const int nrows = min(kPkRows, ld - r0);
    // at least one stage, so documents without pairs still write zero rows
    int c0 = k_lo;
    do {
      const int nc = min(stage_pairs, k_hi - c0);
      __syncthreads();
      if (tid < nc) {
        const int p = g.dlist[c0 + tid];
        const int64_t qi = a.qids[p];
        const int64_t qs = a.qoff[qi];
        st_qs[tid] = qs;
        st_lq[tid] = (int)(a.qoff[qi + 1] - qs);
        st_p[tid] = p;
        st_g[tid] = a.dscore[p];
      }
      for (int t0 = 0; t0 == 0 || t0 < a.slots; t0 += tc) {
        const bool first = (c0 == k_lo && t0 == 0);
        const int ne = nc * tc;
        __syncthreads();
        for (int x = tid; x <= nrows; x += kGroupThreads) start[x] = 0;
        if (tid == 0) n_full = 0;
        __syncthreads();
        // 1. histogram of target rows
        for (int e = tid; e < ne; e += kGroupThreads) {
          const int k = div_small(e, tc, inv_tc);
          const int i = t0 + e - k * tc;
          if (i >= st_lq[k]) continue;
          const int j = a.argmax[(int64_t)st_p[k] * a.slots + i] - r0;
          if (j >= 0 && j < nrows && j + r0 < ld) atomicAdd(&start[j + 1], 1);
        }
        __syncthreads();
        // 2. inclusive scan of start[1..nrows] by wave 0
        if (tid < 64) {
          const int per = (nrows + 63) / 64;
          const int lo = 1 + lane * per;
          const int hi = min(lo + per, nrows + 1);
          int run = 0;
          for (int x = lo; x < hi; ++x) run += start[x];
          int incl = run;
#pragma unroll
          for (int off = 1; off < 64; off <<= 1) {
            const int v = __shfl_up(incl, off);
            if (lane >= off) incl += v;
          }
          int acc = incl - run;
          for (int x = lo; x < hi; ++x) {
            acc += start[x];
            start[x] = acc;
          }
        }
        __syncthreads();
        for (int x = tid; x < nrows; x += kGroupThreads) cursor[x] = start[x];
        __syncthreads();
        // 3. scatter packed entry ids (e | k << 16) into their row buckets
        for (int e = tid; e < ne; e += kGroupThreads) {
          const int k = div_small(e, tc, inv_tc);
          const int i = t0 + e - k * tc;
          if (i >= st_lq[k]) continue;
          const int j = a.argmax[(int64_t)st_p[k] * a.slots + i] - r0;
          if (j >= 0 && j < nrows && j + r0 < ld) ids[atomicAdd(&cursor[j], 1)] = e | (k << 16);
        }
        __syncthreads();
        // 4. Rows with entries are listed in `cursor` (free after the
        // scatter); on the first stage the others are zeroed with coalesced
        // stores (later stages leave them as they are).  Most rows of a short
        // document have no entry, so the groups then walk only the listed
        // rows and wait on far fewer gathers.
        for (int rr = tid; rr < nrows; rr += kGroupThreads)
          if (start[rr + 1] > start[rr]) cursor[atomicAdd(&n_full, 1)] = rr;
        if (first) {
          if constexpr (VEC) {
            // 16-byte pieces, consecutive threads on consecutive pieces
            // (whole lines per wave store), non-temporal: nothing re-reads
            // them.  C4 backward 230.7 -> 190.2 us (bf16 gradients).
            const int upr = dim * O::bytes / 16;  // pieces per row
            const float inv_upr = 1.0f / (float)upr;
            for (int x = tid; x < nrows * upr; x += kGroupThreads) {
              const int rr = div_small(x, upr, inv_upr);
              if (start[rr + 1] == start[rr])
                store16_nt(out_at<O>(a.dd, (ds + r0 + rr) * (int64_t)dim + (x - rr * upr) * (16 / O::bytes)),
                           u32x4_t{0u, 0u, 0u, 0u});
            }
          } else {
            const float zero8[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            const float inv_sl = 1.0f / (float)sl_hi;
            for (int x = tid; x < nrows * sl_hi; x += kGroupThreads) {
              const int rr = div_small(x, sl_hi, inv_sl);
              if (start[rr + 1] == start[rr])
                store8<O>(out_at<O>(a.dd, (ds + r0 + rr) * (int64_t)dim), (x - rr * sl_hi) * 8,
                          dim, VEC, zero8);
            }
          }
        }
        __syncthreads();
        // per-row fp32 sums, one group of G lanes per listed row; a row wider
        // than NS * G slices (dims above 256) is summed in chunks
        const int n_rows_full = n_full;
        for (int i = grp; i < n_rows_full; i += ngroups)
        for (int sc = 0; sc < sl_hi; sc += NS * G) {
          const int rr = cursor[i];
          float acc[NS][8];
          void* dst = out_at<O>(a.dd, (ds + r0 + rr) * (int64_t)dim);
#pragma unroll
          for (int u = 0; u < NS; ++u) {
            const int sl = sc + gl + u * G;
            if (O::bytes == 4 && sl < sl_hi && !first) {  // never taken for 16-bit O
              load8f<F32>(static_cast<const float*>(dst), sl * 8, dim, VEC, acc[u]);
            } else {
#pragma unroll
              for (int x = 0; x < 8; ++x) acc[u][x] = 0.0f;
            }
          }
          const int s_end = start[rr + 1];
          for (int s0 = start[rr]; s0 < s_end; s0 += kDdBlock) {
            const int s1 = min(s0 + kDdBlock, s_end);
            float blk[NS][8];
#pragma unroll
            for (int u = 0; u < NS; ++u)
#pragma unroll
              for (int x = 0; x < 8; ++x) blk[u][x] = 0.0f;
            // KB entries from s; past the bucket's end (masked batches only)
            // an entry repeats entry s with its fragment and weight zeroed
            // (fmaf(0, 0, x) == x exactly).  Full batches of kDdBatch while
            // they last, then pairs: most rows of a sparse document hold one
            // or two entries.
            auto batch = [&](int s, auto masked, auto kb) {
              constexpr bool MASKED = decltype(masked)::value;
              constexpr int KB = decltype(kb)::value;
              const S* row[KB];
              float gx[KB];
              bool ok[KB];
#pragma unroll
              for (int k = 0; k < KB; ++k) {
                ok[k] = !MASKED || s + k < s1;
                const uint32_t v = (uint32_t)ids[ok[k] ? s + k : s];
                const int kk = (int)(v >> 16);
                const int i = t0 + (int)(v & 0xffffu) - kk * tc;
                row[k] = Q + (st_qs[kk] + i) * (int64_t)dim;
                gx[k] = ok[k] ? st_g[kk] : 0.0f;
              }
#pragma unroll
              for (int u = 0; u < NS; ++u) {
                const int sl = sc + gl + u * G;
                if (sl < sl_hi) {
                  Frag<T> v[KB];
#pragma unroll
                  for (int k = 0; k < KB; ++k) {
                    v[k] = load_frag<T>(row[k], sl * 8, dim, VEC);
                    if (MASKED && !ok[k]) v[k] = zero_frag<T>();
                  }
#pragma unroll
                  for (int k = 0; k < KB; ++k)
#pragma unroll
                    for (int x = 0; x < 8; ++x)
                      blk[u][x] = fmaf(gx[k], frag_elem(v[k], x), blk[u][x]);
                }
              }
            };
            int s = s0;
            for (; s + kDdBatch <= s1; s += kDdBatch)
              batch(s, std::false_type{}, std::integral_constant<int, kDdBatch>{});
            for (; s < s1; s += 2) batch(s, std::true_type{}, std::integral_constant<int, 2>{});
#pragma unroll
            for (int u = 0; u < NS; ++u)
#pragma unroll
              for (int x = 0; x < 8; ++x) acc[u][x] += blk[u][x];
          }
#pragma unroll
          for (int u = 0; u < NS; ++u) {
            const int sl = sc + gl + u * G;
            if (sl < sl_hi) {
              if constexpr (VEC)
                store8_nt<O>(dst, sl * 8, acc[u]);
              else
                store8<O>(dst, sl * 8, dim, VEC, acc[u]);
            }
          }
        }
      }
      c0 += nc;
    } while (c0 < k_hi);
  }
}

// dd with a 16-bit output type O for the documents dd_packed_kernel leaves
// (those needing more than one stage of entries).  Workgroups stride over
// blocks of 256 documents, list the block's documents that need this kernel
// (one thread per document), and process the listed ones.  Rows are taken
// kPkAccFloats / dim at a time with their fp32 sums in LDS; a wave adds one
// entry g_k * q_row at a time (lanes over the embedding dimension, LDS
// atomics), over every stage of the document's pairs, then each row is
// rounded to O and written once.  The order of the LDS additions varies, so
// these rows can differ between runs in the last bits.
constexpr int kPkAccFloats = 16384;  // 64 KiB of row sums

template <typename T, typename O>
__global__ __launch_bounds__(kGroupThreads) void dd_packed_multi_kernel(PackedBwdArgs a,
                                                                        PackedGroups g) {
  using S = typename T::storage;
  __shared__ float acc[kPkAccFloats];
  __shared__ int64_t st_qs[kPairStage];
  __shared__ int32_t st_lq[kPairStage];
  __shared__ int32_t st_p[kPairStage];
  __shared__ float st_g[kPairStage];
  __shared__ int listed[kGroupThreads];
  __shared__ int n_listed;
  const int dim = a.dim;
  const int slots = a.slots;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  constexpr int kWaves = kGroupThreads / 64;
  const int rows_per_pass = kPkAccFloats / dim;  // >= 64 for dim <= 256
  const S* __restrict__ Q = static_cast<const S*>(a.q);
  uint16_t* __restrict__ out = static_cast<uint16_t*>(a.dd);
  for (int64_t b0 = (int64_t)blockIdx.x * kGroupThreads; b0 < a.nd;
       b0 += (int64_t)gridDim.x * kGroupThreads) {
    __syncthreads();  // the previous block's list and sums are no longer read
    if (tid == 0) n_listed = 0;
    __syncthreads();
    if (b0 + tid < a.nd) {
      const int64_t di = b0 + tid;
      const int64_t ds = a.doff[di], de = a.doff[di + 1];
      if (ds >= 0 && de > ds && de <= a.total_d &&
          dd_packed_multi_stage(a, g.dstart[di + 1] - g.dstart[di]))
        listed[atomicAdd(&n_listed, 1)] = tid;
    }
    __syncthreads();
    const int n_docs = n_listed;
    // di, and so every branch on it, is uniform over the workgroup
    for (int li = 0; li < n_docs; ++li) {
      const int64_t di = b0 + listed[li];
      const int64_t ds = a.doff[di], de = a.doff[di + 1];
      const int k_lo = g.dstart[di], k_hi = g.dstart[di + 1];
      const int ld = (int)(de - ds);
      for (int r0 = 0; r0 < ld; r0 += rows_per_pass) {
        const int nrows = min(rows_per_pass, ld - r0);
        const int n_el = nrows * dim;
        __syncthreads();  // the previous pass has read its sums
        for (int x = tid; x < n_el; x += kGroupThreads) acc[x] = 0.0f;
        for (int c0 = k_lo; c0 < k_hi; c0 += kPairStage) {
          const int nc = min(kPairStage, k_hi - c0);
          __syncthreads();  // sums zeroed; the previous stage's pairs are no longer read
          if (tid < nc) {
            const int p = g.dlist[c0 + tid];
            const int64_t qi = a.qids[p];
            const int64_t qs = a.qoff[qi];
            st_qs[tid] = qs;
            st_lq[tid] = (int)(a.qoff[qi + 1] - qs);
            st_p[tid] = p;
            st_g[tid] = a.dscore[p];
          }
          __syncthreads();
          // entry e = (pair k, token i); one wave per entry, uniform branches
          const int64_t ne = (int64_t)nc * slots;
          for (int64_t e = wave; e < ne; e += kWaves) {
            const int k = (int)(e / slots);
            const int i = (int)(e - (int64_t)k * slots);
            if (i >= st_lq[k]) continue;
            const int jt = a.argmax[(int64_t)st_p[k] * slots + i];
            if (jt < r0 || jt >= r0 + nrows) continue;
            const int j = jt - r0;
            const S* qrow = Q + (st_qs[k] + i) * (int64_t)dim;
            const float gk = st_g[k];
            for (int x = lane; x < dim; x += 64) {
              float v;
              if constexpr (__is_same(T, BF16))
                v = __uint_as_float((uint32_t)qrow[x] << 16);
              else if constexpr (__is_same(T, F16))
                v = (float)__builtin_bit_cast(_Float16, qrow[x]);
              else
                v = qrow[x];
              atomicAdd(&acc[j * dim + x], gk * v);
            }
          }
        }
        __syncthreads();
        uint16_t* dst = out + (ds + r0) * (int64_t)dim;
        for (int x = tid; x < n_el; x += kGroupThreads) dst[x] = to_out16<O>(acc[x]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Host dispatch
// ---------------------------------------------------------------------------
static bool aligned16b(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

static int pow2_at_least(int x) {
  int p = 1;
  while (p < x) p <<= 1;
  return p;
}

template <typename E>
static void launch_fill(E* p, int64_t n, hipStream_t st) {
  if (n <= 0) return;
  int64_t blocks = (n / (16 / (int64_t)sizeof(E)) + 255) / 256;
  if (blocks < 1) blocks = 1;
  if (blocks > 65535) blocks = 65535;
  hipLaunchKernelGGL(fill_zero_kernel<E>, dim3((unsigned)blocks), dim3(256), 0, st,
                     p, n, aligned16b(p));
}

// n zero gradient elements of 4 (fp32) or 2 (16-bit) bytes
static void launch_fill_grad(void* p, int64_t n, bool out16, hipStream_t st) {
  if (out16)
    launch_fill(static_cast<uint16_t*>(p), n, st);
  else
    launch_fill(static_cast<float*>(p), n, st);
}

// out16: gradients in the input's 16-bit type T instead of fp32.
template <typename T>
static void launch_dq(const DqArgs& a, bool vec, bool out16, hipStream_t st) {
  const int64_t threads = a.rows * a.nslices * a.csplit;
  const dim3 grid((unsigned)((threads + 255) / 256));
  if (out16)
    hipLaunchKernelGGL((dq_gather_kernel<T, T>), grid, dim3(256), 0, st, a, vec);
  else
    hipLaunchKernelGGL((dq_gather_kernel<T, F32>), grid, dim3(256), 0, st, a, vec);
}

// Rows per workgroup of dq_walk_kernel: a power of two, at most
// kWalkMaxRows, with rows x slices <= 256 threads.
static int walk_rows(int nslices) {
  int r = kWalkMaxRows;
  while (r > 1 && r * nslices > 256) r >>= 1;
  return r;
}

template <typename T>
static void launch_dq_walk(const DqArgs& a, bool vec, bool off32, bool out16, hipStream_t st) {
  const int R = walk_rows(a.nslices);
  const dim3 grid((unsigned)((a.rows + R - 1) / R));
  auto go = [&](auto kern) { hipLaunchKernelGGL(kern, grid, dim3(256), 0, st, a, R); };
  if (out16) {
    if (vec && off32) go(dq_walk_kernel<T, true, true, T>);
    else if (vec) go(dq_walk_kernel<T, true, false, T>);
    else if (off32) go(dq_walk_kernel<T, false, true, T>);
    else go(dq_walk_kernel<T, false, false, T>);
  } else {
    if (vec && off32) go(dq_walk_kernel<T, true, true, F32>);
    else if (vec) go(dq_walk_kernel<T, true, false, F32>);
    else if (off32) go(dq_walk_kernel<T, false, true, F32>);
    else go(dq_walk_kernel<T, false, false, F32>);
  }
}

// dq_range_kernel covers vec rows of 2^k slices (dims 8..256), Lq % 8 == 0
// and D below 2 GiB (32-bit byte offsets); returns false otherwise.
template <typename T>
static bool launch_dq_range(const DqArgs& a, float* ws, bool vec, bool off32, bool vec_reduce,
                            bool out16, bool reduce, hipStream_t st) {
  // fp32 fragments do not fit four waves per SIMD: dq_split_kernel takes fp32
  if constexpr (T::bytes == 4) {
    return false;
  } else {
  // 32-bit byte offsets for D (off32) and for argmax (the staging copies)
  const int ns = a.nslices;
  if (!vec || !off32 || a.lq % kRangeItems != 0 || ns > 32 || (ns & (ns - 1)) != 0 ||
      a.rows * a.nb * (int64_t)sizeof(int32_t) >= ((int64_t)1 << 31))
    return false;
  const int rpw = (64 / a.nslices) * kRangeItems;
  const int64_t wgs = (a.rows + 4 * rpw - 1) / (4 * rpw);
  // Below two workgroups per CU (8192 query rows at dim 128) each workgroup
  // walks its range with one wave per SIMD and waits on every gather:
  // dq_split_kernel's smaller workgroups fill the chip instead (same bits).
  // 64 x 512 documents (one GPU's shard of C5 over 8): 46 -> 21 us; 128
  // queries: 112 -> 102 us for the whole backward.
  if (wgs * kXcds < 2 * (int64_t)device_cus()) return false;
  const dim3 grid((unsigned)(wgs * kXcds));
  switch (a.nslices) {
    case 1: hipLaunchKernelGGL((dq_range_kernel<T, 1>), grid, dim3(256), 0, st, a, ws); break;
    case 2: hipLaunchKernelGGL((dq_range_kernel<T, 2>), grid, dim3(256), 0, st, a, ws); break;
    case 4: hipLaunchKernelGGL((dq_range_kernel<T, 4>), grid, dim3(256), 0, st, a, ws); break;
    case 8: hipLaunchKernelGGL((dq_range_kernel<T, 8>), grid, dim3(256), 0, st, a, ws); break;
    case 16: hipLaunchKernelGGL((dq_range_kernel<T, 16>), grid, dim3(256), 0, st, a, ws); break;
    case 32: hipLaunchKernelGGL((dq_range_kernel<T, 32>), grid, dim3(256), 0, st, a, ws); break;
    default: return false;
  }
  if (!reduce) return true;  // the dD launch adds the partial sums
  const int64_t n = a.rows * a.dim;
  const int64_t work = vec_reduce ? n / 4 : n;
  const dim3 rgrid((unsigned)std::max<int64_t>(std::min<int64_t>((work + 255) / 256, 4096), 1));
  if (out16)
    hipLaunchKernelGGL(dq_reduce_kernel<T>, rgrid, dim3(256), 0, st, ws, a.dq, n, vec_reduce);
  else
    hipLaunchKernelGGL(dq_reduce_kernel<F32>, rgrid, dim3(256), 0, st, ws, a.dq, n, vec_reduce);
  return true;
  }
}

template <typename T>
static void launch_dq_split(const DqArgs& a, bool vec, float* ws, bool vec_reduce, bool out16,
                            bool reduce, hipStream_t st) {
  const int rows_per_group = 256 / a.nslices;  // >= 8: dim <= 256
  const int64_t n_groups = (a.rows + rows_per_group - 1) / rows_per_group;
  hipLaunchKernelGGL((dq_split_kernel<T, kDqBatch>), dim3((unsigned)(n_groups * kXcds)),
                     dim3(256), 0, st, a, vec, ws, rows_per_group);
  if (!reduce) return;  // the dD launch adds the partial sums
  const int64_t n = a.rows * a.dim;
  const int64_t work = vec_reduce ? n / 4 : n;
  const dim3 grid((unsigned)std::max<int64_t>(std::min<int64_t>((work + 255) / 256, 4096), 1));
  if (out16)
    hipLaunchKernelGGL(dq_reduce_kernel<T>, grid, dim3(256), 0, st, ws, a.dq, n, vec_reduce);
  else
    hipLaunchKernelGGL(dq_reduce_kernel<F32>, grid, dim3(256), 0, st, ws, a.dq, n, vec_reduce);
}

// Largest dynamic LDS allocation one workgroup may use on the current
// device, queried once per device (64 KB if the query fails).
static size_t max_lds_per_block() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 64 * 1024;
  if (cached[dev] == 0) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess ||
        v <= 0)
      v = 64 * 1024;
    cached[dev] = v;
  }
  return (size_t)cached[dev];
}

template <typename T, bool VEC, int NS, typename O>
static int launch_dd_contrastive_v(const DdArgs& a, size_t lds, hipStream_t st) {
  const auto kern = dd_contrastive_kernel<T, VEC, NS, O>;
  if (lds > 64 * 1024) {
    // once per device and instantiation: allow up to the device's maximum
    static std::atomic<bool> raised[kMaxDevices];
    if (int e = raise_lds_limit((const void*)kern, max_lds_per_block(), "dd_contrastive_kernel",
                                raised))
      return e;
  }
  const int64_t per_part = kXcds / a.parts;
  const int64_t blocks = (a.nb + per_part - 1) / per_part * kXcds;
  hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(kDdThreads), lds, st, a);
  return MAXSIM_OK;
}

template <typename T, typename O>
static int launch_dd_bucket_o(const DdArgs& a, size_t lds, hipStream_t st) {
  const auto kern = dd_bucket_kernel<T, 1, O>;
  if (lds > 64 * 1024) {
    static std::atomic<bool> raised[kMaxDevices];
    if (int e = raise_lds_limit((const void*)kern, max_lds_per_block(), "dd_bucket_kernel",
                                raised))
      return e;
  }
  const int64_t per_part = kXcds / a.parts;
  const int64_t blocks = (a.nb + per_part - 1) / per_part * kXcds;
  hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(kDdThreads), lds, st, a);
  return MAXSIM_OK;
}

template <typename T>
static int launch_dd_bucket(const DdArgs& a, size_t lds, bool out16, hipStream_t st) {
  return out16 ? launch_dd_bucket_o<T, T>(a, lds, st) : launch_dd_bucket_o<T, F32>(a, lds, st);
}

template <typename T, typename O>
static int launch_dd_contrastive_o(const DdArgs& a, bool vec, size_t lds, hipStream_t st) {
  const bool two = a.part_slices > a.group;
  if (vec)
    return two ? launch_dd_contrastive_v<T, true, 2, O>(a, lds, st)
               : launch_dd_contrastive_v<T, true, 1, O>(a, lds, st);
  return two ? launch_dd_contrastive_v<T, false, 2, O>(a, lds, st)
             : launch_dd_contrastive_v<T, false, 1, O>(a, lds, st);
}

template <typename T>
static int launch_dd_contrastive(const DdArgs& a, bool vec, size_t lds, bool out16,
                                 hipStream_t st) {
  return out16 ? launch_dd_contrastive_o<T, T>(a, vec, lds, st)
               : launch_dd_contrastive_o<T, F32>(a, vec, lds, st);
}

template <typename T>
static void launch_dd_padded(const PaddedDdArgs& a, bool out16, hipStream_t st) {
  const dim3 grid((unsigned)((a.npairs * a.nsplit + 3) / 4));
  if constexpr (T::bytes == 2) {
    if (out16) {
      const size_t lds = (size_t)4 * a.am_lds * sizeof(int32_t);
      hipLaunchKernelGGL((dd_padded_kernel<T, T>), grid, dim3(256), lds, st, a);
      return;
    }
  }
  // the fp32 output takes the argmax LDS only on the vec_rows path
  const size_t lds = a.vec_rows ? (size_t)4 * a.am_lds * sizeof(int32_t) : 0;
  hipLaunchKernelGGL((dd_padded_kernel<T, F32>), grid, dim3(256), lds, st, a);
}

// O: output type of the gradients (F32, or T for 16-bit gradients).
template <typename T, typename O>
static void launch_packed_grouped_o(const PackedBwdArgs& a, const PackedGroups& g, bool vec,
                                    int G, hipStream_t st) {
  if (a.nq > 0) {
    const int rows_per_pass = kGroupThreads / std::min(a.nslices, kGroupThreads);
    const dim3 grid((unsigned)a.nq, (unsigned)((a.slots + rows_per_pass - 1) / rows_per_pass));
    if (vec)
      hipLaunchKernelGGL((dq_packed_kernel<T, true, O>), grid, dim3(kGroupThreads), 0, st, a, g);
    else
      hipLaunchKernelGGL((dq_packed_kernel<T, false, O>), grid, dim3(kGroupThreads), 0, st, a, g);
  }
  if (a.nd > 0) {
    const bool two = a.nslices > G;
    const dim3 grid((unsigned)a.nd);
    if (vec && two)
      hipLaunchKernelGGL((dd_packed_kernel<T, true, 2, O>), grid, dim3(kGroupThreads), 0, st, a,
                         g, G);
    else if (vec)
      hipLaunchKernelGGL((dd_packed_kernel<T, true, 1, O>), grid, dim3(kGroupThreads), 0, st, a,
                         g, G);
    else if (two)
      hipLaunchKernelGGL((dd_packed_kernel<T, false, 2, O>), grid, dim3(kGroupThreads), 0, st, a,
                         g, G);
    else
      hipLaunchKernelGGL((dd_packed_kernel<T, false, 1, O>), grid, dim3(kGroupThreads), 0, st, a,
                         g, G);
    if constexpr (O::bytes != 4) {
      const dim3 grid_m((unsigned)std::min<int64_t>((a.nd + kGroupThreads - 1) / kGroupThreads,
                                                    1024));
      hipLaunchKernelGGL((dd_packed_multi_kernel<T, O>), grid_m, dim3(kGroupThreads), 0, st, a,
                         g);
    }
  }
}

template <typename T>
static void launch_packed_grouped(const PackedBwdArgs& a, const PackedGroups& g, bool vec,
                                  int G, bool out16, hipStream_t st) {
  if constexpr (T::bytes == 2) {
    if (out16) {
      launch_packed_grouped_o<T, T>(a, g, vec, G, st);
      return;
    }
  }
  launch_packed_grouped_o<T, F32>(a, g, vec, G, st);
}

template <typename T>
static void launch_packed_bwd(const PackedBwdArgs& a, bool vec, hipStream_t st) {
  const dim3 grid((unsigned)((a.npairs + 3) / 4));
  hipLaunchKernelGGL(packed_bwd_kernel<T>, grid, dim3(256), 0, st, a, vec);
}

#define MAXSIM_DISPATCH(dtype, FN, ...)                        \
  do {                                                         \
    switch (dtype) {                                           \
      case MAXSIM_BFLOAT16: FN<BF16>(__VA_ARGS__); break;      \
      case MAXSIM_FLOAT16: FN<F16>(__VA_ARGS__); break;        \
      default: FN<F32>(__VA_ARGS__); break;                    \
    }                                                          \
  } while (0)

// Largest grid of 256-thread workgroups in one dimension (2^32 - 1 work-items).
constexpr int64_t kMaxBlocks256 = (int64_t)UINT32_MAX / 256;

static int element_bytes(maxsim_dtype dt) { return dt == MAXSIM_FLOAT32 ? 4 : 2; }

// Bytes of the packed backward's grouping workspace: int32 qstart[nq + 1],
// qcur[nq], dstart[nd + 1], dcur[nd], qlist[P], dlist[P].
static size_t packed_workspace_bytes(int64_t nq, int64_t nd, int64_t np) {
  if (nq < 0 || nd < 0 || np < 0) return 0;
  const int64_t ints = 2 * nq + 1 + 2 * nd + 1 + 2 * np;
  return (size_t)ints * sizeof(int32_t);
}

// ---------------------------------------------------------------------------
// Device scratch for maxsim_amd_packed_backward_typed_noalloc: the grouping
// workspace of the packed backward in a file-scope array, for callers that
// cannot allocate (graph capture, serving loops).  Each device holds its own
// copy for the life of the process.  In host code `scratch` names a host-side
// stand-in, never the device memory: the device address comes from
// hipGetSymbolAddress, looked up once per device with that device current,
// and only that address is passed to kernels.  Every call on a device shares
// that device's array, so calls that overlap on one device race; each call
// clears the parts that must start at zero (the group counters) itself.
// ---------------------------------------------------------------------------
constexpr size_t kScratchInts = (size_t)4 << 20;  // 16 MiB
constexpr size_t kScratchBytes = kScratchInts * sizeof(int32_t);
static __device__ __align__(256) int32_t scratch[kScratchInts];

constexpr int kMaxScratchDevices = 64;

static int device_scratch(void** out) {
  int dev = -1;
  const hipError_t ge = hipGetDevice(&dev);
  if (ge != hipSuccess) return fail(MAXSIM_ERR_LAUNCH, "hipGetDevice failed: %s", hipGetErrorString(ge));
  if (dev < 0 || dev >= kMaxScratchDevices)
    return fail(MAXSIM_ERR_UNSUPPORTED, "device index %d beyond the %d this library tracks", dev,
                kMaxScratchDevices);
  static std::mutex mu;
  static void* ptrs[kMaxScratchDevices] = {};
  std::lock_guard<std::mutex> lock(mu);
  if (!ptrs[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(MAXSIM_ERR_LAUNCH, "hipGetSymbolAddress(scratch) failed: %s",
                  hipGetErrorString(e));
    ptrs[dev] = p;
  }
  *out = ptrs[dev];
  return MAXSIM_OK;
}

static int packed_backward_impl(
    maxsim_dtype dtype, maxsim_dtype grad_dtype, const float* dscore, const void* queries,
    int64_t total_q_tokens, const int32_t* query_offsets, int64_t num_queries,
    const void* documents, int64_t total_d_tokens,
    const int32_t* document_offsets, int64_t num_documents,
    const int32_t* pair_query_ids, const int32_t* pair_document_ids,
    int64_t num_pairs, const int32_t* argmax, int64_t max_q_len, int64_t dim,
    void* dqueries, void* ddocuments, void* workspace, size_t workspace_bytes,
    void* stream) {
  if (int e = check_dtype(dtype)) return e;
  if (grad_dtype != MAXSIM_FLOAT32 && grad_dtype != dtype)
    return fail(MAXSIM_ERR_INVALID, "grad_dtype must be FLOAT32 or the input dtype");
  const bool out16 = grad_dtype != MAXSIM_FLOAT32;
  if (total_q_tokens < 0 || num_queries < 0 || total_d_tokens < 0 ||
      num_documents < 0 || num_pairs < 0)
    return fail(MAXSIM_ERR_INVALID, "negative size");
  if (max_q_len <= 0)
    return fail(MAXSIM_ERR_INVALID, "max_q_len must be > 0; got %lld", (long long)max_q_len);
  if (int e = check_dim(dim)) return e;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if ((total_q_tokens > 0 && !dqueries) || (total_d_tokens > 0 && !ddocuments))
    return fail(MAXSIM_ERR_INVALID, "null gradient pointer");
  const size_t ws_need =
      packed_workspace_bytes(num_queries, num_documents, num_pairs);
  const bool grouped = num_pairs > 0 && workspace && workspace_bytes >= ws_need &&
                       max_q_len < (1 << 16) && num_pairs < INT32_MAX;
  // 16-bit gradients are written once per row, which only the grouped
  // kernels do (the atomic path adds into fp32 rows)
  if (out16 && num_pairs > 0 && !grouped)
    return fail(MAXSIM_ERR_UNSUPPORTED,
                "16-bit gradients need the workspace and max_q_len < 65536; use fp32 gradients");
  if (!grouped) {
    if (total_q_tokens > 0) launch_fill_grad(dqueries, total_q_tokens * dim, out16, st);
    if (total_d_tokens > 0) launch_fill_grad(ddocuments, total_d_tokens * dim, out16, st);
    if (int e = check_launch("fill_zero_kernel")) return e;
  }
  if (num_pairs == 0) return MAXSIM_OK;
  if (!dscore || !queries || !documents || !query_offsets || !document_offsets ||
      !pair_query_ids || !pair_document_ids || !argmax)
    return fail(MAXSIM_ERR_INVALID, "null pointer argument");
  const int nslices = (int)((dim + 7) / 8);
  const int eb = element_bytes(dtype);
  const bool vec = (dim % 8 == 0) && aligned16b(queries) && aligned16b(documents) &&
                   ((dim * eb) % 16 == 0);
  PackedBwdArgs a{};
  a.dscore = dscore;
  a.q = queries;
  a.d = documents;
  a.qoff = query_offsets;
  a.doff = document_offsets;
  a.qids = pair_query_ids;
  a.dids = pair_document_ids;
  a.argmax = argmax;
  a.dq = dqueries;
  a.dd = ddocuments;
  a.nq = num_queries;
  a.nd = num_documents;
  a.total_q = total_q_tokens;
  a.total_d = total_d_tokens;
  a.npairs = num_pairs;
  a.slots = (int)max_q_len;
  a.dim = (int)dim;
  a.nslices = nslices;
  a.lanes_per_tok = pow2_at_least(nslices < 64 ? nslices : 64);
  if (!grouped) {
    MAXSIM_DISPATCH(dtype, launch_packed_bwd, a, vec, st);
    return check_launch("packed_bwd_kernel");
  }
  // group the pairs by query and by document (counting sort in the workspace)
  int32_t* w = static_cast<int32_t*>(workspace);
  PackedGroups g{};
  g.qstart = w;
  g.qcur = g.qstart + (num_queries + 1);
  g.dstart = g.qcur + num_queries;
  g.dcur = g.dstart + (num_documents + 1);
  g.qlist = g.dcur + num_documents;
  g.dlist = g.qlist + num_pairs;
  // zero qstart..dstart (qcur is written by the scan) and the gradient rows
  // outside every segment
  {
    const int64_t ng = (num_queries + 1) + num_queries + (num_documents + 1);
    if (out16)
      hipLaunchKernelGGL(packed_init_kernel<uint16_t>, dim3(64), dim3(256), 0, st, g.qstart, ng,
                         static_cast<uint16_t*>(dqueries), query_offsets, num_queries,
                         total_q_tokens, static_cast<uint16_t*>(ddocuments), document_offsets,
                         num_documents, total_d_tokens, (int)dim);
    else
      hipLaunchKernelGGL(packed_init_kernel<float>, dim3(64), dim3(256), 0, st, g.qstart, ng,
                         static_cast<float*>(dqueries), query_offsets, num_queries,
                         total_q_tokens, static_cast<float*>(ddocuments), document_offsets,
                         num_documents, total_d_tokens, (int)dim);
  }
  const int64_t pb = std::min<int64_t>((num_pairs + 255) / 256, 2048);
  hipLaunchKernelGGL(pair_count_kernel, dim3((unsigned)pb), dim3(256), 0, st, a, g);
  hipLaunchKernelGGL(group_scan_kernel, dim3(2), dim3(kScanThreads), 0, st, g, num_queries,
                     num_documents);
  hipLaunchKernelGGL(pair_scatter_kernel, dim3((unsigned)pb), dim3(256), 0, st, a, g);
  if (int e = check_launch("pair grouping kernels")) return e;
  const int G = pow2_at_least(nslices < 16 ? nslices : 16);  // lanes per dd row
  const bool vec_g = vec && aligned16b(dqueries) && aligned16b(ddocuments);
  MAXSIM_DISPATCH(dtype, launch_packed_grouped, a, g, vec_g, G, out16, st);
  return check_launch("dq_packed_kernel / dd_packed_kernel");
}

static int contrastive_backward_impl(
    maxsim_dtype dtype, maxsim_dtype grad_dtype, const float* dscore, const CeGrad& ce,
    const void* queries, int64_t num_queries, int64_t Lq, const void* documents,
    int64_t total_d_tokens, const int32_t* document_offsets, int64_t num_documents,
    const int32_t* argmax, int64_t dim, void* dqueries, void* ddocuments, void* workspace,
    size_t workspace_bytes, void* stream) {
  if (int e = check_dtype(dtype)) return e;
  if (grad_dtype != MAXSIM_FLOAT32 && grad_dtype != dtype)
    return fail(MAXSIM_ERR_INVALID, "grad_dtype must be MAXSIM_FLOAT32 or the input dtype");
  const bool out16 = grad_dtype != MAXSIM_FLOAT32;
  if (num_queries < 0 || num_documents < 0 || total_d_tokens < 0)
    return fail(MAXSIM_ERR_INVALID, "negative size");
  if (Lq <= 0) return fail(MAXSIM_ERR_INVALID, "Lq must be > 0; got %lld", (long long)Lq);
  if (int e = check_dim(dim)) return e;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int nslices = (int)((dim + 7) / 8);
  const int eb = element_bytes(dtype);
  const bool vec = (dim % 8 == 0) && aligned16b(queries) && aligned16b(documents) &&
                   aligned16b(dqueries) && aligned16b(ddocuments) &&
                   ((dim * eb) % 16 == 0);
  if (num_queries > 0 && !dqueries) return fail(MAXSIM_ERR_INVALID, "null dqueries");
  if (total_d_tokens > 0 && !ddocuments) return fail(MAXSIM_ERR_INVALID, "null ddocuments");
  if (num_queries == 0 || num_documents == 0) {
    if (num_queries > 0) launch_fill_grad(dqueries, num_queries * Lq * dim, out16, st);
    if (total_d_tokens > 0) launch_fill_grad(ddocuments, total_d_tokens * dim, out16, st);
    return check_launch("fill_zero_kernel");
  }
  if ((!dscore && !ce.scores) || !queries || !documents || !document_offsets || !argmax)
    return fail(MAXSIM_ERR_INVALID, "null pointer argument");
  if (total_d_tokens <= 0)
    return fail(MAXSIM_ERR_INVALID, "documents must not be empty when Nb > 0");

  // dd plan: one workgroup per document; every row of every valid document is
  // written.  LDS holds the row buckets (2 * (R + 1) ints) and up to E entry
  // ids; use up to 80 KB when the device allows, so C5-sized batches
  // (Nq * Lq = 16384 entries) need a single pass.
  DdArgs da{};
  da.ce = ce;
  da.dscore = dscore;
  da.q = queries;
  da.argmax = argmax;
  da.doff = document_offsets;
  da.dd = ddocuments;
  da.nq = num_queries;
  da.nb = num_documents;
  da.total_d = total_d_tokens;
  da.lq = (int)Lq;
  da.dim = (int)dim;
  da.nslices = nslices;
  // dimension parts: the smallest of 1, 2, 4 that brings each XCD's share of
  // Q to <= 4 MiB (one L2) for 16-bit gradients, <= 2 MiB for fp32 ones,
  // whose dD writes take twice the L2 space; never more parts than slices.
  // Each part buckets every document again.  At C5 (Q = 4 MiB): one part
  // against two, 233.5 against 237.3 us with bf16 gradients, 253.3 against
  // 244.2 us with fp32 ones.
  const int64_t q_bytes = num_queries * Lq * dim * eb;
  const int64_t q_share = out16 ? (int64_t)(4 << 20) : (int64_t)(2 << 20);
  da.parts = 1;
  while (da.parts < 4 && q_bytes / da.parts > q_share && da.parts * 2 <= nslices)
    da.parts *= 2;
  da.part_slices = (nslices + da.parts - 1) / da.parts;
  da.group = 1;
  while (da.group < kDdMaxGroup && da.group < da.part_slices) da.group *= 2;
  da.rows_per_pass = 1024;
  const size_t bucket_bytes = 2 * (size_t)(da.rows_per_pass + 1) * sizeof(int);
  auto entry_cap = [&](size_t cap) {
    const int64_t e = (int64_t)((cap - bucket_bytes) / sizeof(int));
    return std::min<int64_t>(e, 65535);  // packed bucket ids hold x < 2^16
  };
  size_t lds_cap = std::min<size_t>(max_lds_per_block(), 80 * 1024);
  int64_t e_cap = entry_cap(lds_cap);
  // 16-bit output needs every entry in one pass (below): when 80 KB holds
  // too few, take all the LDS a workgroup may have (one workgroup per CU)
  // rather than the fp32 kernels plus a cast.
  if (out16 && (Lq > e_cap || num_queries * (Lq + 1) > e_cap) &&
      max_lds_per_block() > lds_cap) {
    lds_cap = max_lds_per_block();
    e_cap = entry_cap(lds_cap);
  }
  // whole queries per pass when Lq fits (E ids + E / Lq staged dscore values),
  // else one query's tokens in chunks of E (one staged value)
  int64_t qpp = 1;
  if (Lq <= e_cap) {
    qpp = std::min<int64_t>(num_queries, e_cap / Lq);
    while (qpp > 1 && qpp * Lq + qpp > e_cap) --qpp;
    da.entries_per_pass = (int)(qpp * Lq);
  } else {
    da.entries_per_pass = (int)(e_cap - 1);
  }
  // later entry passes add to rows in fp32, so 16-bit output needs one pass
  // (all queries at once, and no query split into token chunks)
  if (out16 && (Lq > e_cap || qpp < num_queries))
    return fail(MAXSIM_ERR_UNSUPPORTED,
                "16-bit gradients need num_queries * Lq <= %lld entries; use fp32",
                (long long)(e_cap * Lq / (Lq + 1)));
  const size_t lds = bucket_bytes + ((size_t)da.entries_per_pass + (size_t)qpp) * sizeof(int);

  // dd_bucket_kernel: every entry of a document in one pass, held 32 per
  // thread, and parts of exactly 2 * G slices with G a power of two <= 16.
  // Decided before dq, whose partial sums it can add (fused reduce).
  bool bucket = false;
  DdArgs ba = da;
  size_t blds = 0;
  {
    const int64_t ne_all = num_queries * Lq;
    // Few documents: more dimension parts (up to one per XCD), so that the
    // launch has about two workgroups per CU; each part buckets its
    // document's entries again, which costs little at such sizes.
    int parts = da.parts;
    while (parts < kXcds && num_documents * parts < 512 && nslices % (parts * 2) == 0)
      parts *= 2;
    const int g2 = nslices / parts;  // one slice per lane
    if (vec && kDdThreads % Lq == 0 && g2 >= 1 && g2 <= kDdMaxGroup && (g2 & (g2 - 1)) == 0 &&
        g2 * parts == nslices && ne_all <= (int64_t)kDdThreads * kBkMaxEntriesPerThread &&
        q_bytes < ((int64_t)1 << 31) &&
        num_queries * num_documents * Lq * (int64_t)sizeof(int32_t) < ((int64_t)1 << 31)) {
      ba.parts = parts;
      ba.part_slices = g2;
      ba.group = g2;
      // the row order reuses the cursor array: kBkClasses + R / 2 <= R + 1
      ba.rows_per_pass = 1024;
      static_assert(kBkClasses + 1024 / 2 <= 1024 + 1, "row order does not fit the cursor array");
      ba.entries_per_pass = (int)ne_all;
      // The deal, where a workgroup's time follows its document's rows: one
      // part (a workgroup takes every slice of its document; with more parts
      // it takes 1 / parts of the rows' work but buckets every entry), and
      // two places per CU (P < nb <= 2 P, places b and b + P on one CU, P
      // the CU count).  Keys are rows >> shift, with twice the mean length
      // below kDealKeys.  Measured (typed backward, interleaved): C5 bf16
      // 222.3 -> 217.3 us, 64-query shard 73.8 -> 68.0 us; the ranking
      // alone costs about 2 us, and C2 (eight parts) lost 1.8 us with it.
      const int cus = device_cus();
      const int64_t places = cus;
      if (parts == 1 && cus % kXcds == 0 && num_documents > places &&
          num_documents <= 2 * places && num_documents <= kDdThreads) {
        ba.deal_places = (int)places;
        const int64_t twice_mean = 2 * total_d_tokens / num_documents;
        int shift = 0;
        while ((twice_mean >> shift) >= kDealKeys) ++shift;
        ba.deal_shift = shift;
      }
      blds = 2 * (size_t)(ba.rows_per_pass + 1) * sizeof(int) +
             ((size_t)ne_all + (size_t)num_queries) * sizeof(int);
      bucket = blds <= max_lds_per_block();
    }
  }

  // dq
  DqArgs qa{};
  qa.ce = ce;
  qa.dscore = dscore;
  qa.q = queries;
  qa.d = documents;
  qa.argmax = argmax;
  qa.dq = dqueries;
  qa.dim = (int)dim;
  qa.nslices = nslices;
  qa.rows = num_queries * Lq;
  qa.lq = (int)Lq;
  qa.doff = document_offsets;
  qa.nb = num_documents;
  qa.total_d = total_d_tokens;
  qa.padded = 0;
  const size_t ws_need = maxsim_amd_contrastive_backward_workspace_size(num_queries, Lq, dim);
  // 32-bit byte offsets of D rows when D is below 2 GiB
  const bool off32 = total_d_tokens * dim * eb < ((int64_t)1 << 31);
  if (workspace && ws_need > 0 && workspace_bytes >= ws_need) {
    float* ws = static_cast<float*>(workspace);
    const bool vec_ws = vec && aligned16b(workspace);
    const bool vec_reduce = ((num_queries * Lq * dim) % 4 == 0) && aligned16b(workspace) &&
                            aligned16b(dqueries);
    bool done = false;
    switch (dtype) {
      case MAXSIM_BFLOAT16: done = launch_dq_range<BF16>(qa, ws, vec_ws, off32, vec_reduce, out16, !bucket, st); break;
      case MAXSIM_FLOAT16: done = launch_dq_range<F16>(qa, ws, vec_ws, off32, vec_reduce, out16, !bucket, st); break;
      default: done = launch_dq_range<F32>(qa, ws, vec_ws, off32, vec_reduce, out16, !bucket, st); break;
    }
    if (!done) MAXSIM_DISPATCH(dtype, launch_dq_split, qa, vec_ws, ws, vec_reduce, out16, !bucket, st);
    if (int e = check_launch("dq_range_kernel / dq_split_kernel")) return e;
    if (bucket) {
      ba.dq_ws = ws;
      ba.dq_out = dqueries;
      ba.dq_n = num_queries * Lq * dim;
      ba.dq_vec = vec_reduce ? 1 : 0;
    }
  } else if (nslices <= 256) {
    MAXSIM_DISPATCH(dtype, launch_dq_walk, qa, vec, off32, out16, st);
    if (int e = check_launch("dq_walk_kernel")) return e;
  } else {
    MAXSIM_DISPATCH(dtype, launch_dq, qa, vec, out16, st);
    if (int e = check_launch("dq_gather_kernel")) return e;
  }

  if (bucket) {
    const int rc = dtype == MAXSIM_BFLOAT16 ? launch_dd_bucket<BF16>(ba, blds, out16, st)
                   : dtype == MAXSIM_FLOAT16 ? launch_dd_bucket<F16>(ba, blds, out16, st)
                                             : launch_dd_bucket<F32>(ba, blds, out16, st);
    if (rc) return rc;
    return check_launch("dd_bucket_kernel");
  }
  const int rc = dtype == MAXSIM_BFLOAT16 ? launch_dd_contrastive<BF16>(da, vec, lds, out16, st)
                 : dtype == MAXSIM_FLOAT16 ? launch_dd_contrastive<F16>(da, vec, lds, out16, st)
                                           : launch_dd_contrastive<F32>(da, vec, lds, out16, st);
  if (rc) return rc;
  return check_launch("dd_contrastive_kernel");
}

}  // namespace maxsim

using namespace maxsim;

extern "C" {

size_t maxsim_amd_contrastive_backward_workspace_size(int64_t num_queries, int64_t Lq,
                                                      int64_t dim) {
  // the split pass keeps a workgroup's rows x slices within 256 threads
  if (num_queries <= 0 || Lq <= 0 || dim <= 0 || dim > kDqSplitMaxDim) return 0;
  return (size_t)kXcds * (size_t)num_queries * (size_t)Lq * (size_t)dim * sizeof(float);
}

int maxsim_amd_contrastive_backward_typed(
    maxsim_dtype dtype, maxsim_dtype grad_dtype, const float* dscore, const void* queries,
    int64_t num_queries, int64_t Lq, const void* documents, int64_t total_d_tokens,
    const int32_t* document_offsets, int64_t num_documents, const int32_t* argmax,
    int64_t dim, void* dqueries, void* ddocuments, void* workspace, size_t workspace_bytes,
    void* stream) {
  clear_error();
  if (!dscore && num_queries > 0 && num_documents > 0)
    return fail(MAXSIM_ERR_INVALID, "null pointer argument");
  return contrastive_backward_impl(dtype, grad_dtype, dscore, CeGrad{}, queries, num_queries, Lq,
                                   documents, total_d_tokens, document_offsets, num_documents,
                                   argmax, dim, dqueries, ddocuments, workspace, workspace_bytes,
                                   stream);
}

int maxsim_amd_contrastive_ce_backward_typed(
    maxsim_dtype dtype, maxsim_dtype grad_dtype, const float* scores, const float* lse,
    const int32_t* targets, const float* grad_loss, int reduction, float inv_temperature,
    const void* queries, int64_t num_queries, int64_t Lq, const void* documents,
    int64_t total_d_tokens, const int32_t* document_offsets, int64_t num_documents,
    const int32_t* argmax, int64_t dim, void* dqueries, void* ddocuments, void* workspace,
    size_t workspace_bytes, void* stream) {
  clear_error();
  if (reduction < MAXSIM_REDUCTION_NONE || reduction > MAXSIM_REDUCTION_SUM)
    return fail(MAXSIM_ERR_INVALID, "unknown reduction %d", reduction);
  if (!(inv_temperature > 0.0f) || !(inv_temperature < INFINITY))
    return fail(MAXSIM_ERR_INVALID, "inv_temperature must be finite and > 0");
  if (num_queries > 0 && num_documents > 0 && (!scores || !lse || !grad_loss))
    return fail(MAXSIM_ERR_INVALID, "null pointer argument");
  if (!targets && num_queries > num_documents)
    return fail(MAXSIM_ERR_INVALID,
                "diagonal targets (targets == NULL) need num_queries <= num_documents");
  CeGrad ce;
  ce.scores = scores;
  ce.lse = lse;
  ce.targets = targets;
  ce.grad_loss = grad_loss;
  ce.per_row = reduction == MAXSIM_REDUCTION_NONE ? 1 : 0;
  ce.inv_t = inv_temperature;
  ce.scale = (reduction == MAXSIM_REDUCTION_MEAN && num_queries > 0) ? 1.0f / (float)num_queries
                                                                     : 1.0f;
  return contrastive_backward_impl(dtype, grad_dtype, nullptr, ce, queries, num_queries, Lq,
                                   documents, total_d_tokens, document_offsets, num_documents,
                                   argmax, dim, dqueries, ddocuments, workspace, workspace_bytes,
                                   stream);
}

int maxsim_amd_contrastive_backward(
    maxsim_dtype dtype, const float* dscore, const void* queries,
    int64_t num_queries, int64_t Lq, const void* documents,
    int64_t total_d_tokens, const int32_t* document_offsets,
    int64_t num_documents, const int32_t* argmax, int64_t dim,
    float* dqueries, float* ddocuments, void* workspace, size_t workspace_bytes,
    void* stream) {
  return maxsim_amd_contrastive_backward_typed(
      dtype, MAXSIM_FLOAT32, dscore, queries, num_queries, Lq, documents, total_d_tokens,
      document_offsets, num_documents, argmax, dim, dqueries, ddocuments, workspace,
      workspace_bytes, stream);
}

int maxsim_amd_padded_backward_typed(
    maxsim_dtype dtype, maxsim_dtype grad_dtype, const float* dscore, const void* queries,
    const void* documents, const int32_t* query_lengths,
    const int32_t* doc_lengths, const int32_t* argmax, int64_t batch,
    int64_t num_candidates, int64_t Lq_max, int64_t Ld_max, int64_t dim,
    void* dqueries, void* ddocuments, void* stream) {
  clear_error();
  if (int e = check_dtype(dtype)) return e;
  if (grad_dtype != MAXSIM_FLOAT32 && grad_dtype != dtype)
    return fail(MAXSIM_ERR_INVALID, "grad_dtype must be FLOAT32 or the input dtype");
  const bool out16 = grad_dtype != MAXSIM_FLOAT32;
  if (batch < 0 || num_candidates < 0) return fail(MAXSIM_ERR_INVALID, "negative size");
  if (Lq_max <= 0 || Ld_max <= 0)
    return fail(MAXSIM_ERR_INVALID, "Lq_max and Ld_max must be > 0");
  if (int e = check_dim(dim)) return e;
  if (batch == 0) return MAXSIM_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (!dqueries || (num_candidates > 0 && !ddocuments))
    return fail(MAXSIM_ERR_INVALID, "null gradient pointer");
  if (num_candidates == 0) {
    launch_fill_grad(dqueries, batch * Lq_max * dim, out16, st);
    return check_launch("fill_zero_kernel");
  }
  if (!dscore || !queries || !documents || !query_lengths || !doc_lengths || !argmax)
    return fail(MAXSIM_ERR_INVALID, "null pointer argument");
  const int nslices = (int)((dim + 7) / 8);
  const int eb = element_bytes(dtype);
  const bool vec = (dim % 8 == 0) && aligned16b(queries) && aligned16b(documents) &&
                   aligned16b(dqueries) && ((dim * eb) % 16 == 0);
  DqArgs qa{};
  qa.dscore = dscore;
  qa.q = queries;
  qa.d = documents;
  qa.argmax = argmax;
  qa.dq = dqueries;
  qa.dim = (int)dim;
  qa.nslices = nslices;
  qa.rows = batch * Lq_max;
  qa.lq = (int)Lq_max;
  qa.qlen = query_lengths;
  qa.dlen = doc_lengths;
  qa.ncand = num_candidates;
  qa.ld_max = (int)Ld_max;
  qa.padded = 1;
  // split each row's candidates over up to 8 lanes until ~128k threads run
  // (keeping at least 8 candidates per lane)
  qa.csplit = 1;
  while (qa.csplit < 8 && qa.rows * nslices * qa.csplit < 131072 &&
         num_candidates >= 16 * qa.csplit)
    qa.csplit *= 2;

  PaddedDdArgs da{};
  da.dscore = dscore;
  da.q = queries;
  da.argmax = argmax;
  da.qlen = query_lengths;
  da.dlen = doc_lengths;
  da.dd = ddocuments;
  da.npairs = batch * num_candidates;
  da.ncand = num_candidates;
  da.lq_max = (int)Lq_max;
  da.ld_max = (int)Ld_max;
  da.dim = (int)dim;
  da.pair = dim % 2 == 0 && reinterpret_cast<uintptr_t>(queries) % 4 == 0 &&
            reinterpret_cast<uintptr_t>(ddocuments) % 4 == 0;
  // Split each candidate's rows over several waves until the launch has
  // about 16k waves (16 per SIMD), keeping at least 16 rows per wave.
  {
    const int64_t npairs = batch * num_candidates;
    const int64_t by_waves = (16384 + npairs - 1) / npairs;
    const int64_t by_rows = (Ld_max + 15) / 16;
    const int64_t ns = std::max<int64_t>(1, std::min(by_waves, by_rows));
    da.rows_per_split = (int)((Ld_max + ns - 1) / ns);
    da.nsplit = (int)((Ld_max + da.rows_per_split - 1) / da.rows_per_split);
  }
  // Both grids are checked before anything is queued: a dispatch holds at
  // most 2^32 - 1 work-items per dimension.
  if ((batch * num_candidates * da.nsplit + 3) / 4 > kMaxBlocks256 ||
      (qa.rows * nslices * qa.csplit + 255) / 256 > kMaxBlocks256)
    return fail(MAXSIM_ERR_UNSUPPORTED, "too many candidates for one launch");
  da.vec_rows = dim % 8 == 0 && 64 % (dim / 8) == 0 && aligned16b(queries) &&
                aligned16b(ddocuments);
  const int64_t am_rest = Lq_max - 64 * kDdAmRegs;
  da.am_lds = (out16 || da.vec_rows) && am_rest > 0 && am_rest <= kDdAmLdsMax ? (int)am_rest : 0;
  MAXSIM_DISPATCH(dtype, launch_dq, qa, vec, out16, st);
  if (int e = check_launch("dq_gather_kernel")) return e;
  MAXSIM_DISPATCH(dtype, launch_dd_padded, da, out16, st);
  return check_launch("dd_padded_kernel");
}

int maxsim_amd_padded_backward(
    maxsim_dtype dtype, const float* dscore, const void* queries,
    const void* documents, const int32_t* query_lengths,
    const int32_t* doc_lengths, const int32_t* argmax, int64_t batch,
    int64_t num_candidates, int64_t Lq_max, int64_t Ld_max, int64_t dim,
    float* dqueries, float* ddocuments, void* stream) {
  return maxsim_amd_padded_backward_typed(dtype, MAXSIM_FLOAT32, dscore, queries, documents,
                                          query_lengths, doc_lengths, argmax, batch,
                                          num_candidates, Lq_max, Ld_max, dim, dqueries,
                                          ddocuments, stream);
}

size_t maxsim_amd_packed_backward_workspace_size(int64_t num_queries, int64_t num_documents,
                                                 int64_t num_pairs) {
  return packed_workspace_bytes(num_queries, num_documents, num_pairs);
}

int maxsim_amd_packed_backward_typed(
    maxsim_dtype dtype, maxsim_dtype grad_dtype, const float* dscore, const void* queries,
    int64_t total_q_tokens, const int32_t* query_offsets, int64_t num_queries,
    const void* documents, int64_t total_d_tokens,
    const int32_t* document_offsets, int64_t num_documents,
    const int32_t* pair_query_ids, const int32_t* pair_document_ids,
    int64_t num_pairs, const int32_t* argmax, int64_t max_q_len, int64_t dim,
    void* dqueries, void* ddocuments, void* workspace, size_t workspace_bytes,
    void* stream) {
  clear_error();
  return packed_backward_impl(dtype, grad_dtype, dscore, queries, total_q_tokens, query_offsets,
                              num_queries, documents, total_d_tokens, document_offsets,
                              num_documents, pair_query_ids, pair_document_ids, num_pairs, argmax,
                              max_q_len, dim, dqueries, ddocuments, workspace, workspace_bytes,
                              stream);
}

int maxsim_amd_packed_backward_typed_noalloc(
    maxsim_dtype dtype, maxsim_dtype grad_dtype, const float* dscore, const void* queries,
    int64_t total_q_tokens, const int32_t* query_offsets, int64_t num_queries,
    const void* documents, int64_t total_d_tokens,
    const int32_t* document_offsets, int64_t num_documents,
    const int32_t* pair_query_ids, const int32_t* pair_document_ids,
    int64_t num_pairs, const int32_t* argmax, int64_t max_q_len, int64_t dim,
    void* dqueries, void* ddocuments, void* stream) {
  clear_error();
  if (num_queries < 0 || num_documents < 0 || num_pairs < 0)
    return fail(MAXSIM_ERR_INVALID, "negative size");
  const size_t need = packed_workspace_bytes(num_queries, num_documents, num_pairs);
  if (need > kScratchBytes)
    return fail(MAXSIM_ERR_UNSUPPORTED,
                "the grouping lists need %zu bytes; the no-allocation entry point holds %zu "
                "(2 * num_queries + 2 * num_documents + 2 * num_pairs + 2 <= %zu); use "
                "maxsim_amd_packed_backward_typed with a workspace",
                need, kScratchBytes, kScratchBytes / sizeof(int32_t));
  // The argument checks of the implementation come first, so bad arguments
  // are rejected without touching the device; the scratch is only needed
  // when there are pairs to group.
  if (int e = check_dtype(dtype)) return e;
  if (grad_dtype != MAXSIM_FLOAT32 && grad_dtype != dtype)
    return fail(MAXSIM_ERR_INVALID, "grad_dtype must be FLOAT32 or the input dtype");
  if (total_q_tokens < 0 || total_d_tokens < 0) return fail(MAXSIM_ERR_INVALID, "negative size");
  if (max_q_len <= 0)
    return fail(MAXSIM_ERR_INVALID, "max_q_len must be > 0; got %lld", (long long)max_q_len);
  if (int e = check_dim(dim)) return e;
  if ((total_q_tokens > 0 && !dqueries) || (total_d_tokens > 0 && !ddocuments))
    return fail(MAXSIM_ERR_INVALID, "null gradient pointer");
  if (num_pairs > 0 && (!dscore || !queries || !documents || !query_offsets ||
                        !document_offsets || !pair_query_ids || !pair_document_ids || !argmax))
    return fail(MAXSIM_ERR_INVALID, "null pointer argument");
  void* ws = nullptr;
  if (num_pairs > 0) {
    if (int e = device_scratch(&ws)) return e;
  }
  return packed_backward_impl(dtype, grad_dtype, dscore, queries, total_q_tokens, query_offsets,
                              num_queries, documents, total_d_tokens, document_offsets,
                              num_documents, pair_query_ids, pair_document_ids, num_pairs, argmax,
                              max_q_len, dim, dqueries, ddocuments, ws, ws ? kScratchBytes : 0,
                              stream);
}

int maxsim_amd_packed_backward(
    maxsim_dtype dtype, const float* dscore, const void* queries,
    int64_t total_q_tokens, const int32_t* query_offsets, int64_t num_queries,
    const void* documents, int64_t total_d_tokens,
    const int32_t* document_offsets, int64_t num_documents,
    const int32_t* pair_query_ids, const int32_t* pair_document_ids,
    int64_t num_pairs, const int32_t* argmax, int64_t max_q_len, int64_t dim,
    float* dqueries, float* ddocuments, void* workspace, size_t workspace_bytes,
    void* stream) {
  return maxsim_amd_packed_backward_typed(
      dtype, MAXSIM_FLOAT32, dscore, queries, total_q_tokens, query_offsets, num_queries,
      documents, total_d_tokens, document_offsets, num_documents, pair_query_ids,
      pair_document_ids, num_pairs, argmax, max_q_len, dim, dqueries, ddocuments, workspace,
      workspace_bytes, stream);
}

}  // extern "C"
