// MaxSim backward kernels for gfx950 and the backward C-ABI entry points.
//
// Given the int32 argmax saved by the forward, the gradient is pure routing
// (reference maxsim.cu:564-613, 1788-1830, 2122-2169):
//     g = dscore[pair], j = argmax[pair, i]
//     dq[query token i]  += g * d[doc token j]
//     dd[doc token j]    += g * q[query token i]
//
// Contrastive and padded layouts are done owner-computes, with no global
// atomics and no zero-fill pass:
//   * dq: one thread per (query token, 8-element slice) gathers the winning
//     document row of every document it was scored against and accumulates
//     in fp32 registers; each dq element is written exactly once.
//   * dd (contrastive): one workgroup per (document, chunk of rows) keeps the
//     chunk's fp32 gradient rows in LDS, scans the argmax entries of that
//     document, and adds g * q for every entry that lands in the chunk with
//     LDS atomics (pre-aggregation); the chunk is then written once.
//   * dd (padded): one wave per (query, candidate) document writes the
//     document's rows once (zeros) and adds its <= Lq contributions in query
//     token order, so the result is deterministic.
// Packed pairs can share queries and documents arbitrarily; there dq and dd
// are zero-filled and accumulated with hardware fp32 global atomics.
#include "maxsim_common.h"
#include "maxsim_host.h"

#include <algorithm>

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

// ---------------------------------------------------------------------------
// Fill (used instead of hipMemsetAsync so the entry points stay capturable).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void fill_zero_kernel(float* p, int64_t n,
                                                        bool vec) {
  const int64_t n4 = vec ? n / 4 : 0;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride)
    reinterpret_cast<float4*>(p)[i] = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int64_t i = n4 * 4 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    p[i] = 0.0f;
}

// ---------------------------------------------------------------------------
// dq gather, contrastive and padded layouts.
// Thread = (query row r, 8-element slice s).  For contrastive, query q has
// rows q*Lq .. and is scored against every document b; for padded, query b
// has rows b*Lq_max .. and candidates p = b*C + c.
// ---------------------------------------------------------------------------
struct DqArgs {
  const float* dscore;
  const void* q;  // unused by the gather itself (kept for symmetry)
  const void* d;
  const int32_t* argmax;
  float* dq;
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
};

template <typename T>
__global__ __launch_bounds__(256) void dq_gather_kernel(DqArgs a, bool vec) {
  using S = typename T::storage;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
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
    const float* gq = a.dscore + qidx * a.nb;
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
        const float gb = (w[u] != 0.0f) ? gq[b] : 0.0f;
#pragma unroll
        for (int e2 = 0; e2 < 8; ++e2)
          acc[e2] = (w[u] != 0.0f) ? fmaf(gb, v[u][e2], acc[e2]) : acc[e2];
      }
    }
  } else {
    const int lqb = a.qlen[qidx];
    if (i < lqb && lqb <= a.lq) {
      for (int64_t c0 = 0; c0 < a.ncand; c0 += U) {
        int64_t src[U];
        float w[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int64_t c = c0 + u;
          src[u] = 0;
          w[u] = 0.0f;
          if (c < a.ncand) {
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
  }
  store8f(a.dq + row * a.dim, k0, a.dim, vec, acc);
}

// ---------------------------------------------------------------------------
// dd, contrastive: one workgroup per document, LDS counting sort.
//
// Document b receives one entry per (query q, token i): row argmax[q, b, i].
// The workgroup buckets those entries by target row in LDS (histogram,
// exclusive scan, scatter of entry ids), then 16-lane groups each own one row
// at a time and sum g[q, b] * q_row over the row's bucket in fp32 registers,
// writing the gradient row once.  No floating-point atomics; every row of the
// document is written (zeros for rows no entry points at).  Documents longer
// than `rows_per_pass` rows and entry sets larger than `entries_per_pass` are
// processed in passes (later entry passes add to the rows already written).
// ---------------------------------------------------------------------------
struct DdArgs {
  const float* dscore;
  const void* q;
  const int32_t* argmax;
  const int32_t* doff;
  float* dd;
  int64_t nq;
  int64_t nb;
  int64_t total_d;
  int lq;
  int dim;
  int nslices;
  int rows_per_pass;     // R: rows bucketed per pass (LDS: 2 * (R + 1) ints)
  int entries_per_pass;  // E: entry ids held per pass (LDS: E ints)
};

constexpr int kDdThreads = 512;
constexpr int kDdGroup = 16;                        // lanes per row
constexpr int kDdGroups = kDdThreads / kDdGroup;    // rows in flight per workgroup
constexpr int kDdMaxSlices = MAXSIM_AMD_MAX_DIM / 8 / kDdGroup;  // per lane

template <typename T>
__global__ __launch_bounds__(kDdThreads) void dd_contrastive_kernel(DdArgs a,
                                                                    bool vec) {
  using S = typename T::storage;
  extern __shared__ int lds_i[];
  const int R = a.rows_per_pass;
  int* start = lds_i;                 // [R + 1]
  int* cursor = start + (R + 1);      // [R + 1]
  int* ids = cursor + (R + 1);        // [E]

  const int64_t b = blockIdx.x;
  const int64_t d0 = a.doff[b], d1 = a.doff[b + 1];
  if (d0 < 0 || d1 <= d0 || d1 > a.total_d) return;
  const int ld = (int)(d1 - d0);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int grp = tid / kDdGroup;
  const int gl = tid % kDdGroup;
  const S* __restrict__ Q = static_cast<const S*>(a.q);
  const int64_t n_entries = a.nq * a.lq;
  const int32_t* am_b = a.argmax + b * a.lq;   // entry (q, i) at am_b[q*nb*lq + i]
  const int64_t am_qstride = a.nb * a.lq;

  for (int r0 = 0; r0 < ld; r0 += R) {
    const int nrows = min(R, ld - r0);
    for (int64_t e0 = 0; e0 < n_entries; e0 += a.entries_per_pass) {
      const int ne = (int)min((int64_t)a.entries_per_pass, n_entries - e0);
      for (int x = tid; x <= nrows; x += kDdThreads) start[x] = 0;
      __syncthreads();
      // 1. histogram of target rows
      for (int x = tid; x < ne; x += kDdThreads) {
        const int64_t e = e0 + x;
        const int64_t qq = e / a.lq;
        const int j = am_b[qq * am_qstride + (e - qq * a.lq)] - r0;
        if (j >= 0 && j < nrows) atomicAdd(&start[j + 1], 1);
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
      // 3. scatter entry ids into their row buckets
      for (int x = tid; x < ne; x += kDdThreads) {
        const int64_t e = e0 + x;
        const int64_t qq = e / a.lq;
        const int j = am_b[qq * am_qstride + (e - qq * a.lq)] - r0;
        if (j >= 0 && j < nrows) ids[atomicAdd(&cursor[j], 1)] = x;
      }
      __syncthreads();
      // 4. per-row fp32 sums, one 16-lane group per row
      for (int rr = grp; rr < nrows; rr += kDdGroups) {
        float acc[kDdMaxSlices][8];
        float* dst = a.dd + (d0 + r0 + rr) * (int64_t)a.dim;
#pragma unroll
        for (int u = 0; u < kDdMaxSlices; ++u) {
          const int sl = gl + u * kDdGroup;
          if (sl < a.nslices && e0 > 0) {
            if (vec) {
              const float4 x0 = *reinterpret_cast<const float4*>(dst + sl * 8);
              const float4 x1 = *reinterpret_cast<const float4*>(dst + sl * 8 + 4);
              acc[u][0] = x0.x; acc[u][1] = x0.y; acc[u][2] = x0.z; acc[u][3] = x0.w;
              acc[u][4] = x1.x; acc[u][5] = x1.y; acc[u][6] = x1.z; acc[u][7] = x1.w;
            } else {
#pragma unroll
              for (int k = 0; k < 8; ++k)
                acc[u][k] = (sl * 8 + k < a.dim) ? dst[sl * 8 + k] : 0.0f;
            }
          } else {
#pragma unroll
            for (int k = 0; k < 8; ++k) acc[u][k] = 0.0f;
          }
        }
        const int s_end = start[rr + 1];
        int s = start[rr];
        // two entries per step keeps two row loads in flight per lane
        for (; s + 1 < s_end; s += 2) {
          const int64_t ea = e0 + ids[s], eb = e0 + ids[s + 1];
          const float ga = a.dscore[(ea / a.lq) * a.nb + b];
          const float gb = a.dscore[(eb / a.lq) * a.nb + b];
#pragma unroll
          for (int u = 0; u < kDdMaxSlices; ++u) {
            const int sl = gl + u * kDdGroup;
            if (sl < a.nslices) {
              float va[8], vb[8];
              load8f<T>(Q + ea * (int64_t)a.dim, sl * 8, a.dim, vec, va);
              load8f<T>(Q + eb * (int64_t)a.dim, sl * 8, a.dim, vec, vb);
#pragma unroll
              for (int k = 0; k < 8; ++k) acc[u][k] = fmaf(gb, vb[k], fmaf(ga, va[k], acc[u][k]));
            }
          }
        }
        if (s < s_end) {
          const int64_t ea = e0 + ids[s];
          const float ga = a.dscore[(ea / a.lq) * a.nb + b];
#pragma unroll
          for (int u = 0; u < kDdMaxSlices; ++u) {
            const int sl = gl + u * kDdGroup;
            if (sl < a.nslices) {
              float va[8];
              load8f<T>(Q + ea * (int64_t)a.dim, sl * 8, a.dim, vec, va);
#pragma unroll
              for (int k = 0; k < 8; ++k) acc[u][k] = fmaf(ga, va[k], acc[u][k]);
            }
          }
        }
#pragma unroll
        for (int u = 0; u < kDdMaxSlices; ++u) {
          const int sl = gl + u * kDdGroup;
          if (sl < a.nslices) store8f(dst, sl * 8, a.dim, vec, acc[u]);
        }
      }
      __syncthreads();
    }
  }
}

// ---------------------------------------------------------------------------
// dd, padded: one wave per (query b, candidate c) document.
// ---------------------------------------------------------------------------
struct PaddedDdArgs {
  const float* dscore;
  const void* q;
  const int32_t* argmax;
  const int32_t* qlen;
  const int32_t* dlen;
  float* dd;
  int64_t npairs;
  int64_t ncand;
  int lq_max;
  int ld_max;
  int dim;
};

template <typename T>
__global__ __launch_bounds__(256) void dd_padded_kernel(PaddedDdArgs a) {
  using S = typename T::storage;
  const int lane = threadIdx.x & 63;
  const int64_t p = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (p >= a.npairs) return;
  const int64_t b = p / a.ncand;
  float* base = a.dd + p * a.ld_max * (int64_t)a.dim;
  const int64_t n = (int64_t)a.ld_max * a.dim;
  for (int64_t x = lane; x < n; x += 64) base[x] = 0.0f;
  const int lqb = a.qlen[b];
  const int ld = a.dlen[p];
  if (lqb < 1 || lqb > a.lq_max || ld < 1 || ld > a.ld_max) return;
  const float g = a.dscore[p];
  const S* __restrict__ Q = static_cast<const S*>(a.q);
  for (int i = 0; i < lqb; ++i) {
    const int j = a.argmax[p * a.lq_max + i];
    if (j < 0 || j >= ld) continue;
    const S* qrow = Q + (b * a.lq_max + i) * (int64_t)a.dim;
    float* drow = base + (int64_t)j * a.dim;
    for (int x = lane; x < a.dim; x += 64) {
      float qv;
      if constexpr (T::bytes == 4) {
        qv = qrow[x];
      } else if constexpr (__is_same(T, BF16)) {
        qv = __uint_as_float((uint32_t)qrow[x] << 16);
      } else {
        qv = (float)__builtin_bit_cast(_Float16, qrow[x]);
      }
      drow[x] = fmaf(g, qv, drow[x]);
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
  float* dq;
  float* dd;
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
      float* dqr = a.dq + (qs + i) * (int64_t)a.dim + sl * 8;
      float* ddr = a.dd + (ds + j) * (int64_t)a.dim + sl * 8;
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

static void launch_fill(float* p, int64_t n, hipStream_t st) {
  if (n <= 0) return;
  int64_t blocks = (n / 4 + 255) / 256;
  if (blocks < 1) blocks = 1;
  if (blocks > 65535) blocks = 65535;
  hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)blocks), dim3(256), 0, st,
                     p, n, aligned16b(p));
}

template <typename T>
static void launch_dq(const DqArgs& a, bool vec, hipStream_t st) {
  const int64_t threads = a.rows * a.nslices;
  const dim3 grid((unsigned)((threads + 255) / 256));
  hipLaunchKernelGGL(dq_gather_kernel<T>, grid, dim3(256), 0, st, a, vec);
}

template <typename T>
static void launch_dd_contrastive(const DdArgs& a, bool vec, size_t lds, hipStream_t st) {
  hipLaunchKernelGGL(dd_contrastive_kernel<T>, dim3((unsigned)a.nb), dim3(kDdThreads), lds,
                     st, a, vec);
}

// Largest dynamic LDS allocation one workgroup may use on this device.
static size_t max_lds_per_block() {
  int dev = 0, v = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 64 * 1024;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess ||
      v <= 0)
    return 64 * 1024;
  return (size_t)v;
}

template <typename T>
static void launch_dd_padded(const PaddedDdArgs& a, hipStream_t st) {
  const dim3 grid((unsigned)((a.npairs + 3) / 4));
  hipLaunchKernelGGL(dd_padded_kernel<T>, grid, dim3(256), 0, st, a);
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

static int element_bytes(maxsim_dtype dt) { return dt == MAXSIM_FLOAT32 ? 4 : 2; }

}  // namespace maxsim

using namespace maxsim;

extern "C" {

int maxsim_amd_contrastive_backward(
    maxsim_dtype dtype, const float* dscore, const void* queries,
    int64_t num_queries, int64_t Lq, const void* documents,
    int64_t total_d_tokens, const int32_t* document_offsets,
    int64_t num_documents, const int32_t* argmax, int64_t dim,
    float* dqueries, float* ddocuments, void* stream) {
  clear_error();
  if (int e = check_dtype(dtype)) return e;
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
    if (num_queries > 0) launch_fill(dqueries, num_queries * Lq * dim, st);
    if (total_d_tokens > 0) launch_fill(ddocuments, total_d_tokens * dim, st);
    return check_launch("fill_zero_kernel");
  }
  if (!dscore || !queries || !documents || !document_offsets || !argmax)
    return fail(MAXSIM_ERR_INVALID, "null pointer argument");
  if (total_d_tokens <= 0)
    return fail(MAXSIM_ERR_INVALID, "documents must not be empty when Nb > 0");

  // dq
  DqArgs qa{};
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
  MAXSIM_DISPATCH(dtype, launch_dq, qa, vec, st);
  if (int e = check_launch("dq_gather_kernel")) return e;

  // dd: one workgroup per document; every row of every valid document is
  // written.  LDS holds the row buckets (2 * (R + 1) ints) and up to E entry
  // ids; use up to 80 KB when the device allows, so C5-sized batches
  // (Nq * Lq = 16384 entries) need a single pass.
  DdArgs da{};
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
  const size_t lds_cap = std::min<size_t>(max_lds_per_block(), 80 * 1024);
  da.rows_per_pass = 1024;
  const size_t bucket_bytes = 2 * (size_t)(da.rows_per_pass + 1) * sizeof(int);
  int64_t e_cap = (int64_t)((lds_cap - bucket_bytes) / sizeof(int));
  if (e_cap > 16384) e_cap = 16384;
  da.entries_per_pass = (int)std::min<int64_t>(e_cap, std::max<int64_t>(num_queries * Lq, 1));
  const size_t lds = bucket_bytes + (size_t)da.entries_per_pass * sizeof(int);
  if (lds > 64 * 1024) {
    (void)hipFuncSetAttribute((const void*)dd_contrastive_kernel<BF16>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    (void)hipFuncSetAttribute((const void*)dd_contrastive_kernel<F16>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    (void)hipFuncSetAttribute((const void*)dd_contrastive_kernel<F32>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    (void)hipGetLastError();
  }
  MAXSIM_DISPATCH(dtype, launch_dd_contrastive, da, vec, lds, st);
  return check_launch("dd_contrastive_kernel");
}

int maxsim_amd_padded_backward(
    maxsim_dtype dtype, const float* dscore, const void* queries,
    const void* documents, const int32_t* query_lengths,
    const int32_t* doc_lengths, const int32_t* argmax, int64_t batch,
    int64_t num_candidates, int64_t Lq_max, int64_t Ld_max, int64_t dim,
    float* dqueries, float* ddocuments, void* stream) {
  clear_error();
  if (int e = check_dtype(dtype)) return e;
  if (batch < 0 || num_candidates < 0) return fail(MAXSIM_ERR_INVALID, "negative size");
  if (Lq_max <= 0 || Ld_max <= 0)
    return fail(MAXSIM_ERR_INVALID, "Lq_max and Ld_max must be > 0");
  if (int e = check_dim(dim)) return e;
  if (batch == 0) return MAXSIM_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (!dqueries || (num_candidates > 0 && !ddocuments))
    return fail(MAXSIM_ERR_INVALID, "null gradient pointer");
  if (num_candidates == 0) {
    launch_fill(dqueries, batch * Lq_max * dim, st);
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
  MAXSIM_DISPATCH(dtype, launch_dq, qa, vec, st);
  if (int e = check_launch("dq_gather_kernel")) return e;

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
  MAXSIM_DISPATCH(dtype, launch_dd_padded, da, st);
  return check_launch("dd_padded_kernel");
}

int maxsim_amd_packed_backward(
    maxsim_dtype dtype, const float* dscore, const void* queries,
    int64_t total_q_tokens, const int32_t* query_offsets, int64_t num_queries,
    const void* documents, int64_t total_d_tokens,
    const int32_t* document_offsets, int64_t num_documents,
    const int32_t* pair_query_ids, const int32_t* pair_document_ids,
    int64_t num_pairs, const int32_t* argmax, int64_t max_q_len, int64_t dim,
    float* dqueries, float* ddocuments, void* stream) {
  clear_error();
  if (int e = check_dtype(dtype)) return e;
  if (total_q_tokens < 0 || num_queries < 0 || total_d_tokens < 0 ||
      num_documents < 0 || num_pairs < 0)
    return fail(MAXSIM_ERR_INVALID, "negative size");
  if (max_q_len <= 0)
    return fail(MAXSIM_ERR_INVALID, "max_q_len must be > 0; got %lld", (long long)max_q_len);
  if (int e = check_dim(dim)) return e;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if ((total_q_tokens > 0 && !dqueries) || (total_d_tokens > 0 && !ddocuments))
    return fail(MAXSIM_ERR_INVALID, "null gradient pointer");
  if (total_q_tokens > 0) launch_fill(dqueries, total_q_tokens * dim, st);
  if (total_d_tokens > 0) launch_fill(ddocuments, total_d_tokens * dim, st);
  if (int e = check_launch("fill_zero_kernel")) return e;
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
  MAXSIM_DISPATCH(dtype, launch_packed_bwd, a, vec, st);
  return check_launch("packed_bwd_kernel");
}

}  // extern "C"
