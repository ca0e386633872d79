// Padded -> packed rows for gfx950 and its C-ABI entry point.
//
// The reference converts padded queries / candidates to the packed layout
// with boolean-mask gathers (torch-ext/maxsim/__init__.py:584-593, inside
// _pack_padded :516-620).  In the padded layout the valid rows of a segment
// are its first rows, one contiguous block, so the conversion is one copy of
// len[s] * row_bytes bytes per segment, from padded + s * max_len * row_bytes
// to packed + off[s] * row_bytes: HBM-bound, 2 * row_bytes of traffic per
// valid row and nothing for the padding.
#include "maxsim_host.h"

#include <algorithm>

namespace maxsim {

// 1024 threads x 4 units in flight x 16 B = 64 KB per pass, two passes per
// workgroup: at the 256k-document shape this copies at ~5.7 TB/s, against
// ~5.1 TB/s with 256 threads and 64 KB chunks (and ~4.9 TB/s for a plain
// device-to-device tensor copy of the same size).
constexpr int kPackThreads = 1024;
constexpr int64_t kPackChunk = 131072;  // bytes per workgroup
constexpr int kPackUnroll = 4;          // copy units in flight per thread

struct PackArgs {
  const char* src;
  char* dst;
  const int32_t* len;
  const int32_t* off;
  int64_t max_len;
  int64_t row_bytes;
  int64_t dst_rows;
};

// Workgroup = (segment, 128 KB chunk of its valid bytes); V is the copy unit
// (16, 8, 4 or 2 bytes), which divides the row size and both base addresses.
template <typename V>
__global__ __launch_bounds__(kPackThreads) void pack_rows_kernel(PackArgs a) {
  const int64_t s = blockIdx.x;
  const int64_t c0 = (int64_t)blockIdx.y * kPackChunk;
  const int64_t o = a.off[s];
  if (o < 0 || o >= a.dst_rows) return;
  // lengths outside [0, max_len] are clamped, and no row lands at or past
  // the packed capacity
  const int64_t len = min(min(max((int64_t)a.len[s], (int64_t)0), a.max_len), a.dst_rows - o);
  const int64_t bytes = len * a.row_bytes;
  if (c0 >= bytes) return;
  const int64_t n = min(kPackChunk, bytes - c0) / (int64_t)sizeof(V);
  const V* __restrict__ src =
      reinterpret_cast<const V*>(a.src + s * a.max_len * a.row_bytes + c0);
  V* __restrict__ dst = reinterpret_cast<V*>(a.dst + o * a.row_bytes + c0);
  int64_t i = threadIdx.x;
  for (; i + (kPackUnroll - 1) * kPackThreads < n; i += kPackUnroll * kPackThreads) {
    V v[kPackUnroll];
#pragma unroll
    for (int u = 0; u < kPackUnroll; ++u) v[u] = src[i + u * kPackThreads];
#pragma unroll
    for (int u = 0; u < kPackUnroll; ++u) dst[i + u * kPackThreads] = v[u];
  }
  for (; i < n; i += kPackThreads) dst[i] = src[i];
}

static int element_size(maxsim_dtype dt) { return dt == MAXSIM_FLOAT32 ? 4 : 2; }

}  // namespace maxsim

using namespace maxsim;

extern "C" {

int maxsim_amd_pack_padded_rows(maxsim_dtype dtype, const void* padded, int64_t num_segments,
                                int64_t max_len, const int32_t* lengths,
                                const int32_t* offsets, int64_t dim, void* packed,
                                int64_t packed_rows, void* stream) {
  clear_error();
  if (int e = check_dtype(dtype)) return e;
  if (num_segments < 0 || max_len < 0 || packed_rows < 0)
    return fail(MAXSIM_ERR_INVALID, "negative size");
  if (dim <= 0) return fail(MAXSIM_ERR_INVALID, "dim must be > 0; got %lld", (long long)dim);
  if (num_segments == 0 || max_len == 0 || packed_rows == 0) return MAXSIM_OK;
  if (!padded || !lengths || !offsets || !packed)
    return fail(MAXSIM_ERR_INVALID, "null pointer argument");
  const int64_t row_bytes = dim * element_size(dtype);
  const int64_t chunks = (max_len * row_bytes + kPackChunk - 1) / kPackChunk;
  if (num_segments > INT32_MAX || chunks > 65535)
    return fail(MAXSIM_ERR_UNSUPPORTED, "padded extent too large");
  PackArgs a{static_cast<const char*>(padded), static_cast<char*>(packed), lengths, offsets,
             max_len, row_bytes, packed_rows};
  const uintptr_t align = reinterpret_cast<uintptr_t>(padded) |
                          reinterpret_cast<uintptr_t>(packed) | (uintptr_t)row_bytes;
  const dim3 grid((unsigned)num_segments, (unsigned)chunks);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if ((align & 15u) == 0)
    hipLaunchKernelGGL(pack_rows_kernel<uint4>, grid, dim3(kPackThreads), 0, st, a);
  else if ((align & 7u) == 0)
    hipLaunchKernelGGL(pack_rows_kernel<uint2>, grid, dim3(kPackThreads), 0, st, a);
  else if ((align & 3u) == 0)
    hipLaunchKernelGGL(pack_rows_kernel<uint32_t>, grid, dim3(kPackThreads), 0, st, a);
  else
    hipLaunchKernelGGL(pack_rows_kernel<uint16_t>, grid, dim3(kPackThreads), 0, st, a);
  return check_launch("pack_rows_kernel");
}

}  // extern "C"
