// Shared device code for the MaxSim kernels (gfx950 / CDNA4).
//
// Tile geometry used by every forward kernel
// ------------------------------------------
// One MFMA output tile is 32 document rows (M) x 32 query tokens (N), built
// from K-chunks of 16 embedding elements:
//   * bf16 / fp16 : one v_mfma_f32_32x32x16_{bf16,f16} per K-chunk
//   * fp32        : eight v_mfma_f32_32x32x2_f32 per K-chunk
// Lane l = c + 32*h (c = l & 31, h = l >> 5) supplies, for K-chunk s,
//   A: document row  (tile_row0 + c), elements [16s + 8h, 16s + 8h + 8)
//   B: query token   (tok0 + c),      elements [16s + 8h, 16s + 8h + 8)
// Because A and B use the same (lane-half, element) -> k mapping, the MFMA
// sums exactly the products q[k] * d[k] over the chunk.  The fp32 path maps
// instruction e of the chunk to k = 16s + 8h + e, which is the same set.
// Accumulator register r of lane l holds
//   S[row = 8*(r>>2) + 4*h + (r&3)][col = c]
// so each lane owns ONE query token and 16 document rows per tile, in
// ascending row order.  The running max/argmax is therefore a per-lane
// register update; the two lane halves are merged once per document.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace maxsim {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kTileRows = 32;   // document rows per MFMA tile
constexpr int kTileCols = 32;   // query tokens per MFMA tile (one "query block")
// gfx950 dispatches workgroup w to XCD w % kXcds; each XCD has its own L2
constexpr int kXcds = 8;
constexpr int kChunk = 16;      // embedding elements per K-chunk

// Element tags (storage is raw bits; arithmetic happens inside MFMA).
struct BF16 { typedef uint16_t storage; static constexpr int bytes = 2; };
struct F16  { typedef uint16_t storage; static constexpr int bytes = 2; };
struct F32  { typedef float    storage; static constexpr int bytes = 4; };

// Per-lane operand fragment for one K-chunk: 8 elements.
template <typename T> struct Frag;
template <> struct Frag<BF16> { uint4 v; };
template <> struct Frag<F16>  { uint4 v; };
template <> struct Frag<F32>  { uint4 lo, hi; };

template <typename T>
__device__ __forceinline__ Frag<T> zero_frag() {
  Frag<T> f;
  if constexpr (T::bytes == 2) {
    f.v = make_uint4(0, 0, 0, 0);
  } else {
    f.lo = make_uint4(0, 0, 0, 0);
    f.hi = make_uint4(0, 0, 0, 0);
  }
  return f;
}

// Load 8 elements [k0, k0+8) of a row.  `vec` means the row pointer plus k0
// is 16-byte aligned and k0 + 8 <= dim; otherwise elements at k >= dim read
// as zero and the load is element-wise.
template <typename T>
__device__ __forceinline__ Frag<T> load_frag(const typename T::storage* row,
                                             int k0, int dim, bool vec) {
  Frag<T> f;
  if (vec) {
    if constexpr (T::bytes == 2) {
      f.v = *reinterpret_cast<const uint4*>(row + k0);
    } else {
      f.lo = *reinterpret_cast<const uint4*>(row + k0);
      f.hi = *reinterpret_cast<const uint4*>(row + k0 + 4);
    }
    return f;
  }
  if constexpr (T::bytes == 2) {
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int k = k0 + 2 * e;
      const uint32_t lo = (k < dim) ? (uint32_t)row[k] : 0u;
      const uint32_t hi = (k + 1 < dim) ? (uint32_t)row[k + 1] : 0u;
      w[e] = lo | (hi << 16);
    }
    f.v = make_uint4(w[0], w[1], w[2], w[3]);
  } else {
    float x[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = (k0 + e < dim) ? row[k0 + e] : 0.0f;
    f.lo = make_uint4(__float_as_uint(x[0]), __float_as_uint(x[1]),
                      __float_as_uint(x[2]), __float_as_uint(x[3]));
    f.hi = make_uint4(__float_as_uint(x[4]), __float_as_uint(x[5]),
                      __float_as_uint(x[6]), __float_as_uint(x[7]));
  }
  return f;
}

// acc += A(32 rows x 16 k) * B(16 k x 32 tokens) for one K-chunk.
__device__ __forceinline__ void mma_chunk(const Frag<BF16>& a,
                                          const Frag<BF16>& b, f32x16& acc) {
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
      __builtin_bit_cast(bf16x8, a.v), __builtin_bit_cast(bf16x8, b.v), acc,
      0, 0, 0);
}
__device__ __forceinline__ void mma_chunk(const Frag<F16>& a,
                                          const Frag<F16>& b, f32x16& acc) {
  acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(
      __builtin_bit_cast(f16x8, a.v), __builtin_bit_cast(f16x8, b.v), acc,
      0, 0, 0);
}
__device__ __forceinline__ void mma_chunk(const Frag<F32>& a,
                                          const Frag<F32>& b, f32x16& acc) {
  const uint32_t av[8] = {a.lo.x, a.lo.y, a.lo.z, a.lo.w,
                          a.hi.x, a.hi.y, a.hi.z, a.hi.w};
  const uint32_t bv[8] = {b.lo.x, b.lo.y, b.lo.z, b.lo.w,
                          b.hi.x, b.hi.y, b.hi.z, b.hi.w};
#pragma unroll
  for (int e = 0; e < 8; ++e)
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(
        __uint_as_float(av[e]), __uint_as_float(bv[e]), acc, 0, 0, 0);
}

// Row (within the 32-row tile) held by accumulator register r of lane-half h.
__device__ __forceinline__ constexpr int acc_row(int r, int h) {
  return 8 * (r >> 2) + 4 * h + (r & 3);
}

// Running max / argmax update for one tile.  Semantics (shared with the
// reference kernels, maxsim.cu:412-443): ascending document order, strict
// `>` so the first index wins ties, NaN never wins (fmaxf ignores NaN and
// `>`/`==` are false for NaN).  `row_base` is tile_row0 + 4*h.
//
// Rows past the end of a document are never masked: the kernels load them
// as copies of the document's last row, whose similarities are bitwise equal
// and come later, so under the strict `>` they can neither raise the max nor
// take the argmax.
//
// The update is branch-free (a max3 tree, then the first register equal to
// the tile max -- sixteen independent compares feeding a select chain --,
// then a conditional commit), so it forms one scheduling region with the
// MFMAs of the next tile and its VALU work can fill the MFMA shadow.
template <bool ARGMAX>
__device__ __forceinline__ void tile_update(const f32x16& acc, float& m,
                                            int& am, int row_base) {
  const float t0 = fmaxf(fmaxf(acc[0], acc[1]), acc[2]);
  const float t1 = fmaxf(fmaxf(acc[3], acc[4]), acc[5]);
  const float t2 = fmaxf(fmaxf(acc[6], acc[7]), acc[8]);
  const float t3 = fmaxf(fmaxf(acc[9], acc[10]), acc[11]);
  const float t4 = fmaxf(fmaxf(acc[12], acc[13]), acc[14]);
  const float t5 = fmaxf(fmaxf(t0, t1), t2);
  const float t6 = fmaxf(fmaxf(t3, t4), acc[15]);
  const float tmax = fmaxf(t5, t6);
  const bool upd = tmax > m;
  m = upd ? tmax : m;
  if constexpr (ARGMAX) {
    bool eq[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) eq[r] = acc[r] == tmax;
    int off = 8 * (15 >> 2) + (15 & 3);
#pragma unroll
    for (int r = 14; r >= 0; --r) off = eq[r] ? (8 * (r >> 2) + (r & 3)) : off;
    am = upd ? row_base + off : am;
  }
}

// Running max with the index search deferred to the end of the document.
// Per tile: the tile max (max3 tree), and when it beats the running max, the
// new max, the base row of that tile (`bt`) and a copy of the tile's 16
// values (`best`) -- 27 VALU instructions, every select reading one mask.
// best_row() then finds the first row of the best tile holding the max, once
// per document.  Same result as tile_update<true>: strict `>` keeps the
// earliest tile, the row search keeps the lowest row within it, and the max
// is always one of the copied values (fmaxf returns one of its operands).
__device__ __forceinline__ void tile_update_deferred(const f32x16& acc, float& m, int& bt,
                                                     f32x16& best, int row_base) {
  const float t0 = fmaxf(fmaxf(acc[0], acc[1]), acc[2]);
  const float t1 = fmaxf(fmaxf(acc[3], acc[4]), acc[5]);
  const float t2 = fmaxf(fmaxf(acc[6], acc[7]), acc[8]);
  const float t3 = fmaxf(fmaxf(acc[9], acc[10]), acc[11]);
  const float t4 = fmaxf(fmaxf(acc[12], acc[13]), acc[14]);
  const float t5 = fmaxf(fmaxf(t0, t1), t2);
  const float t6 = fmaxf(fmaxf(t3, t4), acc[15]);
  const float tmax = fmaxf(t5, t6);
  const bool upd = tmax > m;
  m = upd ? tmax : m;
  bt = upd ? row_base : bt;
#pragma unroll
  for (int r = 0; r < 16; ++r) best[r] = upd ? acc[r] : best[r];
}

// Row index of the running max: bt (< 0 when no tile ever set it -> 0)
// plus the offset of the first copied value equal to m.
__device__ __forceinline__ int best_row(const f32x16& best, float m, int bt) {
  bool eq[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) eq[r] = best[r] == m;
  int off = 8 * (15 >> 2) + (15 & 3);
#pragma unroll
  for (int r = 14; r >= 0; --r) off = eq[r] ? (8 * (r >> 2) + (r & 3)) : off;
  return bt < 0 ? 0 : bt + off;
}

// Merge the two lane halves that own the same query token: larger value
// wins, equal values keep the lower document index.  v_permlane32_swap with
// both operands equal leaves, in every lane l, the value of lane (l & 31)
// in the first result and of lane (l & 31) + 32 in the second, so lanes c
// and c + 32 compute the same merge without an LDS round trip.
__device__ __forceinline__ void merge_halves(float& m, int& am) {
  const auto mv = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, m),
                                                   __builtin_bit_cast(int, m), false, false);
  const auto av = __builtin_amdgcn_permlane32_swap(am, am, false, false);
  const float m_lo = __builtin_bit_cast(float, (int)mv[0]);
  const float m_hi = __builtin_bit_cast(float, (int)mv[1]);
  const int a_lo = (int)av[0], a_hi = (int)av[1];
  const bool hi_wins = m_hi > m_lo || (m_hi == m_lo && a_hi < a_lo);
  m = hi_wins ? m_hi : m_lo;
  am = hi_wins ? a_hi : a_lo;
}

// DPP step: s + (s moved by the DPP control CTRL), rows outside ROW_MASK add 0.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_add(float s) {
  const int t = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, s), CTRL, ROW_MASK, 0xF,
                                            false);
  return s + __builtin_bit_cast(float, t);
}

// Sum of `v` over the 32 lanes of each half with DPP moves (no LDS): pairs
// (quad_perm [1,0,3,2]), quads ([2,3,0,1]), groups of 8 (row_half_mirror),
// rows of 16 (row_mirror), then row 0's total broadcast into row 1 (and row
// 2's into row 3).  The order is fixed, so the result is deterministic; it is
// complete in lanes 16..31 and 48..63 (kHalfSumLane is one of them).
constexpr int kHalfSumLane = 31;
__device__ __forceinline__ float half_sum(float v) {
  v = dpp_add<0xB1, 0xF>(v);
  v = dpp_add<0x4E, 0xF>(v);
  v = dpp_add<0x141, 0xF>(v);
  v = dpp_add<0x140, 0xF>(v);
  return dpp_add<0x142, 0xA>(v);
}

// A global-memory pointer the caller knows to be the same in every lane,
// read back as a scalar and typed in the global address space: loads
// through it with a 32-bit per-lane offset then take the saddr form
// (uniform base in SGPRs + one VGPR offset) instead of a 64-bit address per
// lane.
#define MAXSIM_GLOBAL __attribute__((address_space(1)))
template <typename P>
__device__ __forceinline__ const MAXSIM_GLOBAL P* uniform_gptr(const P* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (const MAXSIM_GLOBAL P*)(((uint64_t)hi << 32) | lo);
}

// 16 bytes at base + off (off a multiple of 16) through a global pointer.
__device__ __forceinline__ uint4 load16(const MAXSIM_GLOBAL char* base, uint32_t off) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 v = *reinterpret_cast<const MAXSIM_GLOBAL u32x4*>(base + off);
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// 32-bit LDS byte address of an LDS pointer (generic -> LDS address space).
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)((__attribute__((address_space(3))) const void*)p);
}

// One wave instruction moving 16 bytes per lane from global memory
// (uniform base + per-lane 32-bit byte offset) straight into LDS at
// m0 + 16 * lane.  m0 is an input operand of the asm ("{m0}"), so the
// compiler itself writes it just before the instruction and knows it is
// read; nothing reserved is clobbered behind its back.  The compiler's
// hazard recognizer does not look inside inline asm, so the asm opens with
// s_nop 4: five wait states cover both a VALU write (readfirstlane) of the
// base SGPRs, which a VMEM read needs five states after, and the compiler's
// SALU write of m0, which an LDS DMA needs one state after.
// (__builtin_amdgcn_global_load_lds would need no asm, but then the
// compiler puts an s_waitcnt vmcnt(0) before every LDS read that follows a
// DMA, since it cannot tell the ring buffers apart, which serialises the
// ring.)
__device__ __forceinline__ void lds_dma16(const void* base, uint32_t off, uint32_t m0) {
  __asm__ __volatile__(
      "s_nop 4\n\t"
      "global_load_lds_dwordx4 %0, %1"
      :
      : "v"(off), "s"(base), "{m0}"(__builtin_amdgcn_readfirstlane(m0))
      : "memory");
}

// The same load with the non-temporal cache policy (`nt`), for data read
// exactly once (the padded candidates' rows): its lines are marked for early
// eviction and leave L2 to the data that is re-read.
__device__ __forceinline__ void lds_dma16_nt(const void* base, uint32_t off, uint32_t m0) {
  __asm__ __volatile__(
      "s_nop 4\n\t"
      "global_load_lds_dwordx4 %0, %1 nt"
      :
      : "v"(off), "s"(base), "{m0}"(__builtin_amdgcn_readfirstlane(m0))
      : "memory");
}

// ---------------------------------------------------------------------------
// Ranking a workgroup's items (at most one per thread) by a small key,
// largest key first, ties by thread index, so that every workgroup that
// ranks the same keys finds the same ranks: the lists that are dealt to
// workgroups longest first.  Each lane sets its bit in a 64-bit mask per
// (wave, key) with one LDS atomic OR; its place among the lanes of equal
// key is the count of bits below its own, the wave's count for the key the
// count of all.  Wave 0 then turns the counts into the counts of the waves
// before and each key's first rank (KEYS / 64 keys per lane).  No loop over
// the distinct keys.
// ---------------------------------------------------------------------------
template <int kWaves, int KEYS>
struct RankScratch {
  static_assert(KEYS == 64 || KEYS == 128, "one or two keys per lane of wave 0");
  static constexpr int kBytes = kWaves * KEYS * 8 + kWaves * KEYS * 4 + KEYS * 4;
  uint64_t* mask;  // [wave][key] lanes holding the key
  int* before;     // [wave][key] items of the key in the waves before
  int* first;      // [key] first rank: items of the larger keys
  __device__ explicit RankScratch(void* lds)
      : mask(static_cast<uint64_t*>(lds)),
        before(reinterpret_cast<int*>(mask + kWaves * KEYS)),
        first(before + kWaves * KEYS) {}
  // Clears the masks; every thread calls it, before rank().
  __device__ void clear() const {
    for (int i = threadIdx.x; i < kWaves * KEYS; i += kWaves * 64) mask[i] = 0;
  }
  // The rank of this thread's item (own: it has one; key in [0, KEYS)), or
  // -1 without one.  Every thread of the workgroup calls it (three barriers,
  // the first of which orders clear() before the atomics).
  __device__ int rank(bool own, int key) const {
    constexpr int KPL = KEYS / 64;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (own) atomicOr(reinterpret_cast<unsigned long long*>(&mask[wave * KEYS + key]),
                      1ull << lane);
    __syncthreads();
    int pos = 0;
    if (own) pos = __popcll(mask[wave * KEYS + key] & ((1ull << lane) - 1ull));
    if (wave == 0) {
      int tot[KPL];
      int sum = 0;
#pragma unroll
      for (int j = 0; j < KPL; ++j) {
        const int k = KEYS - 1 - KPL * lane - j;
        int cnt[kWaves];
#pragma unroll
        for (int w = 0; w < kWaves; ++w) cnt[w] = __popcll(mask[w * KEYS + k]);
        int t = 0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
          before[w * KEYS + k] = t;
          t += cnt[w];
        }
        tot[j] = t;
        sum += t;
      }
      int ci = sum;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int u = __shfl_up(ci, o);
        if (lane >= o) ci += u;
      }
      int run = ci - sum;
#pragma unroll
      for (int j = 0; j < KPL; ++j) {
        first[KEYS - 1 - KPL * lane - j] = run;
        run += tot[j];
      }
    }
    __syncthreads();
    return own ? first[key] + before[wave * KEYS + key] + pos : -1;
  }
};

}  // namespace maxsim
