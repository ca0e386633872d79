// MaxSim forward kernels for gfx950 and the forward C-ABI entry points.
//
// Three families of kernels share the tile math of maxsim_common.h:
//
//  * contrastive_tiled_kernel -- all-pairs scoring (reference K6/K7,
//    maxsim.cu:1227-1595).  A workgroup of 8 waves holds up to 16 query
//    blocks (32 tokens each) in registers and streams the 32-row tiles of a
//    chunk of documents through a ring of four LDS buffers filled by direct
//    global->LDS loads, so each document tile is read from L2 once per 16
//    queries instead of once per pair.  The blockIdx -> (query group, doc
//    chunk) map keeps all query groups of a doc chunk on one XCD so the
//    chunk is fetched into that XCD's L2 once.  Chunks are runs of whole
//    documents of equal work or, with few documents per chunk, documents
//    dealt longest first so that every chunk holds the same tiles.
//
//  * group_docs_kernel + scatter_docs_kernel + doc_chunk_kernel -- packed
//    pairs scored document by document (reference K9, maxsim.cu:1933-2108,
//    with a workspace): the pairs are grouped by document on the device and
//    each document's tiles pass once through an LDS ring shared by up to
//    four of its pairs.
//
//  * pair_kernel -- one wave per run of (query, document) pairs, document
//    rows loaded straight from global memory into MFMA operand registers
//    (reference K1/K2/K3/K5/K9, maxsim.cu:70-322, 647-698, 1933-2010).  Used
//    for padded rerank and packed pairs, whose document tiles are each used
//    by a single query (HBM-bound), and for contrastive shapes the tiled
//    kernel does not cover (Lq > 64).  pair_ring_kernel is its variant for
//    16-bit rows of at most 128 elements and queries of at most 64 tokens:
//    tiles come in through two wave-private LDS slots, two tiles ahead.
//
// Neither kernel writes the [Lq, Ld] similarity matrix anywhere: each
// 32x32 MFMA tile is reduced in registers (tile_update) and discarded.
#include <string>
#include <type_traits>
#include <cstdio>
#include <cstdarg>

#include "maxsim_common.h"
#include "maxsim_host.h"

namespace maxsim {

enum Mode : int { kContrastive = 0, kPadded = 1, kPacked = 2 };

struct FwdArgs {
  const void* q;
  const void* d;
  int dim;
  int mode;
  int64_t npairs;
  int slots;  // argmax row stride (Lq for contrastive, Lq_max, max_q_len)
  // contrastive
  int64_t nb;
  int lq;
  const int32_t* doff;
  int64_t total_d;
  // padded
  const int32_t* qlen;
  const int32_t* dlen;
  int64_t ncand;
  int lq_max;
  int ld_max;
  // packed
  const int32_t* qoff;
  int64_t nq;
  int64_t nd;
  const int32_t* qids;
  const int32_t* dids;
  int64_t total_q;
  // outputs
  float* scores;
  int32_t* argmax;
};

struct Pair {
  int64_t q_row0;
  int64_t d_row0;
  int lq;
  int ld;
  bool ok;
};

// Resolve pair p to row ranges.  Every index read from device memory is
// range-checked so invalid metadata never causes an out-of-bounds access.
__device__ __forceinline__ Pair resolve_pair(const FwdArgs& a, int64_t p) {
  Pair r{0, 0, 0, 0, false};
  if (a.mode == kContrastive) {
    const int64_t q = p / a.nb;
    const int64_t b = p - q * a.nb;
    const int64_t s = a.doff[b], e = a.doff[b + 1];
    r.q_row0 = q * a.lq;
    r.lq = a.lq;
    r.d_row0 = s;
    r.ld = (int)(e - s);
    r.ok = (s >= 0) && (e > s) && (e <= a.total_d);
  } else if (a.mode == kPadded) {
    const int64_t b = p / a.ncand;
    const int lq = a.qlen[b];
    const int ld = a.dlen[p];
    r.q_row0 = b * a.lq_max;
    r.lq = lq;
    r.d_row0 = p * a.ld_max;
    r.ld = ld;
    r.ok = (lq >= 1) && (lq <= a.lq_max) && (ld >= 1) && (ld <= a.ld_max);
  } else {
    const int64_t qi = a.qids[p], di = a.dids[p];
    if (qi < 0 || qi >= a.nq || di < 0 || di >= a.nd) return r;
    const int64_t qs = a.qoff[qi], qe = a.qoff[qi + 1];
    const int64_t ds = a.doff[di], de = a.doff[di + 1];
    r.q_row0 = qs;
    r.lq = (int)(qe - qs);
    r.d_row0 = ds;
    r.ld = (int)(de - ds);
    r.ok = (qs >= 0) && (qe > qs) && (qe <= a.total_q) && (qe - qs <= a.slots) &&
           (ds >= 0) && (de > ds) && (de <= a.total_d);
  }
  return r;
}

__device__ __forceinline__ void write_invalid_pair(const FwdArgs& a, int64_t p,
                                                   int lane) {
  if (lane == 0) a.scores[p] = __builtin_nanf("");
  if (a.argmax)
    for (int t = lane; t < a.slots; t += 64) a.argmax[p * a.slots + t] = 0;
}

// ---------------------------------------------------------------------------
// pair_kernel: each wave scores a run of `ppw` consecutive pairs.
// QB query blocks (32 tokens each) are held in registers; queries longer than
// 32*QB tokens are processed QB blocks at a time, re-streaming the document.
// ---------------------------------------------------------------------------
// VEC (rows are whole 16-byte fragments, 16-byte aligned) is a template
// parameter: as a runtime flag, both load paths were compiled into the tile
// loop, and the element-wise one's bounds checks drove the kernel into
// scalar-register spills.
template <typename T, int KS, int QB, bool ARGMAX, bool VEC>
__global__ __launch_bounds__(256) void pair_kernel(FwdArgs a, int ppw) {
  constexpr bool vec = VEC;
  using S = typename T::storage;
  const int lane = threadIdx.x & 63;
  const int c = lane & 31;
  const int h = lane >> 5;
  // wave-uniform (readfirstlane says so): pair indices stay scalar
  const int64_t wave =
      (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int64_t p_begin = wave * ppw;
  if (p_begin >= a.npairs) return;
  const int64_t p_end = min(p_begin + (int64_t)ppw, a.npairs);
  const S* __restrict__ Q = static_cast<const S*>(a.q);
  const S* __restrict__ D = static_cast<const S*>(a.d);
  const int dim = a.dim;

  Frag<T> qf[QB][KS];
  int64_t loaded_q = -1;
  int loaded_lq = -1, loaded_g = -1;

  // The run is pipelined across pairs: the next pair's rows are resolved
  // while the current one is scored, and its first tile is loaded in place
  // of a prefetch at the current pair's last tile, so a pair starts with its
  // first tile already in flight (queries that change still load here).
  auto load_tile = [&](const Pair& q_pr, int t, Frag<T> (&f)[KS]) __attribute__((always_inline)) {
    const int r = min(t * kTileRows + c, q_pr.ld - 1);
    const S* row = D + (q_pr.d_row0 + r) * (int64_t)dim;
#pragma unroll
    for (int s = 0; s < KS; ++s) f[s] = load_frag<T>(row, kChunk * s + 8 * h, dim, vec);
  };
  Pair pr = resolve_pair(a, p_begin);
  Frag<T> df[KS];
  bool df_ready = false;  // df holds tile 0 of pr
  for (int64_t p = p_begin; p < p_end; ++p) {
    const Pair nx = (p + 1 < p_end) ? resolve_pair(a, p + 1) : Pair{0, 0, 0, 0, false};
    if (!pr.ok) {
      write_invalid_pair(a, p, lane);
      pr = nx;
      df_ready = false;
      continue;
    }
    const int nblk = (pr.lq + kTileCols - 1) / kTileCols;
    const int ntiles = (pr.ld + kTileRows - 1) / kTileRows;
    float score = 0.0f;
    for (int g0 = 0; g0 < nblk; g0 += QB) {
      // query blocks of this pass that hold tokens (wave-uniform); the last
      // pass of a query can have fewer than QB
      const int nact = min(QB, nblk - g0);
      if (pr.q_row0 != loaded_q || pr.lq != loaded_lq || g0 != loaded_g) {
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          if (qb >= nact) break;
          const int tok = min((g0 + qb) * kTileCols + c, pr.lq - 1);
          const S* row = Q + (pr.q_row0 + tok) * (int64_t)dim;
#pragma unroll
          for (int s = 0; s < KS; ++s)
            qf[qb][s] = load_frag<T>(row, kChunk * s + 8 * h, dim, vec);
        }
        loaded_q = pr.q_row0;
        loaded_lq = pr.lq;
        loaded_g = g0;
      }
      float m[QB];
      int am[QB];
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        m[qb] = -__builtin_inff();
        am[qb] = 0;
      }
      if (!df_ready) load_tile(pr, 0, df);
      df_ready = false;
      // after the last tile of the last pass comes the next pair's tile 0
      const bool hand_over = (g0 + QB >= nblk) && nx.ok;
      // The tile walk for NA active query blocks: a pass with fewer blocks
      // than QB (a query of at most 32 tokens under QB = 2) runs no MFMAs and
      // no epilogue for the empty ones.
      auto walk = [&](auto na_const) __attribute__((always_inline)) {
        constexpr int NA = decltype(na_const)::value;
        for (int t = 0; t < ntiles; ++t) {
          Frag<T> nf[KS];
          const bool more = t + 1 < ntiles;
          if (more)
            load_tile(pr, t + 1, nf);
          else if (hand_over)
            load_tile(nx, 0, nf);
          // rows past the document end were loaded as copies of its last row
          // and cannot win (see tile_update), so no masking is needed
          f32x16 acc[NA];
#pragma unroll
          for (int qb = 0; qb < NA; ++qb) {
            acc[qb] = f32x16{};
#pragma unroll
            for (int s = 0; s < KS; ++s) mma_chunk(df[s], qf[qb][s], acc[qb]);
          }
#pragma unroll
          for (int qb = 0; qb < NA; ++qb)
            tile_update<ARGMAX>(acc[qb], m[qb], am[qb], t * kTileRows + 4 * h);
          if (more || hand_over) {
#pragma unroll
            for (int s = 0; s < KS; ++s) df[s] = nf[s];
          }
        }
      };
      if (QB > 1 && nact == 1)
        walk(std::integral_constant<int, 1>{});
      else
        walk(std::integral_constant<int, QB>{});
      df_ready = hand_over;
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        const int blk = g0 + qb;
        if (blk < nblk) {
          merge_halves(m[qb], am[qb]);
          const int tok = blk * kTileCols + c;
          const bool valid = tok < pr.lq;
          score += half_sum(valid ? m[qb] : 0.0f);
          if (ARGMAX && h == 0 && tok < a.slots)
            a.argmax[p * a.slots + tok] = valid ? am[qb] : 0;
        }
      }
    }
    if (ARGMAX) {
      for (int t = nblk * kTileCols + lane; t < a.slots; t += 64)
        a.argmax[p * a.slots + t] = 0;
    }
    if (lane == kHalfSumLane) a.scores[p] = score;
    pr = nx;
  }
}

// ---------------------------------------------------------------------------
// pair_split_kernel: batches with fewer pairs than the chip has SIMDs, where
// pair_kernel's one wave per pair leaves most SIMDs idle (C1: 128 pairs of
// ten fp32 tiles, each tile 64 MFMAs).  One workgroup of kSplitWaves waves
// per pair: for each query block (one in registers), wave w scores tiles w,
// w + kSplitWaves, ... in order, and the waves' per-token maxima are merged
// in LDS (the larger value; on equal values the lower row).  Every tile gets
// the same MFMAs and epilogue as in pair_kernel, and a wave's tiles come in
// row order, so values, indices and the score sums (same order) are
// bit-identical to pair_kernel's.
// ---------------------------------------------------------------------------
constexpr int kSplitWaves = 4;

template <typename T, int KS, bool ARGMAX, bool VEC>
__global__ __launch_bounds__(kSplitWaves * 64) void pair_split_kernel(FwdArgs a) {
  using S = typename T::storage;
  __shared__ float sm[kSplitWaves][kTileCols];
  __shared__ int sa[kSplitWaves][kTileCols];
  const int lane = threadIdx.x & 63;
  const int c = lane & 31;
  const int h = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int64_t p = blockIdx.x;
  if (p >= a.npairs) return;
  const Pair pr = resolve_pair(a, p);
  if (!pr.ok) {
    if (w == 0) write_invalid_pair(a, p, lane);
    return;
  }
  const S* __restrict__ Q = static_cast<const S*>(a.q);
  const S* __restrict__ D = static_cast<const S*>(a.d);
  const int dim = a.dim;
  const int nblk = (pr.lq + kTileCols - 1) / kTileCols;
  const int ntiles = (pr.ld + kTileRows - 1) / kTileRows;
  auto load_tile = [&](int t, Frag<T> (&f)[KS]) __attribute__((always_inline)) {
    const int r = min(t * kTileRows + c, pr.ld - 1);
    const S* row = D + (pr.d_row0 + r) * (int64_t)dim;
#pragma unroll
    for (int s = 0; s < KS; ++s) f[s] = load_frag<T>(row, kChunk * s + 8 * h, dim, VEC);
  };
  float score = 0.0f;
  for (int blk = 0; blk < nblk; ++blk) {
    Frag<T> qf[KS];
    {
      const int tok = min(blk * kTileCols + c, pr.lq - 1);
      const S* row = Q + (pr.q_row0 + tok) * (int64_t)dim;
#pragma unroll
      for (int s = 0; s < KS; ++s) qf[s] = load_frag<T>(row, kChunk * s + 8 * h, dim, VEC);
    }
    float m = -__builtin_inff();
    int am = 0;
    // this wave's tiles, the next one's fragments loading while one is scored
    Frag<T> df[KS];
    if (w < ntiles) load_tile(w, df);
    for (int t = w; t < ntiles; t += kSplitWaves) {
      Frag<T> nf[KS];
      const bool more = t + kSplitWaves < ntiles;
      if (more) load_tile(t + kSplitWaves, nf);
      f32x16 acc = f32x16{};
#pragma unroll
      for (int s = 0; s < KS; ++s) mma_chunk(df[s], qf[s], acc);
      tile_update<ARGMAX>(acc, m, am, t * kTileRows + 4 * h);
      if (more) {
#pragma unroll
        for (int s = 0; s < KS; ++s) df[s] = nf[s];
      }
    }
    merge_halves(m, am);
    if (h == 0) {
      sm[w][c] = m;
      sa[w][c] = am;
    }
    __syncthreads();
    if (w == 0) {
      m = sm[0][c];
      am = sa[0][c];
#pragma unroll
      for (int v = 1; v < kSplitWaves; ++v) {
        const float mv = sm[v][c];
        const int av = sa[v][c];
        const bool wins = mv > m || (mv == m && av < am);
        m = wins ? mv : m;
        am = wins ? av : am;
      }
      const int tok = blk * kTileCols + c;
      const bool valid = tok < pr.lq;
      score += half_sum(valid ? m : 0.0f);
      if (ARGMAX && h == 0 && tok < a.slots) a.argmax[p * a.slots + tok] = valid ? am : 0;
    }
    __syncthreads();  // the LDS slots are written again for the next block
  }
  if (w == 0) {
    if (ARGMAX) {
      for (int t = nblk * kTileCols + lane; t < a.slots; t += 64) a.argmax[p * a.slots + t] = 0;
    }
    if (lane == kHalfSumLane) a.scores[p] = score;
  }
}

// ---------------------------------------------------------------------------
// wide_pair_kernel: embedding dims above kMaxRegDim, where a query block no
// longer fits in registers.  One wave per pair; each 32x32 tile accumulates
// over all K-chunks with both operands loaded per chunk (the query block is
// re-read from L1/L2 for every document tile), kWideBatch chunks in flight.
// Same tile layout, epilogue and semantics as pair_kernel.
// ---------------------------------------------------------------------------
constexpr int kMaxRegDim = 256;  // pair_kernel / tiled kernel: KS <= 16
constexpr int kWideBatch = 4;

template <typename T, bool ARGMAX, bool VEC>
__global__ __launch_bounds__(256) void wide_pair_kernel(FwdArgs a) {
  using S = typename T::storage;
  const int lane = threadIdx.x & 63;
  const int c = lane & 31;
  const int h = lane >> 5;
  const int64_t p =
      (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  if (p >= a.npairs) return;
  const Pair pr = resolve_pair(a, p);
  if (!pr.ok) {
    write_invalid_pair(a, p, lane);
    return;
  }
  const S* __restrict__ Q = static_cast<const S*>(a.q);
  const S* __restrict__ D = static_cast<const S*>(a.d);
  const int dim = a.dim;
  const int ks = (dim + kChunk - 1) / kChunk;
  const int nblk = (pr.lq + kTileCols - 1) / kTileCols;
  const int ntiles = (pr.ld + kTileRows - 1) / kTileRows;
  float score = 0.0f;
  for (int blk = 0; blk < nblk; ++blk) {
    const int tok = blk * kTileCols + c;
    const S* qrow = Q + (pr.q_row0 + min(tok, pr.lq - 1)) * (int64_t)dim;
    float m = -__builtin_inff();
    int am = 0;
    for (int t = 0; t < ntiles; ++t) {
      // rows past the document end repeat its last row and cannot win
      const S* drow = D + (pr.d_row0 + min(t * kTileRows + c, pr.ld - 1)) * (int64_t)dim;
      f32x16 acc = f32x16{};
      for (int s0 = 0; s0 < ks; s0 += kWideBatch) {
        Frag<T> fa[kWideBatch], fb[kWideBatch];
#pragma unroll
        for (int u = 0; u < kWideBatch; ++u) {
          const int k0 = kChunk * (s0 + u) + 8 * h;
          const bool in = s0 + u < ks;
          fa[u] = in ? load_frag<T>(drow, k0, dim, VEC) : zero_frag<T>();
          fb[u] = in ? load_frag<T>(qrow, k0, dim, VEC) : zero_frag<T>();
        }
#pragma unroll
        for (int u = 0; u < kWideBatch; ++u)
          if (s0 + u < ks) mma_chunk(fa[u], fb[u], acc);
      }
      tile_update<ARGMAX>(acc, m, am, t * kTileRows + 4 * h);
    }
    merge_halves(m, am);
    const bool valid = tok < pr.lq;
    score += half_sum(valid ? m : 0.0f);
    if (ARGMAX && h == 0 && tok < a.slots) a.argmax[p * a.slots + tok] = valid ? am : 0;
  }
  if (ARGMAX) {
    for (int t = nblk * kTileCols + lane; t < a.slots; t += 64) a.argmax[p * a.slots + t] = 0;
  }
  if (lane == kHalfSumLane) a.scores[p] = score;
}

// ---------------------------------------------------------------------------
// contrastive_tiled_kernel
// ---------------------------------------------------------------------------
// Workgroup = 8 waves.  Wave w holds NBW query blocks: queries
// [q0 + w*qpw, q0 + (w+1)*qpw), each of nblk = ceil(Lq/32) blocks, with
// qpw * nblk <= NBW.  The workgroup walks the 32-row tiles of its chunk of
// documents in order through a ring of four LDS buffers: tile k+4 is loaded
// straight from global memory into LDS while tile k+2's operand fragments are
// read into registers and tile k+1's MFMAs run, so the max/argmax epilogue of
// tile k overlaps the MFMAs of tile k+1.  In LDS a tile is 32 rows of 16-byte
// pieces; the piece index is XOR-swizzled with the row so the operand reads
// (one row per lane) are bank-conflict free.  Requires dim == KS*16 and
// 16-byte aligned rows (the host routes other shapes to pair_kernel).
constexpr int kTiledWaves = 8;
constexpr int kTiledThreads = kTiledWaves * 64;
constexpr int kTileBuffers = 4;        // LDS tile ring
constexpr int kMaxDocsPerGroup = 2048;  // LDS document list per workgroup
constexpr int kDocTableBytes = 3 * (int)sizeof(int) * kMaxDocsPerGroup;  // rows, end, id
constexpr int kDocWork = 32;            // work of a document beyond its rows, in rows
constexpr int kLptKeys = 128;           // sort keys of the dealt lists: tile counts, clamped
// Dealt lists when chunks average fewer documents than this: with 8 per
// chunk (64 queries x 512 C5 documents) contiguous chunks of whole documents
// hold up to 17 % more tiles than the mean (forward 139.6 -> 128.4 us
// dealt); with 64 (C5) within 2 %, and the ranking costs more (952.7 against
// 955 us)
constexpr int kDealtBelowDocsPerChunk = 32;

struct TiledArgs {
  const void* q;
  const void* d;
  const int32_t* doff;
  int64_t nq;
  int64_t nb;
  int64_t total_d;
  int lq;
  int dim;
  int nblk;   // blocks per query
  int qpw;    // queries per wave
  int n_qg;   // query groups
  int n_dc;   // document chunks
  float* scores;
  int32_t* argmax;
};

// One 16-byte piece per lane from global memory straight into LDS
// (global_load_lds_dwordx4): lane i of the wave writes bytes
// [16*i, 16*i + 16) after `dst`, which must be wave-uniform.  Written as
// inline asm so the compiler does not pair every later LDS read with a
// conservative wait for all loads in flight; the kernel orders these loads
// itself (s_waitcnt vmcnt + s_barrier).  Loads complete in issue order, so
// the compiler's own vmcnt waits stay correct (they can only get stricter).
// The same value, opaque to the optimiser (an empty asm statement): address
// arithmetic that depends on it cannot be hoisted out of the loop, where it
// would keep 64-bit per-lane pointers live across the whole tile walk.
__device__ __forceinline__ int opaque(int v) {
  __asm__ __volatile__("" : "+v"(v));
  return v;
}


template <typename T, int KS>
struct TileGeom {
  static constexpr int kPieceElems = 16 / T::bytes;         // elements / 16 B
  static constexpr int P = KS * kChunk / kPieceElems;       // pieces per row
  static constexpr int SWZ = (P < 16 ? P : 16) - 1;
  static constexpr int kPieces = kTileRows * P;             // per tile
  static constexpr int NP = (kPieces + kTiledThreads - 1) / kTiledThreads;
  static constexpr int kBufPieces = kPieces;                // uint4 per buffer
};

// Position in the (document, tile) walk of a workgroup.  All fields are
// wave-uniform 32-bit values (document offsets are int32), so the walk stays
// in scalar registers.
struct TileCursor {
  int b;          // entry of the workgroup's document list
  int row0;       // its first row
  int ld;         // its length (0 when past the end)
  int t;          // tile within the document
  int id;         // its document index
};

template <typename T, int KS, int NBW, bool ARGMAX>
__global__ __launch_bounds__(kTiledThreads) void contrastive_tiled_kernel(TiledArgs a) {
  using S = typename T::storage;
  using G = TileGeom<T, KS>;
  extern __shared__ uint4 lds[];  // [4][32][P]

  // XCD-aware mapping: consecutive hardware workgroup ids go round-robin over
  // the 8 XCDs; give each XCD a contiguous range of logical ids, ordered
  // query-group fastest, so the workgroups sharing a doc chunk share an L2.
  const int64_t total = (int64_t)a.n_qg * a.n_dc;
  const int64_t per_xcd = gridDim.x / 8;
  const int64_t L = (int64_t)(blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  if (L >= total) return;
  const int qg = (int)(L % a.n_qg);
  const int dc = (int)(L / a.n_qg);

  const int tid = threadIdx.x;
  // wave-uniform; readfirstlane tells the compiler so, which keeps every
  // query index and output address derived from it in scalar registers
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int c = lane & 31;
  const int h = lane >> 5;
  const S* __restrict__ Q = static_cast<const S*>(a.q);
  const S* __restrict__ D = static_cast<const S*>(a.d);
  const int dim = a.dim;

  // ---- query blocks of this wave -> registers
  const int64_t q_first = ((int64_t)qg * kTiledWaves + wave) * a.qpw;
  Frag<T> qf[NBW][KS];
#pragma unroll
  for (int j = 0; j < NBW; ++j) {
    const int64_t q = min(q_first + j / a.nblk, a.nq - 1);
    const int part = j % a.nblk;
    const int tok = min(part * kTileCols + c, a.lq - 1);
    const S* row = Q + (q * a.lq + tok) * (int64_t)dim;
#pragma unroll
    for (int s = 0; s < KS; ++s)
      qf[j][s] = load_frag<T>(row, kChunk * s + 8 * h, dim, true);
  }

  // The documents of chunk dc, as a list in LDS (rows [s, e) and index of
  // entry bl).  Two ways to form the chunks:
  //  * dealt (more than one chunk, fewer than kDealtBelowDocsPerChunk
  //    documents per chunk on average, at most one document per thread):
  //    the documents sorted by tile count, longest
  //    first (ties by index), and dealt in snake order, place p of round r
  //    to chunk p (r even) or n_dc - 1 - p (r odd), so every chunk gets a
  //    near-equal share of the tiles whatever the lengths.  Every workgroup
  //    ranks all documents itself (the same ranks everywhere): one thread
  //    per document, RankScratch (a mask per wave and key set by LDS atomic
  //    ORs, then a scan over the keys);
  //  * contiguous: the documents whose work prefix W(b) = off[b] + kDocWork
  //    * b falls in [dc, dc + 1) * W / n_dc, W = total_d + kDocWork * nb
  //    (rows, plus one tile's worth per document for its last partial tile
  //    and its document-end work), so chunks hold equal work, not equal
  //    counts.  The bounds are counts of documents below each threshold, one
  //    parallel pass over the offsets; counts partition [0, nb) for any
  //    offsets.
  float* __restrict__ scores = a.scores;
  int32_t* __restrict__ argmax_out = a.argmax;
  int* tab_s = reinterpret_cast<int*>(lds + kTileBuffers * G::kBufPieces);
  int* tab_e = tab_s + kMaxDocsPerGroup;
  int* tab_id = tab_e + kMaxDocsPerGroup;
  int n_docs = 0;
  if (a.n_dc > 1 && a.n_dc < a.nb && a.nb <= kTiledThreads &&
      a.nb < (int64_t)kDealtBelowDocsPerChunk * a.n_dc) {
    // scratch in the tile ring, which no load has touched yet (half the
    // keys where the ring is small: 32-element rows)
    constexpr int kRing = kTileBuffers * G::kBufPieces * (int)sizeof(uint4);
    constexpr int kKeys =
        RankScratch<kTiledWaves, kLptKeys>::kBytes <= kRing ? kLptKeys : kLptKeys / 2;
    using Rank = RankScratch<kTiledWaves, kKeys>;
    static_assert(Rank::kBytes <= kRing, "ranking scratch fits the tile ring");
    const Rank rs(lds);
    rs.clear();
    const bool own = tid < a.nb;
    int s0 = 0, e0 = 0, key = 0;
    if (own) {
      s0 = a.doff[tid];
      e0 = a.doff[tid + 1];
      const bool ok = (s0 >= 0) && (e0 > s0) && ((int64_t)e0 <= a.total_d);
      const int t = ok ? (e0 - s0 + kTileRows - 1) / kTileRows : 0;
      key = t < kKeys - 1 ? t : kKeys - 1;
    }
    const int r = rs.rank(own, key);
    const int nc = a.n_dc, nbd = (int)a.nb;
    if (own) {
      const int rd = r / nc, p = r - rd * nc;
      if (((rd & 1) ? nc - 1 - p : p) == dc) {
        tab_s[rd] = s0;
        tab_e[rd] = e0;
        tab_id[rd] = tid;
      }
    }
    const int full = nbd / nc, tail = nbd - full * nc;
    n_docs = full + (tail > 0 && ((full & 1) ? nc - 1 - dc : dc) < tail ? 1 : 0);
  } else {
    __shared__ int chunk_cnt[2];
    if (threadIdx.x < 2) chunk_cnt[threadIdx.x] = 0;
    __syncthreads();
    if (a.n_dc >= a.nb) {
      // one document per chunk: nothing to balance
      if (threadIdx.x == 0) {
        chunk_cnt[0] = dc;
        chunk_cnt[1] = (int)min((int64_t)dc + 1, a.nb);
      }
    } else {
      const int64_t w_all = a.total_d + (int64_t)kDocWork * a.nb;
      const int64_t w_lo = w_all * dc / a.n_dc;
      const int64_t w_hi = w_all * (dc + 1) / a.n_dc;
      int c_lo = 0, c_hi = 0;
      for (int64_t bb = threadIdx.x; bb < a.nb; bb += kTiledThreads) {
        const int64_t w = (int64_t)a.doff[bb] + (int64_t)kDocWork * bb;
        c_lo += w < w_lo ? 1 : 0;
        c_hi += w < w_hi ? 1 : 0;
      }
      if (c_lo) atomicAdd(&chunk_cnt[0], c_lo);
      if (c_hi) atomicAdd(&chunk_cnt[1], c_hi);
    }
    __syncthreads();
    const int64_t b_begin = dc == 0 ? 0 : chunk_cnt[0];
    const int64_t b_end = dc == a.n_dc - 1 ? a.nb : chunk_cnt[1];
    // With non-decreasing offsets consecutive documents are kDocWork apart
    // in W, so the host's chunk count keeps every chunk within the list.
    // Only offsets that decrease or overrun total_d can break that; such a
    // chunk is reported like documents with invalid offsets.
    if (b_end - b_begin > kMaxDocsPerGroup) {
      for (int64_t b = b_begin; b < b_end; ++b) {
#pragma unroll
        for (int j = 0; j < NBW; ++j) {
          const int64_t q = q_first + j / a.nblk;
          if (j >= a.qpw * a.nblk || q >= a.nq) continue;
          const int tok = (j % a.nblk) * kTileCols + c;
          if (ARGMAX && argmax_out && h == 0 && tok < a.lq) argmax_out[(q * a.nb + b) * a.lq + tok] = 0;
          if (j % a.nblk == 0 && lane == 0) scores[q * a.nb + b] = __builtin_nanf("");
        }
      }
      return;
    }
    n_docs = (int)(b_end - b_begin);
    for (int i = tid; i < n_docs; i += kTiledThreads) {
      tab_s[i] = a.doff[b_begin + i];
      tab_e[i] = a.doff[b_begin + i + 1];
      tab_id[i] = (int)(b_begin + i);
    }
  }
  // The list is in LDS once, so the tile walk never issues global loads of
  // its own: the only vector-memory loads in flight are the tile loads,
  // whose completion is tracked by count.
  __syncthreads();
  // Offsets of local document bl (uniform: read back as scalars).
  auto doc_ok = [&](int bl, int& s0, int& ld) {
    const int s = __builtin_amdgcn_readfirstlane(tab_s[bl]);
    const int e = __builtin_amdgcn_readfirstlane(tab_e[bl]);
    s0 = s;
    ld = e - s;
    return (s >= 0) && (e > s) && ((int64_t)e <= a.total_d);
  };
  // One pass over the list, a lane per entry: the tiles to walk, and the
  // documents with invalid offsets (NaN score, zero argmax, never read).
  int ntiles = 0;
  for (int bl0 = 0; bl0 < n_docs; bl0 += 64) {
    const int bl = bl0 + lane;
    bool bad = false;
    if (bl < n_docs) {
      const int s = tab_s[bl], e = tab_e[bl];
      if ((s >= 0) && (e > s) && ((int64_t)e <= a.total_d))
        ntiles += (e - s + kTileRows - 1) / kTileRows;
      else
        bad = true;
    }
    for (uint64_t mb = __ballot(bad); mb; mb &= mb - 1) {
      const int64_t b = __builtin_amdgcn_readfirstlane(tab_id[bl0 + __ffsll((unsigned long long)mb) - 1]);
#pragma unroll
      for (int j = 0; j < NBW; ++j) {
        const int64_t q = q_first + j / a.nblk;
        if (j >= a.qpw * a.nblk || q >= a.nq) continue;
        const int tok = (j % a.nblk) * kTileCols + c;
        if (ARGMAX && argmax_out && h == 0 && tok < a.lq) argmax_out[(q * a.nb + b) * a.lq + tok] = 0;
        if (j % a.nblk == 0 && lane == 0) scores[q * a.nb + b] = __builtin_nanf("");
      }
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) ntiles += __shfl_xor(ntiles, o);
  ntiles = __builtin_amdgcn_readfirstlane(ntiles);
  // First valid document at or after local index bl (cursor at its tile 0).
  auto seek = [&](int bl) -> TileCursor {
    TileCursor cur{n_docs, 0, 0, 0, 0};
    for (; bl < n_docs; ++bl) {
      int s0;
      int ld;
      if (doc_ok(bl, s0, ld)) {
        cur.b = bl;
        cur.row0 = s0;
        cur.ld = ld;
        cur.id = __builtin_amdgcn_readfirstlane(tab_id[bl]);
        break;
      }
    }
    return cur;
  };
  auto advance = [&](TileCursor cur) -> TileCursor {
    if (cur.b >= n_docs) return cur;
    if ((cur.t + 1) * kTileRows < cur.ld) {
      ++cur.t;
      return cur;
    }
    return seek(cur.b + 1);
  };

  // ---- software pipeline
  // LDS holds kNB = 4 tile buffers filled by direct global->LDS loads
  // (global_load_lds_dwordx4: each lane moves one 16-byte piece, a wave
  // instruction fills 1 KB of a buffer; the swizzle is applied by choosing
  // the source address of each slot).  Step k:
  //   (0) issue the first MFMAs of tile k+1 (operands already in registers);
  //   (1) on even k only: wait until this wave's loads of tiles k+2 and k+3
  //       have landed, barrier -- now every wave's loads of both tiles are
  //       in LDS and every wave has finished reading the buffers of tiles k
  //       and k+1 (read two steps earlier, in steps k-2 and k-1) -- and
  //       issue the loads of tiles k+4 and k+5 into those two buffers;
  //   (2) issue the rest of tile k+1's MFMAs into one accumulator set, and
  //       read tile k+2's fragments;
  //   (3) run the max/argmax epilogue of tile k from the other set -- its
  //       VALU work and the LDS reads are interleaved with the MFMAs;
  //   (4) advance the load and epilogue cursors.
  // Loads have two steps to land and operand reads a whole step; no
  // registers are spent on global->LDS staging.  One barrier every two steps
  // (rather than every step) halves the time waves spend waiting for the
  // slowest one; the MFMAs issued before it keep the matrix pipe busy
  // meanwhile.  Vector-memory loads complete in issue order.
  if (ntiles == 0) return;

  constexpr int kNB = kTileBuffers;
  constexpr int kDmaPerTile = G::kPieces / 64;  // wave instructions per tile
  static_assert(G::kPieces % 64 == 0, "tile must be whole wave loads");
  // wave w issues instructions j = w, w + 8, ...; d_w of them per tile
  const int d_w = (kDmaPerTile - wave + kTiledWaves - 1) / kTiledWaves;
  // Per-lane part of each load slot, fixed for the whole walk: the slot's
  // row within the tile and its byte offset within that row (swizzled
  // piece); the LDS destination of wave instruction j is a constant.
  constexpr int kDmaIters = (kDmaPerTile + kTiledWaves - 1) / kTiledWaves;
  int slot_row[kDmaIters];
  uint32_t slot_byte[kDmaIters];
#pragma unroll
  for (int i = 0; i < kDmaIters; ++i) {
    const int slot = (wave + i * kTiledWaves) * 64 + lane;
    const int r = slot / G::P;
    slot_row[i] = r;
    slot_byte[i] = (uint32_t)(((slot - r * G::P) ^ (r & G::SWZ)) * 16);
  }
  const uint32_t row_bytes = (uint32_t)dim * (uint32_t)sizeof(S);
  const uint32_t lds_base = __builtin_amdgcn_readfirstlane(lds_addr(lds));
  auto dma_tile = [&](auto buf_const, const TileCursor& cur) __attribute__((always_inline)) {
    constexpr int BUF = decltype(buf_const)::value;
    if (cur.b >= n_docs) return;
    // uniform tile base; rows past the document end repeat its last row
    const S* base = D + (int64_t)(cur.row0 + cur.t * kTileRows) * dim;
    const int last = cur.ld - 1 - cur.t * kTileRows;
#pragma unroll
    for (int i = 0; i < kDmaIters; ++i) {
      const int j = wave + i * kTiledWaves;
      if (j < kDmaPerTile)
        lds_dma16(base, (uint32_t)min(slot_row[i], last) * row_bytes + slot_byte[i],
                  lds_base + (uint32_t)((BUF * G::kBufPieces + j * 64) * sizeof(uint4)));
    }
  };
  // s_waitcnt vmcnt(n) for the runtime n in {0, 1, 2, 3, 4, 6}; other waits
  // fall back to vmcnt(0).  Encoding (gfx9): vmcnt[3:0] | expcnt[6:4] = 7 |
  // lgkmcnt[11:8] = 15 | vmcnt[5:4] << 14.
  auto wait_vm = [&](int n) __attribute__((always_inline)) {
    switch (n) {
      case 1: __builtin_amdgcn_s_waitcnt(0x0F71); break;
      case 2: __builtin_amdgcn_s_waitcnt(0x0F72); break;
      case 3: __builtin_amdgcn_s_waitcnt(0x0F73); break;
      case 4: __builtin_amdgcn_s_waitcnt(0x0F74); break;
      case 6: __builtin_amdgcn_s_waitcnt(0x0F76); break;
      default: __builtin_amdgcn_s_waitcnt(0x0F70); break;
    }
  };

  // s_barrier without a memory fence (a fence would wait for every load in
  // flight); the empty asm statements keep the compiler from moving memory
  // accesses across it.
  auto barrier = [&]() __attribute__((always_inline)) {
    __asm__ __volatile__("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    __asm__ __volatile__("" ::: "memory");
  };

  // per-lane LDS element offsets of this lane's A fragments in buffer 0
  int aoff[KS * (T::bytes == 2 ? 1 : 2)];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    if constexpr (T::bytes == 2) {
      aoff[s] = c * G::P + ((2 * s + h) ^ (c & G::SWZ));
    } else {
      aoff[2 * s] = c * G::P + ((4 * s + 2 * h) ^ (c & G::SWZ));
      aoff[2 * s + 1] = c * G::P + ((4 * s + 2 * h + 1) ^ (c & G::SWZ));
    }
  }
  auto read_frags = [&](auto buf_const, Frag<T> (&df)[KS]) __attribute__((always_inline)) {
    constexpr int BUF = decltype(buf_const)::value;
    const uint4* tile = lds + BUF * G::kBufPieces;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      if constexpr (T::bytes == 2) {
        df[s].v = tile[aoff[s]];
      } else {
        df[s].lo = tile[aoff[2 * s]];
        df[s].hi = tile[aoff[2 * s + 1]];
      }
    }
  };
  // A tile's NBW * KS MFMAs, issued chain-interleaved (MFMA p accumulates
  // into block p % NBW, chunk p / NBW), so consecutive MFMAs are independent.
  // The first kPreMfma are issued before the step's wait and barrier (they
  // only read registers): the matrix pipe then has work while the waves
  // synchronise and issue the scalar work that follows the barrier.  Three
  // of each block's chunks measured best (one or two: 1-2 % slower).
  constexpr int kPreMfma = (3 * NBW < NBW * KS) ? 3 * NBW : NBW * KS;
  auto mfma_range = [&](auto lo_c, auto hi_c, const Frag<T> (&df)[KS],
                        f32x16 (&acc)[NBW]) __attribute__((always_inline)) {
#pragma unroll
    for (int p = decltype(lo_c)::value; p < decltype(hi_c)::value; ++p) {
      const int j = p % NBW;
      const int s = p / NBW;
      if (s == 0) acc[j] = f32x16{};
      mma_chunk(df[s], qf[j][s], acc[j]);
    }
  };
  auto mfma_pre = [&](const Frag<T> (&df)[KS], f32x16 (&acc)[NBW]) __attribute__((always_inline)) {
    mfma_range(std::integral_constant<int, 0>{}, std::integral_constant<int, kPreMfma>{}, df, acc);
  };
  auto mfma_rest = [&](const Frag<T> (&df)[KS], f32x16 (&acc)[NBW]) __attribute__((always_inline)) {
    mfma_range(std::integral_constant<int, kPreMfma>{}, std::integral_constant<int, NBW * KS>{},
               df, acc);
  };

  float m[NBW];
  int am[NBW];
  int bt[NBW];        // base row of the tile holding the running max (< 0: none)
  f32x16 best[NBW];   // that tile's values (index search deferred to the doc end)
#pragma unroll
  for (int j = 0; j < NBW; ++j) {
    m[j] = -__builtin_inff();
    am[j] = 0;
    bt[j] = -1;
    best[j] = f32x16{};
  }
  auto epilogue = [&](f32x16 (&acc)[NBW], const TileCursor& cur) __attribute__((always_inline)) {
    const int valid = cur.ld - cur.t * kTileRows;
    const int row_base = cur.t * kTileRows + 4 * h;
#pragma unroll
    for (int j = 0; j < NBW; ++j) {
      if constexpr (ARGMAX)
        tile_update_deferred(acc[j], m[j], bt[j], best[j], row_base);
      else
        tile_update<false>(acc[j], m[j], am[j], row_base);
    }
    // Interleave the epilogue's VALU work and the operand reads for the tile
    // after next with the next tile's MFMAs, so one wave keeps the MFMA,
    // VALU and LDS pipes busy at once.
#pragma unroll
    for (int i = 0; i < NBW * KS * (T::bytes == 2 ? 1 : 8); ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (i < KS * (T::bytes == 2 ? 1 : 2)) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, ARGMAX ? 5 : 2, 0);
    }
    if (valid <= kTileRows) {  // last tile of the document
      float part_sum = 0.0f;
#pragma unroll
      for (int j = 0; j < NBW; ++j) {
        const int part = j % a.nblk;
        const int64_t q = q_first + j / a.nblk;
        if constexpr (ARGMAX) am[j] = best_row(best[j], m[j], bt[j]);
        merge_halves(m[j], am[j]);
        const int tok = part * kTileCols + opaque(c);
        const bool vtok = tok < a.lq;
        const float sm = half_sum(vtok ? m[j] : 0.0f);
        part_sum = (part == 0) ? sm : part_sum + sm;
        if ((j < a.qpw * a.nblk) && (q < a.nq)) {
          if (ARGMAX && argmax_out && h == 0 && vtok) argmax_out[(q * a.nb + cur.id) * a.lq + tok] = am[j];
          if (part == a.nblk - 1 && lane == kHalfSumLane) scores[q * a.nb + cur.id] = part_sum;
        }
        m[j] = -__builtin_inff();
        am[j] = 0;
        bt[j] = -1;
      }
    }
  };

  // ---- prologue: loads of tiles 0..3 issued; fragments of tiles 0 and 1
  // in registers; tile 0's MFMAs issued
  TileCursor cc = seek(0);            // tile k (epilogue)
  TileCursor fc = cc;                 // next tile to load
  static_assert(kNB == 4, "prologue issues four tile loads");
  dma_tile(std::integral_constant<int, 0>{}, fc);
  fc = advance(fc);
  dma_tile(std::integral_constant<int, 1>{}, fc);
  fc = advance(fc);
  dma_tile(std::integral_constant<int, 2>{}, fc);
  fc = advance(fc);
  dma_tile(std::integral_constant<int, 3>{}, fc);
  fc = advance(fc);
  wait_vm(ntiles >= kNB ? (kNB - 2) * d_w : 0);
  barrier();
  Frag<T> fr0[KS], fr1[KS];
  f32x16 acc0[NBW], acc1[NBW];
  read_frags(std::integral_constant<int, 0>{}, fr0);
  read_frags(std::integral_constant<int, 1>{}, fr1);
  mfma_pre(fr0, acc0);
  mfma_rest(fr0, acc0);

  // Step k (U = k % 4): fragments of tile k+1 are in registers, tile k's
  // MFMA results in the other accumulator set.
  int k = 0;
  auto step = [&](auto u_const) __attribute__((always_inline)) -> bool {
    constexpr int U = decltype(u_const)::value;
    f32x16 (&acc_cur)[NBW] = (U % 2 == 0) ? acc0 : acc1;
    f32x16 (&acc_nxt)[NBW] = (U % 2 == 0) ? acc1 : acc0;
    Frag<T> (&fr_nxt)[KS] = (U % 2 == 0) ? fr1 : fr0;   // tile k+1
    Frag<T> (&fr_new)[KS] = (U % 2 == 0) ? fr0 : fr1;   // <- tile k+2
    mfma_pre(fr_nxt, acc_nxt);
    if constexpr (U % 2 == 0) {
      // tiles k+2 and k+3 resident (every load of this wave landed), then
      // tiles k+4 and k+5 -> the buffers of tiles k and k+1
      wait_vm(0);
      barrier();
      dma_tile(u_const, fc);
      dma_tile(std::integral_constant<int, U + 1>{}, advance(fc));
    }
    // Past the last tile these reads and MFMAs see stale buffers; their
    // results are never used, and every wave keeps the same barrier count.
    read_frags(std::integral_constant<int, (U + 2) % kNB>{}, fr_new);
    mfma_rest(fr_nxt, acc_nxt);
    epilogue(acc_cur, cc);
    if (k + 1 >= ntiles) return true;
    // The cursor walks (scalar code with branches, document offsets read
    // from LDS) come after the MFMAs and the epilogue, off the path from
    // the barrier to the matrix pipe.
    fc = advance(fc);
    cc = advance(cc);
    ++k;
    return false;
  };
  while (true) {
    if (step(std::integral_constant<int, 0>{})) break;
    if (step(std::integral_constant<int, 1>{})) break;
    if (step(std::integral_constant<int, 2>{})) break;
    if (step(std::integral_constant<int, 3>{})) break;
  }
  // drain: no load may still be writing LDS when the workgroup exits
  __builtin_amdgcn_s_waitcnt(0x0F70);
}

// ---------------------------------------------------------------------------
// pair_ring_kernel: pair_kernel's work split (one wave per run of `ppw`
// pairs, queries of at most two 32-token blocks in registers) with the
// document tiles brought in by direct global->LDS loads into two
// wave-private LDS slots, two tiles ahead, in place of pair_kernel's one tile
// ahead in registers.  Packed pairs and padded candidates miss L2 on nearly
// every tile and the MFMA pipe is mostly idle, so the time is the latency of
// the tile loads: twice the tiles in flight per wave, at no register cost
// (the staging registers are freed).  The load stream runs across pairs:
// the next pair's first tiles load during the current pair's last ones.
// Vector-memory operations complete in order, so any other load would make
// its wait a wait for every tile load before it: a pair's query blocks come
// through the same stream (a query block is a 32-row tile of the same
// layout, read into the B fragments), and the wave's pair metadata is
// resolved once, one pair per lane, and read back with readlane.
// No barriers: each wave owns its slots.  Same MFMA order and tile epilogue
// as pair_kernel, so the results are bit-identical.
// ---------------------------------------------------------------------------
constexpr int kRingSlots = 2;
// 8 waves (128 KB of slots) per workgroup, one workgroup per CU: against 4
// waves (two workgroups per CU), C3 1.70-1.72 against 1.73-1.74 ms.
constexpr int kRingWaves = 8;

// STREAM (padded launches): every candidate row is read by exactly one pair,
// so document tiles are loaded non-temporally; query units, re-read by the
// query's other candidates, and the packed layout's documents, shared by
// pairs, keep the default policy.  C3: 1710 -> 1585 us (1618 us with the
// query units non-temporal too); C4 with non-temporal tiles: 197 -> 214 us.
template <typename T, int KS, bool ARGMAX, bool STREAM>
__global__ __launch_bounds__(kRingWaves * 64) void pair_ring_kernel(FwdArgs a, int ppw) {
  using S = typename T::storage;
  using G = TileGeom<T, KS>;
  static_assert(T::bytes == 2, "16-bit operands: one 16-byte piece per fragment");
  constexpr int QB = 2;
  constexpr int kRPI = 64 / G::P;          // tile rows per wave load instruction
  constexpr int kDma = G::kPieces / 64;    // wave load instructions per tile
  extern __shared__ uint4 lds[];
  const int lane = threadIdx.x & 63;
  const int c = lane & 31;
  const int h = lane >> 5;
  const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int64_t wave = (int64_t)blockIdx.x * kRingWaves + wv;
  const int64_t p_begin = wave * ppw;
  if (p_begin >= a.npairs) return;
  const int64_t p_end = min(p_begin + (int64_t)ppw, a.npairs);
  const S* __restrict__ Q = static_cast<const S*>(a.q);
  const S* __restrict__ D = static_cast<const S*>(a.d);
  const int dim = a.dim;
  const uint32_t row_bytes = (uint32_t)dim * (uint32_t)sizeof(S);
  const uint4* ring = lds + (size_t)wv * kRingSlots * G::kBufPieces;
  const uint32_t ring_lds = __builtin_amdgcn_readfirstlane(lds_addr(ring));
  // lane -> (row within an instruction's rows, piece); slot i*64 + lane of a
  // tile holds piece (lo ^ (row & SWZ)) of row i*kRPI + hi
  const int l_hi = lane / G::P;
  const int l_lo = lane - l_hi * G::P;
  int aoff[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) aoff[s] = c * G::P + ((2 * s + h) ^ (c & G::SWZ));

  // ---- pair metadata: lane i resolves pair p_begin + i once (ppw <= 64,
  // the host's bound), and the walks below read it back with readlane, so
  // no metadata load sits between the tile loads in flight and their waits
  // (vector-memory operations complete in order: waiting for such a load
  // would wait for every tile load issued before it)
  const int npw = (int)(p_end - p_begin);
  Pair mine{0, 0, 0, 0, false};
  if (lane < npw) mine = resolve_pair(a, p_begin + lane);
  auto pair_at = [&](int i) __attribute__((always_inline)) {
    Pair r;
    const uint32_t qlo = __builtin_amdgcn_readlane((int)(uint32_t)mine.q_row0, i);
    const uint32_t qhi = __builtin_amdgcn_readlane((int)(mine.q_row0 >> 32), i);
    const uint32_t dlo = __builtin_amdgcn_readlane((int)(uint32_t)mine.d_row0, i);
    const uint32_t dhi = __builtin_amdgcn_readlane((int)(mine.d_row0 >> 32), i);
    r.q_row0 = (int64_t)(((uint64_t)qhi << 32) | qlo);
    r.d_row0 = (int64_t)(((uint64_t)dhi << 32) | dlo);
    r.lq = __builtin_amdgcn_readlane(mine.lq, i);
    r.ld = __builtin_amdgcn_readlane(mine.ld, i);
    r.ok = __builtin_amdgcn_readlane(mine.ok ? 1 : 0, i) != 0;
    return r;
  };

  // ---- load stream: for each valid pair in order, its query blocks (32
  // token rows each, the B operands), then its document tiles; each unit is
  // one 32-row tile of 16-byte pieces, swizzled alike, in the next slot
  int li = 0;        // pair of the next unit
  int lu = 0;        // unit within that pair
  Pair lpr = pair_at(0);
  while (!lpr.ok && ++li < npw) lpr = pair_at(li);
  int issued = 0;    // units whose loads were issued
  auto dma_next = [&]() __attribute__((always_inline)) {
    if (li >= npw) return;
    const int slot = issued % kRingSlots;
    const int nblk = (lpr.lq + kTileCols - 1) / kTileCols;
    const int ntiles = (lpr.ld + kTileRows - 1) / kTileRows;
    const bool isq = lu < nblk;
    const int t = isq ? lu : lu - nblk;
    const S* base = isq ? Q + (lpr.q_row0 + (int64_t)t * kTileCols) * dim
                        : D + (lpr.d_row0 + (int64_t)t * kTileRows) * dim;
    const int last = (isq ? lpr.lq : lpr.ld) - 1 - t * kTileRows;
#pragma unroll
    for (int i = 0; i < kDma; ++i) {
      const int r = i * kRPI + l_hi;
      const uint32_t off = (uint32_t)min(r, last) * row_bytes +
                           (uint32_t)((l_lo ^ (r & G::SWZ)) * 16);
      const uint32_t dst = ring_lds + (uint32_t)((slot * G::kBufPieces + i * 64) * sizeof(uint4));
      if (STREAM && !isq)
        lds_dma16_nt(base, off, dst);
      else
        lds_dma16(base, off, dst);
    }
    ++issued;
    if (++lu >= nblk + ntiles) {
      lu = 0;
      do {
        ++li;
      } while (li < npw && !(lpr = pair_at(li)).ok);
    }
  };
  // s_waitcnt vmcnt(n), n = kDma (the next unit's loads may be outstanding) or 0
  auto wait_tile = [&](bool next_issued) __attribute__((always_inline)) {
    if (next_issued) {
      if constexpr (kDma == 8) __builtin_amdgcn_s_waitcnt(0x0F78);
      else if constexpr (kDma == 4) __builtin_amdgcn_s_waitcnt(0x0F74);
      else if constexpr (kDma == 2) __builtin_amdgcn_s_waitcnt(0x0F72);
      else __builtin_amdgcn_s_waitcnt(0x0F70);
    } else {
      __builtin_amdgcn_s_waitcnt(0x0F70);
    }
    __asm__ __volatile__("" ::: "memory");
  };
  // the unit's slot has been read into registers: refill it with the unit
  // two ahead (lgkmcnt(0): the reads have completed)
  auto refill = [&]() __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __asm__ __volatile__("" ::: "memory");
    dma_next();
  };
  dma_next();
  dma_next();

  Frag<T> qf[QB][KS];
  int k = 0;  // stream index of the unit being consumed
  for (int i = 0; i < npw; ++i) {
    const int64_t p = p_begin + i;
    const Pair pr = pair_at(i);
    if (!pr.ok) {
      write_invalid_pair(a, p, lane);
      continue;
    }
    const int nblk = (pr.lq + kTileCols - 1) / kTileCols;  // <= QB (host checks)
    const int ntiles = (pr.ld + kTileRows - 1) / kTileRows;
    // query blocks from the stream: the same layout as a document tile, so
    // lane c reads token c's fragments (rows past the query end repeat its
    // last token, as the register loads did)
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      if (qb >= nblk) break;
      wait_tile(issued > k + 1);
      const uint4* tile = ring + (k % kRingSlots) * G::kBufPieces;
#pragma unroll
      for (int s = 0; s < KS; ++s) qf[qb][s].v = tile[aoff[s]];
      ++k;
      refill();
    }
    float m[QB];
    int am[QB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      m[qb] = -__builtin_inff();
      am[qb] = 0;
    }
    auto walk = [&](auto na_const) __attribute__((always_inline)) {
      constexpr int NA = decltype(na_const)::value;
      for (int t = 0; t < ntiles; ++t, ++k) {
        wait_tile(issued > k + 1);
        const uint4* tile = ring + (k % kRingSlots) * G::kBufPieces;
        Frag<T> df[KS];
#pragma unroll
        for (int s = 0; s < KS; ++s) df[s].v = tile[aoff[s]];
        f32x16 acc[NA];
#pragma unroll
        for (int qb = 0; qb < NA; ++qb) {
          acc[qb] = f32x16{};
#pragma unroll
          for (int s = 0; s < KS; ++s) mma_chunk(df[s], qf[qb][s], acc[qb]);
        }
        refill();
#pragma unroll
        for (int qb = 0; qb < NA; ++qb)
          tile_update<ARGMAX>(acc[qb], m[qb], am[qb], t * kTileRows + 4 * h);
      }
    };
    if (nblk == 1)
      walk(std::integral_constant<int, 1>{});
    else
      walk(std::integral_constant<int, QB>{});
    float score = 0.0f;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      if (qb < nblk) {
        merge_halves(m[qb], am[qb]);
        const int tok = qb * kTileCols + c;
        const bool valid = tok < pr.lq;
        score += half_sum(valid ? m[qb] : 0.0f);
        if (ARGMAX && h == 0 && tok < a.slots) a.argmax[p * a.slots + tok] = valid ? am[qb] : 0;
      }
    }
    if (ARGMAX) {
      for (int t = nblk * kTileCols + lane; t < a.slots; t += 64) a.argmax[p * a.slots + t] = 0;
    }
    if (lane == kHalfSumLane) a.scores[p] = score;
  }
  // drain: no load may still be writing LDS when the wave exits
  __builtin_amdgcn_s_waitcnt(0x0F70);
}

// ---------------------------------------------------------------------------
// Packed pairs, document-major (doc_chunk_kernel; needs a workspace).
//
// Packed pairs come in the caller's order (C4: 20,000 pairs drawn uniformly
// over 8,192 documents, about 2.4 per document), so scored pair by pair
// every document is streamed from HBM once per pair that names it, with
// almost no L2 reuse.  Here the pairs are first grouped by document on the
// device (group_docs_kernel) and cut into chunks of at most kChunkPairs
// pairs of one document.  A workgroup of kChunkPairs waves scores a chunk,
// one pair per wave (the query's one or two 32-token blocks in registers, as
// in pair_ring_kernel), while the document's tiles pass once through a ring
// of LDS slots shared by the waves: each wave issues its share of every
// tile's direct global->LDS loads, waits for them, and one barrier per tile
// makes the tile visible to all and frees the slot read one tile before.
// Query blocks travel through the same ring (vector-memory loads complete
// in issue order, so any other load would make its wait a wait for every
// tile in flight).  Chunks are sorted by their document's tile count,
// longest first, and dealt round-robin over a grid that is resident at once,
// so every workgroup gets a similar share and ends on short chunks.
// Each pair sees the same MFMA order and tile epilogue as in pair_kernel,
// so the results are bit-identical whichever kernel scores it.
// ---------------------------------------------------------------------------
constexpr int kChunkPairs = 4;                // pairs per chunk (a set of pair waves)
constexpr int kChunkSets = 1;                 // sets of pair waves, alternating chunks
constexpr int kChunkLoaders = 1;              // loader waves
constexpr int kChunkWaves = kChunkLoaders + kChunkSets * kChunkPairs;
// LDS ring depth, in tiles: at dim 128, 68 KB per workgroup, two per CU
// (C4 forward 124-131 us; 147-155 at depth 6 and three per CU, 179 at depth
// 8 and one per CU, 168-192 with two loader waves)
constexpr int kChunkSlots = 8;
// Tiles per barrier: with two, the pair waves take two tiles between
// barriers and the loader refills two slots after each; C4 forward 133.0
// against 133.7 us with one, i.e. the barriers are not what bounds it.
constexpr int kTilesPerBarrier = 1;


constexpr int kChunkBatch = 64;               // chunks per workgroup, at most
constexpr int kDocGroupThreads = 1024;
// Sort keys: 4 * (63 - the document's tile count, clamped) + the low two
// bits of its id -- longest first; the id bits only spread the atomics of
// documents of one length over four counters (C4's lengths fall into a few
// tile counts, and same-address LDS atomics serialise)
constexpr int kLenClasses = 256;
constexpr int64_t kDocGroupMaxDocs = 16384;   // 1024 per grouping workgroup

// A chunk: the document's rows and, per pair slot, its pair, resolved by
// scatter_docs_kernel; doc_chunk_kernel copies its chunks into LDS.
struct ChunkMeta {
  int d_row0;
  int ld;                      // 0: the document's segment is invalid
  int pad[2];
  int p[kChunkPairs];          // pair id; -1: no pair in this slot
  int q_row0[kChunkPairs];
  int lq[kChunkPairs];         // 0: invalid pair (NaN score)
};
static_assert(sizeof(ChunkMeta) % 16 == 0, "chunks are copied as 16-byte pieces");

// The grouping's workspace (see doc_chunk_ws_bytes for the layout).
constexpr int kGroupWgs = 16;  // grouping workgroups, one range of documents each
struct DocChunks {
  ChunkMeta* recs;   // [max chunks], sorted by their document's length class
  int32_t* nchunks;  // [1]
  int32_t* cnt;      // [nd] pairs per document
  int32_t* rank;     // [npairs] each pair's place among its document's pairs
  int32_t* cpos;     // [nd] each document's first chunk within (range, class)
  int32_t* hist;     // [kGroupWgs][kLenClasses] chunks per (range, class)
  uint8_t* kls;      // [nd] length class
};

// Upper bound on the chunks of a grouping: ceil(c / 4) <= c / 4 + 3 / 4 per
// document with c > 0 pairs, and at most min(nd, npairs) such documents.
static int64_t doc_chunk_bound(int64_t nd, int64_t npairs) {
  return (npairs + kChunkPairs - 1) / kChunkPairs + std::min(nd, npairs);
}

// Documents per grouping range: a multiple of eight, kGroupWgs ranges cover
// all (at most 1024 each since nd <= kDocGroupMaxDocs).
__host__ __device__ __forceinline__ int group_range(int nd) {
  return ((nd + kGroupWgs - 1) / kGroupWgs + 7) & ~7;
}
static_assert(((kDocGroupMaxDocs + kGroupWgs - 1) / kGroupWgs + 7) / 8 * 8 <= 1024,
              "a range fits one batch of eight documents per thread");

// NaN score and zero argmax row for a pair no chunk carries (one thread).
__device__ __forceinline__ void write_unrouted_pair(const FwdArgs& a, int64_t p) {
  a.scores[p] = __builtin_nanf("");
  if (a.argmax)
    for (int t = 0; t < a.slots; ++t) a.argmax[p * a.slots + t] = 0;
}

// group_docs_kernel (kGroupWgs workgroups): workgroup k owns the documents
// of range k.  It reads every pair id and counts the pairs of its range in
// LDS counters (the count before a pair is its place among its document's
// pairs, written out for scatter_docs_kernel), classifies its documents (length class, chunks per class),
// writes its chunks per class to hist[k], and gives each of its documents
// a first chunk within (range, class) by LDS cursors.  scatter_docs_kernel
// turns those into global positions (classes in order, ranges in order
// within a class).  A one-workgroup version took 11.3 us at C4: its time was
// its CU's chain of LDS atomics and round trips.  The ids and offsets are
// loaded up front, 16 bytes per lane where aligned (VEC); a thread owns four
// consecutive pairs per vector and eight consecutive documents.  Pairs whose
// document id is out of range are written off by workgroup 0 (NaN score,
// zero argmax row).  Chunk positions within a (range, class) follow the
// atomics; no result depends on them.
constexpr int kGroupPairVecs = 5;  // 4-pair vectors per thread per batch (20,480 pairs)
constexpr int kGroupDocs = 8;      // consecutive documents per thread

// v[0..3] = p[i0 .. i0 + 3], zero past n (one 16-byte load where VEC and
// whole; p + i0 is then 16-byte aligned since i0 % 4 == 0)
template <bool VEC>
__device__ __forceinline__ void load4_bounded(const int32_t* __restrict__ p, int64_t i0, int64_t n,
                                              int32_t (&v)[4]) {
  if (VEC && i0 + 3 < n) {
    const int4 x = *reinterpret_cast<const int4*>(p + i0);
    v[0] = x.x;
    v[1] = x.y;
    v[2] = x.z;
    v[3] = x.w;
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = i0 + e < n ? p[i0 + e] : 0;
  }
}

// p[d0 .. d0 + 7] = v[0..7] for the entries below n (two 16-byte stores when
// p is 16-byte aligned and all eight are in range)
__device__ __forceinline__ void store8_bounded(int32_t* __restrict__ p, int d0, int n,
                                               const int32_t (&v)[kGroupDocs]) {
  if ((reinterpret_cast<uintptr_t>(p) & 15u) == 0 && d0 + 7 < n) {
    *reinterpret_cast<int4*>(p + d0) = int4{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<int4*>(p + d0 + 4) = int4{v[4], v[5], v[6], v[7]};
  } else {
#pragma unroll
    for (int e = 0; e < kGroupDocs; ++e)
      if (d0 + e < n) p[d0 + e] = v[e];
  }
}

template <bool VEC>
__global__ __launch_bounds__(kDocGroupThreads) void group_docs_kernel(FwdArgs a, DocChunks g) {
  __shared__ int32_t cnt[1024];               // pairs per document of the range
  __shared__ int32_t cls[kLenClasses];        // chunks per class
  __shared__ int32_t cur[kLenClasses];        // cursors per class
  constexpr int T = kDocGroupThreads, UV = kGroupPairVecs, ND = kGroupDocs;
  const int tid = threadIdx.x;
  const int nd = (int)a.nd;
  const int per = group_range(nd);
  const int d_lo = min((int)blockIdx.x * per, nd);
  const int d_hi = min(d_lo + per, nd);
  const int64_t np = a.npairs;
  const bool writer = blockIdx.x == 0;  // writes off the pairs of invalid documents

  // the first batch of pair ids and this thread's eight document extents,
  // loaded before anything waits on them
  int32_t di[UV][4];
  auto load_pairs = [&](int64_t v0) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < UV; ++u) load4_bounded<VEC>(a.dids, 4 * (v0 + (int64_t)u * T), np, di[u]);
  };
  const int d0 = d_lo + ND * tid;  // this thread's documents: d0 .. d0 + 7 (below d_hi)
  int32_t off[ND + 1];
  {
    int32_t lo[4], hi[4];
    const int64_t lim = d0 < d_hi ? (int64_t)nd + 1 : 0;
    load4_bounded<VEC>(a.doff, d0, lim, lo);
    load4_bounded<VEC>(a.doff, d0 + 4, lim, hi);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      off[e] = lo[e];
      off[4 + e] = hi[e];
    }
    off[ND] = d0 < d_hi && d0 + ND <= nd ? a.doff[d0 + ND] : 0;
  }
  load_pairs(tid);
  cnt[tid] = 0;
  if (tid < kLenClasses) {
    cls[tid] = 0;
    cur[tid] = 0;
  }
  // a barrier that waits for this thread's LDS writes only: the loads above
  // are waited for where they are used
  auto lds_barrier = [&]() __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __asm__ __volatile__("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    __asm__ __volatile__("" ::: "memory");
  };
  lds_barrier();

  // 1. pairs per document of the range; workgroup 0 writes off, in a second,
  //    rolled loop (rare), the pairs of a batch holding an out-of-range id
  auto count_batch = [&](int64_t v0) __attribute__((always_inline)) {
    bool bad = false;
#pragma unroll
    for (int u = 0; u < UV; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool in = 4 * (v0 + (int64_t)u * T) + e < np;
        const int32_t d = di[u][e];
        if (in && d >= d_lo && d < d_hi)
          g.rank[4 * (v0 + (int64_t)u * T) + e] = atomicAdd(&cnt[d - d_lo], 1);
        bad |= in && (d < 0 || d >= nd);
      }
    if (writer && bad) {
#pragma unroll 1
      for (int u = 0; u < UV; ++u)
#pragma unroll 1
        for (int e = 0; e < 4; ++e) {
          const int64_t p = 4 * (v0 + (int64_t)u * T) + e;
          if (p >= np) break;
          const int32_t d = a.dids[p];
          if (d < 0 || d >= nd) write_unrouted_pair(a, p);
        }
    }
  };
  const int64_t nv = (np + 3) / 4;
  count_batch(tid);
  for (int64_t v0 = tid + (int64_t)UV * T; v0 < nv; v0 += (int64_t)UV * T) {
    load_pairs(v0);
    count_batch(v0);
  }
  lds_barrier();

  // 2. length class of every document of the range, and chunks per class
  int32_t c8[ND];
  int32_t k8[ND];
  const bool mine = d0 < d_hi;
  if (mine) {
#pragma unroll
    for (int e = 0; e < ND; ++e) {
      const int d = d0 + e;
      const int64_t ld = (int64_t)off[e + 1] - off[e];
      const int64_t t = ld <= 0 ? 0 : (ld + kTileRows - 1) / kTileRows;
      k8[e] = 4 * (63 - (int)(t < 63 ? t : 63)) + (d & 3);
      c8[e] = d < d_hi ? cnt[d - d_lo] : 0;
      if (c8[e] > 0) atomicAdd(&cls[k8[e]], (c8[e] + kChunkPairs - 1) / kChunkPairs);
    }
  }
  lds_barrier();
  if (tid < kLenClasses) g.hist[blockIdx.x * kLenClasses + tid] = cls[tid];

  // 3. each document's first chunk within (range, class), and the copy-out
  if (mine) {
    int32_t p8[ND];
    uint32_t k_lo = 0, k_hi = 0;
#pragma unroll
    for (int e = 0; e < ND; ++e) {
      p8[e] = c8[e] > 0 ? atomicAdd(&cur[k8[e]], (c8[e] + kChunkPairs - 1) / kChunkPairs) : 0;
      if (e < 4)
        k_lo |= (uint32_t)k8[e] << (8 * e);
      else
        k_hi |= (uint32_t)k8[e] << (8 * (e - 4));
    }
    store8_bounded(g.cnt, d0, d_hi, c8);
    store8_bounded(g.cpos, d0, d_hi, p8);
    if (d0 + 7 < d_hi) {
      *reinterpret_cast<uint2*>(g.kls + d0) = uint2{k_lo, k_hi};
    } else {
#pragma unroll
      for (int e = 0; e < ND; ++e)
        if (d0 + e < d_hi) g.kls[d0 + e] = (uint8_t)k8[e];
    }
  }
}

// scatter_docs_kernel (grid-stride, many workgroups): the chunk records.
// Each workgroup first turns the grouping's chunks per (range, class) into
// the first chunk of each (range, class) -- classes in order (longest
// documents first), ranges in order within a class -- in LDS.  Pair k of a
// document (its place from the grouping) then takes slot k % 4 of the
// document's chunk k / 4, and writes its id and its query rows
// there (query length 0 when the pair or its document is invalid); each
// document writes its rows into its chunks and marks the slots past its last
// pair empty.  The order of a document's pairs follows the grouping's
// atomics; no result depends on it.
constexpr int kScatterThreads = 256;
static_assert(kScatterThreads == kLenClasses, "one thread per class in the prologue");
__global__ __launch_bounds__(kScatterThreads) void scatter_docs_kernel(FwdArgs a, DocChunks g) {
  __shared__ int32_t base[kGroupWgs][kLenClasses];
  __shared__ int32_t wsum[kScatterThreads / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  {
    int h[kGroupWgs];
#pragma unroll
    for (int k = 0; k < kGroupWgs; ++k) h[k] = g.hist[k * kLenClasses + tid];
    int tot = 0;
#pragma unroll
    for (int k = 0; k < kGroupWgs; ++k) {
      base[k][tid] = tot;
      tot += h[k];
    }
    // exclusive scan of the class totals over the workgroup
    int inc = tot;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int u = __shfl_up(inc, o);
      if (lane >= o) inc += u;
    }
    if (lane == 63) wsum[wave] = inc;
    __syncthreads();
    int first = inc - tot;
    for (int w = 0; w < wave; ++w) first += wsum[w];
#pragma unroll
    for (int k = 0; k < kGroupWgs; ++k) base[k][tid] += first;
    if (blockIdx.x == 0 && tid == kScatterThreads - 1) g.nchunks[0] = first + tot;
    __syncthreads();
  }
  const int nd = (int)a.nd;
  const int per = group_range(nd);
  const int64_t np = a.npairs;
  const int64_t n = np > nd ? np : nd;
  auto first_chunk = [&](int d) __attribute__((always_inline)) {
    return base[d / per][g.kls[d]] + g.cpos[d];
  };
  auto doc_rows = [&](int64_t d, int& d0, int& ld) __attribute__((always_inline)) {
    const int64_t ds = a.doff[d], de = a.doff[d + 1];
    const bool ok = ds >= 0 && de > ds && de <= a.total_d;
    d0 = ok ? (int)ds : 0;
    ld = ok ? (int)(de - ds) : 0;
  };
  for (int64_t i = (int64_t)blockIdx.x * kScatterThreads + tid; i < n;
       i += (int64_t)gridDim.x * kScatterThreads) {
    if (i < np) {
      const int32_t d = a.dids[i];
      if (d >= 0 && d < nd) {
        const int k = g.rank[i];
        ChunkMeta& r = g.recs[first_chunk(d) + k / kChunkPairs];
        const int j = k % kChunkPairs;
        int d0, ld;
        doc_rows(d, d0, ld);
        int q0 = 0, lq = 0;
        const int64_t qi = a.qids[i];
        if (ld > 0 && qi >= 0 && qi < a.nq) {
          const int64_t qs = a.qoff[qi], qe = a.qoff[qi + 1];
          if (qs >= 0 && qe > qs && qe <= a.total_q && qe - qs <= a.slots) {
            q0 = (int)qs;
            lq = (int)(qe - qs);
          }
        }
        r.p[j] = (int)i;
        r.q_row0[j] = q0;
        r.lq[j] = lq;
      }
    }
    if (i < nd) {
      const int c = g.cnt[i];
      if (c > 0) {
        int d0, ld;
        doc_rows(i, d0, ld);
        const int fc = first_chunk((int)i);
        const int nch = (c + kChunkPairs - 1) / kChunkPairs;
        for (int jc = 0; jc < nch; ++jc) {
          ChunkMeta& r = g.recs[fc + jc];
          r.d_row0 = d0;
          r.ld = ld;
        }
        ChunkMeta& last = g.recs[fc + nch - 1];
        for (int j = c - (nch - 1) * kChunkPairs; j < kChunkPairs; ++j) {
          last.p[j] = -1;
          last.q_row0[j] = 0;
          last.lq[j] = 0;
        }
      }
    }
  }
}

// LDS per workgroup of doc_chunk_kernel (ring + chunk metadata; 68 KB at
// dim 128: two workgroups per CU), and the waves per SIMD its register
// budget is compiled for: a workgroup of five waves takes two wave slots on
// some SIMD, so two workgroups per CU need four slots per SIMD, i.e. at most
// 128 VGPRs (at 154 VGPRs the runtime places one workgroup per CU: C4
// forward 175 against 124-131 us).
template <typename T, int KS>
struct ChunkOcc {
  static constexpr int kLds =
      kChunkSlots * TileGeom<T, KS>::kBufPieces * 16 + kChunkBatch * (int)sizeof(ChunkMeta);
  static constexpr int kWavesPerEu = 2 * ((kChunkWaves + 3) / 4);
};

// Chunk of round r for workgroup b of `grid`: the sorted chunks are dealt
// in snake order (place q, then grid - 1 - q, ...) so that no workgroup takes
// the largest chunk of every round.  With a grid of whole XCD rows the
// places of a round are dealt XCD by XCD (place q to workgroup
// (q % (grid / 8)) * 8 + q / (grid / 8)): the chunks of one document are
// consecutive, so they run at once on one XCD and share its L2.
__device__ __forceinline__ int64_t snake_chunk(int b, int r, int grid) {
  const int q = grid % kXcds == 0 ? (b % kXcds) * (grid / kXcds) + b / kXcds : b;
  return (int64_t)r * grid + ((r & 1) ? grid - 1 - q : q);
}

// s_waitcnt vmcnt(N) (N <= 63); encoding (gfx9): vmcnt[3:0] | expcnt[6:4]
// = 7 | lgkmcnt[11:8] = 15 | vmcnt[5:4] << 14
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt is a 6-bit field");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

// The workgroup: kChunkLoaders loader waves and kChunkSets sets of
// kChunkPairs pair waves.  The loaders issue every global->LDS tile load of
// the ring (each its share of every tile) and nothing else, so their
// vector-memory counters see only the ring and their waits are exact.  Set
// s scores the chunks c with c % kChunkSets == s, wave j of the set pair
// slot j; it loads the query blocks of its next chunk straight into
// registers with ordinary loads (counted by the compiler, behind no tile
// load) as soon as it has finished a chunk, so they arrive while the other
// set scores.  One barrier per tile: the loaders have waited for the tile's
// loads, every pair wave has finished reading the slot of the tile before,
// and the loaders refill that slot.
template <typename T, int KS, bool ARGMAX, bool STREAM>
__global__ __launch_bounds__(kChunkWaves * 64, (ChunkOcc<T, KS>::kWavesPerEu)) void doc_chunk_kernel(
    FwdArgs a, const ChunkMeta* __restrict__ recs, const int32_t* __restrict__ nchunks_p) {
  using S = typename T::storage;
  using G = TileGeom<T, KS>;
  static_assert(T::bytes == 2, "16-bit operands: one 16-byte piece per fragment");
  constexpr int QB = 2;
  constexpr int kRPI = 64 / G::P;                 // tile rows per wave load instruction
  constexpr int kDma = G::kPieces / 64;           // wave load instructions per tile
  constexpr int kDmaL = kDma / kChunkLoaders;     // ... issued by each loader
  static_assert(kDma % kChunkLoaders == 0 && kDmaL >= 1, "tile loads split evenly");
  static_assert(kDmaL * (kChunkSlots - kTilesPerBarrier) <= 63,
                "a loader's tiles in flight fit vmcnt");
  static_assert(kChunkSlots > 2 * kTilesPerBarrier, "a ring deeper than two steps");
  extern __shared__ uint4 lds[];
  ChunkMeta* meta = reinterpret_cast<ChunkMeta*>(lds + kChunkSlots * G::kBufPieces);
  const int lane = threadIdx.x & 63;
  const int c = lane & 31;
  const int h = lane >> 5;
  const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int nch = __builtin_amdgcn_readfirstlane(nchunks_p[0]);
  const int b = blockIdx.x;
  const int grid = gridDim.x;
  // chunks of this workgroup: every full round, plus the last round's if it
  // falls inside; the host sizes the grid so that there are at most
  // kChunkBatch rounds
  const int rounds = nch / grid;
  const int mine =
      min(rounds + (snake_chunk(b, rounds, grid) < nch ? 1 : 0), kChunkBatch);
  if (mine == 0) return;  // whole workgroup
  const S* __restrict__ Q = static_cast<const S*>(a.q);
  const S* __restrict__ D = static_cast<const S*>(a.d);
  const int dim = a.dim;
  const uint32_t row_bytes = (uint32_t)dim * (uint32_t)sizeof(S);

  // ---- chunk records into LDS, one 16-byte piece per thread
  constexpr int kPieces16 = (int)sizeof(ChunkMeta) / 16;
  for (int s = threadIdx.x; s < mine * kPieces16; s += kChunkWaves * 64) {
    const int ci = s / kPieces16, part = s - ci * kPieces16;
    reinterpret_cast<uint4*>(meta + ci)[part] =
        reinterpret_cast<const uint4*>(recs + snake_chunk(b, ci, grid))[part];
  }
  __syncthreads();

  // tiles of chunk ci (wave-uniform): none when no pair of it is valid
  auto chunk_tiles = [&](int ci) __attribute__((always_inline)) {
    const ChunkMeta& m = meta[ci];
    int any = 0;
#pragma unroll
    for (int j = 0; j < kChunkPairs; ++j) any |= __builtin_amdgcn_readfirstlane(m.lq[j]);
    return any > 0 ? (__builtin_amdgcn_readfirstlane(m.ld) + kTileRows - 1) / kTileRows : 0;
  };
  // s_barrier without a fence (a fence would wait for every load in
  // flight); the empty asm statements keep the compiler from moving memory
  // accesses across it
  auto barrier = [&]() __attribute__((always_inline)) {
    __asm__ __volatile__("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    __asm__ __volatile__("" ::: "memory");
  };

  if (wv < kChunkLoaders) {
    // ---- loader waves: the tile stream, kChunkSlots - 1 tiles ahead
    const int l_hi = lane / G::P;
    const int l_lo = lane - l_hi * G::P;
    const uint32_t ring_lds = __builtin_amdgcn_readfirstlane(lds_addr(lds));
    int li = 0, lt = 0;  // chunk and tile of the next load
    int lnt = chunk_tiles(0);
    while (lnt == 0 && ++li < mine) lnt = chunk_tiles(li);
    int issued = 0, lslot = 0;
    auto load_next = [&]() __attribute__((always_inline)) {
      if (li >= mine) return;
      const int d0 = __builtin_amdgcn_readfirstlane(meta[li].d_row0);
      const int ld = __builtin_amdgcn_readfirstlane(meta[li].ld);
      const S* base = D + ((int64_t)d0 + (int64_t)lt * kTileRows) * dim;
      const int last = ld - 1 - lt * kTileRows;
#pragma unroll
      for (int ii = 0; ii < kDmaL; ++ii) {
        const int i = wv * kDmaL + ii;
        const int r = i * kRPI + l_hi;
        const uint32_t off = (uint32_t)min(r, last) * row_bytes +
                             (uint32_t)((l_lo ^ (r & G::SWZ)) * 16);
        const uint32_t dst =
            ring_lds + (uint32_t)((lslot * G::kBufPieces + i * 64) * sizeof(uint4));
        if (STREAM)
          lds_dma16_nt(base, off, dst);
        else
          lds_dma16(base, off, dst);
      }
      ++issued;
      if (++lslot == kChunkSlots) lslot = 0;
      if (++lt >= lnt) {
        lt = 0;
        while (++li < mine && (lnt = chunk_tiles(li)) == 0) {
        }
      }
    };
    // wait until this loader's loads of the tile `ahead` tiles before the
    // newest issued one have landed
    auto wait_tile = [&](int ahead) __attribute__((always_inline)) {
      static_assert(kChunkSlots - 2 <= 14, "wait_tile covers up to 14 tiles ahead");
      switch (ahead) {
        case 1: wait_vmcnt<kDmaL * 1>(); break;
        case 2: wait_vmcnt<kDmaL * 2>(); break;
        case 3: wait_vmcnt<kDmaL * 3>(); break;
        case 4: wait_vmcnt<kDmaL * 4>(); break;
        case 5: wait_vmcnt<kDmaL * 5>(); break;
        case 6: wait_vmcnt<kDmaL * 6>(); break;
        case 7: wait_vmcnt<kDmaL * 7>(); break;
        case 8: wait_vmcnt<kDmaL * 8 <= 63 ? kDmaL * 8 : 0>(); break;
        case 9: wait_vmcnt<kDmaL * 9 <= 63 ? kDmaL * 9 : 0>(); break;
        case 10: wait_vmcnt<kDmaL * 10 <= 63 ? kDmaL * 10 : 0>(); break;
        case 11: wait_vmcnt<kDmaL * 11 <= 63 ? kDmaL * 11 : 0>(); break;
        case 12: wait_vmcnt<kDmaL * 12 <= 63 ? kDmaL * 12 : 0>(); break;
        case 13: wait_vmcnt<kDmaL * 13 <= 63 ? kDmaL * 13 : 0>(); break;
        case 14: wait_vmcnt<kDmaL * 14 <= 63 ? kDmaL * 14 : 0>(); break;
        default: wait_vmcnt<0>(); break;
      }
    };
    // Barrier before tile k when k % kTilesPerBarrier == 0: tiles k ..
    // k + kTilesPerBarrier - 1 have landed, and the pair waves have read the
    // slots of the kTilesPerBarrier tiles before k, which the loads issued
    // after the barrier refill.
    for (int i = 0; i < kChunkSlots - kTilesPerBarrier; ++i) load_next();
    int k = 0;
    for (int ci = 0; ci < mine; ++ci) {
      const int nt = chunk_tiles(ci);
      for (int t = 0; t < nt; ++t, ++k) {
        if (k % kTilesPerBarrier == 0) {
          wait_tile(issued - k - kTilesPerBarrier);
          barrier();
#pragma unroll
          for (int i = 0; i < kTilesPerBarrier; ++i) load_next();
        }
      }
    }
    // drain: no load may still be writing LDS when the wave exits
    wait_vmcnt<0>();
    return;
  }

  // ---- pair waves
  const int pw = wv - kChunkLoaders;
  const int set = pw / kChunkPairs;
  const int j = pw - set * kChunkPairs;  // pair slot
  int aoff[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) aoff[s] = c * G::P + ((2 * s + h) ^ (c & G::SWZ));
  Frag<T> qf[QB][KS];
  // query blocks of this wave's pair in chunk ci into registers: lane (c, h)
  // takes pieces 2s + h of token c (rows past the query end repeat its last
  // token) -- the fragments a tile read of the same rows gives
  auto load_query = [&](int ci) __attribute__((always_inline)) {
    const int mq = __builtin_amdgcn_readfirstlane(meta[ci].lq[j]);
    const int q0 = __builtin_amdgcn_readfirstlane(meta[ci].q_row0[j]);
    const int nblk = (mq + kTileCols - 1) / kTileCols;  // <= QB (host checks)
    const auto* qg = uniform_gptr(reinterpret_cast<const char*>(Q + (int64_t)q0 * dim));
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      if (qb < nblk) {
        const uint32_t row = qb * kTileCols + min(c, mq - 1 - qb * kTileCols);
#pragma unroll
        for (int s = 0; s < KS; ++s)
          qf[qb][s].v = load16(qg, (row * (uint32_t)dim + (2 * s + h) * G::kPieceElems) *
                                       (uint32_t)sizeof(S));
      }
    }
  };
  if (set < mine) load_query(set);
  int cslot = 0;  // slot of the next tile
  int kk = 0;     // the next tile's place in the workgroup's tile stream
  for (int ci = 0; ci < mine; ++ci) {
    const int nt = chunk_tiles(ci);
    if (ci % kChunkSets != set) {
      // the other set's chunk: keep the barriers
      for (int t = 0; t < nt; ++t) {
        if (kk % kTilesPerBarrier == 0) barrier();
        ++kk;
        if (++cslot == kChunkSlots) cslot = 0;
      }
      continue;
    }
    const int p = __builtin_amdgcn_readfirstlane(meta[ci].p[j]);
    const int mq = __builtin_amdgcn_readfirstlane(meta[ci].lq[j]);
    const int nblk = (mq + kTileCols - 1) / kTileCols;
    if (p >= 0 && nblk == 0) write_invalid_pair(a, p, lane);
    float m[QB];
    int am[QB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      m[qb] = -__builtin_inff();
      am[qb] = 0;
    }
    auto walk = [&](auto na_const) __attribute__((always_inline)) {
      constexpr int NA = decltype(na_const)::value;
      auto tile_step = [&](int t) __attribute__((always_inline)) {
        if (kk % kTilesPerBarrier == 0) {
          // this wave's reads of the tiles before have returned
          __builtin_amdgcn_s_waitcnt(0xC07F);
          barrier();
        }
        ++kk;
        if constexpr (NA > 0) {
          const uint4* tile = lds + cslot * G::kBufPieces;
          Frag<T> df[KS];
#pragma unroll
          for (int s = 0; s < KS; ++s) df[s].v = tile[aoff[s]];
          f32x16 acc[NA];
#pragma unroll
          for (int qb = 0; qb < NA; ++qb) {
            acc[qb] = f32x16{};
#pragma unroll
            for (int s = 0; s < KS; ++s) mma_chunk(df[s], qf[qb][s], acc[qb]);
          }
#pragma unroll
          for (int qb = 0; qb < NA; ++qb)
            tile_update<ARGMAX>(acc[qb], m[qb], am[qb], t * kTileRows + 4 * h);
        }
        if (++cslot == kChunkSlots) cslot = 0;
      };
      // The first tile apart: the compiler's waits for the query loads land
      // in it, and the loop over the rest carries none (a wait left in the
      // loop would also wait, every tile, for the stores issued since).
      if (nt > 0) tile_step(0);
      for (int t = 1; t < nt; ++t) tile_step(t);
    };
    if (nblk == 1)
      walk(std::integral_constant<int, 1>{});
    else if (nblk == 2)
      walk(std::integral_constant<int, QB>{});
    else
      walk(std::integral_constant<int, 0>{});
    // this set's next chunk: its query loads go out before this chunk's
    // score and argmax stores, so that the wait for them (vector-memory
    // operations complete in order) does not also wait for the stores
    if (ci + kChunkSets < mine) load_query(ci + kChunkSets);
    if (nblk > 0) {
      float score = 0.0f;
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        if (qb < nblk) {
          merge_halves(m[qb], am[qb]);
          const int tok = qb * kTileCols + c;
          const bool valid = tok < mq;
          score += half_sum(valid ? m[qb] : 0.0f);
          if (ARGMAX && h == 0 && tok < a.slots)
            a.argmax[(int64_t)p * a.slots + tok] = valid ? am[qb] : 0;
        }
      }
      if (ARGMAX) {
        for (int t = nblk * kTileCols + lane; t < a.slots; t += 64)
          a.argmax[(int64_t)p * a.slots + t] = 0;
      }
      if (lane == kHalfSumLane) a.scores[p] = score;
    }
  }
}

// ---------------------------------------------------------------------------
// Host-side dispatch
// ---------------------------------------------------------------------------
static int ks_for_dim(int dim) {
  if (dim <= 32) return 2;
  if (dim <= 64) return 4;
  if (dim <= 128) return 8;
  return 16;
}

static bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

template <typename T, int KS, int QB>
static void launch_pair_qb(const FwdArgs& a, int ppw, bool vec, dim3 grid,
                           hipStream_t st) {
  if (a.argmax && vec)
    hipLaunchKernelGGL((pair_kernel<T, KS, QB, true, true>), grid, dim3(256), 0, st, a, ppw);
  else if (a.argmax)
    hipLaunchKernelGGL((pair_kernel<T, KS, QB, true, false>), grid, dim3(256), 0, st, a, ppw);
  else if (vec)
    hipLaunchKernelGGL((pair_kernel<T, KS, QB, false, true>), grid, dim3(256), 0, st, a, ppw);
  else
    hipLaunchKernelGGL((pair_kernel<T, KS, QB, false, false>), grid, dim3(256), 0, st, a, ppw);
}

template <typename T, int KS>
static void launch_pair_ks(const FwdArgs& a, int max_lq, int ppw, bool vec,
                           dim3 grid, hipStream_t st) {
  // Two query blocks in registers unless that would not fit (fp32, dim 256).
  constexpr bool kTwoFit = (KS * (T::bytes == 2 ? 4 : 8)) <= 64;
  if (max_lq > kTileCols && kTwoFit)
    launch_pair_qb<T, KS, (kTwoFit ? 2 : 1)>(a, ppw, vec, grid, st);
  else
    launch_pair_qb<T, KS, 1>(a, ppw, vec, grid, st);
}

template <typename T>
static void launch_pair(const FwdArgs& a, int max_lq, int ppw, bool vec,
                        hipStream_t st) {
  const int64_t waves = (a.npairs + ppw - 1) / ppw;
  const dim3 grid((unsigned)((waves + 3) / 4));
  switch (ks_for_dim(a.dim)) {
    case 2: launch_pair_ks<T, 2>(a, max_lq, ppw, vec, grid, st); break;
    case 4: launch_pair_ks<T, 4>(a, max_lq, ppw, vec, grid, st); break;
    case 8: launch_pair_ks<T, 8>(a, max_lq, ppw, vec, grid, st); break;
    default: launch_pair_ks<T, 16>(a, max_lq, ppw, vec, grid, st); break;
  }
}

template <typename T, int KS>
static void launch_split_ks(const FwdArgs& a, bool vec, hipStream_t st) {
  const dim3 grid((unsigned)a.npairs);
  const dim3 block(kSplitWaves * 64);
  if (a.argmax && vec)
    hipLaunchKernelGGL((pair_split_kernel<T, KS, true, true>), grid, block, 0, st, a);
  else if (a.argmax)
    hipLaunchKernelGGL((pair_split_kernel<T, KS, true, false>), grid, block, 0, st, a);
  else if (vec)
    hipLaunchKernelGGL((pair_split_kernel<T, KS, false, true>), grid, block, 0, st, a);
  else
    hipLaunchKernelGGL((pair_split_kernel<T, KS, false, false>), grid, block, 0, st, a);
}

template <typename T>
static void launch_split(const FwdArgs& a, bool vec, hipStream_t st) {
  switch (ks_for_dim(a.dim)) {
    case 2: launch_split_ks<T, 2>(a, vec, st); break;
    case 4: launch_split_ks<T, 4>(a, vec, st); break;
    case 8: launch_split_ks<T, 8>(a, vec, st); break;
    default: launch_split_ks<T, 16>(a, vec, st); break;
  }
}

static int pairs_per_wave(int64_t npairs) {
  // Aim for ~16k waves (64 per CU, several rounds of the 8 resident per CU
  // at the two-block kernel's register use) so the last round is a small
  // part of the launch; never below 1.
  int64_t ppw = (npairs + 16383) / 16384;
  if (ppw < 1) ppw = 1;
  if (ppw > 64) ppw = 64;
  return (int)ppw;
}

template <typename T>
static void launch_wide(const FwdArgs& a, bool vec, hipStream_t st) {
  const dim3 grid((unsigned)((a.npairs + 3) / 4));
  if (a.argmax && vec)
    hipLaunchKernelGGL((wide_pair_kernel<T, true, true>), grid, dim3(256), 0, st, a);
  else if (a.argmax)
    hipLaunchKernelGGL((wide_pair_kernel<T, true, false>), grid, dim3(256), 0, st, a);
  else if (vec)
    hipLaunchKernelGGL((wide_pair_kernel<T, false, true>), grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((wide_pair_kernel<T, false, false>), grid, dim3(256), 0, st, a);
}

template <typename T, int KS, bool ARGMAX, bool STREAM>
static int launch_ring_v(const FwdArgs& a, int ppw, dim3 grid, hipStream_t st) {
  using G = TileGeom<T, KS>;
  const size_t lds = (size_t)kRingWaves * kRingSlots * G::kBufPieces * sizeof(uint4);
  const auto kern = pair_ring_kernel<T, KS, ARGMAX, STREAM>;
  if (lds > 64 * 1024) {
    // once per device and instantiation: allow the slots' dynamic LDS
    static std::atomic<bool> raised[kMaxDevices];
    if (int e = raise_lds_limit((const void*)kern, lds, "pair_ring_kernel", raised)) return e;
  }
  hipLaunchKernelGGL(kern, grid, dim3(kRingWaves * 64), lds, st, a, ppw);
  return MAXSIM_OK;
}

template <typename T, int KS>
static int launch_ring_ks(const FwdArgs& a, int ppw, dim3 grid, hipStream_t st) {
  const bool stream = a.mode == kPadded;
  if (a.argmax)
    return stream ? launch_ring_v<T, KS, true, true>(a, ppw, grid, st)
                  : launch_ring_v<T, KS, true, false>(a, ppw, grid, st);
  return stream ? launch_ring_v<T, KS, false, true>(a, ppw, grid, st)
                : launch_ring_v<T, KS, false, false>(a, ppw, grid, st);
}

template <typename T>
static int launch_ring(const FwdArgs& a, int ppw, dim3 grid, hipStream_t st) {
  switch (ks_for_dim(a.dim)) {
    case 2: return launch_ring_ks<T, 2>(a, ppw, grid, st);
    case 4: return launch_ring_ks<T, 4>(a, ppw, grid, st);
    default: return launch_ring_ks<T, 8>(a, ppw, grid, st);
  }
}

// Document-major packed path (doc_chunk_kernel): 16-bit rows of 64 or 128
// elements (four or eight wave loads per tile, split evenly over the four
// waves), queries of at most two 32-token blocks, at most kDocGroupMaxDocs
// documents (one LDS counter each in group_docs_kernel), and enough pairs
// that the grouping launch pays for itself.
constexpr int64_t kDocChunkMinPairs = 4096;
constexpr bool kChunkStream = true;  // document tiles read once: non-temporal

static bool doc_chunk_fits(const FwdArgs& a, maxsim_dtype dtype, int max_lq) {
  const int ks = ks_for_dim(a.dim);
  return a.mode == kPacked && dtype != MAXSIM_FLOAT32 && (ks == 4 || ks == 8) &&
         a.dim == ks * kChunk && aligned16(a.q) && aligned16(a.d) &&
         max_lq <= 2 * kTileCols && a.nd <= kDocGroupMaxDocs &&
         a.npairs >= kDocChunkMinPairs && a.npairs <= INT32_MAX;
}

// Workspace: chunk records (64 bytes) [doc_chunk_bound], nchunks (int32,
// padded to 16 bytes), int32 cnt [nd], cpos [nd], rank [npairs], hist
// [kGroupWgs][kLenClasses] (at a 16-byte boundary), then the length classes
// (bytes) [nd].
static size_t doc_chunk_hist_offset(int64_t nd, int64_t npairs) {
  return (sizeof(ChunkMeta) * (size_t)doc_chunk_bound(nd, npairs) + 16 + 8 * (size_t)nd +
          4 * (size_t)npairs + 15) &
         ~(size_t)15;
}
static size_t doc_chunk_ws_bytes(int64_t nd, int64_t npairs) {
  return doc_chunk_hist_offset(nd, npairs) + sizeof(int32_t) * kGroupWgs * kLenClasses +
         (size_t)nd;
}

// Grid: as many workgroups as the chip holds at once (LDS or registers
// bound it: two per CU at dim 128), so the chunks are dealt in one round;
// more only where one workgroup would otherwise get over kChunkBatch.
template <typename T, int KS, bool ARGMAX>
static int launch_doc_chunk_v(const FwdArgs& a, const DocChunks& g, int64_t bound,
                              hipStream_t st) {
  using G = TileGeom<T, KS>;
  const size_t lds = ChunkOcc<T, KS>::kLds;
  const auto kern = doc_chunk_kernel<T, KS, ARGMAX, kChunkStream>;
  if (lds > 64 * 1024) {
    static std::atomic<bool> raised[kMaxDevices];
    if (int e = raise_lds_limit((const void*)kern, lds, "doc_chunk_kernel", raised)) return e;
  }
  static std::atomic<int> per_cu[kMaxDevices];
  const int64_t resident =
      (int64_t)device_cus() * resident_per_cu((const void*)kern, kChunkWaves * 64, lds, per_cu);
  const int64_t grid = std::max<int64_t>(resident, (bound + kChunkBatch - 1) / kChunkBatch);
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(kChunkWaves * 64), lds, st, a,
                     static_cast<const ChunkMeta*>(g.recs), static_cast<const int32_t*>(g.nchunks));
  return MAXSIM_OK;
}

template <typename T>
static int launch_doc_chunk(const FwdArgs& a, const DocChunks& g, int64_t bound,
                            hipStream_t st) {
  const bool am = a.argmax != nullptr;
  if (ks_for_dim(a.dim) == 8)
    return am ? launch_doc_chunk_v<T, 8, true>(a, g, bound, st)
              : launch_doc_chunk_v<T, 8, false>(a, g, bound, st);
  return am ? launch_doc_chunk_v<T, 4, true>(a, g, bound, st)
            : launch_doc_chunk_v<T, 4, false>(a, g, bound, st);
}

static int run_doc_chunks(const FwdArgs& a, maxsim_dtype dtype, void* workspace,
                          hipStream_t st) {
  const int64_t bound = doc_chunk_bound(a.nd, a.npairs);
  DocChunks g;
  g.recs = static_cast<ChunkMeta*>(workspace);
  g.nchunks = reinterpret_cast<int32_t*>(g.recs + bound);
  g.cnt = g.nchunks + 4;
  g.cpos = g.cnt + a.nd;
  g.rank = g.cpos + a.nd;
  g.hist = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) +
                                      doc_chunk_hist_offset(a.nd, a.npairs));
  g.kls = reinterpret_cast<uint8_t*>(g.hist + kGroupWgs * kLenClasses);
  // the grouping workgroups count, classify and place by document range ...
  const bool vec = aligned16(a.dids) && aligned16(a.doff);
  hipLaunchKernelGGL(vec ? group_docs_kernel<true> : group_docs_kernel<false>, dim3(kGroupWgs),
                     dim3(kDocGroupThreads), 0, st, a, g);
  // ... and the chip scatters the pair ids and the chunk table
  const int64_t n = std::max<int64_t>(a.npairs, a.nd);
  const int64_t sgrid =
      std::min<int64_t>((n + kScatterThreads - 1) / kScatterThreads, 4 * (int64_t)device_cus());
  hipLaunchKernelGGL(scatter_docs_kernel, dim3((unsigned)sgrid), dim3(kScatterThreads), 0, st, a,
                     g);
  if (int e = check_launch("group_docs_kernel / scatter_docs_kernel")) return e;
  const int rc = dtype == MAXSIM_BFLOAT16 ? launch_doc_chunk<BF16>(a, g, bound, st)
                                          : launch_doc_chunk<F16>(a, g, bound, st);
  if (rc) return rc;
  return check_launch("doc_chunk_kernel");
}

static int run_pair(const FwdArgs& a, maxsim_dtype dtype, int max_lq,
                    hipStream_t st) {
  if (a.dim > kMaxRegDim) {
    // one wave per pair, four per workgroup
    if ((a.npairs + 3) / 4 > (int64_t)UINT32_MAX / 256)
      return fail(MAXSIM_ERR_UNSUPPORTED, "too many pairs for one launch");
    const bool vec = (a.dim % kChunk == 0) && aligned16(a.q) && aligned16(a.d);
    switch (dtype) {
      case MAXSIM_BFLOAT16: launch_wide<BF16>(a, vec, st); break;
      case MAXSIM_FLOAT16: launch_wide<F16>(a, vec, st); break;
      default: launch_wide<F32>(a, vec, st); break;
    }
    return check_launch("wide_pair_kernel");
  }
  const int ppw = pairs_per_wave(a.npairs);
  const bool vec = (a.dim == ks_for_dim(a.dim) * kChunk) && aligned16(a.q) &&
                   aligned16(a.d);
  // Fewer pairs than SIMDs: a workgroup per pair, its tiles split over the
  // workgroup's waves (the same bits as pair_kernel).
  if (a.npairs < (int64_t)4 * device_cus()) {
    switch (dtype) {
      case MAXSIM_BFLOAT16: launch_split<BF16>(a, vec, st); break;
      case MAXSIM_FLOAT16: launch_split<F16>(a, vec, st); break;
      default: launch_split<F32>(a, vec, st); break;
    }
    return check_launch("pair_split_kernel");
  }
  // 16-bit rows of at most 128 elements, queries of at most two blocks:
  // the LDS-ring variant (two tiles in flight per wave)
  if (dtype != MAXSIM_FLOAT32 && vec && ks_for_dim(a.dim) <= 8 && max_lq <= 2 * kTileCols &&
      a.mode != kContrastive) {
    // Above 32k pairs the ring takes one pair per wave (C3, 256k pairs:
    // 1.74 ms, against 1.75 / 1.77 / 1.78 / 1.83 ms at 2 / 4 / 8 / 16 pairs
    // per wave); below, the ~16k-wave rule (C4: 2 pairs per wave, 195 us,
    // against 203-206 us at one).
    const int ppw_r = a.npairs > 32768 ? 1 : ppw;
    const int64_t waves = (a.npairs + ppw_r - 1) / ppw_r;
    const dim3 grid((unsigned)((waves + kRingWaves - 1) / kRingWaves));
    const int rc = dtype == MAXSIM_BFLOAT16 ? launch_ring<BF16>(a, ppw_r, grid, st)
                                            : launch_ring<F16>(a, ppw_r, grid, st);
    if (rc) return rc;
    return check_launch("pair_ring_kernel");
  }
  switch (dtype) {
    case MAXSIM_BFLOAT16: launch_pair<BF16>(a, max_lq, ppw, vec, st); break;
    case MAXSIM_FLOAT16: launch_pair<F16>(a, max_lq, ppw, vec, st); break;
    default: launch_pair<F32>(a, max_lq, ppw, vec, st); break;
  }
  return check_launch("pair_kernel");
}


// Blocks per wave for the tiled kernel, per (dtype width, KS): the query
// fragments (NBW * KS * {4,8} VGPRs) must leave room for the document
// fragments and accumulators at two waves per SIMD.
template <typename T, int KS>
constexpr int tiled_nbw() {
  return (KS * (T::bytes == 2 ? 4 : 8) * 2 <= 64) ? 2 : 1;
}

template <typename T, int KS>
static void launch_tiled_ks(TiledArgs a, hipStream_t st) {
  if constexpr (4 * 32 * KS * 16 * T::bytes + kDocTableBytes > 64 * 1024) {
    return;  // excluded by tiled_supported(): four buffers would exceed 64 KB
  } else {
  constexpr int NBW = tiled_nbw<T, KS>();
  using G = TileGeom<T, KS>;
  a.qpw = NBW / a.nblk;
  const int64_t q_per_wg = (int64_t)a.qpw * kTiledWaves;
  a.n_qg = (int)((a.nq + q_per_wg - 1) / q_per_wg);
  // About one workgroup per CU, each streaming one long tile sequence: its
  // query group against a chunk of documents holding an equal share of the
  // work (the chunks are found on the device), so every CU finishes at the
  // same time and pays for one pipeline fill.  More chunks when needed to keep
  // each chunk within the LDS offset table (documents are >= kDocWork apart
  // in the work measure).
  const int64_t w_all = a.total_d + (int64_t)kDocWork * a.nb;
  const int64_t per_table = (int64_t)kDocWork * (kMaxDocsPerGroup - 1);
  int64_t n_dc = (device_cus() + a.n_qg - 1) / a.n_qg;
  n_dc = std::max<int64_t>(n_dc, (w_all + per_table - 1) / per_table);
  n_dc = std::max<int64_t>(1, std::min<int64_t>(n_dc, a.nb));
  a.n_dc = (int)n_dc;
  const int64_t total = (int64_t)a.n_qg * a.n_dc;
  const int64_t per_xcd = (total + 7) / 8;
  const dim3 grid((unsigned)(per_xcd * 8));
  const size_t lds = kTileBuffers * G::kBufPieces * sizeof(uint4) + kDocTableBytes;
  // Score-only calls use the same kernel with argmax == nullptr: a variant
  // without the index search needs more registers under this schedule and
  // spills, which costs far more than the search.
  hipLaunchKernelGGL((contrastive_tiled_kernel<T, KS, NBW, true>), grid,
                     dim3(kTiledThreads), lds, st, a);
  }
}

template <typename T>
static bool tiled_supported(int dim, int lq) {
  const int ks = ks_for_dim(dim);
  // four LDS tile buffers of 32 rows x ks*16 elements (plus the document
  // list) must fit in 64 KB
  if (4 * 32 * ks * 16 * T::bytes + kDocTableBytes > 64 * 1024) return false;
  int nbw = 1;
  switch (ks) {
    case 2: nbw = tiled_nbw<T, 2>(); break;
    case 4: nbw = tiled_nbw<T, 4>(); break;
    case 8: nbw = tiled_nbw<T, 8>(); break;
    default: nbw = tiled_nbw<T, 16>(); break;
  }
  const int nblk = (lq + kTileCols - 1) / kTileCols;
  return nblk <= nbw;
}

template <typename T>
static void launch_tiled(const TiledArgs& a, hipStream_t st) {
  switch (ks_for_dim(a.dim)) {
    case 2: launch_tiled_ks<T, 2>(a, st); break;
    case 4: launch_tiled_ks<T, 4>(a, st); break;
    case 8: launch_tiled_ks<T, 8>(a, st); break;
    default: launch_tiled_ks<T, 16>(a, st); break;
  }
}

static int run_contrastive(maxsim_dtype dtype, const void* q, int64_t nq,
                           int64_t lq, const void* d, int64_t total_d,
                           const int32_t* doff, int64_t nb, int64_t dim,
                           float* scores, int32_t* argmax, hipStream_t st) {
  const bool vec = (dim == ks_for_dim((int)dim) * kChunk) && aligned16(q) &&
                   aligned16(d);
  bool tiled = false;
  switch (dtype) {
    case MAXSIM_BFLOAT16: tiled = tiled_supported<BF16>((int)dim, (int)lq); break;
    case MAXSIM_FLOAT16: tiled = tiled_supported<F16>((int)dim, (int)lq); break;
    default: tiled = tiled_supported<F32>((int)dim, (int)lq); break;
  }
  // The tiled kernel stages whole 16-byte pieces: it needs dim == KS*16 and
  // aligned rows; other shapes take the pair kernel.
  if (tiled && vec) {
    TiledArgs a{};
    a.q = q;
    a.d = d;
    a.doff = doff;
    a.nq = nq;
    a.nb = nb;
    a.total_d = total_d;
    a.lq = (int)lq;
    a.dim = (int)dim;
    a.nblk = (int)((lq + kTileCols - 1) / kTileCols);
    a.scores = scores;
    a.argmax = argmax;
    switch (dtype) {
      case MAXSIM_BFLOAT16: launch_tiled<BF16>(a, st); break;
      case MAXSIM_FLOAT16: launch_tiled<F16>(a, st); break;
      default: launch_tiled<F32>(a, st); break;
    }
    return check_launch("contrastive_tiled_kernel");
  }
  FwdArgs a{};
  a.q = q;
  a.d = d;
  a.dim = (int)dim;
  a.mode = kContrastive;
  a.npairs = nq * nb;
  a.slots = (int)lq;
  a.nb = nb;
  a.lq = (int)lq;
  a.doff = doff;
  a.total_d = total_d;
  a.scores = scores;
  a.argmax = argmax;
  return run_pair(a, dtype, (int)lq, st);
}

}  // namespace maxsim

using namespace maxsim;

// ---------------------------------------------------------------------------
// C ABI -- forward entry points
// ---------------------------------------------------------------------------
extern "C" {

int maxsim_amd_contrastive_forward_with_argmax(
    maxsim_dtype dtype, const void* queries, int64_t num_queries, int64_t Lq,
    const void* documents, int64_t total_d_tokens,
    const int32_t* document_offsets, int64_t num_documents, int64_t dim,
    float* scores, int32_t* argmax, void* stream) {
  clear_error();
  if (int e = check_dtype(dtype)) return e;
  if (num_queries < 0 || num_documents < 0 || total_d_tokens < 0)
    return fail(MAXSIM_ERR_INVALID, "negative size");
  if (Lq <= 0) return fail(MAXSIM_ERR_INVALID, "Lq must be > 0; got %lld", (long long)Lq);
  if (int e = check_dim(dim)) return e;
  if (num_queries == 0 || num_documents == 0) return MAXSIM_OK;
  if (!queries || !documents || !document_offsets || !scores)
    return fail(MAXSIM_ERR_INVALID, "null pointer argument");
  if (num_queries * num_documents > (int64_t)1 << 40 || Lq > (1 << 20))
    return fail(MAXSIM_ERR_UNSUPPORTED, "problem too large");
  return run_contrastive(dtype, queries, num_queries, Lq, documents,
                         total_d_tokens, document_offsets, num_documents, dim,
                         scores, argmax, static_cast<hipStream_t>(stream));
}

int maxsim_amd_contrastive_forward(maxsim_dtype dtype, const void* queries,
                                   int64_t num_queries, int64_t Lq,
                                   const void* documents,
                                   int64_t total_d_tokens,
                                   const int32_t* document_offsets,
                                   int64_t num_documents, int64_t dim,
                                   float* scores, void* stream) {
  return maxsim_amd_contrastive_forward_with_argmax(
      dtype, queries, num_queries, Lq, documents, total_d_tokens,
      document_offsets, num_documents, dim, scores, nullptr, stream);
}

int maxsim_amd_padded_forward_with_argmax(
    maxsim_dtype dtype, const void* queries, const int32_t* query_lengths,
    const void* documents, const int32_t* doc_lengths, int64_t batch,
    int64_t num_candidates, int64_t Lq_max, int64_t Ld_max, int64_t dim,
    float* scores, int32_t* argmax, void* stream) {
  clear_error();
  if (int e = check_dtype(dtype)) return e;
  if (batch < 0 || num_candidates < 0)
    return fail(MAXSIM_ERR_INVALID, "negative size");
  if (Lq_max <= 0 || Ld_max <= 0)
    return fail(MAXSIM_ERR_INVALID, "Lq_max and Ld_max must be > 0");
  if (int e = check_dim(dim)) return e;
  if (batch == 0 || num_candidates == 0) return MAXSIM_OK;
  if (!queries || !documents || !query_lengths || !doc_lengths || !scores)
    return fail(MAXSIM_ERR_INVALID, "null pointer argument");
  if (Lq_max > (1 << 20) || Ld_max > ((int64_t)1 << 30))
    return fail(MAXSIM_ERR_UNSUPPORTED, "padded extent too large");
  FwdArgs a{};
  a.q = queries;
  a.d = documents;
  a.dim = (int)dim;
  a.mode = kPadded;
  a.npairs = batch * num_candidates;
  a.slots = (int)Lq_max;
  a.qlen = query_lengths;
  a.dlen = doc_lengths;
  a.ncand = num_candidates;
  a.lq_max = (int)Lq_max;
  a.ld_max = (int)Ld_max;
  a.scores = scores;
  a.argmax = argmax;
  return run_pair(a, dtype, (int)Lq_max, static_cast<hipStream_t>(stream));
}

int maxsim_amd_padded_forward(maxsim_dtype dtype, const void* queries,
                              const int32_t* query_lengths,
                              const void* documents,
                              const int32_t* doc_lengths, int64_t batch,
                              int64_t num_candidates, int64_t Lq_max,
                              int64_t Ld_max, int64_t dim, float* scores,
                              void* stream) {
  return maxsim_amd_padded_forward_with_argmax(
      dtype, queries, query_lengths, documents, doc_lengths, batch,
      num_candidates, Lq_max, Ld_max, dim, scores, nullptr, stream);
}

static int packed_forward_impl(
    maxsim_dtype dtype, const void* queries, int64_t total_q_tokens,
    const int32_t* query_offsets, int64_t num_queries, const void* documents,
    int64_t total_d_tokens, const int32_t* document_offsets,
    int64_t num_documents, const int32_t* pair_query_ids,
    const int32_t* pair_document_ids, int64_t num_pairs, int64_t dim,
    int64_t max_q_len, float* scores, int32_t* argmax, void* workspace,
    size_t workspace_bytes, void* stream) {
  if (int e = check_dtype(dtype)) return e;
  if (total_q_tokens < 0 || num_queries < 0 || total_d_tokens < 0 ||
      num_documents < 0 || num_pairs < 0)
    return fail(MAXSIM_ERR_INVALID, "negative size");
  if (max_q_len <= 0)
    return fail(MAXSIM_ERR_INVALID, "max_q_len must be > 0; got %lld",
                (long long)max_q_len);
  if (int e = check_dim(dim)) return e;
  if (num_pairs == 0) return MAXSIM_OK;
  if (!queries || !documents || !query_offsets || !document_offsets ||
      !pair_query_ids || !pair_document_ids || !scores)
    return fail(MAXSIM_ERR_INVALID, "null pointer argument");
  // max_q_len sizes the argmax rows; without argmax it only bounds the
  // segment lengths, and any bound >= the number of query rows is the same
  // bound, so it is clamped instead of rejected.
  if (argmax && max_q_len > (1 << 20))
    return fail(MAXSIM_ERR_UNSUPPORTED, "max_q_len too large");
  if (!argmax) max_q_len = std::min<int64_t>(max_q_len, std::max<int64_t>(total_q_tokens, 1));
  if (max_q_len > INT32_MAX)
    return fail(MAXSIM_ERR_UNSUPPORTED, "more than 2^31 - 1 query rows");
  FwdArgs a{};
  a.q = queries;
  a.d = documents;
  a.dim = (int)dim;
  a.mode = kPacked;
  a.npairs = num_pairs;
  a.slots = (int)max_q_len;
  a.qoff = query_offsets;
  a.nq = num_queries;
  a.doff = document_offsets;
  a.nd = num_documents;
  a.qids = pair_query_ids;
  a.dids = pair_document_ids;
  a.total_q = total_q_tokens;
  a.total_d = total_d_tokens;
  a.scores = scores;
  a.argmax = argmax;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (workspace && (reinterpret_cast<uintptr_t>(workspace) & 15u) == 0 &&
      workspace_bytes >= doc_chunk_ws_bytes(num_documents, num_pairs) &&
      doc_chunk_fits(a, dtype, (int)max_q_len))
    return run_doc_chunks(a, dtype, workspace, st);
  return run_pair(a, dtype, (int)max_q_len, st);
}

int maxsim_amd_packed_forward_with_argmax(
    maxsim_dtype dtype, const void* queries, int64_t total_q_tokens,
    const int32_t* query_offsets, int64_t num_queries, const void* documents,
    int64_t total_d_tokens, const int32_t* document_offsets,
    int64_t num_documents, const int32_t* pair_query_ids,
    const int32_t* pair_document_ids, int64_t num_pairs, int64_t dim,
    int64_t max_q_len, float* scores, int32_t* argmax, void* stream) {
  clear_error();
  return packed_forward_impl(dtype, queries, total_q_tokens, query_offsets, num_queries,
                             documents, total_d_tokens, document_offsets, num_documents,
                             pair_query_ids, pair_document_ids, num_pairs, dim, max_q_len,
                             scores, argmax, nullptr, 0, stream);
}

size_t maxsim_amd_packed_forward_workspace_size(int64_t num_documents, int64_t num_pairs) {
  if (num_documents < 0 || num_pairs < 0) return 0;
  return doc_chunk_ws_bytes(num_documents, num_pairs);
}

int maxsim_amd_packed_forward_with_argmax_ws(
    maxsim_dtype dtype, const void* queries, int64_t total_q_tokens,
    const int32_t* query_offsets, int64_t num_queries, const void* documents,
    int64_t total_d_tokens, const int32_t* document_offsets,
    int64_t num_documents, const int32_t* pair_query_ids,
    const int32_t* pair_document_ids, int64_t num_pairs, int64_t dim,
    int64_t max_q_len, float* scores, int32_t* argmax, void* workspace,
    size_t workspace_bytes, void* stream) {
  clear_error();
  return packed_forward_impl(dtype, queries, total_q_tokens, query_offsets, num_queries,
                             documents, total_d_tokens, document_offsets, num_documents,
                             pair_query_ids, pair_document_ids, num_pairs, dim, max_q_len,
                             scores, argmax, workspace, workspace_bytes, stream);
}

int maxsim_amd_forward(maxsim_dtype dtype, const void* queries,
                       int64_t total_q_tokens, const int32_t* query_offsets,
                       int64_t num_queries, const void* documents,
                       int64_t total_d_tokens, const int32_t* document_offsets,
                       int64_t num_documents, const int32_t* pair_query_ids,
                       const int32_t* pair_document_ids, int64_t num_pairs,
                       int64_t dim, int64_t max_q_len, float* scores,
                       void* stream) {
  return maxsim_amd_packed_forward_with_argmax(
      dtype, queries, total_q_tokens, query_offsets, num_queries, documents,
      total_d_tokens, document_offsets, num_documents, pair_query_ids,
      pair_document_ids, num_pairs, dim, max_q_len, scores, nullptr, stream);
}

}  // extern "C"
