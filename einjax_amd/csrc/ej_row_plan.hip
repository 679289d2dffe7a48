// Join and segment plan of a sparse einsum whose operands are both sorted
// relations, row by row, in three launches and without sorting.
//
// The reference joins with a dict and groups the pairs by output coordinate
// with a second dict and a sort (execution/sparse_dispatch.py:29-82,
// :129-171).  When both relations' coordinates are strictly increasing in
// lexicographic order, the rhs's join dims lead, and the output is the lhs's
// leading dims followed by the rhs's dims after its join dims (the structure
// of the dense plan, with a sparse rhs), both results follow row by row, as
// in Gustavson's sparse matrix product:
//  - the lhs tiles that share their output (leading) coordinates form a
//    contiguous run; lhs tile t meets the rhs "row" of its join key J(t), the
//    contiguous range of rhs tiles with that key, in rhs order.  The pairs
//    of the reference's join are therefore run by run, lhs tile by lhs tile,
//    row tile by row tile;
//  - the segments of run r are the distinct free indices F (the rhs dims
//    after the join dims, linearised) among the rows its tiles meet, in
//    ascending order, which is the reference's sorted output order;
//  - segment (r, F) holds one pair for each tile of the run whose row holds
//    F, in lhs order: the reference's accumulation order (pair order).
//
// Launches (all on the caller's stream; each reads what the one before
// wrote):
//  row_index_kernel  the rhs row table rows[J] = first rhs tile whose join
//                    key is >= J (rows[GJ] = n_rhs), one run-start bit per
//                    lhs tile, and the data checks (both relations inside
//                    their grids and strictly increasing, lhs join
//                    coordinates inside the rhs grid); a failure sets bit 0
//                    of scal[6];
//                    It also keeps each rhs tile's free index (fidx);
//  row_count_kernel  per run: its pair count and its number of distinct
//                    free indices (a bitmap in LDS), and per lhs tile its row
//                    (tile_a, tile_len);
//  row_fill_kernel   every block adds up the runs' counts (P, U and the bases
//                    of its own runs); per run: the free-index histogram of
//                    its pairs, its segments (offsets and coordinates) and its
//                    pairs placed stably by free index.  Block 0 publishes the
//                    counts; the last block to finish clears scal[6 .. 7].
// A run's tiles are read kRowChunk at a time into a pair table in LDS, and
// its pairs mapped to their tiles kRowMapWindow at a time (each tile marks
// its first pair, a running maximum fills in the rest); a run of at most
// kRowChunk tiles and kRowCache pairs keeps its pairs' tiles and free
// indices in LDS for both of the fill's walks.
#include "ej_internal.h"

namespace ej {
namespace {

constexpr int kRowThreads = 512;
constexpr int kRowWaves = kRowThreads / 64;
constexpr int kRowMaxLhs = 16384;               // run-start bits held in LDS
constexpr int kRowMaxWords = kRowMaxLhs / 64;
constexpr int kRowMaxFree = 8192;               // free-index bitmap / histogram in LDS
constexpr int64_t kRowMaxJoin = 65536;          // entries of the rhs row table
constexpr int kRowMaxRuns = 8192;
constexpr int kRowMaxBlocks = 1024;             // count / fill blocks (runs strided over them)
constexpr int kRowRunsPerBlock = kRowMaxRuns / kRowMaxBlocks;
constexpr int kRowCountBits = 21;               // P and U in the published word
constexpr int kRowChunk = 1024;                 // run tiles per pair table
constexpr int kRowChunkBits = 10;
constexpr int kRowTPT = kRowChunk / kRowThreads;  // table tiles per thread
constexpr int kRowCache = 8192;                 // pairs of a run kept in LDS between walks
constexpr int kRowQuarterFree = kRowMaxFree / kRowWaves;  // free indices of the per-wave scatter
constexpr int kRowMapWindow = 4096;             // pairs mapped to their tiles at a time
constexpr int kRowLoads = 8;                    // free-index loads per thread in flight
constexpr int kRowPreRuns = 4;                  // run counts per thread loaded up front
static_assert((1 << kRowChunkBits) == kRowChunk, "binary search depth");

// Every count and grid extent fits 32 bits (checked on the host).
struct RowSpec {
  int32_t lncols, rncols;
  int32_t nk;     // join keys: rhs dims 0 .. nk-1
  int32_t nlo;    // output dims taken from the lhs: lhs dims 0 .. nlo-1
  int32_t n_out;  // nlo + (rncols - nk)
  int32_t ldim[EJ_MAX_KEYS];   // lhs dim joined with rhs dim i
  int32_t lgrid[EJ_MAX_DIMS];
  int32_t rgrid[EJ_MAX_DIMS];
  int32_t GJ;       // join keys: prod rgrid[0 .. nk)
  int32_t NK;       // free indices: prod rgrid[nk .. rncols)
  int32_t fbits;    // bits of a free index: NK <= 2^fbits
  int32_t n_lhs, n_rhs;
  int32_t max_runs;  // bound on the runs: min(n_lhs, prod lgrid[0 .. nlo))
  int64_t cap_p, cap_u;
};

__device__ inline int32_t clamp_coord(int32_t c, int32_t g) { return c < 0 ? 0 : (c >= g ? g - 1 : c); }

// Exclusive prefix sum over the block's threads in order, and the block's
// total (the row plan's scans: DPP within waves, LDS across them).  Every
// thread calls it.
__device__ inline int64_t row_block_sum(int64_t v, int64_t *total) {
  __shared__ int64_t wave_tot[kRowWaves];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t inc = wave_inclusive_sum(v);
  if (lane == 63) wave_tot[wave] = inc;
  lds_barrier();
  int64_t off = 0, all = 0;
#pragma unroll
  for (int w = 0; w < kRowWaves; ++w) {
    const int64_t t = wave_tot[w];
    off += w < wave ? t : 0;
    all += t;
  }
  lds_barrier();  // wave_tot is reused by the next call
  *total = all;
  return off + inc - v;
}

// Join key of rhs coordinates (clamped into the grid).
template <int RD>
__device__ inline uint32_t rhs_join_key(const int32_t *cv, const RowSpec &s) {
  uint32_t J = 0;
#pragma unroll
  for (int i = 0; i < RD; ++i)
    if (i < s.nk)
      J = J * static_cast<uint32_t>(s.rgrid[i]) + static_cast<uint32_t>(clamp_coord(cv[i], s.rgrid[i]));
  return J;
}

// Join key of lhs tile t (its join coordinates over the rhs grid, clamped).
__device__ inline uint32_t lhs_join_key(const int32_t *__restrict__ lc, int t, int lncols,
                                        const RowSpec &s) {
  uint32_t J = 0;
  for (int i = 0; i < s.nk; ++i)
    J = J * static_cast<uint32_t>(s.rgrid[i]) +
        static_cast<uint32_t>(clamp_coord(lc[t * lncols + s.ldim[i]], s.rgrid[i]));
  return J;
}

// Rows [a, b) of join key J, clamped into [0, n_rhs] with a <= b, so that
// data that failed a check (the row table then has gaps) stays in bounds.
__device__ inline void row_bounds(const int32_t *__restrict__ rows, uint32_t J, const RowSpec &s,
                                  int *a, int *b) {
  int x = rows[J], y = rows[J + 1];
  x = x < 0 ? 0 : (x > s.n_rhs ? s.n_rhs : x);
  y = y < x ? x : (y > s.n_rhs ? s.n_rhs : y);
  *a = x;
  *b = y;
}

template <int LN, int RN>
__global__ __launch_bounds__(kRowThreads) void row_index_kernel(
    const int32_t *__restrict__ lc, const int32_t *__restrict__ rc, RowSpec s,
    int32_t *__restrict__ rows, unsigned long long *__restrict__ bits, int32_t *__restrict__ fidx,
    int64_t *__restrict__ scal) {
  constexpr int LD = LN ? LN : EJ_MAX_DIMS, RD = RN ? RN : EJ_MAX_DIMS;
  const int lncols = LN ? LN : s.lncols, rncols = RN ? RN : s.rncols;
  const int g = blockIdx.x * kRowThreads + threadIdx.x;
  int bad = 0;
  // ---- rhs tile g: its share of the row table ------------------------------
  if (g < s.n_rhs) {
    int32_t cv[RD], pv[RD];
#pragma unroll
    for (int d = 0; d < RD; ++d) cv[d] = d < rncols ? rc[g * rncols + d] : 0;
#pragma unroll
    for (int d = 0; d < RD; ++d) pv[d] = d < rncols && g > 0 ? rc[(g - 1) * rncols + d] : 0;
#pragma unroll
    for (int d = 0; d < RD; ++d)
      if (d < rncols && (cv[d] < 0 || cv[d] >= s.rgrid[d])) bad = 1;
    if (g > 0) {
      int cmp = 0;
#pragma unroll
      for (int d = 0; d < RD; ++d)
        if (d < rncols && cmp == 0 && cv[d] != pv[d]) cmp = cv[d] < pv[d] ? -1 : 1;
      if (cmp <= 0) bad = 1;  // strictly increasing
    }
    const int J = static_cast<int>(rhs_join_key<RD>(cv, s));
    const int lo = g == 0 ? 0 : static_cast<int>(rhs_join_key<RD>(pv, s)) + 1;
    uint32_t F = 0;
#pragma unroll
    for (int d = 0; d < RD; ++d)
      if (d >= s.nk && d < rncols)
        F = F * static_cast<uint32_t>(s.rgrid[d]) + static_cast<uint32_t>(clamp_coord(cv[d], s.rgrid[d]));
    fidx[g] = static_cast<int32_t>(F);
    for (int x = lo; x <= J; ++x) rows[x] = g;  // keys (J(g-1), J(g)] start at g
    if (g == s.n_rhs - 1)
      for (int x = J + 1; x <= s.GJ; ++x) rows[x] = s.n_rhs;
  }
  // ---- lhs tile g: checks and its run-start bit ----------------------------
  bool newrun = false;
  if (g < s.n_lhs) {
    int32_t cv[LD], pv[LD];
#pragma unroll
    for (int d = 0; d < LD; ++d) cv[d] = d < lncols ? lc[g * lncols + d] : 0;
#pragma unroll
    for (int d = 0; d < LD; ++d) pv[d] = d < lncols && g > 0 ? lc[(g - 1) * lncols + d] : 0;
#pragma unroll
    for (int d = 0; d < LD; ++d)
      if (d < lncols && (cv[d] < 0 || cv[d] >= s.lgrid[d])) bad = 1;
#pragma unroll
    for (int i = 0; i < EJ_MAX_KEYS; ++i)
      if (i < s.nk) {
        int32_t c = 0;
#pragma unroll
        for (int d = 0; d < LD; ++d) c = d == s.ldim[i] ? cv[d] : c;
        if (c >= s.rgrid[i]) bad = 1;  // no rhs row to meet
      }
    newrun = g == 0;
    if (g > 0) {
      int cmp = 0;
#pragma unroll
      for (int d = 0; d < LD; ++d)
        if (d < lncols && cmp == 0 && cv[d] != pv[d]) cmp = cv[d] < pv[d] ? -1 : 1;
      if (cmp <= 0) bad = 1;
#pragma unroll
      for (int d = 0; d < LD; ++d) newrun = newrun || (d < s.nlo && cv[d] != pv[d]);
    }
  }
  const unsigned long long word = __ballot(newrun);
  if ((threadIdx.x & 63) == 0 && g < s.n_lhs) bits[g >> 6] = word;
  if (__syncthreads_or(bad) && threadIdx.x == 0)
    atomicOr(reinterpret_cast<unsigned long long *>(scal + 6), 1ull);
}

// The run-start bits in LDS and the runs started before each word (thread
// tid holds word tid: at most kRowMaxWords <= kRowThreads words); returns
// the number of runs.  Every thread of the block calls it.
static_assert(kRowMaxWords <= kRowThreads, "one run-start word per thread");
__device__ inline int load_runs(const unsigned long long *__restrict__ bits, const RowSpec &s,
                                unsigned long long *sbits, int32_t *wbase) {
  const int tid = threadIdx.x;
  const int nwords = (s.n_lhs + 63) / 64;
  const unsigned long long b = tid < nwords ? bits[tid] : 0ull;
  int64_t total = 0;
  const int64_t before = row_block_sum(__popcll(b), &total);
  if (tid < nwords) {
    sbits[tid] = b;
    wbase[tid] = static_cast<int32_t>(before);
  }
  __syncthreads();
  return static_cast<int>(total);
}

// First lhs tile of run r (r < nruns): the r-th set bit.
__device__ inline int run_first(int r, int nwords, const unsigned long long *sbits,
                                const int32_t *wbase) {
  int lo = 0, hi = nwords - 1;  // last word whose base is <= r
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (wbase[mid] <= r) lo = mid; else hi = mid - 1;
  }
  // the k-th set bit of the word: halve the window by popcounts
  const unsigned long long b = sbits[lo];
  int k = r - wbase[lo], pos = 0;
#pragma unroll
  for (int w = 32; w >= 1; w >>= 1) {
    const int c = __popcll((b >> pos) & ((1ull << w) - 1ull));
    if (k >= c) {
      k -= c;
      pos += w;
    }
  }
  return lo * 64 + pos;
}

// A run's tiles are taken kRowChunk at a time (thread tid holds chunk tiles
// kRowTPT * tid .. + kRowTPT - 1).  The chunk's pair table: row_a[c], the
// rhs tile where chunk tile c's row starts, and pre[c], the chunk's pairs
// before tile c (pre[kRowChunk] = the chunk's pairs; tiles past the chunk's
// end hold no pair).  Every thread calls it; returns the chunk's pair count.
__device__ inline int chunk_table(const int *a, const int *len, int32_t *row_a, int32_t *pre) {
  int loc = 0, lp[kRowTPT];
#pragma unroll
  for (int j = 0; j < kRowTPT; ++j) {
    lp[j] = loc;
    loc += len[j];
  }
  int64_t tot = 0;
  const int base = static_cast<int>(row_block_sum(loc, &tot));
#pragma unroll
  for (int j = 0; j < kRowTPT; ++j) {
    row_a[kRowTPT * threadIdx.x + j] = a[j];
    pre[kRowTPT * threadIdx.x + j] = base + lp[j];
  }
  if (threadIdx.x == 0) pre[kRowChunk] = static_cast<int>(tot);
  __syncthreads();
  return static_cast<int>(tot);
}

// Chunk tile and free index of one chunk pair p < n (the uncached walks of
// long runs; kept small, as they run rarely).
__device__ inline void one_pair(int p, const int32_t *row_a, const int32_t *pre,
                                const int32_t *__restrict__ fidx, int *x, int *f) {
  int lo = 0, hi = kRowChunk - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (pre[mid] <= p) lo = mid; else hi = mid - 1;
  }
  *x = lo;
  *f = fidx[row_a[lo] + (p - pre[lo])];
}

// Inclusive maximum scan of v >= 0 across the 64 lanes of a wave, with DPP
// moves (row shifts within 16 lanes, then the row broadcasts of lanes 15 and
// 31) rather than LDS-routed shuffles.  Lanes a move does not reach take 0.
__device__ inline int wave_inclusive_max(int v) {
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false));  // row_shr:1
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false));  // row_shr:2
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false));  // row_shr:4
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false));  // row_shr:8
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false));  // row_bcast:15
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false));  // row_bcast:31
  return v;
}

// Block-wide exclusive maximum of v (-1 for thread 0); *total = the
// maximum over the block.  Every thread calls it.
__device__ inline int block_exclusive_max(int v, int *total) {
  __shared__ int wave_max[kRowWaves];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int inc = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int o = __shfl_up(inc, d, 64);
    if (lane >= d) inc = max(inc, o);
  }
  if (lane == 63) wave_max[wave] = inc;
  lds_barrier();
  int before = -1, all = -1;
#pragma unroll
  for (int w = 0; w < kRowWaves; ++w) {
    const int m = wave_max[w];
    if (w < wave) before = max(before, m);
    all = max(all, m);
  }
  int ex = __shfl_up(inc, 1, 64);
  if (lane == 0) ex = -1;
  lds_barrier();  // wave_max is reused by the next call
  *total = all;
  return max(before, ex);
}

// Chunk tiles of the chunk pairs [w0, w0 + n).  Each chunk tile with pairs
// marks its first pair (as tile + 1), then a running maximum fills in the
// rest: wave w scans the positions [w * span, (w + 1) * span), 64 at a time
// (lane l on position base + l) and four steps together, so that their LDS
// reads and DPP scans overlap, carrying each step's maximum to the next.
// The waves' carries are joined into wbefore[w] (the maximum before wave
// w's positions); the tile of pair w0 + i is then max(map[i], wbefore[i /
// span]) - 1, which readers form (map_tile).  carry_in is the previous
// window's carry (tile + 1 of pair w0 - 1; 0 for the first window); returns
// this window's.  Work per wave grows with the pairs, not with a fixed number
// of positions per thread.
struct PairMap {
  int span;
  int carry;
};

__device__ inline PairMap map_pairs(int w0, int n, int carry_in, const int32_t *pre, uint16_t *map,
                                    int32_t *wbefore) {
  __shared__ int32_t wcarry[kRowWaves];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int p = tid; p < n; p += kRowThreads) map[p] = 0;
  lds_barrier();
#pragma unroll
  for (int j = 0; j < kRowTPT; ++j) {
    const int c = kRowTPT * tid + j;
    const int a = pre[c], b = pre[c + 1];
    if (b > a && a >= w0 && a < w0 + n) map[a - w0] = static_cast<uint16_t>(c + 1);
  }
  lds_barrier();
  const int span = (n + kRowThreads - 1) / kRowThreads * 64;
  const int q0 = wave * span, q1 = min(n, q0 + span);
  int carry = 0;
  for (int b0 = q0; b0 < q1; b0 += 4 * 64) {  // uniform within the wave
    int v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int p = b0 + 64 * u + lane;
      v[u] = p < q1 ? static_cast<int>(map[p]) : 0;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = wave_inclusive_max(v[u]);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      v[u] = max(v[u], carry);
      carry = __builtin_amdgcn_readlane(v[u], 63);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int p = b0 + 64 * u + lane;
      if (p < q1) map[p] = static_cast<uint16_t>(v[u]);
    }
  }
  if (lane == 0) wcarry[wave] = carry;
  lds_barrier();
  int all = carry_in;
  if (tid < kRowWaves) {
    int before = carry_in;
    for (int w = 0; w < tid; ++w) before = max(before, wcarry[w]);
    wbefore[tid] = before;
  }
#pragma unroll
  for (int w = 0; w < kRowWaves; ++w) all = max(all, wcarry[w]);
  lds_barrier();
  return PairMap{span, all};
}

// The tile of mapped pair i (see map_pairs).
__device__ inline int map_tile(const uint16_t *map, const int32_t *wbefore, int span, int i) {
  return max(static_cast<int>(map[i]), wbefore[i / span]) - 1;
}

template <int LN, int RN>
__global__ __launch_bounds__(kRowThreads) void row_count_kernel(
    const int32_t *__restrict__ lc, RowSpec s, const int32_t *__restrict__ rows,
    const unsigned long long *__restrict__ bits, const int32_t *__restrict__ fidx,
    int32_t *__restrict__ tile_a, int32_t *__restrict__ tile_len, int64_t *__restrict__ run_pc,
    int32_t *__restrict__ run_sc, const int64_t *__restrict__ scal) {
  const int lncols = LN ? LN : s.lncols;
  __shared__ unsigned long long sbits[kRowMaxWords];
  __shared__ int32_t wbase[kRowMaxWords];
  __shared__ uint32_t fmap[kRowMaxFree / 32];
  __shared__ int32_t row_a[kRowChunk], pre[kRowChunk + 1];
  __shared__ uint16_t map[kRowMapWindow];
  __shared__ int32_t wbefore[kRowWaves];
  if (scal[6] != 0) return;  // the data failed a check: nothing to count
  const int tid = threadIdx.x;
  const int nruns = load_runs(bits, s, sbits, wbase);
  const int nwords = (s.n_lhs + 63) / 64;
  const int fwords = (s.NK + 31) / 32;
  for (int r = blockIdx.x; r < nruns && r < s.max_runs; r += gridDim.x) {
    const int rs = run_first(r, nwords, sbits, wbase);
    const int re = r + 1 < nruns ? run_first(r + 1, nwords, sbits, wbase) : s.n_lhs;
    for (int w = tid; w < fwords; w += kRowThreads) fmap[w] = 0;
    int64_t pc = 0;
    for (int tb = rs; tb < re; tb += kRowChunk) {
      uint32_t J[kRowTPT];
      int a[kRowTPT], len[kRowTPT];
#pragma unroll
      for (int j = 0; j < kRowTPT; ++j) {
        const int t = tb + kRowTPT * tid + j;
        J[j] = t < re ? lhs_join_key(lc, t, lncols, s) : 0u;
      }
#pragma unroll
      for (int j = 0; j < kRowTPT; ++j) {
        const int t = tb + kRowTPT * tid + j;
        int b = 0;
        a[j] = 0;
        if (t < re) row_bounds(rows, J[j], s, &a[j], &b);
        len[j] = b - a[j];
      }
      const int cp = chunk_table(a, len, row_a, pre);
#pragma unroll
      for (int j = 0; j < kRowTPT; ++j) {  // stored after the table's barriers
        const int t = tb + kRowTPT * tid + j;
        if (t < re) {
          tile_a[t] = a[j];
          tile_len[t] = len[j];
        }
      }
      for (int w0 = 0, carry = 0; w0 < cp; w0 += kRowMapWindow) {
        const int n = min(kRowMapWindow, cp - w0);
        const PairMap pm = map_pairs(w0, n, carry, pre, map, wbefore);
        carry = pm.carry;
        for (int i0 = 0; i0 < n; i0 += kRowLoads * kRowThreads) {
          int f[kRowLoads];
#pragma unroll
          for (int u = 0; u < kRowLoads; ++u) {
            const int i = i0 + u * kRowThreads + tid;
            const int x = i < n ? map_tile(map, wbefore, pm.span, i) : 0;
            f[u] = i < n ? fidx[row_a[x] + (w0 + i - pre[x])] : -1;
          }
#pragma unroll
          for (int u = 0; u < kRowLoads; ++u)
            if (f[u] >= 0) atomicOr(&fmap[f[u] >> 5], 1u << (f[u] & 31));
        }
        lds_barrier();  // map is rebuilt for the next window
      }
      lds_barrier();  // the table is rebuilt for the next chunk
      pc += cp;
    }
    int mine = 0;
    for (int w = tid; w < fwords; w += kRowThreads) mine += __popc(fmap[w]);
    int64_t sc = 0;
    row_block_sum(mine, &sc);
    if (tid == 0) {
      run_pc[r] = pc;
      run_sc[r] = static_cast<int32_t>(sc);
    }
    lds_barrier();  // fmap is cleared for the next run
  }
}

template <int LN, int RN>
__global__ __launch_bounds__(kRowThreads) void row_fill_kernel(
    const int32_t *__restrict__ lc, RowSpec s, const unsigned long long *__restrict__ bits,
    const int32_t *__restrict__ fidx, const int32_t *__restrict__ tile_a,
    const int32_t *__restrict__ tile_len, const int64_t *__restrict__ run_pc,
    const int32_t *__restrict__ run_sc, int64_t *__restrict__ lidx, int64_t *__restrict__ ridx,
    int32_t *__restrict__ out_coords, int32_t *__restrict__ seg_offsets,
    int64_t *__restrict__ scal, int64_t *__restrict__ host_counts, int64_t ticket) {
  const int lncols = LN ? LN : s.lncols, rncols = RN ? RN : s.rncols;
  __shared__ unsigned long long sbits[kRowMaxWords];
  __shared__ int32_t wbase[kRowMaxWords];
  __shared__ int32_t hist[kRowMaxFree];  // per free index: count, then cursor
  __shared__ int32_t row_a[kRowChunk], pre[kRowChunk + 1];
  __shared__ uint16_t fcache[kRowCache], xcache[kRowCache];  // a cached run's pairs
  __shared__ int32_t wbefore[kRowWaves];
  __shared__ int64_t my_pb[kRowRunsPerBlock], my_pc[kRowRunsPerBlock];
  __shared__ int32_t my_sb[kRowRunsPerBlock];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool failed = scal[6] != 0;
  // The runs' counts, for up to kRowThreads * kRowPreRuns runs loaded before
  // the run-start bits (they do not depend on them).
  const bool pre_counts = s.max_runs <= kRowThreads * kRowPreRuns;
  int64_t pcv[kRowPreRuns];
  int32_t scv[kRowPreRuns];
#pragma unroll
  for (int j = 0; j < kRowPreRuns; ++j) {
    const int r = j * kRowThreads + tid;
    const bool in = !failed && pre_counts && r < s.max_runs;
    pcv[j] = in ? run_pc[r] : 0;
    scv[j] = in ? run_sc[r] : 0;
  }
  int nruns = 0;
  int64_t P = 0, U = 0;
  // The first chunk of this block's first run, loaded beside the counts.
  int pre_a[kRowTPT] = {}, pre_len[kRowTPT] = {};
  if (!failed) {
    nruns = load_runs(bits, s, sbits, wbase);
    if (nruns > s.max_runs) nruns = s.max_runs;  // cannot happen for data inside its grid
    if (static_cast<int>(blockIdx.x) < nruns) {
      const int nwords = (s.n_lhs + 63) / 64;
      const int r = blockIdx.x;
      const int rs = run_first(r, nwords, sbits, wbase);
      const int re = r + 1 < nruns ? run_first(r + 1, nwords, sbits, wbase) : s.n_lhs;
#pragma unroll
      for (int j = 0; j < kRowTPT; ++j) {
        const int t = rs + kRowTPT * tid + j;
        pre_a[j] = t < re ? tile_a[t] : 0;
        pre_len[j] = t < re ? tile_len[t] : 0;
      }
    }
    // P, U and the bases of this block's runs r = blockIdx.x + k * gridDim.x:
    // the runs' counts scanned in steps of kRowThreads runs.
    for (int c = 0, j = 0; c < nruns; c += kRowThreads, ++j) {
      const int r = c + tid;
      int64_t pv = 0, sv = 0;
      if (pre_counts) {
#pragma unroll
        for (int i = 0; i < kRowPreRuns; ++i)
          if (i == j && r < nruns) {
            pv = pcv[i];
            sv = scv[i];
          }
      } else if (r < nruns) {
        pv = run_pc[r];
        sv = run_sc[r];
      }
      int64_t ptot = 0, stot = 0;
      const int64_t pb = row_block_sum(pv, &ptot);
      const int64_t sb = row_block_sum(sv, &stot);
      if (r < nruns && r >= static_cast<int>(blockIdx.x) &&
          (r - static_cast<int>(blockIdx.x)) % static_cast<int>(gridDim.x) == 0) {
        const int k = (r - static_cast<int>(blockIdx.x)) / static_cast<int>(gridDim.x);
        if (k < kRowRunsPerBlock) {
          my_pb[k] = P + pb;
          my_pc[k] = pv;
          my_sb[k] = static_cast<int32_t>(U + sb);
        }
      }
      P += ptot;
      U += stot;
    }
    __syncthreads();
  }
  const int64_t lim = int64_t(1) << kRowCountBits;
  const bool bound = !failed && (P > s.cap_p || U > s.cap_u || P >= lim || U >= lim);
  // ---- counts: published by block 0 (every block holds the same totals) ----
  if (blockIdx.x == 0 && tid == 0) {
    const int64_t flag = (failed ? 1 : 0) | (bound ? 2 : 0);
    const int64_t u_dev = flag ? 0 : U;
    scal[0] = u_dev;
    scal[1] = flag;
    scal[2] = P < s.cap_p ? P : s.cap_p;
    scal[3] = 0;
    scal[4] = P;
    scal[5] = 0;
    if (host_counts) {
      const unsigned long long pw = static_cast<unsigned long long>(P < lim ? P : lim - 1);
      const unsigned long long uw = static_cast<unsigned long long>(U < lim ? U : lim - 1);
      __hip_atomic_store(reinterpret_cast<unsigned long long *>(host_counts + 6),
                         (static_cast<unsigned long long>(ticket) << 44) |
                             (static_cast<unsigned long long>(flag) << 42) | (pw << 21) | uw,
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
  }
  if (!failed && !bound) {
    const int fbits = s.fbits;
    const int NK = s.NK;
    const int nwords = (s.n_lhs + 63) / 64;
    const uint64_t lt = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    for (int r = blockIdx.x, k = 0; r < nruns && k < kRowRunsPerBlock; r += gridDim.x, ++k) {
      const int rs = run_first(r, nwords, sbits, wbase);
      const int re = r + 1 < nruns ? run_first(r + 1, nwords, sbits, wbase) : s.n_lhs;
      const int64_t PB = my_pb[k];
      const int SB = my_sb[k];
      const int npairs = static_cast<int>(my_pc[k]);
      // A run of at most kRowChunk tiles and kRowCache pairs is looked up once:
      // its pairs' free indices and chunk tiles stay in LDS for both walks.
      const bool cached = re - rs <= kRowChunk && npairs <= kRowCache;
      // Cached with at most kRowQuarterFree free indices: wave w places the
      // pairs of part w of the run's kRowWaves equal parts on its own
      // cursors (hist as [kRowWaves][NK]), without barriers between its steps.
      const bool quarters = cached && NK <= kRowQuarterFree;
      const int qlen = (npairs + kRowWaves - 1) / kRowWaves;
      const int hn = quarters ? kRowWaves * NK : NK;
      for (int f = tid; f < hn; f += kRowThreads) hist[f] = 0;
      lds_barrier();
      // The chunk table (one round of loads; the first chunk of the first
      // run was loaded with the counts).
      auto table = [&](int tb) {
        int a[kRowTPT], len[kRowTPT];
#pragma unroll
        for (int j = 0; j < kRowTPT; ++j) {
          const int t = tb + kRowTPT * tid + j;
          a[j] = k == 0 && tb == rs ? pre_a[j] : (t < re ? tile_a[t] : 0);
          len[j] = k == 0 && tb == rs ? pre_len[j] : (t < re ? tile_len[t] : 0);
        }
        return chunk_table(a, len, row_a, pre);
      };
      // Pairs [p0, p0 + kRowThreads) of a chunk (pair order), placed stably
      // by free index: the waves take turns; the lanes of a wave with the
      // same free index (found by ballots over its bits) rank by lane.
      auto place = [&](int tb, int p, bool valid, uint32_t F, int x) {
        uint64_t peers = __ballot(valid);
        for (int b = 0; b < fbits; ++b) {
          const bool bit = (F >> b) & 1u;
          const uint64_t m = __ballot(bit);
          peers &= bit ? m : ~m;
        }
        for (int w = 0; w < kRowWaves; ++w) {
          if (wave == w && valid) {
            const int base = hist[F];
            const int rank = __popcll(peers & lt);
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            if (rank == 0) hist[F] = base + __popcll(peers);
            const int64_t qpos = PB + base + rank;
            lidx[qpos] = tb + x;
            ridx[qpos] = row_a[x] + (p - pre[x]);
          }
          lds_barrier();
        }
      };
      // ---- pass 0: the free-index histogram of the run's pairs --------------
      if (cached) {
        // the run's pairs are positions [0, npairs) of its one chunk; xcache
        // holds each pair's tile
        table(rs);
        const PairMap pm = map_pairs(0, npairs, 0, pre, xcache, wbefore);
        for (int i0 = 0; i0 < npairs; i0 += kRowLoads * kRowThreads) {
          int f[kRowLoads], x[kRowLoads];
#pragma unroll
          for (int u = 0; u < kRowLoads; ++u) {
            const int p = i0 + u * kRowThreads + tid;
            x[u] = p < npairs ? map_tile(xcache, wbefore, pm.span, p) : 0;
            f[u] = p < npairs ? fidx[row_a[x[u]] + (p - pre[x[u]])] : -1;
          }
#pragma unroll
          for (int u = 0; u < kRowLoads; ++u)
            if (f[u] >= 0) {
              const int p = i0 + u * kRowThreads + tid;
              fcache[p] = static_cast<uint16_t>(f[u]);
              xcache[p] = static_cast<uint16_t>(x[u]);  // the tile itself from here on
              atomicAdd(&hist[(quarters ? (p / qlen) * NK : 0) + f[u]], 1);
            }
        }
      } else {
        for (int tb = rs; tb < re; tb += kRowChunk) {
          const int cp = table(tb);
          for (int p = tid; p < cp; p += kRowThreads) {
            int x, f;
            one_pair(p, row_a, pre, fidx, &x, &f);
            atomicAdd(&hist[f], 1);
          }
          lds_barrier();  // the table is rebuilt for the next chunk
        }
      }
      __syncthreads();
      // ---- segments: the free indices present, ascending --------------------
      // Thread tid takes free indices [tid * per, (tid + 1) * per).
      {
        const int per = (NK + kRowThreads - 1) / kRowThreads;
        const int f0 = min(NK, tid * per), f1 = min(NK, f0 + per);
        const int nq = quarters ? kRowWaves : 1;
        auto count = [&](int f) {
          int h = 0;
          for (int w = 0; w < nq; ++w) h += hist[w * NK + f];
          return h;
        };
        int cnt = 0, segs = 0;
        for (int f = f0; f < f1; ++f) {
          const int h = count(f);
          cnt += h;
          segs += h > 0 ? 1 : 0;
        }
        int64_t tot = 0;
        int off = static_cast<int>(row_block_sum(cnt, &tot));
        int u = SB + static_cast<int>(row_block_sum(segs, &tot));
        for (int f = f0; f < f1; ++f) {
          const int h = count(f);
          if (h > 0) {
            seg_offsets[u] = static_cast<int32_t>(PB + off);
            int32_t *oc = out_coords + static_cast<int64_t>(u) * s.n_out;
            for (int d = 0; d < s.nlo; ++d) oc[d] = lc[rs * lncols + d];
            uint32_t rem = static_cast<uint32_t>(f);
            for (int d = rncols - 1; d >= s.nk; --d) {
              const uint32_t gd = static_cast<uint32_t>(s.rgrid[d]), qd = rem / gd;
              oc[s.nlo + (d - s.nk)] = static_cast<int32_t>(rem - qd * gd);
              rem = qd;
            }
            ++u;
          }
          // the cursors of free index f (per quarter), from the run's first pair
          for (int w = 0, c = off; w < nq; ++w) {
            const int hw = hist[w * NK + f];
            hist[w * NK + f] = c;
            c += hw;
          }
          off += h;
        }
        if (r == nruns - 1 && tid == 0) seg_offsets[U] = static_cast<int32_t>(P);
      }
      lds_barrier();
      // ---- pass 1: the pairs, placed stably by free index -------------------
      if (quarters) {
        const int q0 = wave * qlen, q1 = min(npairs, q0 + qlen);
        int32_t *cur = hist + wave * NK;
        // each step reads the next step's pair ahead, so that only the cursor's
        // read and write stay on the step's critical path
        int p = q0 + lane;
        bool valid = p < q1;
        uint32_t F = valid ? fcache[p] : 0u;
        int x = valid ? xcache[p] : 0;
        for (int b0 = q0; b0 < q1; b0 += 64) {  // uniform within the wave
          const int pn = b0 + 64 + lane;
          const bool vn = pn < q1;
          const uint32_t Fn = vn ? fcache[pn] : 0u;
          const int xn = vn ? xcache[pn] : 0;
          const int rt = row_a[x] + (p - pre[x]);
          uint64_t peers = __ballot(valid);
          for (int b = 0; b < fbits; ++b) {
            const bool bit = (F >> b) & 1u;
            const uint64_t m = __ballot(bit);
            peers &= bit ? m : ~m;
          }
          if (valid) {
            const int base = cur[F];
            const int rank = __popcll(peers & lt);
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            if (rank == 0) cur[F] = base + __popcll(peers);
            const int64_t qpos = PB + base + rank;
            lidx[qpos] = rs + x;
            ridx[qpos] = rt;
          }
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // cur before the next step
          p = pn;
          valid = vn;
          F = Fn;
          x = xn;
        }
      } else if (cached) {
        for (int p0 = 0; p0 < npairs; p0 += kRowThreads) {
          const int p = p0 + tid;
          const bool valid = p < npairs;
          place(rs, p, valid, valid ? fcache[p] : 0u,
                valid ? xcache[p] : 0);
        }
      } else {
        for (int tb = rs; tb < re; tb += kRowChunk) {
          const int cp = table(tb);
          for (int p0 = 0; p0 < cp; p0 += kRowThreads) {
            const int p = p0 + tid;
            int x = 0, f = 0;
            if (p < cp) one_pair(p, row_a, pre, fidx, &x, &f);
            place(tb, p, p < cp, static_cast<uint32_t>(f), x);
          }
          lds_barrier();  // the table is rebuilt for the next chunk
        }
      }
      lds_barrier();  // hist and the caches are reused by the next run
    }
  }
  // ---- the last block clears the failure word and the meeting word --------
  if (tid == 0) {
    unsigned long long *meet = reinterpret_cast<unsigned long long *>(scal + 7);
    const unsigned long long prev = atomicAdd(meet, 1ull);
    if (prev == static_cast<unsigned long long>(gridDim.x - 1)) {
      scal[6] = 0;
      scal[7] = 0;  // ready for the next call
    }
  }
}

using RowIndexKernel = void (*)(const int32_t *, const int32_t *, RowSpec, int32_t *,
                                unsigned long long *, int32_t *, int64_t *);
using RowCountKernel = void (*)(const int32_t *, RowSpec, const int32_t *,
                                const unsigned long long *, const int32_t *, int32_t *, int32_t *,
                                int64_t *, int32_t *, const int64_t *);
using RowFillKernel = void (*)(const int32_t *, RowSpec, const unsigned long long *,
                               const int32_t *, const int32_t *, const int32_t *, const int64_t *,
                               const int32_t *, int64_t *, int64_t *, int32_t *, int32_t *,
                               int64_t *, int64_t *, int64_t);

struct RowKernels {
  RowIndexKernel index;
  RowCountKernel count;
  RowFillKernel fill;
};

template <int LN, int RN>
RowKernels row_kernels_t() {
  return {row_index_kernel<LN, RN>, row_count_kernel<LN, RN>, row_fill_kernel<LN, RN>};
}

template <int LN>
RowKernels row_kernels_for_rhs(int rn) {
  switch (rn) {
    case 2: return row_kernels_t<LN, 2>();
    case 3: return row_kernels_t<LN, 3>();
    default: return row_kernels_t<0, 0>();
  }
}

// Specialised for the common ranks (lhs 2 or 3, rhs 2 or 3), else general.
RowKernels row_kernels_for(int ln, int rn) {
  switch (ln) {
    case 2: return row_kernels_for_rhs<2>(rn);
    case 3: return row_kernels_for_rhs<3>(rn);
    default: return row_kernels_t<0, 0>();
  }
}

struct RowWorkspace {
  int32_t *rows;
  unsigned long long *bits;
  int32_t *fidx;
  int32_t *tile_a, *tile_len;
  int64_t *run_pc;
  int32_t *run_sc;
};

size_t row_workspace(void *base, int64_t n_lhs, int64_t n_rhs, int64_t n_join, RowWorkspace *w) {
  Carver c(base);
  RowWorkspace r;
  r.rows = c.take<int32_t>(n_join + 1);
  r.bits = c.take<unsigned long long>((n_lhs + 63) / 64);
  r.fidx = c.take<int32_t>(n_rhs);
  r.tile_a = c.take<int32_t>(n_lhs);
  r.tile_len = c.take<int32_t>(n_lhs);
  r.run_pc = c.take<int64_t>(n_lhs);
  r.run_sc = c.take<int32_t>(n_lhs);
  if (w) *w = r;
  return c.off;
}

}  // namespace
}  // namespace ej

using namespace ej;

extern "C" int ej_row_plan_workspace_size(int64_t n_lhs, int64_t n_rhs, int64_t n_join,
                                          size_t *bytes) {
  clear_error();
  EJ_CHECK_ARG(bytes, "null bytes");
  EJ_CHECK_ARG(n_lhs >= 1 && n_lhs <= kRowMaxLhs, "n_lhs outside [1, %d]", kRowMaxLhs);
  EJ_CHECK_ARG(n_rhs >= 1 && n_rhs < (int64_t(1) << 31), "n_rhs outside [1, 2^31)");
  EJ_CHECK_ARG(n_join >= 1 && n_join <= kRowMaxJoin, "join grid outside [1, %lld]",
               (long long)kRowMaxJoin);
  *bytes = row_workspace(nullptr, n_lhs, n_rhs, n_join, nullptr);
  return EJ_OK;
}

extern "C" int ej_row_plan_async(const int32_t *lhs_coords, int64_t n_lhs, int32_t lhs_ncols,
                                 const int32_t *rhs_coords, int64_t n_rhs, int32_t rhs_ncols,
                                 int32_t n_keys, const int32_t *lhs_dims, const int32_t *rhs_dims,
                                 const int64_t *lhs_grid, const int64_t *rhs_grid, int32_t n_out,
                                 const int32_t *agg_src, const int32_t *agg_dim, int64_t *lhs_idx,
                                 int64_t *rhs_idx, int64_t pair_capacity, int32_t *out_coords,
                                 int32_t *seg_offsets, int64_t seg_capacity, void *workspace,
                                 size_t workspace_bytes, int64_t *dev_counts, int64_t *counts,
                                 int32_t counts_direct, ej_stream_t stream_) {
  clear_error();
  hipStream_t stream = as_stream(stream_);
  EJ_CHECK_ARG(lhs_coords && rhs_coords && lhs_idx && rhs_idx && out_coords && seg_offsets &&
                   workspace && dev_counts && counts && lhs_grid && rhs_grid,
               "null pointer argument");
  EJ_CHECK_ARG(lhs_ncols >= 1 && lhs_ncols <= EJ_MAX_DIMS && rhs_ncols >= 1 &&
                   rhs_ncols <= EJ_MAX_DIMS,
               "coordinate rank outside [1, %d]", EJ_MAX_DIMS);
  EJ_CHECK_ARG(n_keys >= 1 && n_keys <= rhs_ncols && n_keys <= EJ_MAX_KEYS,
               "the row plan needs 1 .. rhs rank join keys");
  EJ_CHECK_ARG(lhs_dims && rhs_dims && (agg_src || n_out == 0) && (agg_dim || n_out == 0),
               "null key arrays");
  EJ_CHECK_ARG(counts_direct >= 0 && counts_direct < (1 << 20),
               "counts_direct (the ticket) outside [0, 2^20)");
  EJ_CHECK_ARG(pair_capacity >= 1 && seg_capacity >= 1, "capacities must be positive");
  RowSpec s{};
  s.lncols = lhs_ncols;
  s.rncols = rhs_ncols;
  s.nk = n_keys;
  int nlo = 0;
  EJ_TRY(run_plan_structure("the row plan", n_keys, lhs_dims, rhs_dims, lhs_ncols, rhs_ncols,
                            n_out, agg_src, agg_dim, s.ldim, &nlo));
  s.nlo = nlo;
  s.n_out = n_out;
  int64_t GJ = 1, NK = 1, runs = 1;
  for (int d = 0; d < rhs_ncols; ++d) {
    EJ_CHECK_ARG(rhs_grid[d] >= 1 && rhs_grid[d] < (int64_t(1) << 31), "bad rhs grid");
    s.rgrid[d] = static_cast<int32_t>(rhs_grid[d]);
    if (d < n_keys) GJ = std::min(GJ * rhs_grid[d], int64_t(1) << 40);
    else NK = std::min(NK * rhs_grid[d], int64_t(1) << 40);
  }
  for (int d = 0; d < lhs_ncols; ++d) {
    EJ_CHECK_ARG(lhs_grid[d] >= 1 && lhs_grid[d] < (int64_t(1) << 31), "bad lhs grid");
    s.lgrid[d] = static_cast<int32_t>(lhs_grid[d]);
    if (d < nlo) runs = std::min(runs * lhs_grid[d], int64_t(1) << 40);
  }
  runs = std::min(runs, n_lhs);
  if (n_lhs < 1 || n_lhs > kRowMaxLhs || n_rhs < 1 || n_rhs >= (int64_t(1) << 31) ||
      GJ > kRowMaxJoin || NK > kRowMaxFree || runs > kRowMaxRuns) {
    set_error("the row plan needs 1 .. %d lhs tiles, a nonempty rhs, at most %lld rhs join "
              "keys, %d free indices and %d runs",
              kRowMaxLhs, (long long)kRowMaxJoin, kRowMaxFree, kRowMaxRuns);
    return EJ_E_UNSUPPORTED;
  }
  s.GJ = static_cast<int32_t>(GJ);
  s.NK = static_cast<int32_t>(NK);
  int fb = 0;
  while ((int64_t(1) << fb) < NK) ++fb;
  s.fbits = fb;
  s.n_lhs = static_cast<int32_t>(n_lhs);
  s.n_rhs = static_cast<int32_t>(n_rhs);
  s.max_runs = static_cast<int32_t>(runs);
  s.cap_p = pair_capacity;
  s.cap_u = seg_capacity;
  RowWorkspace w;
  const size_t need = row_workspace(workspace, n_lhs, n_rhs, GJ, &w);
  if (workspace_bytes < need) {
    set_error("row plan workspace %zu < %zu bytes", workspace_bytes, need);
    return EJ_E_CAPACITY;
  }
  int64_t *direct = nullptr;
  if (counts_direct) EJ_HIP(hipHostGetDevicePointer(reinterpret_cast<void **>(&direct), counts, 0));
  const RowKernels k = row_kernels_for(lhs_ncols, rhs_ncols);
  const int64_t n1 = ceil_div(std::max(n_lhs, n_rhs), kRowThreads);
  hipLaunchKernelGGL(k.index, dim3(static_cast<unsigned>(n1)), dim3(kRowThreads), 0, stream,
                     lhs_coords, rhs_coords, s, w.rows, w.bits, w.fidx, dev_counts);
  EJ_LAUNCH_CHECK();
  const unsigned nb = static_cast<unsigned>(std::min<int64_t>(runs, kRowMaxBlocks));
  hipLaunchKernelGGL(k.count, dim3(nb), dim3(kRowThreads), 0, stream, lhs_coords, s, w.rows,
                     w.bits, w.fidx, w.tile_a, w.tile_len, w.run_pc, w.run_sc, dev_counts);
  EJ_LAUNCH_CHECK();
  hipLaunchKernelGGL(k.fill, dim3(nb), dim3(kRowThreads), 0, stream, lhs_coords, s, w.bits,
                     w.fidx, w.tile_a, w.tile_len, w.run_pc, w.run_sc, lhs_idx, rhs_idx,
                     out_coords, seg_offsets, dev_counts, direct, int64_t(counts_direct));
  EJ_LAUNCH_CHECK();
  if (!direct)
    EJ_HIP(hipMemcpyAsync(counts, dev_counts, 6 * sizeof(int64_t), hipMemcpyDeviceToHost, stream));
  return EJ_OK;
}
