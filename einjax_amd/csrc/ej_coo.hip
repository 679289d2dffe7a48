// COO ingest, COO-to-tile bucketing and per-tile-shape occupancy statistics.
//
// Reference: SparseTensor (tensor/sparse.py:93-231).
//   _extract_coo (:234-270): the elements != 0 of a dense array as int32
//     indices in row-major order (np.nonzero) plus float64 values;
//   to_relation (:160-219) for COO input: entries whose value is 0 are
//     dropped (:184-187), the rest are grouped by tile coordinate in
//     lexicographic order (np.unique(axis=0), :204-206) and scattered into
//     zero tiles (:210-212); an element listed twice keeps its last entry,
//     as numpy's fancy assignment leaves it;
//   _compute_sparsity_metrics (:124-158) for the tile shapes of BaseTensor
//     (tensor/base.py:39-49): num_tuples = number of distinct tile
//     coordinates idx // tile_shape over the nonzero entries, value_count[l]
//     = number of distinct idx[l] // tile_shape[l].
//
// Dense to COO: each wave owns a run of 64 * V * kCooRounds elements (V
// elements = one 16-byte load per lane per round); a count pass, an
// exclusive scan of the per-wave counts and a fill pass that compacts with
// a wave prefix sum keep the row-major order without sorting.
//
// COO to tiles: one 64-bit key per entry, (tile index << wbits) | offset in
// the tile, with dropped entries keyed past every tile; a stable radix sort
// orders the entries by tile, then by element, then by input position;
// tile-start flags and their scan number the tiles; the last entry of each
// run of equal keys writes its value.
//
// Statistics: num_tuples of a tile shape is the number of set bits of its
// occupancy map (one bit per tile of the grid).  The map of a tile shape
// equals the map of a finer tile shape pooled by OR along one dimension:
// every tile shape except (1, ..., 1) has a parent that divides its last
// tile extent above 1 by that extent's smallest prime factor.  The maps are
// built along that tree in depth-first order on a stack inside the
// workspace, so the live maps are the ancestors of the current one (at most
// about twice the finest map).  value_count[l] of a tile shape t is
// num_tuples of the tile shape that equals the tensor shape in every
// dimension except l, where it is t[l]: its grid is one tile wide in every
// other dimension.  Those shapes join the tree.  For COO input, a tile
// shape whose grid has more than bitmap_cap tiles is counted instead by
// sorting the tile keys of the entries and counting distinct keys, and the
// largest maps below the cap are built by marking the entries' tiles.
#include "ej_internal.h"

#include <algorithm>
#include <array>
#include <map>
#include <vector>

namespace ej {
namespace {

// ---- element access (T = double, float, or uint16_t holding bfloat16) ----
__device__ inline bool nz(double x) { return x != 0.0; }  // NaN != 0 holds
__device__ inline bool nz(float x) { return x != 0.0f; }
__device__ inline bool nz(uint16_t x) { return (x & 0x7fffu) != 0; }  // +-0 are zero
__device__ inline double as_f64(double x) { return x; }
__device__ inline double as_f64(float x) { return static_cast<double>(x); }
__device__ inline double as_f64(uint16_t x) {
  return static_cast<double>(__uint_as_float(static_cast<uint32_t>(x) << 16));
}
// Tile element written for a nonzero entry: every dtype is kept.
__device__ inline double tile_val(double x) { return x; }
__device__ inline float tile_val(float x) { return x; }
__device__ inline uint16_t tile_val(uint16_t x) { return x; }

int elem_size(int32_t dtype) { return dtype == EJ_F64 ? 8 : dtype == EJ_F32 ? 4 : 2; }

__device__ inline int wave_sum_i32(int v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, 64);
  return v;
}

__device__ inline int wave_incl_i32(int v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int o = __shfl_up(v, d, 64);
    if (lane >= d) v += o;
  }
  return v;
}

// Adds the block's total of v to *acc: one atomic per 256-thread block.
// Every thread of the block calls it.
__device__ inline void block_add(unsigned long long *acc, int64_t v) {
  __shared__ int64_t part[4];
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, 64);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = v;
  __syncthreads();
  if (threadIdx.x == 0) {
    const int64_t t = part[0] + part[1] + part[2] + part[3];
    if (t) atomicAdd(acc, static_cast<unsigned long long>(t));
  }
}

// Counters of the statistics sit 128 bytes apart, so the atomics of
// different tile shapes never contend for one cache line.
constexpr int64_t kCountStride = 16;

// Number of bytes of w that are nonzero, for bytes holding 0 or 1.
__device__ inline int bytes_set(uint32_t w) { return static_cast<int>((w * 0x01010101u) >> 24); }

// Sets bit t of a bit map for every lane with valid set, with one atomic per
// distinct map word of the wave (skipped when its bits are already set):
// neighbouring entries mostly fall in the same word, which would otherwise
// take one contended atomic per entry.  Every lane of the wave calls it.
__device__ inline void wave_set_bit(uint32_t *map, uint64_t t, bool valid) {
  const int lane = threadIdx.x & 63;
  uint64_t my_word = valid ? (t >> 5) : ~uint64_t(0);
  const uint32_t my_bit = valid ? 1u << (t & 31) : 0u;
  for (;;) {
    const uint64_t active = __ballot(my_word != ~uint64_t(0));
    if (!active) break;
    const int leader = __ffsll(static_cast<unsigned long long>(active)) - 1;
    const uint64_t lw = __shfl(my_word, leader, 64);
    const bool same = my_word == lw;
    uint32_t bits = same ? my_bit : 0u;
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) bits |= __shfl_xor(bits, d, 64);
    if (lane == leader && (map[lw] & bits) != bits) atomicOr(&map[lw], bits);
    if (same) my_word = ~uint64_t(0);
  }
}

template <typename T>
__global__ void fill_zero_kernel(T *p, int64_t n) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (; i < n; i += stride) p[i] = T(0);
}

// Grid-stride launches: at most 32 blocks per CU (one atomic per block).
inline unsigned stride_grid(int64_t work, int64_t cap_blocks = 8192) {
  int64_t g = ceil_div(work > 0 ? work : 1, kBlock);
  return static_cast<unsigned>(g < cap_blocks ? g : cap_blocks);
}

// ---------------------------------------------------------------------------
// Dense to COO.
constexpr int kCooRounds = 4;

template <typename T> constexpr int vec_elems() { return 16 / static_cast<int>(sizeof(T)); }
template <typename T> constexpr int64_t wave_run() {
  return static_cast<int64_t>(kCooRounds) * 64 * vec_elems<T>();
}

struct DenseShape {
  int32_t nd;
  int64_t ext[EJ_MAX_DIMS];
};

// V consecutive elements from index i (a multiple of V); a 16-byte load when
// the base is aligned and the group is whole.
template <typename T>
__device__ inline void load_group(const T *__restrict__ p, int64_t i, int64_t n, bool vec,
                                  T (&v)[vec_elems<T>()]) {
  constexpr int V = vec_elems<T>();
  if (vec && i + V <= n) {
    const uint4 w = *reinterpret_cast<const uint4 *>(p + i);
    __builtin_memcpy(&v[0], &w, 16);
  } else {
#pragma unroll
    for (int k = 0; k < V; ++k) v[k] = i + k < n ? p[i + k] : T(0);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void coo_count_kernel(const T *__restrict__ dense, int64_t n,
                                                        int64_t n_runs, bool vec,
                                                        int64_t *__restrict__ counts) {
  constexpr int V = vec_elems<T>();
  const int lane = threadIdx.x & 63;
  const int64_t s = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (s >= n_runs) return;  // whole waves leave together
  const int64_t base = s * wave_run<T>();
  T v[kCooRounds][V];
#pragma unroll
  for (int r = 0; r < kCooRounds; ++r)
    load_group(dense, base + static_cast<int64_t>(r * 64 + lane) * V, n, vec, v[r]);
  int c = 0;
#pragma unroll
  for (int r = 0; r < kCooRounds; ++r)
#pragma unroll
    for (int k = 0; k < V; ++k) c += nz(v[r][k]) ? 1 : 0;
  c = wave_sum_i32(c);
  if (lane == 0) counts[s] = c;
}

template <typename T>
__global__ __launch_bounds__(256) void coo_fill_kernel(const T *__restrict__ dense, int64_t n,
                                                       int64_t n_runs, bool vec, DenseShape sh,
                                                       const int64_t *__restrict__ excl,
                                                       int64_t nnz_cap,
                                                       int32_t *__restrict__ idx,
                                                       double *__restrict__ vals) {
  constexpr int V = vec_elems<T>();
  const int lane = threadIdx.x & 63;
  const int64_t s = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (s >= n_runs) return;
  const int64_t base = s * wave_run<T>();
  int64_t off = excl[s];
  for (int r = 0; r < kCooRounds; ++r) {
    const int64_t i0 = base + static_cast<int64_t>(r * 64 + lane) * V;
    T v[V];
    load_group(dense, i0, n, vec, v);
    int c = 0;
#pragma unroll
    for (int k = 0; k < V; ++k) c += nz(v[k]) ? 1 : 0;
    const int incl = wave_incl_i32(c);
    const int total = __shfl(incl, 63, 64);
    if (c) {
      int64_t pos = off + incl - c;
      int64_t co[EJ_MAX_DIMS];
      int64_t t = i0;
#pragma unroll
      for (int d = EJ_MAX_DIMS - 1; d >= 0; --d) {
        co[d] = 0;
        if (d < sh.nd) {
          co[d] = t % sh.ext[d];
          t /= sh.ext[d];
        }
      }
#pragma unroll
      for (int k = 0; k < V; ++k) {
        if (nz(v[k]) && pos < nnz_cap) {
#pragma unroll
          for (int d = 0; d < EJ_MAX_DIMS; ++d)
            if (d < sh.nd) idx[pos * sh.nd + d] = static_cast<int32_t>(co[d]);
          vals[pos] = as_f64(v[k]);
          ++pos;
        }
        bool carry = true;  // next element in row-major order
#pragma unroll
        for (int d = EJ_MAX_DIMS - 1; d >= 0; --d) {
          if (d < sh.nd && carry) {
            if (++co[d] == sh.ext[d]) co[d] = 0;
            else carry = false;
          }
        }
      }
    }
    off += total;
  }
}

struct ExtractWs {
  int64_t *scalars, *counts, *excl;
  void *scan_ws;
  size_t bytes;
};

ExtractWs carve_extract(void *base, int64_t n_runs) {
  Carver c(base);
  ExtractWs w;
  w.scalars = c.take<int64_t>(4);
  w.counts = c.take<int64_t>(n_runs);
  w.excl = c.take<int64_t>(n_runs);
  w.scan_ws = c.take<char>(static_cast<int64_t>(scan_workspace_bytes(n_runs)));
  w.bytes = c.off;
  return w;
}

int dense_shape(int32_t ndim, const int64_t *shape, DenseShape *sh, int64_t *n) {
  EJ_CHECK_ARG(ndim >= 1 && ndim <= EJ_MAX_DIMS, "ndim=%d outside [1, %d]", ndim, EJ_MAX_DIMS);
  EJ_CHECK_ARG(shape, "shape is null");
  sh->nd = ndim;
  int64_t total = 1;
  for (int d = 0; d < ndim; ++d) {
    EJ_CHECK_ARG(shape[d] >= 0 && shape[d] <= INT32_MAX, "shape[%d]=%lld outside [0, 2^31)", d,
                 (long long)shape[d]);
    sh->ext[d] = shape[d];
    total *= shape[d];
  }
  *n = total;
  return EJ_OK;
}

int64_t extract_runs(int64_t n, int32_t dtype) {
  const int64_t run = static_cast<int64_t>(kCooRounds) * 64 * (16 / elem_size(dtype));
  return ceil_div(n, run);
}

// ---------------------------------------------------------------------------
// COO to tiles.
struct CooGeom {
  int32_t nd;
  int64_t shape[EJ_MAX_DIMS], tile[EJ_MAX_DIMS], grid[EJ_MAX_DIMS];
  int64_t tile_elems, n_tiles;
  int32_t wbits;      // bits of the offset inside a tile
  int32_t bits;       // key bits the sort orders
  uint64_t sentinel;  // key of a dropped entry: n_tiles << wbits
};

int bits_for(uint64_t values) {  // bits for keys in [0, values)
  int b = 0;
  while (b < 64 && (uint64_t(1) << b) < values) ++b;
  return b;
}

int make_coo_geom(int32_t ndim, const int64_t *shape, const int64_t *tile, CooGeom *g) {
  EJ_CHECK_ARG(ndim >= 1 && ndim <= EJ_MAX_DIMS, "ndim=%d outside [1, %d]", ndim, EJ_MAX_DIMS);
  EJ_CHECK_ARG(shape && tile, "null shape");
  g->nd = ndim;
  unsigned __int128 tiles = 1, elems = 1;
  for (int d = 0; d < ndim; ++d) {
    EJ_CHECK_ARG(tile[d] >= 1 && shape[d] >= 0 && shape[d] <= INT32_MAX,
                 "bad extent in dim %d", d);
    EJ_CHECK_ARG(shape[d] % tile[d] == 0,
                 "tile_shape[%d]=%lld does not evenly divide shape[%d]=%lld", d,
                 (long long)tile[d], d, (long long)shape[d]);
    g->shape[d] = shape[d];
    g->tile[d] = tile[d];
    g->grid[d] = shape[d] / tile[d];
    tiles *= static_cast<uint64_t>(g->grid[d]);
    elems *= static_cast<uint64_t>(tile[d]);
  }
  if (tiles >= (static_cast<unsigned __int128>(1) << 62) ||
      elems >= (static_cast<unsigned __int128>(1) << 62)) {
    set_error("tile grid or tile too large for 64-bit keys");
    return EJ_E_UNSUPPORTED;
  }
  g->n_tiles = static_cast<int64_t>(tiles);
  g->tile_elems = static_cast<int64_t>(elems);
  g->wbits = bits_for(static_cast<uint64_t>(g->tile_elems));
  const int tbits = bits_for(static_cast<uint64_t>(g->n_tiles) + 1);
  if (tbits + g->wbits > 63) {
    set_error("tile index and in-tile offset need %d bits; at most 63 are supported",
              tbits + g->wbits);
    return EJ_E_UNSUPPORTED;
  }
  g->bits = tbits + g->wbits;
  g->sentinel = static_cast<uint64_t>(g->n_tiles) << g->wbits;
  return EJ_OK;
}

template <typename T>
__global__ __launch_bounds__(256) void coo_keys_kernel(const int32_t *__restrict__ idx,
                                                       const T *__restrict__ vals, int64_t nnz,
                                                       CooGeom g, uint64_t *__restrict__ keys,
                                                       int32_t *__restrict__ order,
                                                       int64_t *bad) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= nnz) return;
  uint64_t tkey = 0, wkey = 0;
  bool ok = true;
#pragma unroll
  for (int d = 0; d < EJ_MAX_DIMS; ++d) {
    if (d < g.nd) {
      int64_t c = idx[i * g.nd + d];
      if (c < 0 || c >= g.shape[d]) {
        ok = false;
        c = 0;
      }
      const uint32_t cu = static_cast<uint32_t>(c), tu = static_cast<uint32_t>(g.tile[d]);
      tkey = tkey * static_cast<uint64_t>(g.grid[d]) + cu / tu;
      wkey = wkey * static_cast<uint64_t>(tu) + cu % tu;
    }
  }
  const bool keep = nz(vals[i]);
  if (keep && !ok) *bad = 1;
  keys[i] = keep && ok ? (tkey << g.wbits) | wkey : g.sentinel;
  order[i] = static_cast<int32_t>(i);
}

__global__ __launch_bounds__(256) void coo_tile_flags_kernel(const uint64_t *__restrict__ keys,
                                                             int64_t nnz, uint64_t sentinel,
                                                             int wbits,
                                                             int64_t *__restrict__ flags) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= nnz) return;
  const uint64_t k = keys[i];
  flags[i] = k != sentinel && (i == 0 || (keys[i - 1] >> wbits) != (k >> wbits)) ? 1 : 0;
}

template <typename T, typename U>
__global__ __launch_bounds__(256) void coo_scatter_kernel(
    const uint64_t *__restrict__ keys, const int32_t *__restrict__ order,
    const int64_t *__restrict__ flags, const int64_t *__restrict__ excl,
    const T *__restrict__ vals, int64_t nnz, CooGeom g, int64_t n_tiles,
    int32_t *__restrict__ coords, U *__restrict__ tiles) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= nnz) return;
  const uint64_t k = keys[i];
  if (k == g.sentinel) return;
  const int64_t slot = excl[i] + flags[i] - 1;
  if (slot < 0 || slot >= n_tiles) return;
  if (flags[i]) {
    uint64_t t = k >> g.wbits;
#pragma unroll
    for (int d = EJ_MAX_DIMS - 1; d >= 0; --d) {
      if (d < g.nd) {
        const uint64_t gd = static_cast<uint64_t>(g.grid[d]);
        coords[slot * g.nd + d] = static_cast<int32_t>(t % gd);
        t /= gd;
      }
    }
  }
  if (i + 1 < nnz && keys[i + 1] == k) return;  // a later entry of this element wins
  const uint64_t w = k & ((uint64_t(1) << g.wbits) - 1);
  tiles[slot * g.tile_elems + static_cast<int64_t>(w)] = tile_val(vals[order[i]]);
}

struct CooWs {
  int64_t *scalars;  // [0] tile count, [1] range flag
  uint64_t *keys, *keys_alt;
  int32_t *order, *order_alt;
  int64_t *flags, *excl;
  void *sort_ws, *scan_ws;
  size_t bytes;
};

CooWs carve_coo(void *base, int64_t nnz) {
  Carver c(base);
  CooWs w;
  w.scalars = c.take<int64_t>(4);
  w.keys = c.take<uint64_t>(nnz);
  w.keys_alt = c.take<uint64_t>(nnz);
  w.order = c.take<int32_t>(nnz);
  w.order_alt = c.take<int32_t>(nnz);
  w.flags = c.take<int64_t>(nnz);
  w.excl = c.take<int64_t>(nnz);
  w.sort_ws = c.take<char>(static_cast<int64_t>(sort_workspace_bytes(nnz)));
  w.scan_ws = c.take<char>(static_cast<int64_t>(scan_workspace_bytes(nnz)));
  w.bytes = c.off;
  return w;
}

// COO to tiles without sorting, for fp32 or float64 tiles on grids of at most 2^30
// tiles: every entry marks its tile in a byte-per-tile flag array with a
// plain store (concurrent stores write the same value, and no two tiles
// share a byte, so no atomics); the flags are packed into a bit map whose
// word popcounts are scanned, so a tile's slot is the number of occupied
// tiles before it and slots follow the lexicographic tile order; each
// element of the output takes the value of the largest entry index that
// names it (atomicMax of the index, kept in the output buffer until the
// values are resolved), which is the last entry, as the sorted path keeps it.
constexpr int64_t kCooMapMaxTiles = int64_t(1) << 30;

bool coo_map_path(int32_t dtype, const CooGeom &g) {
  return dtype != EJ_BF16 && g.n_tiles <= kCooMapMaxTiles;
}

struct CooMapWs {
  int64_t *scalars;  // [0] tile count, [1] range flag
  uint8_t *flags;    // one byte per tile, padded to whole map words
  uint32_t *map;
  int64_t *cnt, *prefix;
  void *scan_ws;
  size_t bytes;
};

CooMapWs carve_coo_map(void *base, int64_t n_tiles) {
  const int64_t words = (n_tiles + 31) / 32;
  Carver c(base);
  CooMapWs w;
  w.scalars = c.take<int64_t>(4);
  w.flags = c.take<uint8_t>(words * 32);
  w.map = c.take<uint32_t>(words);
  w.cnt = c.take<int64_t>(words);
  w.prefix = c.take<int64_t>(words);
  w.scan_ws = c.take<char>(static_cast<int64_t>(scan_workspace_bytes(words)));
  w.bytes = c.off;
  return w;
}

// Tile index and in-tile offset of entry i; false for an entry whose value
// is 0, or that lies outside the tensor (then *bad is set).
template <typename T>
__device__ inline bool coo_entry(const int32_t *__restrict__ idx, const T *__restrict__ vals,
                                 int64_t i, const CooGeom &g, int64_t *bad, uint64_t *tile,
                                 uint64_t *within) {
  if (!nz(vals[i])) return false;
  uint64_t tkey = 0, wkey = 0;
  bool ok = true;
#pragma unroll
  for (int d = 0; d < EJ_MAX_DIMS; ++d) {
    if (d < g.nd) {
      const int64_t c = idx[i * g.nd + d];
      if (c < 0 || c >= g.shape[d]) ok = false;
      const uint32_t cu = static_cast<uint32_t>(c), tu = static_cast<uint32_t>(g.tile[d]);
      tkey = tkey * static_cast<uint64_t>(g.grid[d]) + cu / tu;
      wkey = wkey * static_cast<uint64_t>(tu) + cu % tu;
    }
  }
  if (!ok) {
    *bad = 1;
    return false;
  }
  *tile = tkey;
  *within = wkey;
  return true;
}

template <typename T>
__global__ __launch_bounds__(256) void coo_tile_mark_kernel(const int32_t *__restrict__ idx,
                                                            const T *__restrict__ vals,
                                                            int64_t nnz, CooGeom g,
                                                            uint8_t *__restrict__ flags,
                                                            int64_t *bad) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= nnz) return;
  uint64_t t, w;
  if (coo_entry(idx, vals, i, g, bad, &t, &w) && !flags[t]) flags[t] = 1;
}

// Map word j from flags [32j, 32j + 32), and its popcount.
__global__ __launch_bounds__(256) void pack_flags_kernel(const uint8_t *__restrict__ flags,
                                                         int64_t words,
                                                         uint32_t *__restrict__ map,
                                                         int64_t *__restrict__ cnt) {
  const int64_t j = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (j >= words) return;
  const uint4 *src = reinterpret_cast<const uint4 *>(flags + j * 32);
  const uint4 a = src[0], b = src[1];
  const uint32_t f[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  uint32_t bits = 0;
#pragma unroll
  for (int q = 0; q < 8; ++q) {
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if ((f[q] >> (8 * k)) & 0xffu) bits |= 1u << (4 * q + k);
  }
  map[j] = bits;
  cnt[j] = __popc(bits);
}

__global__ void fill_i32_kernel(int32_t *p, int64_t n, int32_t v) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    p[i] = v;
}

__global__ void fill_i64_kernel(long long *p, int64_t n, long long v) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    p[i] = v;
}

// W: the winner's integer type, as wide as the tile element (int32 for fp32
// tiles, long long for float64 tiles), so the winners live in the output.
template <typename T, typename W>
__global__ __launch_bounds__(256) void coo_winner_kernel(const int32_t *__restrict__ idx,
                                                         const T *__restrict__ vals, int64_t nnz,
                                                         CooGeom g,
                                                         const uint32_t *__restrict__ map,
                                                         const int64_t *__restrict__ prefix,
                                                         int64_t n_slots, int64_t *bad,
                                                         W *__restrict__ win) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= nnz) return;
  uint64_t t, w;
  if (!coo_entry(idx, vals, i, g, bad, &t, &w)) return;
  const uint32_t word = map[t >> 5];
  const int64_t slot = prefix[t >> 5] + __popc(word & ((1u << (t & 31)) - 1u));
  if (slot < n_slots) atomicMax(&win[slot * g.tile_elems + static_cast<int64_t>(w)], W(i));
}

// In place: the entry index each element holds becomes that entry's value
// (T, fp32 or float64), or +0.0 where no entry names the element.
template <typename T, typename W>
__global__ __launch_bounds__(256) void coo_resolve_kernel(const T *__restrict__ vals,
                                                          W *__restrict__ tiles, int64_t elems) {
  static_assert(sizeof(T) == sizeof(W), "winners are held in the output elements");
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < elems;
       e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const W wi = tiles[e];
    const T f = wi >= 0 ? tile_val(vals[wi]) : T(0);
    tiles[e] = __builtin_bit_cast(W, f);
  }
}

__global__ __launch_bounds__(256) void coo_map_coords_kernel(const uint32_t *__restrict__ map,
                                                             const int64_t *__restrict__ prefix,
                                                             int64_t words, CooGeom g,
                                                             int64_t n_slots,
                                                             int32_t *__restrict__ coords) {
  const int64_t j = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (j >= words) return;
  uint32_t bits = map[j];
  int64_t slot = prefix[j];
  while (bits && slot < n_slots) {
    const int k = __ffs(bits) - 1;
    uint64_t t = static_cast<uint64_t>(j) * 32 + k;
#pragma unroll
    for (int d = EJ_MAX_DIMS - 1; d >= 0; --d) {
      if (d < g.nd) {
        const uint64_t gd = static_cast<uint64_t>(g.grid[d]);
        coords[slot * g.nd + d] = static_cast<int32_t>(t % gd);
        t /= gd;
      }
    }
    ++slot;
    bits &= bits - 1;
  }
}

// ---------------------------------------------------------------------------
// Statistics.
struct TileIdx {  // mixed-radix tile index of an element for one tile shape
  int32_t nd;
  int64_t shape[EJ_MAX_DIMS];
  int64_t tile[EJ_MAX_DIMS];
  int64_t grid[EJ_MAX_DIMS];
  int64_t cells;  // tiles in the grid
};

// Occupancy maps hold one bit per tile of a grid, row-major, packed into
// 32-bit words (bit i of the map is bit i % 32 of word i / 32); bits past the
// last tile are zero.

template <typename T>
__global__ __launch_bounds__(256) void dense_bits_kernel(const T *__restrict__ dense, int64_t n,
                                                         bool vec, uint32_t *__restrict__ map,
                                                         unsigned long long *count) {
  // Each wave takes chunks of 4 rounds x 64 lanes x E elements, one 16-byte
  // load per lane and round (consecutive lanes read consecutive bytes); the
  // E flag bits of LPW neighbouring lanes are or-ed into one map word by
  // shuffles and stored by the first of them.
  constexpr int E = 16 / static_cast<int>(sizeof(T));  // elements per load
  constexpr int LPW = 32 / E;                           // lanes per map word
  constexpr int R = 4;
  constexpr int64_t CHUNK = int64_t(R) * 64 * E;
  const int lane = threadIdx.x & 63;
  const int64_t words = (n + 31) / 32;
  const int64_t chunks = (n + CHUNK - 1) / CHUNK;
  const int64_t n_waves = static_cast<int64_t>(gridDim.x) * 4;
  int64_t c = 0;
  for (int64_t ch = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6); ch < chunks;
       ch += n_waves) {
    const int64_t base = ch * CHUNK;
    T v[R][E];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t i = base + static_cast<int64_t>(r * 64 + lane) * E;
      if (vec && i + E <= n) {
        const uint4 x = *reinterpret_cast<const uint4 *>(dense + i);
        __builtin_memcpy(&v[r][0], &x, 16);
      } else {
#pragma unroll
        for (int k = 0; k < E; ++k) v[r][k] = i + k < n ? dense[i + k] : T(0);
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      uint32_t b = 0;
#pragma unroll
      for (int k = 0; k < E; ++k) b |= (nz(v[r][k]) ? 1u : 0u) << k;
      b <<= E * (lane % LPW);
#pragma unroll
      for (int d = 1; d < LPW; d <<= 1) b |= __shfl_xor(b, d, 64);
      const int64_t widx = (base + static_cast<int64_t>(r * 64 + lane) * E) >> 5;
      if (lane % LPW == 0 && widx < words) {
        map[widx] = b;
        c += __popc(b);
      }
    }
  }
  block_add(count, c);
}

// Pooling by OR: in [outer][n_out * p][inner] -> out [outer][n_out][inner],
// sizes in tiles (bits).
struct PoolGeom {
  int64_t outer, n_out, p, inner, total;  // total = outer * n_out * inner
};

// inner % 128 == 0: 128 outputs (one 16-byte vector) per thread.
template <typename I>
__global__ __launch_bounds__(256) void pool_bits_vec_kernel(const uint32_t *__restrict__ in,
                                                            uint32_t *__restrict__ out,
                                                            PoolGeom g, unsigned long long *count) {
  const I vecs = static_cast<I>(g.total / 128);
  const I inner = static_cast<I>(g.inner), n_out = static_cast<I>(g.n_out),
          p = static_cast<I>(g.p);
  int64_t c = 0;
  for (I w = static_cast<I>(blockIdx.x) * blockDim.x + threadIdx.x; w < vecs;
       w += static_cast<I>(gridDim.x) * blockDim.x) {
    const I o = w * 128;
    const I r = o % inner, t = o / inner;
    const I j = t % n_out, a = t / n_out;
    const uint4 *src = reinterpret_cast<const uint4 *>(in) + ((a * n_out + j) * p * inner + r) / 128;
    const I step = inner / 128;
    uint4 acc = make_uint4(0u, 0u, 0u, 0u);
    for (I q = 0; q < p; ++q) {
      const uint4 x = src[q * step];
      acc.x |= x.x;
      acc.y |= x.y;
      acc.z |= x.z;
      acc.w |= x.w;
    }
    reinterpret_cast<uint4 *>(out)[w] = acc;
    c += __popc(acc.x) + __popc(acc.y) + __popc(acc.z) + __popc(acc.w);
  }
  block_add(count, c);
}

// inner % 32 == 0: one output word per thread.
template <typename I>
__global__ __launch_bounds__(256) void pool_bits_word_kernel(const uint32_t *__restrict__ in,
                                                             uint32_t *__restrict__ out,
                                                             PoolGeom g,
                                                             unsigned long long *count) {
  const I words = static_cast<I>(g.total / 32);
  const I inner = static_cast<I>(g.inner), n_out = static_cast<I>(g.n_out),
          p = static_cast<I>(g.p);
  int64_t c = 0;
  for (I w = static_cast<I>(blockIdx.x) * blockDim.x + threadIdx.x; w < words;
       w += static_cast<I>(gridDim.x) * blockDim.x) {
    const I o = w * 32;
    const I r = o % inner, t = o / inner;
    const I j = t % n_out, a = t / n_out;
    const uint32_t *src = in + ((a * n_out + j) * p * inner + r) / 32;
    const I step = inner / 32;
    uint32_t acc = 0;
    for (I q = 0; q < p; ++q) acc |= src[q * step];
    out[w] = acc;
    c += __popc(acc);
  }
  block_add(count, c);
}

// Any geometry: one output word per thread, assembled bit by bit.
__global__ __launch_bounds__(256) void pool_bits_any_kernel(const uint32_t *__restrict__ in,
                                                            uint32_t *__restrict__ out,
                                                            PoolGeom g,
                                                            unsigned long long *count) {
  const int64_t words = (g.total + 31) / 32;
  int64_t c = 0;
  for (int64_t w = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; w < words;
       w += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    uint32_t acc = 0;
    for (int b = 0; b < 32; ++b) {
      const int64_t o = w * 32 + b;
      if (o >= g.total) break;
      const int64_t r = o % g.inner, t = o / g.inner;
      const int64_t j = t % g.n_out, a = t / g.n_out;
      const int64_t i0 = (a * g.n_out + j) * g.p * g.inner + r;
      uint32_t any = 0;
      for (int64_t q = 0; q < g.p && !any; ++q) {
        const int64_t i = i0 + q * g.inner;
        any = (in[i >> 5] >> (i & 31)) & 1u;
      }
      acc |= any << b;
    }
    out[w] = acc;
    c += __popc(acc);
  }
  block_add(count, c);
}

// Power-of-two pooling along the last dimension, counted without writing
// the maps: each wave reads 16384 consecutive map bits (256 per lane, four
// 64-bit words) and counts the nonempty groups of 2^k bits for k = 1 ..
// levels (<= 14) into count[k - 1]; groups never cross a row because
// 2^levels divides the row length.  Levels 1-6 are folded inside each word,
// 7-8 across a lane's four words, 9-14 across the wave's ballot; waves need
// no barrier.  With write_level == 14 the map pooled by 2^14 (one bit per
// wave chunk) is or-ed into out, which the caller zeroes, for the next pass
// of a longer chain.
constexpr int kChainMax = 14;
constexpr int64_t kChainChunk = int64_t(64) * 256;  // bits per wave chunk

struct ChainArgs {
  int32_t levels;
  int32_t write_level;
  unsigned long long *count[kChainMax];
};

// Bits at positions that are multiples of 2^k, k = 1 .. 6.
__device__ inline uint64_t level_mask(int k) {
  switch (k) {
    case 1: return 0x5555555555555555ull;
    case 2: return 0x1111111111111111ull;
    case 3: return 0x0101010101010101ull;
    case 4: return 0x0001000100010001ull;
    case 5: return 0x0000000100000001ull;
    default: return 0x0000000000000001ull;
  }
}

__global__ __launch_bounds__(256) void pool_chain_kernel(const uint32_t *__restrict__ in,
                                                         int64_t S, ChainArgs a,
                                                         uint32_t *__restrict__ out) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int64_t cnt[kChainMax];
#pragma unroll
  for (int k = 0; k < kChainMax; ++k) cnt[k] = 0;
  const int64_t chunks = (S + kChainChunk - 1) / kChainChunk;
  const int64_t n_waves = static_cast<int64_t>(gridDim.x) * 4;
  for (int64_t ch = static_cast<int64_t>(blockIdx.x) * 4 + wave; ch < chunks; ch += n_waves) {
    const int64_t base = ch * kChainChunk + static_cast<int64_t>(lane) * 256;
    uint64_t m[4] = {0, 0, 0, 0};
    if (base + 256 <= S) {
      const uint4 *src = reinterpret_cast<const uint4 *>(in) + (base >> 7);
      const uint4 v0 = src[0], v1 = src[1];
      m[0] = static_cast<uint64_t>(v0.x) | static_cast<uint64_t>(v0.y) << 32;
      m[1] = static_cast<uint64_t>(v0.z) | static_cast<uint64_t>(v0.w) << 32;
      m[2] = static_cast<uint64_t>(v1.x) | static_cast<uint64_t>(v1.y) << 32;
      m[3] = static_cast<uint64_t>(v1.z) | static_cast<uint64_t>(v1.w) << 32;
    } else if (base < S) {
      // the map allocation is padded to 256 bytes: these words are inside it
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t b = base + 64 * r;
        if (b < S) {
          m[r] = reinterpret_cast<const uint64_t *>(in)[b >> 6];
          if (S - b < 64) m[r] &= (uint64_t(1) << (S - b)) - 1;
        }
      }
    }
    uint64_t g[4] = {m[0], m[1], m[2], m[3]};
#pragma unroll
    for (int k = 1; k <= 6; ++k) {
      int c = 0;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        g[r] = (g[r] | (g[r] >> (1 << (k - 1)))) & level_mask(k);
        c += __popcll(g[r]);
      }
      cnt[k - 1] += c;
    }
    // g[r] now holds bit 0 = word r nonempty
    cnt[6] += (g[0] | g[1]) + (g[2] | g[3]);
    const bool any = (g[0] | g[1] | g[2] | g[3]) != 0;
    cnt[7] += any ? 1 : 0;
    const uint64_t B = __ballot(any);
    uint64_t gb = B;
#pragma unroll
    for (int k = 9; k <= 14; ++k) {
      gb = (gb | (gb >> (1 << (k - 9)))) & level_mask(k - 8);
      if (lane == 0) cnt[k - 1] += __popcll(gb);
    }
    if (a.write_level == kChainMax && lane == 0 && B != 0)
      atomicOr(&out[ch >> 5], 1u << (ch & 31));
  }
  // Block totals (levels 1-8 summed over the lanes, 9-14 held by lane 0),
  // then one atomic per level and block.
  __shared__ int64_t part[4][kChainMax];
#pragma unroll
  for (int k = 0; k < kChainMax; ++k) {
    int64_t v = cnt[k];
    if (k < 8) {
#pragma unroll
      for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, 64);
    }
    if (lane == 0) part[wave][k] = v;
  }
  __syncthreads();
  if (threadIdx.x < kChainMax && static_cast<int>(threadIdx.x) < a.levels) {
    const int k = threadIdx.x;
    const int64_t t = part[0][k] + part[1][k] + part[2][k] + part[3][k];
    if (t) atomicAdd(a.count[k], static_cast<unsigned long long>(t));
  }
}

// A run of poolings by 2 along the next-to-last dimension, each pooled map
// counted along its last-dimension chain, in one pass: each wave takes one
// 16384-bit chunk (256 bits per lane) of 2^H consecutive rows of the input
// map (a row = the last dimension's map bits, a multiple of 16384), ors them
// pairwise level by level in registers, counts the nonempty groups of 2^k
// bits of every pooled row for k = 1 .. levels[h] as pool_chain_kernel does
// (and, for h >= 1, the pooled map's own bits), and writes only the level-H
// row.  Level 0's chain is counted when `first` is set (its map's own bits
// were counted by its producer).  Counts: per lane, then one atomic per
// counter and block.
constexpr int kBandMax = 3;  // row levels per launch: bands of 8 rows

struct BandArgs {
  int32_t H, first;
  int32_t levels[kBandMax + 1];
  int64_t rows_out, row_bits;
  unsigned long long *chain[kBandMax + 1][kChainMax];
  unsigned long long *pop[kBandMax + 1];
};

__global__ __launch_bounds__(256) void band_chain_kernel(const uint32_t *__restrict__ in,
                                                         BandArgs a, uint32_t *__restrict__ out) {
  constexpr int NR = 1 << kBandMax;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int H = a.H, nb = 1 << H;
  const int64_t cpr = a.row_bits / kChainChunk;  // chunks per row
  const int64_t items = a.rows_out * cpr;
  uint32_t cnt[kBandMax + 1][kChainMax + 1];  // [h][0]: the map's bits, [h][k]: chain level k
#pragma unroll
  for (int h = 0; h <= kBandMax; ++h)
#pragma unroll
    for (int k = 0; k <= kChainMax; ++k) cnt[h][k] = 0;
  auto count = [&](const uint64_t (&m)[4], int h) {
    cnt[h][0] += __popcll(m[0]) + __popcll(m[1]) + __popcll(m[2]) + __popcll(m[3]);
    uint64_t g[4] = {m[0], m[1], m[2], m[3]};
#pragma unroll
    for (int k = 1; k <= 6; ++k) {
      uint32_t c = 0;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        g[r] = (g[r] | (g[r] >> (1 << (k - 1)))) & level_mask(k);
        c += __popcll(g[r]);
      }
      cnt[h][k] += c;
    }
    cnt[h][7] += static_cast<uint32_t>((g[0] | g[1]) + (g[2] | g[3]));
    const bool any = (g[0] | g[1] | g[2] | g[3]) != 0;
    cnt[h][8] += any ? 1u : 0u;
    uint64_t gb = __ballot(any);
#pragma unroll
    for (int k = 9; k <= 14; ++k) {
      gb = (gb | (gb >> (1 << (k - 9)))) & level_mask(k - 8);
      if (lane == 0) cnt[h][k] += __popcll(gb);
    }
  };
  const int64_t n_waves = static_cast<int64_t>(gridDim.x) * 4;
  for (int64_t it = static_cast<int64_t>(blockIdx.x) * 4 + wave; it < items; it += n_waves) {
    const int64_t band = it / cpr, c = it - band * cpr;
    uint64_t m[NR][4];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      if (r < nb) {
        const uint4 *src = reinterpret_cast<const uint4 *>(in) +
                           ((band * nb + r) * a.row_bits + c * kChainChunk + lane * 256) / 128;
        const uint4 v0 = src[0], v1 = src[1];
        m[r][0] = static_cast<uint64_t>(v0.x) | static_cast<uint64_t>(v0.y) << 32;
        m[r][1] = static_cast<uint64_t>(v0.z) | static_cast<uint64_t>(v0.w) << 32;
        m[r][2] = static_cast<uint64_t>(v1.x) | static_cast<uint64_t>(v1.y) << 32;
        m[r][3] = static_cast<uint64_t>(v1.z) | static_cast<uint64_t>(v1.w) << 32;
      }
    }
    if (a.first) {
#pragma unroll
      for (int r = 0; r < NR; ++r)
        if (r < nb) count(m[r], 0);
    }
#pragma unroll
    for (int h = 1; h <= kBandMax; ++h) {
      if (h <= H) {
#pragma unroll
        for (int i = 0; i < (NR >> h); ++i) {
          if (i < (nb >> h)) {
#pragma unroll
            for (int q = 0; q < 4; ++q) m[i][q] = m[2 * i][q] | m[2 * i + 1][q];
            count(m[i], h);
          }
        }
      }
    }
    uint4 *dst = reinterpret_cast<uint4 *>(out) + (band * a.row_bits + c * kChainChunk + lane * 256) / 128;
    dst[0] = make_uint4(static_cast<uint32_t>(m[0][0]), static_cast<uint32_t>(m[0][0] >> 32),
                        static_cast<uint32_t>(m[0][1]), static_cast<uint32_t>(m[0][1] >> 32));
    dst[1] = make_uint4(static_cast<uint32_t>(m[0][2]), static_cast<uint32_t>(m[0][2] >> 32),
                        static_cast<uint32_t>(m[0][3]), static_cast<uint32_t>(m[0][3] >> 32));
  }
  // Block totals: bits and levels 1-8 summed over the lanes, 9-14 held by lane 0.
  __shared__ unsigned long long part[4][kBandMax + 1][kChainMax + 1];
#pragma unroll
  for (int h = 0; h <= kBandMax; ++h)
#pragma unroll
    for (int k = 0; k <= kChainMax; ++k) {
      unsigned long long v = cnt[h][k];
      if (k <= 8) {
#pragma unroll
        for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, 64);
      }
      if (lane == 0) part[wave][h][k] = v;
    }
  __syncthreads();
  for (int e = threadIdx.x; e < (kBandMax + 1) * (kChainMax + 1); e += 256) {
    const int h = e / (kChainMax + 1), k = e % (kChainMax + 1);
    if (h > H) continue;
    unsigned long long *dst = nullptr;
    if (k == 0) dst = h >= 1 ? a.pop[h] : nullptr;
    else if (k <= a.levels[h] && (h >= 1 || a.first)) dst = a.chain[h][k - 1];
    const unsigned long long t = part[0][h][k] + part[1][h][k] + part[2][h][k] + part[3][h][k];
    if (dst && t) atomicAdd(dst, t);
  }
}

// The same for map rows shorter than a chunk (256 .. 8192 bits, whole
// chunks in the map): a chunk holds 16384 / row_bits consecutive rows, row r
// in lanes [r lpr, (r + 1) lpr) with lpr = row_bits / 256, and 2^H <= that
// many rows form a band inside it.  Level h ors each lane with the lane
// lpr 2^(h-1) away (every lane of a group of 2^h rows then holds the group's
// or); the first row's lanes of each group count it, the others are masked.
__global__ __launch_bounds__(256) void band_chain_small_kernel(const uint32_t *__restrict__ in,
                                                               BandArgs a,
                                                               uint32_t *__restrict__ out) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int H = a.H;
  const int lpr = static_cast<int>(a.row_bits / 256);
  const int row = lane / lpr;
  const int64_t chunks = (a.rows_out << H) * a.row_bits / kChainChunk;
  uint32_t cnt[kBandMax + 1][kChainMax + 1];
#pragma unroll
  for (int h = 0; h <= kBandMax; ++h)
#pragma unroll
    for (int k = 0; k <= kChainMax; ++k) cnt[h][k] = 0;
  auto count = [&](const uint64_t (&m)[4], bool live, int h) {
    uint64_t g[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) g[r] = live ? m[r] : 0;
    cnt[h][0] += __popcll(g[0]) + __popcll(g[1]) + __popcll(g[2]) + __popcll(g[3]);
#pragma unroll
    for (int k = 1; k <= 6; ++k) {
      uint32_t c = 0;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        g[r] = (g[r] | (g[r] >> (1 << (k - 1)))) & level_mask(k);
        c += __popcll(g[r]);
      }
      cnt[h][k] += c;
    }
    cnt[h][7] += static_cast<uint32_t>((g[0] | g[1]) + (g[2] | g[3]));
    const bool any = (g[0] | g[1] | g[2] | g[3]) != 0;
    cnt[h][8] += any ? 1u : 0u;
    uint64_t gb = __ballot(any);
#pragma unroll
    for (int k = 9; k <= 14; ++k) {
      gb = (gb | (gb >> (1 << (k - 9)))) & level_mask(k - 8);
      if (lane == 0) cnt[h][k] += __popcll(gb);
    }
  };
  auto xor_lanes = [](uint64_t v, int d) {
    const uint32_t lo = __shfl_xor(static_cast<uint32_t>(v), d, 64);
    const uint32_t hi = __shfl_xor(static_cast<uint32_t>(v >> 32), d, 64);
    return static_cast<uint64_t>(lo) | static_cast<uint64_t>(hi) << 32;
  };
  const int64_t n_waves = static_cast<int64_t>(gridDim.x) * 4;
  for (int64_t ch = static_cast<int64_t>(blockIdx.x) * 4 + wave; ch < chunks; ch += n_waves) {
    const uint4 *src = reinterpret_cast<const uint4 *>(in) + (ch * kChainChunk + lane * 256) / 128;
    const uint4 v0 = src[0], v1 = src[1];
    uint64_t m[4];
    m[0] = static_cast<uint64_t>(v0.x) | static_cast<uint64_t>(v0.y) << 32;
    m[1] = static_cast<uint64_t>(v0.z) | static_cast<uint64_t>(v0.w) << 32;
    m[2] = static_cast<uint64_t>(v1.x) | static_cast<uint64_t>(v1.y) << 32;
    m[3] = static_cast<uint64_t>(v1.z) | static_cast<uint64_t>(v1.w) << 32;
    if (a.first) count(m, true, 0);
#pragma unroll
    for (int h = 1; h <= kBandMax; ++h) {
      if (h <= H) {
#pragma unroll
        for (int q = 0; q < 4; ++q) m[q] |= xor_lanes(m[q], lpr << (h - 1));
        count(m, (row & ((1 << h) - 1)) == 0, h);
      }
    }
    if ((row & ((1 << H) - 1)) == 0) {
      const int64_t bit = ch * (kChainChunk >> H) + static_cast<int64_t>(row >> H) * a.row_bits +
                          static_cast<int64_t>(lane % lpr) * 256;
      uint4 *dst = reinterpret_cast<uint4 *>(out) + bit / 128;
      dst[0] = make_uint4(static_cast<uint32_t>(m[0]), static_cast<uint32_t>(m[0] >> 32),
                          static_cast<uint32_t>(m[1]), static_cast<uint32_t>(m[1] >> 32));
      dst[1] = make_uint4(static_cast<uint32_t>(m[2]), static_cast<uint32_t>(m[2] >> 32),
                          static_cast<uint32_t>(m[3]), static_cast<uint32_t>(m[3] >> 32));
    }
  }
  __shared__ unsigned long long part[4][kBandMax + 1][kChainMax + 1];
#pragma unroll
  for (int h = 0; h <= kBandMax; ++h)
#pragma unroll
    for (int k = 0; k <= kChainMax; ++k) {
      unsigned long long v = cnt[h][k];
      if (k <= 8) {
#pragma unroll
        for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, 64);
      }
      if (lane == 0) part[wave][h][k] = v;
    }
  __syncthreads();
  for (int e = threadIdx.x; e < (kBandMax + 1) * (kChainMax + 1); e += 256) {
    const int h = e / (kChainMax + 1), k = e % (kChainMax + 1);
    if (h > H) continue;
    unsigned long long *dst = nullptr;
    if (k == 0) dst = h >= 1 ? a.pop[h] : nullptr;
    else if (k <= a.levels[h] && (h >= 1 || a.first)) dst = a.chain[h][k - 1];
    const unsigned long long t = part[0][h][k] + part[1][h][k] + part[2][h][k] + part[3][h][k];
    if (dst && t) atomicAdd(dst, t);
  }
}

// Tile index of entry i for the tile shape in ti; false when the entry is
// dropped (value 0) or lies outside the tensor (then *bad is set).
template <typename T>
__device__ inline bool entry_tile(const int32_t *__restrict__ idx, const T *__restrict__ vals,
                                  int64_t i, const TileIdx &ti, int64_t *bad, uint64_t *tile) {
  if (!nz(vals[i])) return false;
  uint64_t t = 0;
  bool ok = true;
#pragma unroll
  for (int d = 0; d < EJ_MAX_DIMS; ++d) {
    if (d < ti.nd) {
      const int64_t c = idx[i * ti.nd + d];
      if (c < 0 || c >= ti.shape[d]) ok = false;
      t = t * static_cast<uint64_t>(ti.grid[d]) +
          static_cast<uint32_t>(c) / static_cast<uint32_t>(ti.tile[d]);
    }
  }
  if (!ok) {
    *bad = 1;
    return false;
  }
  *tile = t;
  return true;
}

template <typename T>
__global__ __launch_bounds__(256) void coo_mark_kernel(const int32_t *__restrict__ idx,
                                                       const T *__restrict__ vals, int64_t nnz,
                                                       TileIdx ti, uint32_t *__restrict__ map,
                                                       int64_t *bad) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  uint64_t t = 0;
  const bool keep = i < nnz && entry_tile(idx, vals, i, ti, bad, &t);
  wave_set_bit(map, t, keep);
}

__global__ __launch_bounds__(256) void map_count_kernel(const uint32_t *__restrict__ words,
                                                        int64_t n_words,
                                                        unsigned long long *count) {
  int64_t c = 0;
  for (int64_t w = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; w < n_words;
       w += static_cast<int64_t>(gridDim.x) * blockDim.x)
    c += __popc(words[w]);
  block_add(count, c);
}

template <typename T>
__global__ __launch_bounds__(256) void stat_keys_kernel(const int32_t *__restrict__ idx,
                                                        const T *__restrict__ vals, int64_t nnz,
                                                        TileIdx ti, uint64_t *__restrict__ keys,
                                                        int64_t *bad) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= nnz) return;
  uint64_t t;
  keys[i] = entry_tile(idx, vals, i, ti, bad, &t) ? t : static_cast<uint64_t>(ti.cells);
}

__global__ __launch_bounds__(256) void distinct_count_kernel(const uint64_t *__restrict__ keys,
                                                             int64_t nnz, uint64_t sentinel,
                                                             unsigned long long *count) {
  int64_t c = 0;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < nnz;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const uint64_t k = keys[i];
    c += k != sentinel && (i == 0 || keys[i - 1] != k) ? 1 : 0;
  }
  block_add(count, c);
}

// ---- the plan --------------------------------------------------------------
// kChain: a power-of-two last tile extent pooled from its parent by 2 along
// the last dimension; counted by pool_chain_kernel from the nearest
// materialised ancestor, never materialised itself.
enum NodeKind { kDenseRoot, kCooRoot, kPool, kSorted, kChain };

struct StatNode {
  std::array<int64_t, EJ_MAX_DIMS> ts;
  int64_t cells = 1;   // tiles in the grid
  int parent = -1;
  int pdim = -1;       // dimension pooled from the parent
  int64_t pfac = 1;    // pooling factor
  int kind = kPool;
  std::vector<int> kids;
  size_t off = 0;      // map offset on the stack
  size_t tmp_off = 0;  // chain maps of a chain longer than kChainMax levels
};

struct StatsPlan {
  int nd = 0;
  int64_t shape[EJ_MAX_DIMS] = {};
  std::vector<StatNode> nodes;
  std::vector<int> req;   // node of each requested tile shape
  std::vector<int> proj;  // node of (scheme, dim): value_count source
  std::vector<int> roots; // map roots in execution order
  size_t stack_bytes = 0;
  bool any_sorted = false;
};

// Ascending prime factors of n (trial division once per dimension).
std::vector<int64_t> prime_factors(int64_t n) {
  std::vector<int64_t> ps;
  for (int64_t p = 2; p * p <= n; ++p) {
    if (n % p == 0) {
      ps.push_back(p);
      while (n % p == 0) n /= p;
    }
  }
  if (n > 1) ps.push_back(n);
  return ps;
}

// Chain nodes below v, in level order.
std::vector<int> chain_of(const StatsPlan &pl, int v) {
  std::vector<int> c;
  int cur = v;
  for (;;) {
    int next = -1;
    for (int k : pl.nodes[cur].kids)
      if (pl.nodes[k].kind == kChain) next = k;
    if (next < 0) break;
    c.push_back(next);
    cur = next;
  }
  return c;
}

// Bytes of a map of `cells` bits: whole 32-bit words, padded to 256 bytes.
size_t map_bytes(int64_t cells) {
  return align_up(static_cast<size_t>((cells + 31) / 32) * 4, 256);
}

void layout(StatsPlan &pl, int v, size_t base) {
  StatNode &nd = pl.nodes[v];
  nd.off = base;
  size_t top = base + map_bytes(nd.cells);
  // maps handed from one chain kernel to the next
  nd.tmp_off = top;
  const size_t levels = chain_of(pl, v).size();
  int64_t cells = nd.cells;
  for (size_t done = kChainMax; done < levels; done += kChainMax) {
    cells >>= kChainMax;
    top += map_bytes(cells);
  }
  if (top > pl.stack_bytes) pl.stack_bytes = top;
  for (int k : pl.nodes[v].kids)
    if (pl.nodes[k].kind != kChain) layout(pl, k, top);
}

// dense: nnz < 0.  cap: largest map in bytes for COO input (<= 0: default).
int make_plan(int32_t ndim, const int64_t *shape, int64_t n_schemes, const int64_t *tile_shapes,
              bool dense, int64_t cap, StatsPlan *pl) {
  EJ_CHECK_ARG(ndim >= 1 && ndim <= EJ_MAX_DIMS, "ndim=%d outside [1, %d]", ndim, EJ_MAX_DIMS);
  EJ_CHECK_ARG(shape, "shape is null");
  EJ_CHECK_ARG(n_schemes >= 0, "n_schemes < 0");
  EJ_CHECK_ARG(n_schemes == 0 || tile_shapes, "tile_shapes is null");
  pl->nd = ndim;
  unsigned __int128 total = 1;
  for (int d = 0; d < ndim; ++d) {
    EJ_CHECK_ARG(shape[d] >= 1 && shape[d] <= INT32_MAX, "shape[%d]=%lld outside [1, 2^31)", d,
                 (long long)shape[d]);
    pl->shape[d] = shape[d];
    total *= static_cast<uint64_t>(shape[d]);
  }
  if (total >= (static_cast<unsigned __int128>(1) << 62)) {
    set_error("tensor has 2^62 or more elements");
    return EJ_E_UNSUPPORTED;
  }
  if (cap <= 0) cap = int64_t(1) << 32;
  if (dense) cap = INT64_MAX;
  std::vector<std::vector<int64_t>> primes(ndim);
  for (int d = 0; d < ndim; ++d) primes[d] = prime_factors(shape[d]);

  std::map<std::array<int64_t, EJ_MAX_DIMS>, int> ids;
  auto insert = [&](const std::array<int64_t, EJ_MAX_DIMS> &ts) -> int {
    auto it = ids.find(ts);
    if (it != ids.end()) return it->second;
    StatNode n;
    n.ts = ts;
    for (int d = 0; d < ndim; ++d) n.cells *= shape[d] / ts[d];
    const int id = static_cast<int>(pl->nodes.size());
    pl->nodes.push_back(std::move(n));
    ids.emplace(ts, id);
    return id;
  };
  pl->req.resize(static_cast<size_t>(n_schemes));
  pl->proj.resize(static_cast<size_t>(n_schemes) * ndim);
  for (int64_t s = 0; s < n_schemes; ++s) {
    std::array<int64_t, EJ_MAX_DIMS> ts{};
    for (int d = 0; d < EJ_MAX_DIMS; ++d) ts[d] = 1;
    for (int d = 0; d < ndim; ++d) {
      const int64_t t = tile_shapes[s * ndim + d];
      EJ_CHECK_ARG(t >= 1 && shape[d] % t == 0,
                   "tile shape %lld: extent %lld does not divide shape[%d]=%lld",
                   (long long)s, (long long)t, d, (long long)shape[d]);
      ts[d] = t;
    }
    pl->req[s] = insert(ts);
    for (int l = 0; l < ndim; ++l) {
      std::array<int64_t, EJ_MAX_DIMS> pj = ts;
      for (int d = 0; d < ndim; ++d)
        if (d != l) pj[d] = shape[d];
      pl->proj[s * ndim + l] = insert(pj);
    }
  }
  // Close under the parent relation (the vector grows while it is walked).
  for (size_t v = 0; v < pl->nodes.size(); ++v) {
    std::array<int64_t, EJ_MAX_DIMS> ts = pl->nodes[v].ts;
    int d = ndim - 1;
    while (d >= 0 && ts[d] == 1) --d;
    if (d < 0) continue;  // (1, ..., 1)
    int64_t p = ts[d];
    for (int64_t q : primes[d])
      if (ts[d] % q == 0) {
        p = q;
        break;
      }
    ts[d] /= p;
    const int par = insert(ts);
    pl->nodes[v].parent = par;
    pl->nodes[v].pdim = d;
    pl->nodes[v].pfac = p;
  }
  // Kinds, parents before children (a parent has more cells).
  std::vector<int> order(pl->nodes.size());
  for (size_t v = 0; v < order.size(); ++v) order[v] = static_cast<int>(v);
  std::sort(order.begin(), order.end(), [&](int a, int b) {
    return pl->nodes[a].cells != pl->nodes[b].cells ? pl->nodes[a].cells > pl->nodes[b].cells
                                                    : a < b;
  });
  for (int v : order) {
    StatNode &n = pl->nodes[v];
    if (dense) {
      n.kind = n.parent < 0 ? kDenseRoot : kPool;
    } else if (n.cells > cap) {
      n.kind = kSorted;
      pl->any_sorted = true;
    } else {
      n.kind = n.parent < 0 || pl->nodes[n.parent].kind == kSorted ? kCooRoot : kPool;
    }
    if (n.kind == kPool && n.pdim == ndim - 1 && n.pfac == 2 &&
        (n.ts[ndim - 1] & (n.ts[ndim - 1] - 1)) == 0)
      n.kind = kChain;
    if (n.kind == kPool || n.kind == kChain) pl->nodes[n.parent].kids.push_back(v);
    if (n.kind == kDenseRoot || n.kind == kCooRoot) pl->roots.push_back(v);
  }
  for (int r : pl->roots) layout(*pl, r, 0);
  return EJ_OK;
}

// The plan of the last statistics request on this thread: a workspace query
// and the call that follows it with the same arguments build it once.
struct PlanCache {
  bool valid = false;
  std::vector<int64_t> key;
  StatsPlan plan;
};
thread_local PlanCache g_plan_cache;

int cached_plan(int32_t ndim, const int64_t *shape, int64_t n_schemes,
                const int64_t *tile_shapes, bool dense, int64_t cap, const StatsPlan **out) {
  std::vector<int64_t> key;
  if (ndim >= 1 && ndim <= EJ_MAX_DIMS && shape && n_schemes >= 0 &&
      (n_schemes == 0 || tile_shapes)) {
    key.reserve(static_cast<size_t>(4 + ndim + n_schemes * ndim));
    key.push_back(ndim);
    key.push_back(dense ? 1 : 0);
    key.push_back(dense ? 0 : cap);
    key.push_back(n_schemes);
    key.insert(key.end(), shape, shape + ndim);
    key.insert(key.end(), tile_shapes, tile_shapes + n_schemes * ndim);
    if (g_plan_cache.valid && g_plan_cache.key == key) {
      *out = &g_plan_cache.plan;
      return EJ_OK;
    }
  }
  g_plan_cache.valid = false;
  g_plan_cache.plan = StatsPlan();
  EJ_TRY(make_plan(ndim, shape, n_schemes, tile_shapes, dense, cap, &g_plan_cache.plan));
  g_plan_cache.key = std::move(key);
  g_plan_cache.valid = true;
  *out = &g_plan_cache.plan;
  return EJ_OK;
}

struct StatsWs {
  unsigned long long *counts;  // one per node, then the range flag
  uint32_t *stack;
  uint64_t *keys, *keys_alt;
  int32_t *vals, *vals_alt;
  void *sort_ws;
  size_t bytes;
};

StatsWs carve_stats(void *base, const StatsPlan &pl, int64_t nnz) {
  Carver c(base);
  StatsWs w{};
  w.counts = c.take<unsigned long long>((static_cast<int64_t>(pl.nodes.size()) + 1) * kCountStride);
  w.stack = c.take<uint32_t>(static_cast<int64_t>(pl.stack_bytes / 4));
  if (pl.any_sorted) {
    w.keys = c.take<uint64_t>(nnz);
    w.keys_alt = c.take<uint64_t>(nnz);
    w.vals = c.take<int32_t>(nnz);
    w.vals_alt = c.take<int32_t>(nnz);
    w.sort_ws = c.take<char>(static_cast<int64_t>(sort_workspace_bytes(nnz)));
  }
  w.bytes = c.off;
  return w;
}

TileIdx tile_idx(const StatsPlan &pl, const StatNode &n) {
  TileIdx ti{};
  ti.nd = pl.nd;
  for (int d = 0; d < pl.nd; ++d) {
    ti.shape[d] = pl.shape[d];
    ti.tile[d] = n.ts[d];
    ti.grid[d] = pl.shape[d] / n.ts[d];
  }
  ti.cells = n.cells;
  return ti;
}

int launch_pool(const StatsPlan &pl, const StatNode &child, const uint32_t *in, uint32_t *out,
                unsigned long long *count, hipStream_t stream) {
  const StatNode &par = pl.nodes[child.parent];
  PoolGeom g;
  const int d = child.pdim;
  g.p = child.pfac;
  g.n_out = pl.shape[d] / child.ts[d];
  g.outer = 1;
  for (int e = 0; e < d; ++e) g.outer *= pl.shape[e] / child.ts[e];
  g.inner = 1;
  for (int e = d + 1; e < pl.nd; ++e) g.inner *= pl.shape[e] / child.ts[e];
  g.total = child.cells;
  const bool small = par.cells < (int64_t(1) << 31);
  if (g.inner % 128 == 0) {
    const int64_t vecs = g.total / 128;
    if (small)
      hipLaunchKernelGGL(pool_bits_vec_kernel<uint32_t>, dim3(stride_grid(vecs)), dim3(kBlock), 0,
                         stream, in, out, g, count);
    else
      hipLaunchKernelGGL(pool_bits_vec_kernel<int64_t>, dim3(stride_grid(vecs)), dim3(kBlock), 0,
                         stream, in, out, g, count);
  } else if (g.inner % 32 == 0) {
    const int64_t words = g.total / 32;
    if (small)
      hipLaunchKernelGGL(pool_bits_word_kernel<uint32_t>, dim3(stride_grid(words)), dim3(kBlock),
                         0, stream, in, out, g, count);
    else
      hipLaunchKernelGGL(pool_bits_word_kernel<int64_t>, dim3(stride_grid(words)), dim3(kBlock), 0,
                         stream, in, out, g, count);
  } else {
    hipLaunchKernelGGL(pool_bits_any_kernel, dim3(stride_grid(ceil_div(g.total, 32))),
                       dim3(kBlock), 0, stream, in, out, g, count);
  }
  EJ_LAUNCH_CHECK();
  return EJ_OK;
}

int run_chain(const StatsPlan &pl, int v, const StatsWs &w, hipStream_t stream) {
  const std::vector<int> chain = chain_of(pl, v);
  const StatNode &n = pl.nodes[v];
  const uint32_t *src = w.stack + n.off / 4;
  int64_t S = n.cells;
  uint32_t *tmp = w.stack + n.tmp_off / 4;
  for (size_t done = 0; done < chain.size(); done += kChainMax) {
    ChainArgs a{};
    a.levels = static_cast<int32_t>(std::min<size_t>(kChainMax, chain.size() - done));
    const bool more = done + kChainMax < chain.size();
    a.write_level = more ? kChainMax : 0;
    for (int k = 0; k < a.levels; ++k) a.count[k] = w.counts + chain[done + k] * kCountStride;
    if (more) {  // the next pass's map is or-ed together: start from zero
      const int64_t words = static_cast<int64_t>(map_bytes(S >> kChainMax) / 4);
      hipLaunchKernelGGL(fill_zero_kernel<uint32_t>, dim3(stride_grid(words)), dim3(kBlock), 0,
                         stream, tmp, words);
      EJ_LAUNCH_CHECK();
    }
    const int64_t blocks = ceil_div(ceil_div(S, kChainChunk), 4);
    hipLaunchKernelGGL(pool_chain_kernel,
                       dim3(static_cast<unsigned>(std::min<int64_t>(blocks, 4096))), dim3(256), 0,
                       stream, src, S, a, tmp);
    EJ_LAUNCH_CHECK();
    if (more) {
      src = tmp;
      S >>= kChainMax;
      tmp += map_bytes(S) / 4;
    }
  }
  return EJ_OK;
}

// The kid of v pooled from it by 2 along dimension nd - 2, or -1.
int row_pool_kid(const StatsPlan &pl, int v) {
  if (pl.nd < 2) return -1;
  for (int k : pl.nodes[v].kids) {
    const StatNode &c = pl.nodes[k];
    if (c.kind == kPool && c.pdim == pl.nd - 2 && c.pfac == 2) return k;
  }
  return -1;
}

// From materialised node v, a run of up to kBandMax row poolings (v's row
// pool kid, its row pool kid, ...) whose inner nodes have no kids but their
// chain and their row pool, every chain of at most kChainMax levels: one
// launch counts the chains of the run (v's unless chain_done) and the inner
// and last nodes' bits, and writes the last node's map.  Map rows of whole
// chunks take band_chain_kernel; rows of 256 .. 8192 bits in a map of whole
// chunks take band_chain_small_kernel, with at most a chunk's rows per
// band.  *end = the last node, or -1 when no run applies.
int run_band(const StatsPlan &pl, int v, bool chain_done, const StatsWs &w, hipStream_t stream,
             int *end) {
  *end = -1;
  if (pl.nd < 2) return EJ_OK;
  const int64_t row_bits = pl.shape[pl.nd - 1] / pl.nodes[v].ts[pl.nd - 1];
  const bool whole = row_bits % kChainChunk == 0;
  const bool small = !whole && row_bits >= 256 && kChainChunk % row_bits == 0 &&
                     pl.nodes[v].cells % kChainChunk == 0;
  if ((!whole && !small) || chain_of(pl, v).size() > static_cast<size_t>(kChainMax))
    return EJ_OK;
  int hmax = kBandMax;
  if (small)
    while (hmax > 0 && (int64_t(1) << hmax) > kChainChunk / row_bits) --hmax;
  std::vector<int> run{v};
  while (static_cast<int>(run.size()) <= hmax) {
    const int u = run.back();
    const int k = row_pool_kid(pl, u);
    if (k < 0 || chain_of(pl, k).size() > static_cast<size_t>(kChainMax)) break;
    if (u != v) {  // u becomes an inner node: nothing else may need its map
      bool pure = true;
      for (int c : pl.nodes[u].kids) pure = pure && (c == k || pl.nodes[c].kind == kChain);
      if (!pure) break;
    }
    run.push_back(k);
  }
  const int H = static_cast<int>(run.size()) - 1;
  if (H < 1) return EJ_OK;
  BandArgs a{};
  a.H = H;
  a.first = chain_done ? 0 : 1;
  a.row_bits = row_bits;
  a.rows_out = pl.nodes[run[H]].cells / row_bits;
  for (int h = 0; h <= H; ++h) {
    const std::vector<int> ch = chain_of(pl, run[h]);
    a.levels[h] = static_cast<int32_t>(ch.size());
    for (size_t k = 0; k < ch.size(); ++k) a.chain[h][k] = w.counts + ch[k] * kCountStride;
    a.pop[h] = h >= 1 ? w.counts + run[h] * kCountStride : nullptr;
  }
  const int64_t items = small ? pl.nodes[v].cells / kChainChunk
                              : a.rows_out * (row_bits / kChainChunk);
  const dim3 grid(static_cast<unsigned>(std::min<int64_t>(ceil_div(items, 4), 4096)));
  if (small)
    hipLaunchKernelGGL(band_chain_small_kernel, grid, dim3(256), 0, stream,
                       w.stack + pl.nodes[v].off / 4, a, w.stack + pl.nodes[run[H]].off / 4);
  else
    hipLaunchKernelGGL(band_chain_kernel, grid, dim3(256), 0, stream,
                       w.stack + pl.nodes[v].off / 4, a, w.stack + pl.nodes[run[H]].off / 4);
  EJ_LAUNCH_CHECK();
  *end = run[H];
  return EJ_OK;
}

int run_subtree(const StatsPlan &pl, int v, const StatsWs &w, hipStream_t stream,
                bool chain_done = false) {
  const StatNode &n = pl.nodes[v];
  int end = -1;
  EJ_TRY(run_band(pl, v, chain_done, w, stream, &end));
  // The band run's last map sits where v's row pool kid's subtree would, and
  // v's other kids reuse that stack space: its subtree runs first.
  if (end >= 0) EJ_TRY(run_subtree(pl, end, w, stream, true));
  const int banded = end >= 0 ? row_pool_kid(pl, v) : -1;  // handled by the band run
  bool chained = chain_done || end >= 0;
  for (int k : n.kids) {
    const StatNode &kid = pl.nodes[k];
    if (kid.kind == kChain) {
      if (!chained) EJ_TRY(run_chain(pl, v, w, stream));
      chained = true;
      continue;
    }
    if (k == banded) continue;
    EJ_TRY(launch_pool(pl, kid, w.stack + n.off / 4, w.stack + kid.off / 4,
                       w.counts + k * kCountStride, stream));
    EJ_TRY(run_subtree(pl, k, w, stream));
  }
  return EJ_OK;
}

template <typename T>
int run_stats(const StatsPlan &pl, const StatsWs &w, const T *dense, int64_t n_dense,
              const int32_t *idx, const T *vals, int64_t nnz, hipStream_t stream) {
  const int64_t n_counts = (static_cast<int64_t>(pl.nodes.size()) + 1) * kCountStride;
  int64_t *bad = reinterpret_cast<int64_t *>(w.counts + pl.nodes.size() * kCountStride);
  hipLaunchKernelGGL(fill_zero_kernel<unsigned long long>, dim3(stride_grid(n_counts)),
                     dim3(kBlock), 0, stream, w.counts, n_counts);
  EJ_LAUNCH_CHECK();
  if (pl.any_sorted) {
    for (size_t v = 0; v < pl.nodes.size(); ++v) {
      const StatNode &n = pl.nodes[v];
      if (n.kind != kSorted) continue;
      const TileIdx ti = tile_idx(pl, n);
      hipLaunchKernelGGL(stat_keys_kernel<T>, dim3(grid_for(nnz)), dim3(kBlock), 0, stream, idx,
                         vals, nnz, ti, w.keys, bad);
      EJ_LAUNCH_CHECK();
      EJ_TRY(sort_pairs_u64(w.keys, w.vals, w.keys_alt, w.vals_alt, nnz,
                            bits_for(static_cast<uint64_t>(n.cells) + 1), w.sort_ws, stream));
      hipLaunchKernelGGL(distinct_count_kernel, dim3(stride_grid(nnz)), dim3(kBlock), 0, stream,
                         w.keys, nnz, static_cast<uint64_t>(n.cells), w.counts + v * kCountStride);
      EJ_LAUNCH_CHECK();
    }
  }
  for (int r : pl.roots) {
    const StatNode &n = pl.nodes[r];
    uint32_t *map = w.stack + n.off / 4;
    if (n.kind == kDenseRoot) {
      const bool vec = (reinterpret_cast<uintptr_t>(dense) % 16) == 0;
      const int64_t chunk = 4 * 64 * (16 / static_cast<int64_t>(sizeof(T)));
      hipLaunchKernelGGL(dense_bits_kernel<T>,
                         dim3(static_cast<unsigned>(std::min<int64_t>(
                             std::max<int64_t>(ceil_div(ceil_div(n_dense, chunk), 4), 1), 8192))),
                         dim3(kBlock), 0, stream, dense, n_dense, vec, map,
                         w.counts + r * kCountStride);
    } else {
      const int64_t words = static_cast<int64_t>(map_bytes(n.cells) / 4);
      hipLaunchKernelGGL(fill_zero_kernel<uint32_t>, dim3(stride_grid(words)), dim3(kBlock), 0,
                         stream, map, words);
      EJ_LAUNCH_CHECK();
      hipLaunchKernelGGL(coo_mark_kernel<T>, dim3(grid_for(nnz)), dim3(kBlock), 0, stream, idx,
                         vals, nnz, tile_idx(pl, n), map, bad);
      EJ_LAUNCH_CHECK();
      hipLaunchKernelGGL(map_count_kernel, dim3(stride_grid(words)), dim3(kBlock), 0, stream,
                         map, words, w.counts + r * kCountStride);
    }
    EJ_LAUNCH_CHECK();
    EJ_TRY(run_subtree(pl, r, w, stream));
  }
  return EJ_OK;
}

int finish_stats(const StatsPlan &pl, const StatsWs &w, int64_t *num_tuples,
                 int64_t *value_count, hipStream_t stream) {
  std::vector<unsigned long long> host((pl.nodes.size() + 1) * kCountStride);
  EJ_HIP(hipMemcpyAsync(host.data(), w.counts, host.size() * sizeof(unsigned long long),
                        hipMemcpyDeviceToHost, stream));
  EJ_HIP(hipStreamSynchronize(stream));
  if (host[pl.nodes.size() * kCountStride]) {
    set_error("a nonzero entry has an index outside the tensor shape");
    return EJ_E_RANGE;
  }
  for (size_t s = 0; s < pl.req.size(); ++s) {
    num_tuples[s] = static_cast<int64_t>(host[pl.req[s] * kCountStride]);
    for (int l = 0; l < pl.nd; ++l)
      value_count[s * pl.nd + l] =
          static_cast<int64_t>(host[pl.proj[s * pl.nd + l] * kCountStride]);
  }
  return EJ_OK;
}

}  // namespace
}  // namespace ej

using namespace ej;

// ---- dense to COO ------------------------------------------------------------
extern "C" int ej_extract_coo_workspace_size(int32_t ndim, const int64_t *shape, int32_t dtype,
                                             size_t *bytes) {
  clear_error();
  EJ_CHECK_ARG(bytes, "bytes is null");
  EJ_CHECK_ARG(dtype == EJ_F32 || dtype == EJ_BF16 || dtype == EJ_F64, "unknown dtype %d", dtype);
  DenseShape sh;
  int64_t n;
  EJ_TRY(dense_shape(ndim, shape, &sh, &n));
  *bytes = carve_extract(nullptr, extract_runs(n, dtype)).bytes;
  return EJ_OK;
}

extern "C" int ej_extract_coo_count(const void *dense, int32_t dtype, int32_t ndim,
                                    const int64_t *shape, void *workspace,
                                    size_t workspace_bytes, int64_t *nnz, ej_stream_t stream_) {
  clear_error();
  hipStream_t stream = as_stream(stream_);
  EJ_CHECK_ARG(nnz, "nnz is null");
  EJ_CHECK_ARG(dtype == EJ_F32 || dtype == EJ_BF16 || dtype == EJ_F64, "unknown dtype %d", dtype);
  DenseShape sh;
  int64_t n;
  EJ_TRY(dense_shape(ndim, shape, &sh, &n));
  if (n == 0) {
    *nnz = 0;
    return EJ_OK;
  }
  EJ_CHECK_ARG(dense, "dense is null");
  const int64_t runs = extract_runs(n, dtype);
  ExtractWs w = carve_extract(workspace, runs);
  EJ_CHECK_ARG(workspace && workspace_bytes >= w.bytes, "workspace too small: %zu < %zu bytes",
               workspace_bytes, w.bytes);
  const bool vec = (reinterpret_cast<uintptr_t>(dense) & 15u) == 0;
  const dim3 grid(static_cast<unsigned>(ceil_div(runs, 4)));
  if (dtype == EJ_F64)
    hipLaunchKernelGGL(coo_count_kernel<double>, grid, dim3(256), 0, stream,
                       static_cast<const double *>(dense), n, runs, vec, w.counts);
  else if (dtype == EJ_F32)
    hipLaunchKernelGGL(coo_count_kernel<float>, grid, dim3(256), 0, stream,
                       static_cast<const float *>(dense), n, runs, vec, w.counts);
  else
    hipLaunchKernelGGL(coo_count_kernel<uint16_t>, grid, dim3(256), 0, stream,
                       static_cast<const uint16_t *>(dense), n, runs, vec, w.counts);
  EJ_LAUNCH_CHECK();
  EJ_TRY(scan_exclusive_i64(w.counts, w.excl, runs, w.scalars, w.scan_ws, stream));
  int64_t host = 0;
  EJ_HIP(hipMemcpyAsync(&host, w.scalars, sizeof(int64_t), hipMemcpyDeviceToHost, stream));
  EJ_HIP(hipStreamSynchronize(stream));
  *nnz = host;
  return EJ_OK;
}

extern "C" int ej_extract_coo_fill(const void *dense, int32_t dtype, int32_t ndim,
                                   const int64_t *shape, const void *workspace,
                                   size_t workspace_bytes, int64_t nnz, int32_t *indices,
                                   double *values, int64_t capacity, ej_stream_t stream_) {
  clear_error();
  hipStream_t stream = as_stream(stream_);
  EJ_CHECK_ARG(dtype == EJ_F32 || dtype == EJ_BF16 || dtype == EJ_F64, "unknown dtype %d", dtype);
  DenseShape sh;
  int64_t n;
  EJ_TRY(dense_shape(ndim, shape, &sh, &n));
  EJ_CHECK_ARG(nnz >= 0 && nnz <= n, "nnz out of range");
  if (capacity < nnz) {
    set_error("capacity %lld < %lld nonzeros", (long long)capacity, (long long)nnz);
    return EJ_E_CAPACITY;
  }
  if (nnz == 0) return EJ_OK;
  EJ_CHECK_ARG(dense && indices && values, "null pointer argument");
  const int64_t runs = extract_runs(n, dtype);
  ExtractWs w = carve_extract(const_cast<void *>(workspace), runs);
  EJ_CHECK_ARG(workspace && workspace_bytes >= w.bytes, "workspace too small");
  const bool vec = (reinterpret_cast<uintptr_t>(dense) & 15u) == 0;
  const dim3 grid(static_cast<unsigned>(ceil_div(runs, 4)));
  if (dtype == EJ_F64)
    hipLaunchKernelGGL(coo_fill_kernel<double>, grid, dim3(256), 0, stream,
                       static_cast<const double *>(dense), n, runs, vec, sh, w.excl, nnz,
                       indices, values);
  else if (dtype == EJ_F32)
    hipLaunchKernelGGL(coo_fill_kernel<float>, grid, dim3(256), 0, stream,
                       static_cast<const float *>(dense), n, runs, vec, sh, w.excl, nnz,
                       indices, values);
  else
    hipLaunchKernelGGL(coo_fill_kernel<uint16_t>, grid, dim3(256), 0, stream,
                       static_cast<const uint16_t *>(dense), n, runs, vec, sh, w.excl, nnz,
                       indices, values);
  EJ_LAUNCH_CHECK();
  return EJ_OK;
}

// ---- COO to tiles --------------------------------------------------------------
extern "C" int ej_bucket_coo_workspace_size(int64_t nnz, int32_t dtype, int32_t ndim,
                                            const int64_t *shape, const int64_t *tile_shape,
                                            size_t *bytes) {
  clear_error();
  EJ_CHECK_ARG(bytes, "bytes is null");
  EJ_CHECK_ARG(dtype == EJ_F32 || dtype == EJ_BF16 || dtype == EJ_F64, "unknown dtype %d", dtype);
  EJ_CHECK_ARG(nnz >= 0 && nnz <= INT32_MAX, "nnz=%lld outside [0, 2^31)", (long long)nnz);
  CooGeom g;
  EJ_TRY(make_coo_geom(ndim, shape, tile_shape, &g));
  *bytes = coo_map_path(dtype, g) ? carve_coo_map(nullptr, g.n_tiles).bytes
                                  : carve_coo(nullptr, nnz).bytes;
  return EJ_OK;
}

extern "C" int ej_bucket_coo_count(const int32_t *indices, const void *values, int32_t dtype,
                                   int64_t nnz, int32_t ndim, const int64_t *shape,
                                   const int64_t *tile_shape, void *workspace,
                                   size_t workspace_bytes, int64_t *n_tiles,
                                   ej_stream_t stream_) {
  clear_error();
  hipStream_t stream = as_stream(stream_);
  EJ_CHECK_ARG(n_tiles, "n_tiles is null");
  EJ_CHECK_ARG(dtype == EJ_F32 || dtype == EJ_BF16 || dtype == EJ_F64, "unknown dtype %d", dtype);
  EJ_CHECK_ARG(nnz >= 0 && nnz <= INT32_MAX, "nnz=%lld outside [0, 2^31)", (long long)nnz);
  CooGeom g;
  EJ_TRY(make_coo_geom(ndim, shape, tile_shape, &g));
  if (nnz == 0 || g.n_tiles == 0) {
    *n_tiles = 0;
    return EJ_OK;
  }
  EJ_CHECK_ARG(indices && values, "null pointer argument");
  const dim3 grid(grid_for(nnz));
  if (coo_map_path(dtype, g)) {
    CooMapWs w = carve_coo_map(workspace, g.n_tiles);
    EJ_CHECK_ARG(workspace && workspace_bytes >= w.bytes,
                 "workspace too small: %zu < %zu bytes", workspace_bytes, w.bytes);
    const int64_t words = (g.n_tiles + 31) / 32;
    hipLaunchKernelGGL(fill_zero_kernel<int64_t>, dim3(1), dim3(64), 0, stream, w.scalars,
                       int64_t(4));
    EJ_LAUNCH_CHECK();
    hipLaunchKernelGGL(fill_zero_kernel<uint32_t>, dim3(stride_grid(words * 8)), dim3(kBlock),
                       0, stream, reinterpret_cast<uint32_t *>(w.flags), words * 8);
    EJ_LAUNCH_CHECK();
    if (dtype == EJ_F64)
      hipLaunchKernelGGL(coo_tile_mark_kernel<double>, grid, dim3(kBlock), 0, stream, indices,
                         static_cast<const double *>(values), nnz, g, w.flags, w.scalars + 1);
    else
      hipLaunchKernelGGL(coo_tile_mark_kernel<float>, grid, dim3(kBlock), 0, stream, indices,
                         static_cast<const float *>(values), nnz, g, w.flags, w.scalars + 1);
    EJ_LAUNCH_CHECK();
    hipLaunchKernelGGL(pack_flags_kernel, dim3(grid_for(words)), dim3(kBlock), 0, stream,
                       w.flags, words, w.map, w.cnt);
    EJ_LAUNCH_CHECK();
    EJ_TRY(scan_exclusive_i64(w.cnt, w.prefix, words, w.scalars, w.scan_ws, stream));
    int64_t host[2] = {0, 0};
    EJ_HIP(hipMemcpyAsync(host, w.scalars, 2 * sizeof(int64_t), hipMemcpyDeviceToHost, stream));
    EJ_HIP(hipStreamSynchronize(stream));
    if (host[1]) {
      set_error("a nonzero entry has an index outside the tensor shape");
      return EJ_E_RANGE;
    }
    *n_tiles = host[0];
    return EJ_OK;
  }
  CooWs w = carve_coo(workspace, nnz);
  EJ_CHECK_ARG(workspace && workspace_bytes >= w.bytes, "workspace too small: %zu < %zu bytes",
               workspace_bytes, w.bytes);
  hipLaunchKernelGGL(fill_zero_kernel<int64_t>, dim3(1), dim3(64), 0, stream, w.scalars,
                     int64_t(4));
  EJ_LAUNCH_CHECK();
  // Keys go to the alternate buffers when the sort takes an odd number of
  // passes, so the sorted result lands in keys / order without a copy.
  const bool alt = radix_passes(g.bits) % 2 == 1;
  uint64_t *k0 = alt ? w.keys_alt : w.keys;
  int32_t *o0 = alt ? w.order_alt : w.order;
  if (dtype == EJ_F64)
    hipLaunchKernelGGL(coo_keys_kernel<double>, grid, dim3(kBlock), 0, stream, indices,
                       static_cast<const double *>(values), nnz, g, k0, o0, w.scalars + 1);
  else if (dtype == EJ_F32)
    hipLaunchKernelGGL(coo_keys_kernel<float>, grid, dim3(kBlock), 0, stream, indices,
                       static_cast<const float *>(values), nnz, g, k0, o0, w.scalars + 1);
  else
    hipLaunchKernelGGL(coo_keys_kernel<uint16_t>, grid, dim3(kBlock), 0, stream, indices,
                       static_cast<const uint16_t *>(values), nnz, g, k0, o0, w.scalars + 1);
  EJ_LAUNCH_CHECK();
  EJ_TRY(sort_pairs_u64(w.keys, w.order, w.keys_alt, w.order_alt, nnz, g.bits, w.sort_ws, stream,
                        alt));
  hipLaunchKernelGGL(coo_tile_flags_kernel, grid, dim3(kBlock), 0, stream, w.keys, nnz,
                     g.sentinel, g.wbits, w.flags);
  EJ_LAUNCH_CHECK();
  EJ_TRY(scan_exclusive_i64(w.flags, w.excl, nnz, w.scalars, w.scan_ws, stream));
  int64_t host[2] = {0, 0};
  EJ_HIP(hipMemcpyAsync(host, w.scalars, 2 * sizeof(int64_t), hipMemcpyDeviceToHost, stream));
  EJ_HIP(hipStreamSynchronize(stream));
  if (host[1]) {
    set_error("a nonzero entry has an index outside the tensor shape");
    return EJ_E_RANGE;
  }
  *n_tiles = host[0];
  return EJ_OK;
}

extern "C" int ej_bucket_coo_fill(const int32_t *indices, const void *values, int32_t dtype,
                                  int64_t nnz, int32_t ndim, const int64_t *shape,
                                  const int64_t *tile_shape, const void *workspace,
                                  size_t workspace_bytes, int64_t n_tiles, int32_t *coords,
                                  void *tiles, int64_t capacity, ej_stream_t stream_) {
  clear_error();
  hipStream_t stream = as_stream(stream_);
  EJ_CHECK_ARG(dtype == EJ_F32 || dtype == EJ_BF16 || dtype == EJ_F64, "unknown dtype %d", dtype);
  EJ_CHECK_ARG(nnz >= 0 && nnz <= INT32_MAX, "nnz=%lld outside [0, 2^31)", (long long)nnz);
  CooGeom g;
  EJ_TRY(make_coo_geom(ndim, shape, tile_shape, &g));
  EJ_CHECK_ARG(n_tiles >= 0 && n_tiles <= nnz && n_tiles <= g.n_tiles, "n_tiles out of range");
  if (capacity < n_tiles) {
    set_error("tile capacity %lld < %lld tiles", (long long)capacity, (long long)n_tiles);
    return EJ_E_CAPACITY;
  }
  if (n_tiles == 0) return EJ_OK;
  EJ_CHECK_ARG(values && coords && tiles, "null pointer argument");
  const int64_t elems = n_tiles * g.tile_elems;
  const dim3 grid(grid_for(nnz));
  if (coo_map_path(dtype, g)) {
    EJ_CHECK_ARG(indices, "null pointer argument");
    CooMapWs w = carve_coo_map(const_cast<void *>(workspace), g.n_tiles);
    EJ_CHECK_ARG(workspace && workspace_bytes >= w.bytes, "workspace too small");
    const int64_t words = (g.n_tiles + 31) / 32;
    if (dtype == EJ_F64) {
      long long *win = static_cast<long long *>(tiles);
      hipLaunchKernelGGL(fill_i64_kernel, dim3(stride_grid(elems)), dim3(kBlock), 0, stream, win,
                         elems, -1ll);
      EJ_LAUNCH_CHECK();
      hipLaunchKernelGGL((coo_winner_kernel<double, long long>), grid, dim3(kBlock), 0, stream,
                         indices, static_cast<const double *>(values), nnz, g, w.map, w.prefix,
                         n_tiles, w.scalars + 1, win);
      EJ_LAUNCH_CHECK();
      hipLaunchKernelGGL((coo_resolve_kernel<double, long long>), dim3(stride_grid(elems)),
                         dim3(kBlock), 0, stream, static_cast<const double *>(values), win,
                         elems);
    } else {
      int32_t *win = static_cast<int32_t *>(tiles);
      hipLaunchKernelGGL(fill_i32_kernel, dim3(stride_grid(elems)), dim3(kBlock), 0, stream, win,
                         elems, int32_t(-1));
      EJ_LAUNCH_CHECK();
      hipLaunchKernelGGL((coo_winner_kernel<float, int32_t>), grid, dim3(kBlock), 0, stream,
                         indices, static_cast<const float *>(values), nnz, g, w.map, w.prefix,
                         n_tiles, w.scalars + 1, win);
      EJ_LAUNCH_CHECK();
      hipLaunchKernelGGL((coo_resolve_kernel<float, int32_t>), dim3(stride_grid(elems)),
                         dim3(kBlock), 0, stream, static_cast<const float *>(values), win, elems);
    }
    EJ_LAUNCH_CHECK();
    hipLaunchKernelGGL(coo_map_coords_kernel, dim3(grid_for(words)), dim3(kBlock), 0, stream,
                       w.map, w.prefix, words, g, n_tiles, coords);
    EJ_LAUNCH_CHECK();
    return EJ_OK;
  }
  CooWs w = carve_coo(const_cast<void *>(workspace), nnz);
  EJ_CHECK_ARG(workspace && workspace_bytes >= w.bytes, "workspace too small");
  if (dtype == EJ_BF16) {
    hipLaunchKernelGGL(fill_zero_kernel<uint16_t>, dim3(stride_grid(elems)), dim3(kBlock), 0,
                       stream, static_cast<uint16_t *>(tiles), elems);
    EJ_LAUNCH_CHECK();
    hipLaunchKernelGGL((coo_scatter_kernel<uint16_t, uint16_t>), grid, dim3(kBlock), 0, stream,
                       w.keys, w.order, w.flags, w.excl, static_cast<const uint16_t *>(values),
                       nnz, g, n_tiles, coords, static_cast<uint16_t *>(tiles));
  } else if (dtype == EJ_F64) {
    hipLaunchKernelGGL(fill_zero_kernel<double>, dim3(stride_grid(elems)), dim3(kBlock), 0,
                       stream, static_cast<double *>(tiles), elems);
    EJ_LAUNCH_CHECK();
    hipLaunchKernelGGL((coo_scatter_kernel<double, double>), grid, dim3(kBlock), 0, stream,
                       w.keys, w.order, w.flags, w.excl, static_cast<const double *>(values),
                       nnz, g, n_tiles, coords, static_cast<double *>(tiles));
  } else {
    hipLaunchKernelGGL(fill_zero_kernel<float>, dim3(stride_grid(elems)), dim3(kBlock), 0,
                       stream, static_cast<float *>(tiles), elems);
    EJ_LAUNCH_CHECK();
    hipLaunchKernelGGL((coo_scatter_kernel<float, float>), grid, dim3(kBlock), 0, stream,
                       w.keys, w.order, w.flags, w.excl, static_cast<const float *>(values),
                       nnz, g, n_tiles, coords, static_cast<float *>(tiles));
  }
  EJ_LAUNCH_CHECK();
  return EJ_OK;
}

// ---- statistics --------------------------------------------------------------
extern "C" int ej_scheme_stats_workspace_size(int32_t ndim, const int64_t *shape,
                                              int64_t n_schemes, const int64_t *tile_shapes,
                                              int64_t nnz, int64_t bitmap_cap, size_t *bytes) {
  clear_error();
  EJ_CHECK_ARG(bytes, "bytes is null");
  EJ_CHECK_ARG(nnz <= INT32_MAX, "nnz=%lld outside [0, 2^31)", (long long)nnz);
  const StatsPlan *pp = nullptr;
  EJ_TRY(cached_plan(ndim, shape, n_schemes, tile_shapes, nnz < 0, bitmap_cap, &pp));
  const StatsPlan &pl = *pp;
  *bytes = carve_stats(nullptr, pl, nnz < 0 ? 0 : nnz).bytes;
  return EJ_OK;
}

extern "C" int ej_scheme_stats_dense(const void *dense, int32_t dtype, int32_t ndim,
                                     const int64_t *shape, int64_t n_schemes,
                                     const int64_t *tile_shapes, void *workspace,
                                     size_t workspace_bytes, int64_t *num_tuples,
                                     int64_t *value_count, ej_stream_t stream_) {
  clear_error();
  hipStream_t stream = as_stream(stream_);
  EJ_CHECK_ARG(dtype == EJ_F32 || dtype == EJ_BF16 || dtype == EJ_F64, "unknown dtype %d", dtype);
  const StatsPlan *pp = nullptr;
  EJ_TRY(cached_plan(ndim, shape, n_schemes, tile_shapes, true, 0, &pp));
  const StatsPlan &pl = *pp;
  if (n_schemes == 0) return EJ_OK;
  EJ_CHECK_ARG(dense && num_tuples && value_count, "null pointer argument");
  StatsWs w = carve_stats(workspace, pl, 0);
  EJ_CHECK_ARG(workspace && workspace_bytes >= w.bytes, "workspace too small: %zu < %zu bytes",
               workspace_bytes, w.bytes);
  int64_t n = 1;
  for (int d = 0; d < ndim; ++d) n *= shape[d];
  if (dtype == EJ_F64)
    EJ_TRY(run_stats<double>(pl, w, static_cast<const double *>(dense), n, nullptr, nullptr, 0,
                             stream));
  else if (dtype == EJ_F32)
    EJ_TRY(run_stats<float>(pl, w, static_cast<const float *>(dense), n, nullptr, nullptr, 0,
                            stream));
  else
    EJ_TRY(run_stats<uint16_t>(pl, w, static_cast<const uint16_t *>(dense), n, nullptr, nullptr,
                               0, stream));
  return finish_stats(pl, w, num_tuples, value_count, stream);
}

extern "C" int ej_scheme_stats_coo(const int32_t *indices, const void *values, int32_t dtype,
                                   int64_t nnz, int32_t ndim, const int64_t *shape,
                                   int64_t n_schemes, const int64_t *tile_shapes,
                                   int64_t bitmap_cap, void *workspace, size_t workspace_bytes,
                                   int64_t *num_tuples, int64_t *value_count,
                                   ej_stream_t stream_) {
  clear_error();
  hipStream_t stream = as_stream(stream_);
  EJ_CHECK_ARG(dtype == EJ_F32 || dtype == EJ_BF16 || dtype == EJ_F64, "unknown dtype %d", dtype);
  EJ_CHECK_ARG(nnz >= 0 && nnz <= INT32_MAX, "nnz=%lld outside [0, 2^31)", (long long)nnz);
  const StatsPlan *pp = nullptr;
  EJ_TRY(cached_plan(ndim, shape, n_schemes, tile_shapes, false, bitmap_cap, &pp));
  const StatsPlan &pl = *pp;
  if (n_schemes == 0) return EJ_OK;
  EJ_CHECK_ARG(num_tuples && value_count, "null pointer argument");
  if (nnz == 0) {
    for (int64_t s = 0; s < n_schemes; ++s) {
      num_tuples[s] = 0;
      for (int l = 0; l < ndim; ++l) value_count[s * ndim + l] = 0;
    }
    return EJ_OK;
  }
  EJ_CHECK_ARG(indices && values, "null pointer argument");
  StatsWs w = carve_stats(workspace, pl, nnz);
  EJ_CHECK_ARG(workspace && workspace_bytes >= w.bytes, "workspace too small: %zu < %zu bytes",
               workspace_bytes, w.bytes);
  if (dtype == EJ_F64)
    EJ_TRY(run_stats<double>(pl, w, nullptr, 0, indices, static_cast<const double *>(values), nnz,
                             stream));
  else if (dtype == EJ_F32)
    EJ_TRY(run_stats<float>(pl, w, nullptr, 0, indices, static_cast<const float *>(values), nnz,
                            stream));
  else
    EJ_TRY(run_stats<uint16_t>(pl, w, nullptr, 0, indices, static_cast<const uint16_t *>(values),
                               nnz, stream));
  return finish_stats(pl, w, num_tuples, value_count, stream);
}
