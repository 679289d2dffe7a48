// Coordinate-to-tile bucketing of a dense tensor, and its inverse.
//
// Reference: SparseTensor.to_relation (tensor/sparse.py:160-219) takes the
// nonzero elements (values != 0, :184-187), computes idx // tile and
// idx % tile (:200-201), orders the distinct tile coordinates
// lexicographically with np.unique(axis=0) (:204-206) and scatters the
// nonzero values into zero tiles (:210-212).  For a dense row-major input
// the lexicographic order of tile coordinates is the row-major order of the
// tile grid, so no sort is needed:
//   count: one pass over the dense tensor flags every tile holding an
//          element != 0; an exclusive scan of the flags gives each kept
//          tile its slot and the tile count T;
//   fill:  one workgroup per kept tile copies it into the packed
//          [T, *tile] array (zeros normalised to +0.0, as the reference's
//          scatter into np.zeros leaves them) and writes its coordinates.
#include "ej_internal.h"

namespace ej {
namespace {

struct BucketGeom {
  int32_t nd;
  int64_t shape[EJ_MAX_DIMS], tile[EJ_MAX_DIMS], grid[EJ_MAX_DIMS];
  int64_t dstride[EJ_MAX_DIMS];  // dense row-major strides
  int64_t tile_elems, n_tiles;   // elements per tile, tiles in the grid
  int64_t inner;                 // tile[nd-1]: contiguous run length in HBM
  int64_t rows;                  // tile_elems / inner
};

int make_geom(int32_t ndim, const int64_t *shape, const int64_t *tile, BucketGeom *g) {
  EJ_CHECK_ARG(ndim >= 1 && ndim <= EJ_MAX_DIMS, "ndim=%d outside [1, %d]", ndim, EJ_MAX_DIMS);
  EJ_CHECK_ARG(shape && tile, "null shape");
  g->nd = ndim;
  g->tile_elems = 1;
  g->n_tiles = 1;
  for (int d = 0; d < ndim; ++d) {
    EJ_CHECK_ARG(tile[d] >= 1 && shape[d] >= 0, "bad extent in dim %d", d);
    EJ_CHECK_ARG(shape[d] % tile[d] == 0, "tile_shape[%d]=%lld does not evenly divide shape[%d]=%lld",
                 d, (long long)tile[d], d, (long long)shape[d]);
    g->shape[d] = shape[d];
    g->tile[d] = tile[d];
    g->grid[d] = shape[d] / tile[d];
    g->tile_elems *= tile[d];
    g->n_tiles *= g->grid[d];
  }
  int64_t s = 1;
  for (int d = ndim - 1; d >= 0; --d) {
    g->dstride[d] = s;
    s *= shape[d];
  }
  g->inner = tile[ndim - 1];
  g->rows = g->tile_elems / g->inner;
  return EJ_OK;
}

// Dense offset of the first element of tile t (row-major tile id).
__device__ inline int64_t tile_origin(const BucketGeom &g, int64_t t) {
  int64_t off = 0;
  for (int d = g.nd - 1; d >= 0; --d) {
    int64_t c = t % g.grid[d];
    t /= g.grid[d];
    off += c * g.tile[d] * g.dstride[d];
  }
  return off;
}

// Dense offset (relative to the tile origin) of row r of a tile, where a row
// is a run of `inner` contiguous elements.
__device__ inline int64_t row_offset(const BucketGeom &g, int64_t r) {
  int64_t off = 0;
  for (int d = g.nd - 2; d >= 0; --d) {
    int64_t c = r % g.tile[d];
    r /= g.tile[d];
    off += c * g.dstride[d];
  }
  return off;
}

__device__ inline bool nonzero(double x) { return x != 0.0; }  // NaN != 0 holds
__device__ inline bool nonzero(float x) { return x != 0.0f; }
__device__ inline bool nonzero(uint16_t x) { return (x & 0x7fffu) != 0; }  // bf16: +-0 are zero
// Tile element as stored: zeros become +0.0 (the reference scatters the
// nonzero values into np.zeros tiles); every dtype keeps its precision.
__device__ inline double stored(double x) { return x == 0.0 ? 0.0 : x; }
__device__ inline float stored(float x) { return x == 0.0f ? 0.0f : x; }
__device__ inline uint16_t stored(uint16_t x) { return (x & 0x7fffu) ? x : 0; }

// One workgroup per tile: rows are spread over the threads, the innermost
// run is read contiguously.
template <typename T>
__global__ __launch_bounds__(256) void tile_flags_kernel(const T *__restrict__ dense,
                                                         BucketGeom g, int64_t *flags) {
  const int64_t t = blockIdx.x;
  const T *base = dense + tile_origin(g, t);
  int any = 0;
  const int64_t total = g.tile_elems;
  for (int64_t e = threadIdx.x; e < total && !any; e += 256) {
    const int64_t r = e / g.inner, c = e % g.inner;
    if (nonzero(base[row_offset(g, r) + c])) any = 1;
  }
  any = __syncthreads_or(any);
  if (threadIdx.x == 0) flags[t] = any ? 1 : 0;
}

// Vectorised forms for tiles whose rows are whole 16-byte vectors (vpr
// vectors per row, vpr a power of two <= 256): thread t owns vector column
// t % vpr and rows t / vpr, t / vpr + 256 / vpr, ...; a thread issues all its
// loads before testing them, so the loads overlap.  MODE 0 = bf16, 1 = fp32,
// 2 = fp64 input (fp32 tiles out).  ND2: rank-2 tensors (row offset = r *
// row pitch); otherwise rows are decoded over the outer tile dimensions.
template <int MODE>
__device__ inline uint32_t nz_vec(uint4 x) {
  if constexpr (MODE == 0) {
    const uint32_t m = 0x7fff7fffu;
    return (x.x & m) | (x.y & m) | (x.z & m) | (x.w & m);
  } else if constexpr (MODE == 1) {
    const uint32_t m = 0x7fffffffu;
    return (x.x & m) | (x.y & m) | (x.z & m) | (x.w & m);
  } else {
    return (x.x | (x.y & 0x7fffffffu)) | (x.z | (x.w & 0x7fffffffu));
  }
}

template <int MODE, bool ND2>
__global__ __launch_bounds__(256) void tile_flags_vec_kernel(const unsigned char *__restrict__ dense,
                                                             BucketGeom g, int vpr,
                                                             int64_t row_pitch,
                                                             int64_t *flags) {
  constexpr int ESZ = MODE == 0 ? 2 : MODE == 1 ? 4 : 8;
  constexpr int U = 8;
  const int64_t t = blockIdx.x;
  const unsigned char *base = dense + tile_origin(g, t) * ESZ;
  const int c = threadIdx.x & (vpr - 1);
  const int rstep = 256 / vpr;
  uint32_t any = 0;
  // The trip count is the same for every thread (the loop holds a barrier).
  for (int64_t rb = 0; rb < g.rows; rb += static_cast<int64_t>(rstep) * U) {
    const int64_t r0 = rb + threadIdx.x / vpr;
    uint4 x[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t r = r0 + static_cast<int64_t>(u) * rstep;
      if (r < g.rows) {
        const int64_t roff = ND2 ? r * row_pitch : row_offset(g, r) * ESZ;
        x[u] = *reinterpret_cast<const uint4 *>(base + roff + c * 16);
      } else {
        x[u] = make_uint4(0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) any |= nz_vec<MODE>(x[u]);
    if (__syncthreads_or(any != 0)) break;
  }
  any = __syncthreads_or(any != 0);
  if (threadIdx.x == 0) flags[t] = any ? 1 : 0;
}

__device__ inline uint32_t zero_norm_bf16x2(uint32_t w) {
  const uint32_t lo = (w & 0x7fffu) ? (w & 0xffffu) : 0u;
  const uint32_t hi = (w & 0x7fff0000u) ? (w & 0xffff0000u) : 0u;
  return lo | hi;
}
__device__ inline uint32_t zero_norm_f32(uint32_t w) { return (w & 0x7fffffffu) ? w : 0u; }

template <int MODE, bool ND2>
__global__ __launch_bounds__(256) void tile_copy_vec_kernel(const unsigned char *__restrict__ dense,
                                                            BucketGeom g, int vpr,
                                                            int64_t row_pitch,
                                                            const int64_t *tile_of_slot,
                                                            const int64_t *counted,
                                                            int32_t *coords,
                                                            unsigned char *__restrict__ values) {
  constexpr int ESZ = MODE == 0 ? 2 : MODE == 1 ? 4 : 8;
  const int64_t slot = blockIdx.x;
  if (slot >= *counted) return;
  const int64_t t = tile_of_slot[slot];
  if (threadIdx.x == 0) {
    int64_t tt = t;
    for (int d = g.nd - 1; d >= 0; --d) {
      coords[slot * g.nd + d] = static_cast<int32_t>(tt % g.grid[d]);
      tt /= g.grid[d];
    }
  }
  const unsigned char *base = dense + tile_origin(g, t) * ESZ;
  unsigned char *dst = values + slot * g.tile_elems * ESZ;
  const int c = threadIdx.x & (vpr - 1);
  const int rstep = 256 / vpr;
  const int per_vec = 16 / ESZ;  // input elements per vector
  for (int64_t r = threadIdx.x / vpr; r < g.rows; r += rstep) {
    const int64_t roff = ND2 ? r * row_pitch : row_offset(g, r) * ESZ;
    const uint4 x = *reinterpret_cast<const uint4 *>(base + roff + c * 16);
    unsigned char *o = dst + (r * g.inner + static_cast<int64_t>(c) * per_vec) * ESZ;
    if constexpr (MODE == 0) {
      *reinterpret_cast<uint4 *>(o) = make_uint4(zero_norm_bf16x2(x.x), zero_norm_bf16x2(x.y),
                                                 zero_norm_bf16x2(x.z), zero_norm_bf16x2(x.w));
    } else if constexpr (MODE == 1) {
      *reinterpret_cast<uint4 *>(o) = make_uint4(zero_norm_f32(x.x), zero_norm_f32(x.y),
                                                 zero_norm_f32(x.z), zero_norm_f32(x.w));
    } else {  // float64: a word pair is zero when both halves are, ignoring the sign bit
      const bool z0 = (x.x | (x.y & 0x7fffffffu)) == 0u;
      const bool z1 = (x.z | (x.w & 0x7fffffffu)) == 0u;
      *reinterpret_cast<uint4 *>(o) = make_uint4(z0 ? 0u : x.x, z0 ? 0u : x.y, z1 ? 0u : x.z,
                                                 z1 ? 0u : x.w);
    }
  }
}

// Vector geometry: vectors per tile row, or 0 when the vector kernels do
// not apply (row not a whole number of 16-byte vectors, misaligned pitch).
int vec_shape(const BucketGeom &g, int esz, const void *dense, int64_t *row_pitch) {
  const int64_t inner_b = g.inner * esz;
  if (inner_b % 16 != 0 || (reinterpret_cast<uintptr_t>(dense) & 15u) != 0) return 0;
  const int64_t vpr = inner_b / 16;
  if (vpr > 256 || (vpr & (vpr - 1)) != 0) return 0;
  const int64_t pitch = g.nd >= 2 ? g.dstride[g.nd - 2] * esz : 0;
  if (pitch % 16 != 0) return 0;
  *row_pitch = pitch;
  return static_cast<int>(vpr);
}

__global__ void slot_map_kernel(const int64_t *flags, const int64_t *excl, int64_t n,
                                int64_t *tile_of_slot) {
  int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t < n && flags[t]) tile_of_slot[excl[t]] = t;
}

template <typename T, typename U>
__global__ __launch_bounds__(256) void tile_copy_kernel(const T *__restrict__ dense, BucketGeom g,
                                                        const int64_t *tile_of_slot,
                                                        const int64_t *counted, int32_t *coords,
                                                        U *__restrict__ values) {
  const int64_t slot = blockIdx.x;
  if (slot >= *counted) return;  // only slots the count filled in
  int64_t t = tile_of_slot[slot];
  if (threadIdx.x == 0) {
    int64_t tt = t;
    for (int d = g.nd - 1; d >= 0; --d) {
      coords[slot * g.nd + d] = static_cast<int32_t>(tt % g.grid[d]);
      tt /= g.grid[d];
    }
  }
  const T *base = dense + tile_origin(g, t);
  U *dst = values + slot * g.tile_elems;
  for (int64_t e = threadIdx.x; e < g.tile_elems; e += 256) {
    const int64_t r = e / g.inner, c = e % g.inner;
    dst[e] = stored(base[row_offset(g, r) + c]);
  }
}

template <typename T>
__global__ void fill_zero_kernel(T *p, int64_t n) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (; i < n; i += stride) p[i] = T(0);
}

template <typename T>
__global__ __launch_bounds__(256) void scatter_tiles_kernel(const int32_t *coords,
                                                            const T *__restrict__ values,
                                                            BucketGeom g, T *__restrict__ dense) {
  const int64_t slot = blockIdx.x;
  int64_t origin = 0;
  for (int d = 0; d < g.nd; ++d) {
    const int64_t c = coords[slot * g.nd + d];
    if (c < 0 || c >= g.grid[d]) return;  // outside the grid: skipped
    origin += c * g.tile[d] * g.dstride[d];
  }
  const T *src = values + slot * g.tile_elems;
  for (int64_t e = threadIdx.x; e < g.tile_elems; e += 256) {
    const int64_t r = e / g.inner, c = e % g.inner;
    dense[origin + row_offset(g, r) + c] = src[e];
  }
}

struct BucketWs {
  int64_t *scalars, *flags, *excl, *tile_of_slot;
  void *scan_ws;
  size_t bytes;
};

BucketWs carve_bucket(void *base, int64_t n_tiles) {
  Carver c(base);
  BucketWs w;
  w.scalars = c.take<int64_t>(4);
  w.flags = c.take<int64_t>(n_tiles);
  w.excl = c.take<int64_t>(n_tiles);
  w.tile_of_slot = c.take<int64_t>(n_tiles);
  w.scan_ws = c.take<char>(static_cast<int64_t>(scan_workspace_bytes(n_tiles)));
  w.bytes = c.off;
  return w;
}

}  // namespace
}  // namespace ej

using namespace ej;

extern "C" int ej_bucket_workspace_size(int32_t ndim, const int64_t *shape,
                                        const int64_t *tile_shape, size_t *bytes) {
  clear_error();
  EJ_CHECK_ARG(bytes, "bytes is null");
  BucketGeom g;
  EJ_TRY(make_geom(ndim, shape, tile_shape, &g));
  *bytes = carve_bucket(nullptr, g.n_tiles).bytes;
  return EJ_OK;
}

extern "C" int ej_bucket_dense_count(const void *dense, int32_t dtype, int32_t ndim,
                                     const int64_t *shape, const int64_t *tile_shape,
                                     void *workspace, size_t workspace_bytes, int64_t *n_tiles,
                                     ej_stream_t stream_) {
  clear_error();
  hipStream_t stream = as_stream(stream_);
  EJ_CHECK_ARG(n_tiles, "n_tiles is null");
  EJ_CHECK_ARG(dtype == EJ_F32 || dtype == EJ_BF16 || dtype == EJ_F64, "unknown dtype %d", dtype);
  BucketGeom g;
  EJ_TRY(make_geom(ndim, shape, tile_shape, &g));
  if (g.n_tiles == 0 || g.tile_elems == 0) {
    *n_tiles = 0;
    return EJ_OK;
  }
  EJ_CHECK_ARG(g.n_tiles < (int64_t(1) << 32), "tile grid too large for one launch");
  EJ_CHECK_ARG(dense, "dense is null");
  BucketWs w = carve_bucket(workspace, g.n_tiles);
  EJ_CHECK_ARG(workspace && workspace_bytes >= w.bytes, "workspace too small: %zu < %zu bytes",
               workspace_bytes, w.bytes);
  const int esz = dtype == EJ_F64 ? 8 : dtype == EJ_F32 ? 4 : 2;
  const int mode = dtype == EJ_F64 ? 2 : dtype == EJ_F32 ? 1 : 0;
  int64_t pitch = 0;
  const int vpr = vec_shape(g, esz, dense, &pitch);
  const dim3 grid(static_cast<unsigned>(g.n_tiles));
  const unsigned char *db = static_cast<const unsigned char *>(dense);
  if (vpr > 0) {
#define EJ_FLAGS(M, N2) hipLaunchKernelGGL((tile_flags_vec_kernel<M, N2>), grid, dim3(256), 0, stream, db, g, vpr, pitch, w.flags)
    if (g.nd == 2) {
      if (mode == 0) EJ_FLAGS(0, true); else if (mode == 1) EJ_FLAGS(1, true); else EJ_FLAGS(2, true);
    } else {
      if (mode == 0) EJ_FLAGS(0, false); else if (mode == 1) EJ_FLAGS(1, false); else EJ_FLAGS(2, false);
    }
#undef EJ_FLAGS
  } else if (dtype == EJ_F64)
    hipLaunchKernelGGL(tile_flags_kernel<double>, grid, dim3(256), 0, stream,
                       static_cast<const double *>(dense), g, w.flags);
  else if (dtype == EJ_F32)
    hipLaunchKernelGGL(tile_flags_kernel<float>, grid, dim3(256), 0, stream,
                       static_cast<const float *>(dense), g, w.flags);
  else
    hipLaunchKernelGGL(tile_flags_kernel<uint16_t>, grid, dim3(256), 0, stream,
                       static_cast<const uint16_t *>(dense), g, w.flags);
  EJ_LAUNCH_CHECK();
  EJ_TRY(scan_exclusive_i64(w.flags, w.excl, g.n_tiles, w.scalars, w.scan_ws, stream));
  hipLaunchKernelGGL(slot_map_kernel, dim3(grid_for(g.n_tiles)), dim3(kBlock), 0, stream, w.flags,
                     w.excl, g.n_tiles, w.tile_of_slot);
  EJ_LAUNCH_CHECK();
  int64_t host = 0;
  EJ_HIP(hipMemcpyAsync(&host, w.scalars, sizeof(int64_t), hipMemcpyDeviceToHost, stream));
  EJ_HIP(hipStreamSynchronize(stream));
  *n_tiles = host;
  return EJ_OK;
}

extern "C" int ej_bucket_dense_fill(const void *dense, int32_t dtype, int32_t ndim,
                                    const int64_t *shape, const int64_t *tile_shape,
                                    const void *workspace, size_t workspace_bytes,
                                    int64_t n_tiles, int32_t *coords, void *values,
                                    int64_t capacity, ej_stream_t stream_) {
  clear_error();
  hipStream_t stream = as_stream(stream_);
  EJ_CHECK_ARG(dtype == EJ_F32 || dtype == EJ_BF16 || dtype == EJ_F64, "unknown dtype %d", dtype);
  BucketGeom g;
  EJ_TRY(make_geom(ndim, shape, tile_shape, &g));
  EJ_CHECK_ARG(n_tiles >= 0 && n_tiles <= g.n_tiles, "n_tiles out of range");
  if (capacity < n_tiles) {
    set_error("tile capacity %lld < %lld tiles", (long long)capacity, (long long)n_tiles);
    return EJ_E_CAPACITY;
  }
  if (n_tiles == 0) return EJ_OK;
  EJ_CHECK_ARG(dense && coords && values, "null pointer argument");
  BucketWs w = carve_bucket(const_cast<void *>(workspace), g.n_tiles);
  EJ_CHECK_ARG(workspace && workspace_bytes >= w.bytes, "workspace too small");
  const int esz = dtype == EJ_F64 ? 8 : dtype == EJ_F32 ? 4 : 2;
  const int mode = dtype == EJ_F64 ? 2 : dtype == EJ_F32 ? 1 : 0;
  int64_t pitch = 0;
  const int vpr = vec_shape(g, esz, dense, &pitch);
  const dim3 grid(static_cast<unsigned>(n_tiles));
  const bool out_aligned = (reinterpret_cast<uintptr_t>(values) & 15u) == 0;
  if (vpr > 0 && out_aligned) {
    const unsigned char *db = static_cast<const unsigned char *>(dense);
    unsigned char *vb = static_cast<unsigned char *>(values);
#define EJ_COPY(M, N2) hipLaunchKernelGGL((tile_copy_vec_kernel<M, N2>), grid, dim3(256), 0, stream, db, g, vpr, pitch, w.tile_of_slot, w.scalars, coords, vb)
    if (g.nd == 2) {
      if (mode == 0) EJ_COPY(0, true); else if (mode == 1) EJ_COPY(1, true); else EJ_COPY(2, true);
    } else {
      if (mode == 0) EJ_COPY(0, false); else if (mode == 1) EJ_COPY(1, false); else EJ_COPY(2, false);
    }
#undef EJ_COPY
  } else if (dtype == EJ_F64)
    hipLaunchKernelGGL((tile_copy_kernel<double, double>), grid, dim3(256), 0, stream,
                       static_cast<const double *>(dense), g, w.tile_of_slot, w.scalars, coords,
                       static_cast<double *>(values));
  else if (dtype == EJ_F32)
    hipLaunchKernelGGL((tile_copy_kernel<float, float>), grid, dim3(256), 0, stream,
                       static_cast<const float *>(dense), g, w.tile_of_slot, w.scalars, coords,
                       static_cast<float *>(values));
  else
    hipLaunchKernelGGL((tile_copy_kernel<uint16_t, uint16_t>), grid, dim3(256), 0, stream,
                       static_cast<const uint16_t *>(dense), g, w.tile_of_slot, w.scalars, coords,
                       static_cast<uint16_t *>(values));
  EJ_LAUNCH_CHECK();
  return EJ_OK;
}

extern "C" int ej_relation_to_dense(const int32_t *coords, const void *values, int64_t n_tiles,
                                    int32_t dtype, int32_t ndim, const int64_t *shape,
                                    const int64_t *tile_shape, void *dense,
                                    ej_stream_t stream_) {
  clear_error();
  hipStream_t stream = as_stream(stream_);
  EJ_CHECK_ARG(dtype == EJ_F32 || dtype == EJ_BF16 || dtype == EJ_F64, "unknown dtype %d", dtype);
  BucketGeom g;
  EJ_TRY(make_geom(ndim, shape, tile_shape, &g));
  EJ_CHECK_ARG(n_tiles >= 0 && n_tiles < (int64_t(1) << 32), "n_tiles out of range");
  int64_t total = 1;
  for (int d = 0; d < ndim; ++d) total *= shape[d];
  if (total == 0) return EJ_OK;
  EJ_CHECK_ARG(dense, "dense is null");
  const unsigned zb = static_cast<unsigned>(ceil_div(total, 256) < 65536 ? ceil_div(total, 256) : 65536);
  if (dtype == EJ_F64)
    hipLaunchKernelGGL(fill_zero_kernel<double>, dim3(zb), dim3(256), 0, stream,
                       static_cast<double *>(dense), total);
  else if (dtype == EJ_F32)
    hipLaunchKernelGGL(fill_zero_kernel<float>, dim3(zb), dim3(256), 0, stream,
                       static_cast<float *>(dense), total);
  else
    hipLaunchKernelGGL(fill_zero_kernel<uint16_t>, dim3(zb), dim3(256), 0, stream,
                       static_cast<uint16_t *>(dense), total);
  EJ_LAUNCH_CHECK();
  if (n_tiles == 0) return EJ_OK;
  EJ_CHECK_ARG(coords && values, "null pointer argument");
  if (dtype == EJ_F64)
    hipLaunchKernelGGL(scatter_tiles_kernel<double>, dim3(static_cast<unsigned>(n_tiles)),
                       dim3(256), 0, stream, coords, static_cast<const double *>(values), g,
                       static_cast<double *>(dense));
  else if (dtype == EJ_F32)
    hipLaunchKernelGGL(scatter_tiles_kernel<float>, dim3(static_cast<unsigned>(n_tiles)), dim3(256),
                       0, stream, coords, static_cast<const float *>(values), g,
                       static_cast<float *>(dense));
  else
    hipLaunchKernelGGL(scatter_tiles_kernel<uint16_t>, dim3(static_cast<unsigned>(n_tiles)),
                       dim3(256), 0, stream, coords, static_cast<const uint16_t *>(values), g,
                       static_cast<uint16_t *>(dense));
  EJ_LAUNCH_CHECK();
  return EJ_OK;
}
