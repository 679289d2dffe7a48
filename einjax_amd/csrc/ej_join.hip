// Tile-coordinate join, per-pair output coordinates and the segment plan.
//
// Join (reference: coordinate_join, execution/sparse_dispatch.py:29-82, and
// coordinate_join_sorted, kernels/pallas_gather.py:79-174):
//   1. the join columns of every coordinate row are packed into one int64
//      mixed-radix key (key order == lexicographic tuple order);
//   2. the build side is stably radix-sorted by key (stable = original index
//      ascending inside a key, the order the reference's dict lists keep);
//   3. every probe row binary-searches its equal range -> count;
//   4. exclusive scan of the counts -> output offsets, total = P;
//   5. fill: one thread per output pair locates its probe row by a binary
//      search over the offsets (balanced under skewed keys) and writes the
//      pair.  Probe order EJ_ORDER_PROBE: probe side = rhs in index order,
//      giving the hash join's order.  EJ_ORDER_SORTED: both sides sorted,
//      probe side = lhs in sorted order, giving the sort-merge order.
#include "ej_internal.h"

namespace ej {

namespace {

__global__ void pack_keys_kernel(const int32_t *coords, int64_t n, KeySpec ks, uint64_t *keys,
                                 int *bad) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  int b = 0;
  keys[i] = pack_key(coords + i * ks.ncols, ks, &b);
  if (b) atomicOr(bad, 1);
}

__device__ inline int64_t lower_bound_u64(const uint64_t *a, int64_t n, uint64_t x) {
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    int64_t mid = (lo + hi) >> 1;
    if (a[mid] < x) lo = mid + 1; else hi = mid;
  }
  return lo;
}

__device__ inline int64_t upper_bound_u64(const uint64_t *a, int64_t n, uint64_t x) {
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    int64_t mid = (lo + hi) >> 1;
    if (a[mid] <= x) lo = mid + 1; else hi = mid;
  }
  return lo;
}

// Largest j with offs[j] <= q (offs ascending, offs[0] == 0).
__device__ inline int64_t owner_of(const int64_t *offs, int64_t n, int64_t q) {
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    int64_t mid = (lo + hi) >> 1;
    if (offs[mid] <= q) lo = mid + 1; else hi = mid;
  }
  return lo - 1;
}

__global__ void probe_count_kernel(const uint64_t *probe_keys, int64_t n_probe,
                                   const uint64_t *build_sorted, int64_t n_build, int64_t *lo_out,
                                   int64_t *cnt_out) {
  int64_t j = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (j >= n_probe) return;
  uint64_t k = probe_keys[j];
  int64_t lo = lower_bound_u64(build_sorted, n_build, k);
  int64_t hi = upper_bound_u64(build_sorted, n_build, k);
  lo_out[j] = lo;
  cnt_out[j] = hi - lo;
}

// EJ_ORDER_PROBE fill: pair q belongs to rhs row j = owner_of(offs, q).
__global__ void fill_probe_order_kernel(const int64_t *offs, int64_t n_rhs, const int64_t *lo,
                                        const int32_t *lhs_perm, int64_t n_pairs,
                                        const int64_t *counted, int64_t *lhs_idx,
                                        int64_t *rhs_idx) {
  int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (q >= n_pairs || q >= *counted) return;
  int64_t j = owner_of(offs, n_rhs, q);
  int64_t t = q - offs[j];
  lhs_idx[q] = lhs_perm[lo[j] + t];
  rhs_idx[q] = j;
}

// EJ_ORDER_SORTED fill: pair q belongs to sorted lhs position p.
__global__ void fill_sorted_order_kernel(const int64_t *offs, int64_t n_lhs, const int64_t *lo,
                                         const int32_t *lhs_perm, const int32_t *rhs_perm,
                                         int64_t n_pairs, const int64_t *counted,
                                         int64_t *lhs_idx, int64_t *rhs_idx) {
  int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (q >= n_pairs || q >= *counted) return;
  int64_t p = owner_of(offs, n_lhs, q);
  int64_t t = q - offs[p];
  lhs_idx[q] = lhs_perm[p];
  rhs_idx[q] = rhs_perm[lo[p] + t];
}

__global__ void fill_cross_kernel(int64_t n_rhs, int64_t n_pairs, int64_t *lhs_idx,
                                  int64_t *rhs_idx) {
  int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (q >= n_pairs) return;
  lhs_idx[q] = q / n_rhs;
  rhs_idx[q] = q % n_rhs;
}

// Workspace layout shared by ej_join_count and ej_join_fill.
struct JoinWs {
  int64_t *scalars;  // [0] = P, [1] = bad-coordinate flag (as int)
  uint64_t *lkeys, *lkeys_alt, *rkeys, *rkeys_alt;
  int32_t *lperm, *lperm_alt, *rperm, *rperm_alt;
  int64_t *lo, *cnt, *offs;
  void *sort_ws, *scan_ws;
  size_t bytes;
};

JoinWs carve_join(void *base, int64_t n_lhs, int64_t n_rhs, int32_t order) {
  Carver c(base);
  JoinWs w;
  const int64_t n_probe = order == EJ_ORDER_SORTED ? n_lhs : n_rhs;
  w.scalars = c.take<int64_t>(4);
  w.lkeys = c.take<uint64_t>(n_lhs);
  w.lkeys_alt = c.take<uint64_t>(n_lhs);
  w.rkeys = c.take<uint64_t>(n_rhs);
  w.rkeys_alt = c.take<uint64_t>(n_rhs);
  w.lperm = c.take<int32_t>(n_lhs);
  w.lperm_alt = c.take<int32_t>(n_lhs);
  w.rperm = c.take<int32_t>(n_rhs);
  w.rperm_alt = c.take<int32_t>(n_rhs);
  w.lo = c.take<int64_t>(n_probe);
  w.cnt = c.take<int64_t>(n_probe);
  w.offs = c.take<int64_t>(n_probe);
  int64_t nmax = n_lhs > n_rhs ? n_lhs : n_rhs;
  w.sort_ws = c.take<char>(static_cast<int64_t>(sort_workspace_bytes(nmax)));
  w.scan_ws = c.take<char>(static_cast<int64_t>(scan_workspace_bytes(n_probe)));
  w.bytes = c.off;
  return w;
}

int check_keyspec(int32_t n_keys, const int32_t *dims, int32_t ncols, const int64_t *radices,
                  const char *side, KeySpec *ks) {
  EJ_CHECK_ARG(n_keys >= 0 && n_keys <= EJ_MAX_KEYS, "n_keys=%d outside [0, %d]", n_keys,
               EJ_MAX_KEYS);
  EJ_CHECK_ARG(ncols >= 0 && ncols <= EJ_MAX_DIMS, "%s ncols=%d outside [0, %d]", side, ncols,
               EJ_MAX_DIMS);
  ks->n = n_keys;
  ks->ncols = ncols;
  for (int i = 0; i < n_keys; ++i) {
    EJ_CHECK_ARG(dims && dims[i] >= 0 && dims[i] < ncols, "%s join dim %d out of range", side, i);
    EJ_CHECK_ARG(radices && radices[i] > 0, "radix %d must be positive", i);
    ks->dims[i] = dims[i];
    ks->radix[i] = radices[i];
  }
  return EJ_OK;
}

}  // namespace

}  // namespace ej

using namespace ej;

extern "C" int ej_join_workspace_size(int64_t n_lhs, int64_t n_rhs, int32_t order, size_t *bytes) {
  clear_error();
  EJ_CHECK_ARG(bytes, "bytes is null");
  EJ_CHECK_ARG(n_lhs >= 0 && n_rhs >= 0, "negative relation size");
  EJ_CHECK_ARG(order == EJ_ORDER_PROBE || order == EJ_ORDER_SORTED, "unknown join order %d",
               order);
  *bytes = carve_join(nullptr, n_lhs, n_rhs, order).bytes;
  return EJ_OK;
}

extern "C" int ej_join_count(const int32_t *lhs_coords, int64_t n_lhs, int32_t lhs_ncols,
                             const int32_t *rhs_coords, int64_t n_rhs, int32_t rhs_ncols,
                             int32_t n_keys, const int32_t *lhs_dims, const int32_t *rhs_dims,
                             const int64_t *radices, int32_t order, void *workspace,
                             size_t workspace_bytes, int64_t *n_pairs, ej_stream_t stream_) {
  clear_error();
  hipStream_t stream = as_stream(stream_);
  EJ_CHECK_ARG(n_pairs, "n_pairs is null");
  EJ_CHECK_ARG(n_lhs >= 0 && n_rhs >= 0, "negative relation size");
  EJ_CHECK_ARG(n_lhs < (int64_t(1) << 31) && n_rhs < (int64_t(1) << 31),
               "relations are limited to 2^31 - 1 tiles");
  EJ_CHECK_ARG(order == EJ_ORDER_PROBE || order == EJ_ORDER_SORTED, "unknown join order %d",
               order);
  KeySpec lks, rks;
  EJ_TRY(check_keyspec(n_keys, lhs_dims, lhs_ncols, radices, "lhs", &lks));
  EJ_TRY(check_keyspec(n_keys, rhs_dims, rhs_ncols, radices, "rhs", &rks));
  if (n_keys == 0 || n_lhs == 0 || n_rhs == 0) {
    // Cross product (lhs-major) or an empty side: size known on the host.
    unsigned __int128 p = n_keys == 0 ? static_cast<unsigned __int128>(n_lhs) * n_rhs : 0;
    if (p >= (static_cast<unsigned __int128>(1) << 62)) {
      set_error("cross product too large");
      return EJ_E_UNSUPPORTED;
    }
    *n_pairs = static_cast<int64_t>(p);
    return EJ_OK;
  }
  EJ_CHECK_ARG(lhs_coords && rhs_coords, "coordinate pointer is null");
  int bits = 0;
  EJ_TRY(key_bits(radices, n_keys, &bits));
  JoinWs w = carve_join(workspace, n_lhs, n_rhs, order);
  EJ_CHECK_ARG(workspace && workspace_bytes >= w.bytes, "workspace too small: %zu < %zu bytes",
               workspace_bytes, w.bytes);

  EJ_HIP(hipMemsetAsync(w.scalars, 0, 4 * sizeof(int64_t), stream));
  int *bad = reinterpret_cast<int *>(w.scalars + 1);
  hipLaunchKernelGGL(pack_keys_kernel, dim3(grid_for(n_lhs)), dim3(kBlock), 0, stream, lhs_coords,
                     n_lhs, lks, w.lkeys, bad);
  EJ_LAUNCH_CHECK();
  hipLaunchKernelGGL(pack_keys_kernel, dim3(grid_for(n_rhs)), dim3(kBlock), 0, stream, rhs_coords,
                     n_rhs, rks, w.rkeys, bad);
  EJ_LAUNCH_CHECK();
  EJ_TRY(fill_iota_i32(w.lperm, n_lhs, stream));
  EJ_TRY(sort_pairs_u64(w.lkeys, w.lperm, w.lkeys_alt, w.lperm_alt, n_lhs, bits, w.sort_ws,
                        stream));
  int64_t n_probe;
  if (order == EJ_ORDER_PROBE) {
    n_probe = n_rhs;
    hipLaunchKernelGGL(probe_count_kernel, dim3(grid_for(n_rhs)), dim3(kBlock), 0, stream,
                       w.rkeys, n_rhs, w.lkeys, n_lhs, w.lo, w.cnt);
  } else {
    EJ_TRY(fill_iota_i32(w.rperm, n_rhs, stream));
    EJ_TRY(sort_pairs_u64(w.rkeys, w.rperm, w.rkeys_alt, w.rperm_alt, n_rhs, bits, w.sort_ws,
                          stream));
    n_probe = n_lhs;
    hipLaunchKernelGGL(probe_count_kernel, dim3(grid_for(n_lhs)), dim3(kBlock), 0, stream,
                       w.lkeys, n_lhs, w.rkeys, n_rhs, w.lo, w.cnt);
  }
  EJ_LAUNCH_CHECK();
  EJ_TRY(scan_exclusive_i64(w.cnt, w.offs, n_probe, w.scalars, w.scan_ws, stream));
  int64_t host[2] = {0, 0};
  EJ_HIP(hipMemcpyAsync(host, w.scalars, 2 * sizeof(int64_t), hipMemcpyDeviceToHost, stream));
  EJ_HIP(hipStreamSynchronize(stream));
  if (host[1] != 0) {
    set_error("a join-key coordinate lies outside [0, radix)");
    return EJ_E_RANGE;
  }
  *n_pairs = host[0];
  return EJ_OK;
}

extern "C" int ej_join_fill(int64_t n_lhs, int64_t n_rhs, int32_t n_keys, int32_t order,
                            const void *workspace, size_t workspace_bytes, int64_t n_pairs,
                            int64_t *lhs_idx, int64_t *rhs_idx, int64_t capacity,
                            ej_stream_t stream_) {
  clear_error();
  hipStream_t stream = as_stream(stream_);
  EJ_CHECK_ARG(n_pairs >= 0, "negative n_pairs");
  if (capacity < n_pairs) {
    set_error("pair capacity %lld < %lld matched pairs", (long long)capacity, (long long)n_pairs);
    return EJ_E_CAPACITY;
  }
  if (n_pairs == 0) return EJ_OK;
  EJ_CHECK_ARG(lhs_idx && rhs_idx, "output pointer is null");
  if (n_keys == 0) {
    EJ_CHECK_ARG(n_rhs > 0 && n_pairs == n_lhs * n_rhs, "cross product size mismatch");
    hipLaunchKernelGGL(fill_cross_kernel, dim3(grid_for(n_pairs)), dim3(kBlock), 0, stream, n_rhs,
                       n_pairs, lhs_idx, rhs_idx);
    EJ_LAUNCH_CHECK();
    return EJ_OK;
  }
  JoinWs w = carve_join(const_cast<void *>(workspace), n_lhs, n_rhs, order);
  EJ_CHECK_ARG(workspace && workspace_bytes >= w.bytes, "workspace too small");
  if (order == EJ_ORDER_PROBE) {
    hipLaunchKernelGGL(fill_probe_order_kernel, dim3(grid_for(n_pairs)), dim3(kBlock), 0, stream,
                       w.offs, n_rhs, w.lo, w.lperm, n_pairs, w.scalars, lhs_idx, rhs_idx);
  } else {
    hipLaunchKernelGGL(fill_sorted_order_kernel, dim3(grid_for(n_pairs)), dim3(kBlock), 0, stream,
                       w.offs, n_lhs, w.lo, w.lperm, w.rperm, n_pairs, w.scalars, lhs_idx,
                       rhs_idx);
  }
  EJ_LAUNCH_CHECK();
  return EJ_OK;
}

// ---------------------------------------------------------------------------
// Output coordinates and the segment plan.

namespace ej {
namespace {

struct AggSpec {
  int32_t n;
  int32_t lncols, rncols;
  int64_t n_lhs, n_rhs;
  int32_t src[EJ_MAX_KEYS];
  int32_t dim[EJ_MAX_KEYS];
  int64_t radix[EJ_MAX_KEYS];
};

int check_agg(int32_t n_out, const int32_t *agg_src, const int32_t *agg_dim, int64_t n_lhs,
              int32_t lncols, int64_t n_rhs, int32_t rncols, const int64_t *radices, AggSpec *a) {
  EJ_CHECK_ARG(n_out >= 0 && n_out <= EJ_MAX_KEYS, "n_out=%d outside [0, %d]", n_out,
               EJ_MAX_KEYS);
  EJ_CHECK_ARG(n_lhs >= 0 && n_rhs >= 0, "negative relation size");
  EJ_CHECK_ARG(lncols >= 0 && lncols <= EJ_MAX_DIMS && rncols >= 0 && rncols <= EJ_MAX_DIMS,
               "coordinate rank outside [0, %d]", EJ_MAX_DIMS);
  a->n = n_out;
  a->n_lhs = n_lhs;
  a->n_rhs = n_rhs;
  a->lncols = lncols;
  a->rncols = rncols;
  for (int d = 0; d < n_out; ++d) {
    EJ_CHECK_ARG(agg_src && agg_dim, "agg arrays are null");
    EJ_CHECK_ARG(agg_src[d] == 0 || agg_src[d] == 1, "agg source %d must be 0 or 1", d);
    int nc = agg_src[d] == 0 ? lncols : rncols;
    EJ_CHECK_ARG(agg_dim[d] >= 0 && agg_dim[d] < nc, "agg dim %d out of range", d);
    a->src[d] = agg_src[d];
    a->dim[d] = agg_dim[d];
    a->radix[d] = radices ? radices[d] : 1;
    if (radices) EJ_CHECK_ARG(radices[d] > 0, "output radix %d must be positive", d);
  }
  return EJ_OK;
}

__global__ void output_coords_kernel(const int32_t *lc, const int32_t *rc, const int64_t *li,
                                     const int64_t *ri, int64_t n, AggSpec a, int32_t *out) {
  int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (p >= n) return;
  if (li[p] < 0 || li[p] >= a.n_lhs || ri[p] < 0 || ri[p] >= a.n_rhs) {
    for (int d = 0; d < a.n; ++d) out[p * a.n + d] = -1;
    return;
  }
  const int32_t *lrow = lc + li[p] * a.lncols;
  const int32_t *rrow = rc + ri[p] * a.rncols;
  for (int d = 0; d < a.n; ++d) out[p * a.n + d] = a.src[d] == 0 ? lrow[a.dim[d]] : rrow[a.dim[d]];
}

__global__ void pair_keys_kernel(const int32_t *lc, const int32_t *rc, const int64_t *li,
                                 const int64_t *ri, int64_t n, AggSpec a, uint64_t *keys,
                                 int *bad) {
  int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (p >= n) return;
  if (li[p] < 0 || li[p] >= a.n_lhs || ri[p] < 0 || ri[p] >= a.n_rhs) {
    keys[p] = 0;
    atomicOr(bad, 1);
    return;
  }
  const int32_t *lrow = lc + li[p] * a.lncols;
  const int32_t *rrow = rc + ri[p] * a.rncols;
  uint64_t key = 0;
  bool b = false;
  for (int d = 0; d < a.n; ++d) {
    int64_t c = a.src[d] == 0 ? lrow[a.dim[d]] : rrow[a.dim[d]];
    if (c < 0 || c >= a.radix[d]) {
      b = true;
      c = 0;
    }
    key = key * static_cast<uint64_t>(a.radix[d]) + static_cast<uint64_t>(c);
  }
  keys[p] = key;
  if (b) atomicOr(bad, 1);
}

__global__ void seg_flags_kernel(const uint64_t *skeys, int64_t n, int64_t *flags) {
  int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (q >= n) return;
  flags[q] = (q == 0 || skeys[q] != skeys[q - 1]) ? 1 : 0;
}

__global__ void seg_fill_kernel(const uint64_t *skeys, const int32_t *sperm, const int64_t *flags,
                                const int64_t *excl, int64_t n, int64_t n_seg, AggSpec a,
                                int32_t *out_coords, int32_t *seg_offsets, int32_t *perm,
                                int32_t *seg_ids) {
  int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (q >= n) return;
  const int64_t seg = excl[q] + flags[q] - 1;
  perm[q] = sperm[q];
  if (seg_ids) seg_ids[sperm[q]] = static_cast<int32_t>(seg);
  if (flags[q] && seg < n_seg) {
    seg_offsets[seg] = static_cast<int32_t>(q);
    uint64_t key = skeys[q];
    for (int d = a.n - 1; d >= 0; --d) {
      uint64_t r = static_cast<uint64_t>(a.radix[d]);
      out_coords[seg * a.n + d] = static_cast<int32_t>(key % r);
      key /= r;
    }
  }
  if (q == 0) seg_offsets[n_seg] = static_cast<int32_t>(n);
}

struct SegWs {
  int64_t *scalars;  // [0] = U, [1] = bad flag
  uint64_t *keys, *keys_alt;
  int32_t *perm, *perm_alt;
  int64_t *flags, *excl;
  void *sort_ws, *scan_ws;
  size_t bytes;
};

SegWs carve_seg(void *base, int64_t n) {
  Carver c(base);
  SegWs w;
  w.scalars = c.take<int64_t>(4);
  w.keys = c.take<uint64_t>(n);
  w.keys_alt = c.take<uint64_t>(n);
  w.perm = c.take<int32_t>(n);
  w.perm_alt = c.take<int32_t>(n);
  w.flags = c.take<int64_t>(n);
  w.excl = c.take<int64_t>(n);
  w.sort_ws = c.take<char>(static_cast<int64_t>(sort_workspace_bytes(n)));
  w.scan_ws = c.take<char>(static_cast<int64_t>(scan_workspace_bytes(n)));
  w.bytes = c.off;
  return w;
}

}  // namespace
}  // namespace ej

extern "C" int ej_output_coords(const int32_t *lhs_coords, int64_t n_lhs, int32_t lhs_ncols,
                                const int32_t *rhs_coords, int64_t n_rhs, int32_t rhs_ncols,
                                const int64_t *lhs_idx, const int64_t *rhs_idx, int64_t n_pairs,
                                int32_t n_out, const int32_t *agg_src, const int32_t *agg_dim,
                                int32_t *out, ej_stream_t stream_) {
  clear_error();
  AggSpec a;
  EJ_TRY(check_agg(n_out, agg_src, agg_dim, n_lhs, lhs_ncols, n_rhs, rhs_ncols, nullptr, &a));
  EJ_CHECK_ARG(n_pairs >= 0, "negative n_pairs");
  if (n_pairs == 0 || n_out == 0) return EJ_OK;
  EJ_CHECK_ARG(lhs_coords && rhs_coords && lhs_idx && rhs_idx && out, "null pointer argument");
  hipLaunchKernelGGL(output_coords_kernel, dim3(grid_for(n_pairs)), dim3(kBlock), 0,
                     as_stream(stream_), lhs_coords, rhs_coords, lhs_idx, rhs_idx, n_pairs, a, out);
  EJ_LAUNCH_CHECK();
  return EJ_OK;
}

extern "C" int ej_segment_workspace_size(int64_t n_pairs, size_t *bytes) {
  clear_error();
  EJ_CHECK_ARG(bytes && n_pairs >= 0, "bad arguments");
  *bytes = carve_seg(nullptr, n_pairs).bytes;
  return EJ_OK;
}

extern "C" int ej_segment_count(const int32_t *lhs_coords, int64_t n_lhs, int32_t lhs_ncols,
                                const int32_t *rhs_coords, int64_t n_rhs, int32_t rhs_ncols,
                                const int64_t *lhs_idx, const int64_t *rhs_idx, int64_t n_pairs,
                                int32_t n_out, const int32_t *agg_src, const int32_t *agg_dim,
                                const int64_t *radices, void *workspace, size_t workspace_bytes,
                                int64_t *n_segments, ej_stream_t stream_) {
  clear_error();
  hipStream_t stream = as_stream(stream_);
  EJ_CHECK_ARG(n_segments, "n_segments is null");
  EJ_CHECK_ARG(n_pairs >= 0 && n_pairs < (int64_t(1) << 31), "n_pairs must lie in [0, 2^31)");
  EJ_CHECK_ARG(radices || n_out == 0, "radices is null");
  AggSpec a;
  EJ_TRY(check_agg(n_out, agg_src, agg_dim, n_lhs, lhs_ncols, n_rhs, rhs_ncols, radices, &a));
  if (n_pairs == 0) {
    *n_segments = 0;
    return EJ_OK;
  }
  EJ_CHECK_ARG(lhs_coords && rhs_coords && lhs_idx && rhs_idx, "null pointer argument");
  int bits = 0;
  EJ_TRY(key_bits(a.radix, n_out, &bits));
  SegWs w = carve_seg(workspace, n_pairs);
  EJ_CHECK_ARG(workspace && workspace_bytes >= w.bytes, "workspace too small: %zu < %zu bytes",
               workspace_bytes, w.bytes);
  EJ_HIP(hipMemsetAsync(w.scalars, 0, 4 * sizeof(int64_t), stream));
  int *bad = reinterpret_cast<int *>(w.scalars + 1);
  hipLaunchKernelGGL(pair_keys_kernel, dim3(grid_for(n_pairs)), dim3(kBlock), 0, stream,
                     lhs_coords, rhs_coords, lhs_idx, rhs_idx, n_pairs, a, w.keys, bad);
  EJ_LAUNCH_CHECK();
  EJ_TRY(fill_iota_i32(w.perm, n_pairs, stream));
  EJ_TRY(sort_pairs_u64(w.keys, w.perm, w.keys_alt, w.perm_alt, n_pairs, bits, w.sort_ws, stream));
  hipLaunchKernelGGL(seg_flags_kernel, dim3(grid_for(n_pairs)), dim3(kBlock), 0, stream, w.keys,
                     n_pairs, w.flags);
  EJ_LAUNCH_CHECK();
  EJ_TRY(scan_exclusive_i64(w.flags, w.excl, n_pairs, w.scalars, w.scan_ws, stream));
  int64_t host[2] = {0, 0};
  EJ_HIP(hipMemcpyAsync(host, w.scalars, 2 * sizeof(int64_t), hipMemcpyDeviceToHost, stream));
  EJ_HIP(hipStreamSynchronize(stream));
  if (host[1] != 0) {
    set_error("a pair index or an output coordinate lies outside [0, radix)");
    return EJ_E_RANGE;
  }
  *n_segments = host[0];
  return EJ_OK;
}

extern "C" int ej_segment_fill(int64_t n_pairs, int64_t n_segments, int32_t n_out,
                               const int64_t *radices, const void *workspace,
                               size_t workspace_bytes, int32_t *out_coords, int32_t *seg_offsets,
                               int32_t *perm, int32_t *seg_ids, int64_t capacity,
                               ej_stream_t stream_) {
  clear_error();
  hipStream_t stream = as_stream(stream_);
  EJ_CHECK_ARG(n_pairs >= 0 && n_segments >= 0 && n_segments <= n_pairs, "bad sizes");
  if (capacity < n_segments) {
    set_error("segment capacity %lld < %lld segments", (long long)capacity,
              (long long)n_segments);
    return EJ_E_CAPACITY;
  }
  if (n_pairs == 0) {
    if (seg_offsets) EJ_HIP(hipMemsetAsync(seg_offsets, 0, sizeof(int32_t), stream));
    return EJ_OK;
  }
  EJ_CHECK_ARG(seg_offsets && perm && (out_coords || n_out == 0), "null output pointer");
  AggSpec a;
  a.n = n_out;
  EJ_CHECK_ARG(n_out >= 0 && n_out <= EJ_MAX_KEYS, "bad n_out");
  for (int d = 0; d < n_out; ++d) a.radix[d] = radices[d];
  SegWs w = carve_seg(const_cast<void *>(workspace), n_pairs);
  EJ_CHECK_ARG(workspace && workspace_bytes >= w.bytes, "workspace too small");
  hipLaunchKernelGGL(seg_fill_kernel, dim3(grid_for(n_pairs)), dim3(kBlock), 0, stream, w.keys,
                     w.perm, w.flags, w.excl, n_pairs, n_segments, a, out_coords, seg_offsets,
                     perm, seg_ids);
  EJ_LAUNCH_CHECK();
  return EJ_OK;
}

// ---------------------------------------------------------------------------
// Column ranges of a coordinate array (used to size key radices when a
// caller passes bare coordinates without grid metadata).

namespace ej {
namespace {

__global__ void range_init_kernel(int32_t *lo_hi, int32_t ncols) {
  int c = threadIdx.x;
  if (c < ncols) {
    lo_hi[2 * c] = INT32_MAX;
    lo_hi[2 * c + 1] = INT32_MIN;
  }
}

__global__ __launch_bounds__(256) void range_kernel(const int32_t *coords, int64_t n,
                                                    int32_t ncols, int32_t *lo_hi) {
  __shared__ int32_t slo[EJ_MAX_DIMS], shi[EJ_MAX_DIMS];
  if (threadIdx.x < ncols) {
    slo[threadIdx.x] = INT32_MAX;
    shi[threadIdx.x] = INT32_MIN;
  }
  __syncthreads();
  const int64_t total = n * ncols;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    const int c = static_cast<int>(i % ncols);
    atomicMin(&slo[c], coords[i]);
    atomicMax(&shi[c], coords[i]);
  }
  __syncthreads();
  if (threadIdx.x < ncols) {
    atomicMin(&lo_hi[2 * threadIdx.x], slo[threadIdx.x]);
    atomicMax(&lo_hi[2 * threadIdx.x + 1], shi[threadIdx.x]);
  }
}

}  // namespace
}  // namespace ej

extern "C" int ej_coords_range(const int32_t *coords, int64_t n, int32_t ncols, int32_t *lo_hi,
                               void *workspace, size_t workspace_bytes, ej_stream_t stream_) {
  clear_error();
  hipStream_t stream = as_stream(stream_);
  EJ_CHECK_ARG(lo_hi, "lo_hi is null");
  EJ_CHECK_ARG(ncols >= 0 && ncols <= EJ_MAX_DIMS, "ncols outside [0, %d]", EJ_MAX_DIMS);
  EJ_CHECK_ARG(n >= 0, "negative n");
  if (n == 0 || ncols == 0) {
    for (int c = 0; c < ncols; ++c) {
      lo_hi[2 * c] = 0;
      lo_hi[2 * c + 1] = -1;
    }
    return EJ_OK;
  }
  EJ_CHECK_ARG(coords, "coords is null");
  EJ_CHECK_ARG(workspace && workspace_bytes >= sizeof(int32_t) * 2 * ncols,
               "workspace too small");
  int32_t *dev = static_cast<int32_t *>(workspace);
  hipLaunchKernelGGL(range_init_kernel, dim3(1), dim3(64), 0, stream, dev, ncols);
  EJ_LAUNCH_CHECK();
  const int64_t total = n * ncols;
  const unsigned blocks = static_cast<unsigned>(ceil_div(total, 256) < 1024 ? ceil_div(total, 256) : 1024);
  hipLaunchKernelGGL(range_kernel, dim3(blocks), dim3(256), 0, stream, coords, n, ncols, dev);
  EJ_LAUNCH_CHECK();
  EJ_HIP(hipMemcpyAsync(lo_hi, dev, sizeof(int32_t) * 2 * ncols, hipMemcpyDeviceToHost, stream));
  EJ_HIP(hipStreamSynchronize(stream));
  return EJ_OK;
}
