// Device-wide scan and stable LSD radix sort built from wave64 ballot and
// prefix primitives, plus the library's error state and version entry points.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "ej_internal.h"

namespace ej {

static thread_local std::string g_error;

void set_error(const char *fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
}

void clear_error() { g_error.clear(); }

bool fault_injected(const char *site) {
  const char *env = getenv("EJ_INJECT_FAULT");
  if (!env || !*env) return false;
  const size_t n = strlen(site);
  for (const char *p = env; *p;) {
    const char *end = strchr(p, ',');
    const size_t len = end ? static_cast<size_t>(end - p) : strlen(p);
    if (len == n && strncmp(p, site, n) == 0) return true;
    if (!end) break;
    p = end + 1;
  }
  return false;
}

__global__ void zero_words_kernel(uint32_t *p, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    p[i] = 0u;
}

int zero_async(void *p, size_t bytes, hipStream_t stream) {
  const int64_t n = static_cast<int64_t>(bytes / 4);
  if (n <= 0) return EJ_OK;
  const int64_t g = ceil_div(n, kBlock);
  hipLaunchKernelGGL(zero_words_kernel, dim3(static_cast<unsigned>(g < 1024 ? g : 1024)),
                     dim3(kBlock), 0, stream, static_cast<uint32_t *>(p), n);
  EJ_LAUNCH_CHECK();
  return EJ_OK;
}

int key_bits(const int64_t *radix, int n, int *bits) {
  // prod(radix) must stay below 2^63 so that packed keys are exact.
  unsigned __int128 prod = 1;
  for (int i = 0; i < n; ++i) {
    if (radix[i] <= 0) {
      set_error("key radix %d is %lld; radices must be positive", i, (long long)radix[i]);
      return EJ_E_INVAL;
    }
    prod *= static_cast<unsigned __int128>(radix[i]);
    if (prod > (static_cast<unsigned __int128>(1) << 63)) {
      set_error("packed key space exceeds 2^63 (product of radices too large)");
      return EJ_E_UNSUPPORTED;
    }
  }
  int b = 0;
  while ((static_cast<unsigned __int128>(1) << b) < prod) ++b;
  *bits = b;
  return EJ_OK;
}

// ---------------------------------------------------------------------------
// Scan.  Up to kFastScanMax values: the two-launch reduce-then-scan.  Longer:
// each block scans kScanTile consecutive values (8 per thread), writes the
// block total, the totals are scanned recursively and added back.
__global__ __launch_bounds__(kBlock) void scan_tiles_kernel(const int64_t *in, int64_t *out,
                                                            int64_t *tile_sums, int64_t n,
                                                            const int64_t *n_dev) {
  n = live_count(n, n_dev);
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile +
                       static_cast<int64_t>(threadIdx.x) * kScanItems;
  int64_t v[kScanItems];
  int64_t s = 0;
#pragma unroll
  for (int i = 0; i < kScanItems; ++i) {
    int64_t idx = base + i;
    v[i] = idx < n ? in[idx] : 0;
    s += v[i];
  }
  int64_t tot;
  int64_t run = block_exclusive_sum<kBlock>(s, &tot);
#pragma unroll
  for (int i = 0; i < kScanItems; ++i) {
    int64_t idx = base + i;
    if (idx < n) out[idx] = run;
    run += v[i];
  }
  if (threadIdx.x == 0) tile_sums[blockIdx.x] = tot;
}

__global__ __launch_bounds__(kBlock) void scan_add_kernel(int64_t *out, const int64_t *tile_offs,
                                                          int64_t n, const int64_t *n_dev) {
  n = live_count(n, n_dev);
  const int64_t off = tile_offs[blockIdx.x];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile;
  for (int i = threadIdx.x; i < kScanTile; i += kBlock) {
    int64_t idx = base + i;
    if (idx < n) out[idx] += off;
  }
}

__global__ void scan_total_kernel(const int64_t *in, const int64_t *out, int64_t n,
                                  const int64_t *n_dev, int64_t *total) {
  n = live_count(n, n_dev);
  *total = n > 0 ? out[n - 1] + in[n - 1] : 0;
}

size_t scan_workspace_bytes(int64_t n) {
  size_t bytes = 0;
  while (n > 1) {
    int64_t tiles = ceil_div(n, kScanTile);
    bytes += align_up(sizeof(int64_t) * tiles * 2, 256);
    if (tiles == 1) break;
    n = tiles;
  }
  return bytes + 256;
}

int scan_exclusive_i64(const int64_t *in, int64_t *out, int64_t n, int64_t *total, void *ws,
                       hipStream_t stream, const int64_t *n_dev) {
  if (n <= 0) {
    if (total) EJ_TRY(zero_async(total, sizeof(int64_t), stream));
    return EJ_OK;
  }
  if (n <= kFastScanMax) {
    launch_fast_scan(LoadI64{in}, NoEmit{}, n, n_dev, static_cast<int64_t *>(ws), out, total,
                     stream);
    EJ_LAUNCH_CHECK();
    return EJ_OK;
  }
  const int64_t tiles = ceil_div(n, kScanTile);
  char *w = static_cast<char *>(ws);
  int64_t *sums = reinterpret_cast<int64_t *>(w);
  int64_t *sums_scanned = sums + tiles;
  char *rest = w + align_up(sizeof(int64_t) * tiles * 2, 256);
  hipLaunchKernelGGL(scan_tiles_kernel, dim3(static_cast<unsigned>(tiles)), dim3(kBlock), 0,
                     stream, in, out, sums, n, n_dev);
  EJ_LAUNCH_CHECK();
  if (tiles > 1) {
    EJ_TRY(scan_exclusive_i64(sums, sums_scanned, tiles, nullptr, rest, stream));
    hipLaunchKernelGGL(scan_add_kernel, dim3(static_cast<unsigned>(tiles)), dim3(kBlock), 0,
                       stream, out, sums_scanned, n, n_dev);
    EJ_LAUNCH_CHECK();
  }
  if (total) {
    hipLaunchKernelGGL(scan_total_kernel, dim3(1), dim3(1), 0, stream, in, out, n, n_dev,
                       total);
    EJ_LAUNCH_CHECK();
  }
  return EJ_OK;
}

// ---------------------------------------------------------------------------
// Radix sort: 8-bit digits; each block takes a tile of kBlock * ITEMS keys,
// ITEMS in {1, 2, 4, 8} chosen per sort so that short sequences spread over
// many blocks (fewer serial rounds per block).
//   pass 1: per-block digit histogram;
//   pass 2: stable scatter.  Each block first derives its starting offset
//           per digit.  Up to kInlineOffsetBlocks blocks: the histogram is
//           stored block-major (hist[block][digit]) and every block reads it
//           directly (digit totals scanned across the 256 digits plus the
//           counts of earlier blocks).  More blocks: it is stored digit-major
//           (hist[digit][block]) and one device-wide exclusive scan of it
//           supplies the offsets.
//           Ranks inside a round of 256 keys come from wave64 ballots (peer
//           mask of equal digits + popcount of lower lanes) and a per-digit
//           prefix over the four waves in LDS.
constexpr int kRadixBits = 8;
constexpr int kRadix = 1 << kRadixBits;
constexpr int kMaxSortItems = 8;
#ifndef EJ_INLINE_OFFSET_BLOCKS
#define EJ_INLINE_OFFSET_BLOCKS 32
#endif
constexpr int64_t kInlineOffsetBlocks = EJ_INLINE_OFFSET_BLOCKS;
static_assert(kRadix == kBlock, "one thread per digit in the scatter bookkeeping");

template <int ITEMS>
__global__ __launch_bounds__(kBlock) void radix_hist_kernel(const uint64_t *keys, int64_t n,
                                                            const int64_t *n_dev, int shift,
                                                            int64_t *hist, int64_t nblocks,
                                                            bool digit_major) {
  n = live_count(n, n_dev);
  __shared__ int counts[kRadix];
  counts[threadIdx.x] = 0;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kBlock * ITEMS;
  uint64_t k[ITEMS];
#pragma unroll
  for (int r = 0; r < ITEMS; ++r) {
    int64_t i = base + r * kBlock + threadIdx.x;
    k[r] = i < n ? keys[i] : 0;
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < ITEMS; ++r) {
    int64_t i = base + r * kBlock + threadIdx.x;
    if (i < n) atomicAdd(&counts[(k[r] >> shift) & (kRadix - 1)], 1);
  }
  __syncthreads();
  const int64_t at = digit_major ? static_cast<int64_t>(threadIdx.x) * nblocks + blockIdx.x
                                 : static_cast<int64_t>(blockIdx.x) * kRadix + threadIdx.x;
  hist[at] = counts[threadIdx.x];
}

// offs == nullptr: offsets are derived from the block-major hist.
template <int ITEMS>
__global__ __launch_bounds__(kBlock) void radix_scatter_kernel(
    const uint64_t *__restrict__ kin, const int32_t *__restrict__ vin, uint64_t *__restrict__ kout,
    int32_t *__restrict__ vout, int64_t n, const int64_t *n_dev, int shift,
    const int64_t *__restrict__ hist, const int64_t *__restrict__ offs, int64_t nblocks) {
  n = live_count(n, n_dev);
  __shared__ int64_t base_off[kRadix];
  __shared__ int wcount[kBlock / 64][kRadix];
  __shared__ int wprefix[kBlock / 64][kRadix];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  const int64_t tile0 = static_cast<int64_t>(blockIdx.x) * kBlock * ITEMS;
  uint64_t kk[ITEMS];
  int32_t vv[ITEMS];
#pragma unroll
  for (int r = 0; r < ITEMS; ++r) {
    const int64_t i = tile0 + r * kBlock + tid;
    kk[r] = i < n ? kin[i] : 0;
    vv[r] = i < n ? vin[i] : 0;
  }
  if (offs) {
    base_off[tid] = offs[static_cast<int64_t>(tid) * nblocks + blockIdx.x];
  } else {
    int64_t before = 0, digit_total = 0;
#pragma unroll 8
    for (int64_t b = 0; b < nblocks; ++b) {
      const int64_t c = hist[b * kRadix + tid];
      digit_total += c;
      before += b < static_cast<int64_t>(blockIdx.x) ? c : 0;
    }
    int64_t all;
    base_off[tid] = block_exclusive_sum<kBlock>(digit_total, &all) + before;
  }
#pragma unroll
  for (int r = 0; r < ITEMS; ++r) {
#pragma unroll
    for (int w = 0; w < kBlock / 64; ++w) wcount[w][tid] = 0;
    __syncthreads();
    const int64_t i = tile0 + r * kBlock + tid;
    const bool valid = i < n;
    const uint64_t k = kk[r];
    const int d = static_cast<int>((k >> shift) & (kRadix - 1));
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int b = 0; b < kRadixBits; ++b) {
      int bit = (d >> b) & 1;
      uint64_t m = __ballot(bit);
      peers &= bit ? m : ~m;
    }
    const int rank = __popcll(peers & lt_mask);
    if (valid && rank == 0) wcount[wave][d] = __popcll(peers);
    __syncthreads();
    int run = 0;
#pragma unroll
    for (int w = 0; w < kBlock / 64; ++w) {
      wprefix[w][tid] = run;
      run += wcount[w][tid];
    }
    __syncthreads();
    if (valid) {
      int64_t pos = base_off[d] + wprefix[wave][d] + rank;
      kout[pos] = k;
      vout[pos] = vv[r];
    }
    __syncthreads();
    base_off[tid] += run;
  }
}

__global__ void copy_pairs_kernel(const uint64_t *ks, const int32_t *vs, uint64_t *kd,
                                  int32_t *vd, int64_t n, const int64_t *n_dev) {
  n = live_count(n, n_dev);
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) {
    kd[i] = ks[i];
    vd[i] = vs[i];
  }
}

// Keys per thread for a sort of n keys: the fewest rounds per block that keep
// the grid within kInlineOffsetBlocks blocks, else the largest tile.
int sort_items(int64_t n) {
  for (int items = 1; items < kMaxSortItems; items *= 2)
    if (ceil_div(n, static_cast<int64_t>(kBlock) * items) <= kInlineOffsetBlocks) return items;
  return kMaxSortItems;
}

// Covers every sort of up to n keys: below 8 * kBlock * kInlineOffsetBlocks
// keys a sort uses at most kInlineOffsetBlocks blocks, above it the block
// count grows with n.
size_t sort_workspace_bytes(int64_t n) {
  int64_t nblocks = ceil_div(n > 0 ? n : 1, static_cast<int64_t>(kBlock) * sort_items(n));
  if (nblocks < kInlineOffsetBlocks) nblocks = kInlineOffsetBlocks;
  int64_t h = nblocks * kRadix;
  return align_up(sizeof(int64_t) * h * 2, 256) + scan_workspace_bytes(h);
}

int radix_passes(int bits) { return bits <= 0 ? 0 : (bits + kRadixBits - 1) / kRadixBits; }

SortTiling sort_tiling(int64_t n) {
  SortTiling t;
  t.tile = static_cast<int64_t>(kBlock) * sort_items(n);
  t.nblocks = ceil_div(n, t.tile);
  t.inline_offsets = t.nblocks <= kInlineOffsetBlocks;
  return t;
}

template <int ITEMS>
int sort_passes(uint64_t *&ks, int32_t *&vs, uint64_t *&kd, int32_t *&vd, int64_t n, int bits,
                void *ws, hipStream_t stream, const int64_t *n_dev, bool first_hist_given) {
  const int64_t nblocks = ceil_div(n, static_cast<int64_t>(kBlock) * ITEMS);
  const int64_t h = nblocks * kRadix;
  char *w = static_cast<char *>(ws);
  int64_t *hist = reinterpret_cast<int64_t *>(w);
  int64_t *offs = hist + h;
  void *scan_ws = w + align_up(sizeof(int64_t) * h * 2, 256);
  const bool inline_offs = nblocks <= kInlineOffsetBlocks;
  for (int shift = 0; shift < bits; shift += kRadixBits) {
    if (shift > 0 || !first_hist_given || !inline_offs) {
      hipLaunchKernelGGL(radix_hist_kernel<ITEMS>, dim3(static_cast<unsigned>(nblocks)),
                         dim3(kBlock), 0, stream, ks, n, n_dev, shift, hist, nblocks,
                         !inline_offs);
      EJ_LAUNCH_CHECK();
    }
    if (!inline_offs) EJ_TRY(scan_exclusive_i64(hist, offs, h, nullptr, scan_ws, stream));
    hipLaunchKernelGGL(radix_scatter_kernel<ITEMS>, dim3(static_cast<unsigned>(nblocks)),
                       dim3(kBlock), 0, stream, ks, vs, kd, vd, n, n_dev, shift, hist,
                       inline_offs ? nullptr : offs, nblocks);
    EJ_LAUNCH_CHECK();
    uint64_t *tk = ks; ks = kd; kd = tk;
    int32_t *tv = vs; vs = vd; vd = tv;
  }
  return EJ_OK;
}

int sort_pairs_u64(uint64_t *keys, int32_t *vals, uint64_t *keys_alt, int32_t *vals_alt,
                   int64_t n, int bits, void *ws, hipStream_t stream, bool input_in_alt,
                   const int64_t *n_dev, bool first_hist_given) {
  uint64_t *ks = input_in_alt ? keys_alt : keys, *kd = input_in_alt ? keys : keys_alt;
  int32_t *vs = input_in_alt ? vals_alt : vals, *vd = input_in_alt ? vals : vals_alt;
  if (n > 1 && bits > 0) {
    switch (sort_items(n)) {
      case 1:
        EJ_TRY(sort_passes<1>(ks, vs, kd, vd, n, bits, ws, stream, n_dev, first_hist_given));
        break;
      case 2:
        EJ_TRY(sort_passes<2>(ks, vs, kd, vd, n, bits, ws, stream, n_dev, first_hist_given));
        break;
      case 4:
        EJ_TRY(sort_passes<4>(ks, vs, kd, vd, n, bits, ws, stream, n_dev, first_hist_given));
        break;
      default:
        EJ_TRY(sort_passes<8>(ks, vs, kd, vd, n, bits, ws, stream, n_dev, first_hist_given));
        break;
    }
  }
  if (ks != keys && n > 0) {
    hipLaunchKernelGGL(copy_pairs_kernel, dim3(grid_for(n)), dim3(kBlock), 0, stream, ks, vs,
                       keys, vals, n, n_dev);
    EJ_LAUNCH_CHECK();
  }
  return EJ_OK;
}

}  // namespace ej

extern "C" int ej_version(void) { return EJ_ABI_VERSION; }

extern "C" int ej_host_alloc(size_t bytes, void **host_ptr) {
  ej::clear_error();
  if (!host_ptr || bytes == 0) {
    ej::set_error("ej_host_alloc: null pointer or zero size");
    return EJ_E_INVAL;
  }
  *host_ptr = nullptr;
  const bool injected = ej::fault_injected("host_alloc");
  const hipError_t e = injected ? hipErrorOutOfMemory
                                : hipHostMalloc(host_ptr, bytes,
                                                hipHostMallocMapped | hipHostMallocCoherent);
  if (e != hipSuccess) {
    ej::set_error("hipHostMalloc failed: %s%s", hipGetErrorString(e),
                  injected ? " (injected by EJ_INJECT_FAULT)" : "");
    return EJ_E_HIP;
  }
  return EJ_OK;
}

extern "C" int ej_host_free(void *host_ptr) {
  ej::clear_error();
  if (!host_ptr) return EJ_OK;
  const hipError_t e = hipHostFree(host_ptr);
  if (e != hipSuccess) {
    ej::set_error("hipHostFree failed: %s", hipGetErrorString(e));
    return EJ_E_HIP;
  }
  return EJ_OK;
}

extern "C" const char *ej_last_error(void) { return ej::g_error.c_str(); }
