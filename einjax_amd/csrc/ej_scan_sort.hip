// Device-wide scan and stable LSD radix sort built from wave64 ballot and
// prefix primitives, plus the library's error state and version entry points.
#include <stdarg.h>
#include <stdio.h>

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
// Scan: each block scans kScanTile consecutive values (8 per thread), writes
// the block total, the totals are scanned recursively and added back.
constexpr int kScanItems = 8;
constexpr int kScanTile = kBlock * kScanItems;

// Inclusive prefix sum across the 64 lanes of a wave.
__device__ inline int64_t wave_inclusive_sum(int64_t v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    int64_t o = __shfl_up(v, d, 64);
    if (lane >= d) v += o;
  }
  return v;
}

// Exclusive prefix of v across the block; *block_total receives the sum.
__device__ inline int64_t block_exclusive_sum(int64_t v, int64_t *block_total) {
  __shared__ int64_t wave_tot[kBlock / 64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int64_t inc = wave_inclusive_sum(v);
  if (lane == 63) wave_tot[wave] = inc;
  __syncthreads();
  int64_t wave_off = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < kBlock / 64; ++w) {
    int64_t t = wave_tot[w];
    if (w < wave) wave_off += t;
    tot += t;
  }
  __syncthreads();
  *block_total = tot;
  return wave_off + inc - v;
}

__global__ __launch_bounds__(kBlock) void scan_tiles_kernel(const int64_t *in, int64_t *out,
                                                            int64_t *tile_sums, int64_t n) {
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
  int64_t run = block_exclusive_sum(s, &tot);
#pragma unroll
  for (int i = 0; i < kScanItems; ++i) {
    int64_t idx = base + i;
    if (idx < n) out[idx] = run;
    run += v[i];
  }
  if (threadIdx.x == 0) tile_sums[blockIdx.x] = tot;
}

__global__ __launch_bounds__(kBlock) void scan_add_kernel(int64_t *out, const int64_t *tile_offs,
                                                          int64_t n) {
  const int64_t off = tile_offs[blockIdx.x];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile;
  for (int i = threadIdx.x; i < kScanTile; i += kBlock) {
    int64_t idx = base + i;
    if (idx < n) out[idx] += off;
  }
}

__global__ void scan_total_kernel(const int64_t *in, const int64_t *out, int64_t n,
                                  int64_t *total) {
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
                       hipStream_t stream) {
  if (n <= 0) {
    if (total) EJ_HIP(hipMemsetAsync(total, 0, sizeof(int64_t), stream));
    return EJ_OK;
  }
  const int64_t tiles = ceil_div(n, kScanTile);
  char *w = static_cast<char *>(ws);
  int64_t *sums = reinterpret_cast<int64_t *>(w);
  int64_t *sums_scanned = sums + tiles;
  char *rest = w + align_up(sizeof(int64_t) * tiles * 2, 256);
  hipLaunchKernelGGL(scan_tiles_kernel, dim3(static_cast<unsigned>(tiles)), dim3(kBlock), 0,
                     stream, in, out, sums, n);
  EJ_LAUNCH_CHECK();
  if (tiles > 1) {
    EJ_TRY(scan_exclusive_i64(sums, sums_scanned, tiles, nullptr, rest, stream));
    hipLaunchKernelGGL(scan_add_kernel, dim3(static_cast<unsigned>(tiles)), dim3(kBlock), 0,
                       stream, out, sums_scanned, n);
    EJ_LAUNCH_CHECK();
  }
  if (total) {
    hipLaunchKernelGGL(scan_total_kernel, dim3(1), dim3(1), 0, stream, in, out, n, total);
    EJ_LAUNCH_CHECK();
  }
  return EJ_OK;
}

// ---------------------------------------------------------------------------
// Radix sort: 8-bit digits, tiles of kSortTile keys per block.
//   pass 1: per-block digit histogram, stored digit-major so that one
//           exclusive scan yields every block's starting offset per digit;
//   pass 2: scan;
//   pass 3: stable scatter.  Ranks inside a round of 256 keys come from
//           wave64 ballots (peer mask of equal digits + popcount of lower
//           lanes) and a per-digit prefix over the four waves in LDS.
constexpr int kRadixBits = 8;
constexpr int kRadix = 1 << kRadixBits;
constexpr int kSortItems = 8;
constexpr int kSortTile = kBlock * kSortItems;
static_assert(kRadix == kBlock, "one thread per digit in the scatter bookkeeping");

__global__ __launch_bounds__(kBlock) void radix_hist_kernel(const uint64_t *keys, int64_t n,
                                                            int shift, int64_t *hist,
                                                            int64_t nblocks) {
  __shared__ int counts[kRadix];
  counts[threadIdx.x] = 0;
  __syncthreads();
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kSortTile;
#pragma unroll
  for (int r = 0; r < kSortItems; ++r) {
    int64_t i = base + r * kBlock + threadIdx.x;
    if (i < n) atomicAdd(&counts[(keys[i] >> shift) & (kRadix - 1)], 1);
  }
  __syncthreads();
  hist[static_cast<int64_t>(threadIdx.x) * nblocks + blockIdx.x] = counts[threadIdx.x];
}

__global__ __launch_bounds__(kBlock) void radix_scatter_kernel(
    const uint64_t *kin, const int32_t *vin, uint64_t *kout, int32_t *vout, int64_t n, int shift,
    const int64_t *offs, int64_t nblocks) {
  __shared__ int64_t base_off[kRadix];
  __shared__ int wcount[kBlock / 64][kRadix];
  __shared__ int wprefix[kBlock / 64][kRadix];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  base_off[tid] = offs[static_cast<int64_t>(tid) * nblocks + blockIdx.x];
  const int64_t tile0 = static_cast<int64_t>(blockIdx.x) * kSortTile;
  for (int r = 0; r < kSortItems; ++r) {
#pragma unroll
    for (int w = 0; w < kBlock / 64; ++w) wcount[w][tid] = 0;
    __syncthreads();
    const int64_t i = tile0 + r * kBlock + tid;
    const bool valid = i < n;
    uint64_t k = valid ? kin[i] : 0;
    int32_t v = valid ? vin[i] : 0;
    int d = static_cast<int>((k >> shift) & (kRadix - 1));
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
      vout[pos] = v;
    }
    __syncthreads();
    base_off[tid] += run;
  }
}

__global__ void iota_kernel(int32_t *v, int64_t n) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) v[i] = static_cast<int32_t>(i);
}

__global__ void copy_pairs_kernel(const uint64_t *ks, const int32_t *vs, uint64_t *kd,
                                  int32_t *vd, int64_t n) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) {
    kd[i] = ks[i];
    vd[i] = vs[i];
  }
}

int fill_iota_i32(int32_t *v, int64_t n, hipStream_t stream) {
  if (n <= 0) return EJ_OK;
  hipLaunchKernelGGL(iota_kernel, dim3(grid_for(n)), dim3(kBlock), 0, stream, v, n);
  EJ_LAUNCH_CHECK();
  return EJ_OK;
}

size_t sort_workspace_bytes(int64_t n) {
  int64_t nblocks = ceil_div(n > 0 ? n : 1, kSortTile);
  int64_t h = nblocks * kRadix;
  return align_up(sizeof(int64_t) * h * 2, 256) + scan_workspace_bytes(h);
}

int sort_pairs_u64(uint64_t *keys, int32_t *vals, uint64_t *keys_alt, int32_t *vals_alt,
                   int64_t n, int bits, void *ws, hipStream_t stream) {
  if (n <= 1 || bits <= 0) return EJ_OK;
  const int64_t nblocks = ceil_div(n, kSortTile);
  const int64_t h = nblocks * kRadix;
  char *w = static_cast<char *>(ws);
  int64_t *hist = reinterpret_cast<int64_t *>(w);
  int64_t *offs = hist + h;
  void *scan_ws = w + align_up(sizeof(int64_t) * h * 2, 256);
  uint64_t *ks = keys, *kd = keys_alt;
  int32_t *vs = vals, *vd = vals_alt;
  for (int shift = 0; shift < bits; shift += kRadixBits) {
    hipLaunchKernelGGL(radix_hist_kernel, dim3(static_cast<unsigned>(nblocks)), dim3(kBlock), 0,
                       stream, ks, n, shift, hist, nblocks);
    EJ_LAUNCH_CHECK();
    EJ_TRY(scan_exclusive_i64(hist, offs, h, nullptr, scan_ws, stream));
    hipLaunchKernelGGL(radix_scatter_kernel, dim3(static_cast<unsigned>(nblocks)), dim3(kBlock),
                       0, stream, ks, vs, kd, vd, n, shift, offs, nblocks);
    EJ_LAUNCH_CHECK();
    uint64_t *tk = ks; ks = kd; kd = tk;
    int32_t *tv = vs; vs = vd; vd = tv;
  }
  if (ks != keys) {
    hipLaunchKernelGGL(copy_pairs_kernel, dim3(grid_for(n)), dim3(kBlock), 0, stream, ks, vs,
                       keys, vals, n);
    EJ_LAUNCH_CHECK();
  }
  return EJ_OK;
}

}  // namespace ej

extern "C" int ej_version(void) { return EJ_ABI_VERSION; }

extern "C" const char *ej_last_error(void) { return ej::g_error.c_str(); }
