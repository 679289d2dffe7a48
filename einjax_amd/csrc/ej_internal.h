// Internal helpers shared by the HIP translation units of libejhip.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include <string>

#include "../../include/einjax_hip.h"

namespace ej {

// ---- error reporting ------------------------------------------------------
void set_error(const char *fmt, ...);
void clear_error();

#define EJ_CHECK_ARG(cond, ...)                                                \
  do {                                                                         \
    if (!(cond)) {                                                             \
      ::ej::set_error(__VA_ARGS__);                                            \
      return EJ_E_INVAL;                                                       \
    }                                                                          \
  } while (0)

#define EJ_HIP(expr)                                                           \
  do {                                                                         \
    hipError_t e_ = (expr);                                                    \
    if (e_ != hipSuccess) {                                                    \
      ::ej::set_error("%s failed: %s (%s:%d)", #expr, hipGetErrorString(e_),   \
                      __FILE__, __LINE__);                                     \
      return EJ_E_HIP;                                                         \
    }                                                                          \
  } while (0)

// ---- fault injection -----------------------------------------------------
// EJ_INJECT_FAULT (environment, read at every check): a comma-separated list
// of sites that then fail as if the HIP runtime had returned an error there:
//   host_alloc  hipHostMalloc in ej_host_alloc (hipErrorOutOfMemory)
//   launch      every kernel launch check (hipErrorLaunchFailure; the
//               kernel itself was enqueued)
// It lets tests drive the EJ_E_HIP paths, status and message, without a
// failing device.  Unset, every check is a plain hipGetLastError.
bool fault_injected(const char *site);

#define EJ_LAUNCH_CHECK()                                                      \
  do {                                                                         \
    const bool inj_ = ::ej::fault_injected("launch");                          \
    hipError_t e_ = inj_ ? hipErrorLaunchFailure : hipGetLastError();          \
    if (e_ != hipSuccess) {                                                    \
      ::ej::set_error("kernel launch failed: %s%s (%s:%d)",                    \
                      hipGetErrorString(e_),                                   \
                      inj_ ? " (injected by EJ_INJECT_FAULT)" : "", __FILE__,  \
                      __LINE__);                                               \
      return EJ_E_HIP;                                                         \
    }                                                                          \
  } while (0)

#define EJ_TRY(expr)                                                           \
  do {                                                                         \
    int s_ = (expr);                                                           \
    if (s_ != EJ_OK) return s_;                                                \
  } while (0)

inline hipStream_t as_stream(ej_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// Carves aligned sub-buffers out of a caller-supplied workspace.  With a
// null base it only measures.
struct Carver {
  char *base;
  size_t off = 0;
  explicit Carver(void *b) : base(static_cast<char *>(b)) {}
  template <typename T> T *take(int64_t n) {
    off = align_up(off, 256);
    T *p = base ? reinterpret_cast<T *>(base + off) : nullptr;
    off += sizeof(T) * static_cast<size_t>(n > 0 ? n : 1);
    return p;
  }
};

// ---- small by-value kernel argument blocks ---------------------------------
struct KeySpec {            // mixed-radix packing of selected coordinate columns
  int32_t n;                // number of key columns
  int32_t ncols;            // columns per coordinate row
  int32_t dims[EJ_MAX_KEYS];
  int64_t radix[EJ_MAX_KEYS];
};

// Radix bits needed for keys in [0, prod(radix)); 0 keys -> 0 bits.
int key_bits(const int64_t *radix, int n, int *bits);

// ---- device-wide primitives (ej_scan_sort.hip) ----------------------------
// Exclusive scan of n int64 values; total (device scalar) may be null.
// n_dev (optional): device-side count clipping n.
size_t scan_workspace_bytes(int64_t n);
int scan_exclusive_i64(const int64_t *in, int64_t *out, int64_t n, int64_t *total,
                       void *ws, hipStream_t stream, const int64_t *n_dev = nullptr);

// Stable LSD radix sort of (key, value) pairs on the low `bits` key bits.
// The input lies in keys/vals, or in keys_alt/vals_alt when input_in_alt;
// the result always ends in keys/vals.  A caller that packs its input into
// the alt buffers when radix_passes(bits) is odd saves the final copy.
size_t sort_workspace_bytes(int64_t n);
int radix_passes(int bits);
// n_dev (optional): device-side count clipping n (keys beyond it stay put).
// first_hist_given: the digit histogram of the first pass (bits 0-7) is
// already in the workspace (see sort_tiling), so that pass skips its
// histogram launch.
int sort_pairs_u64(uint64_t *keys, int32_t *vals, uint64_t *keys_alt, int32_t *vals_alt,
                   int64_t n, int bits, void *ws, hipStream_t stream,
                   bool input_in_alt = false, const int64_t *n_dev = nullptr,
                   bool first_hist_given = false);
// Tiling of a sort of n keys: tile = keys per block, nblocks blocks; when
// inline_offsets, the first int64s of the workspace hold the digit histogram
// block-major (hist[block * 256 + digit]), which a producer of the keys may
// fill itself (zeroed first, then counts of keys [block * tile, ...) that lie
// below the live count) and pass first_hist_given.
struct SortTiling {
  int64_t tile, nblocks;
  bool inline_offsets;
};
SortTiling sort_tiling(int64_t n);

// The fused segment einsum (ej_einsum.hip) with a run order: segments per
// group of the launch that follows an order for this descriptor and segment
// count (0: the launch follows none), and the einsum itself given the order
// (run_order[0] = live groups, run_order[1 + b] = the group block b runs).
int segment_einsum_order_group(const ej_einsum_desc *d, int32_t dtype, int64_t n_seg,
                               const void *A, const void *B);
int segment_einsum_ordered(const ej_einsum_desc *d, int32_t dtype, const void *A, const void *B,
                           int64_t n_a_tiles, int64_t n_b_tiles, const int64_t *lidx,
                           const int64_t *ridx, const int32_t *perm, const int32_t *seg_off,
                           int64_t n_seg, const int32_t *run_order, int32_t order_group,
                           void *out, hipStream_t stream);

// The fused segment einsum for an fp32 lhs (k-contiguous [m][k] tiles) with
// an exactly-bf16 rhs (k-contiguous [n][k] tiles), 128 x 128 output blocks:
// the lhs is split into three bf16 terms per value and every product runs
// as three bf16 MFMAs with fp32 sums (ej_einsum.hip).  EJ_E_UNSUPPORTED
// (nothing launched) for other layouts; the caller then widens the rhs.
bool segment_einsum_split_ok(const ej_einsum_desc *d, const void *A, const void *B);
int segment_einsum_split(const ej_einsum_desc *d, const float *A, const uint16_t *B,
                         int64_t n_a_tiles, int64_t n_b_tiles, const int64_t *lidx,
                         const int64_t *ridx, const int32_t *perm, const int32_t *seg_off,
                         int64_t n_seg, const int32_t *run_order, int32_t order_group, void *out,
                         hipStream_t stream);

// The same for an exactly-bf16 lhs with free-dimension-contiguous [k][m]
// tiles against an fp32 rhs [k][n] (the rhs is split), one segment per
// workgroup.
bool segment_einsum_split_b_ok(const ej_einsum_desc *d, const void *A, const void *B);
int segment_einsum_split_b(const ej_einsum_desc *d, const uint16_t *A, const float *B,
                           int64_t n_a_tiles, int64_t n_b_tiles, const int64_t *lidx,
                           const int64_t *ridx, const int32_t *perm, const int32_t *seg_off,
                           int64_t n_seg, void *out, hipStream_t stream);

// Structure shared by the closed-form plans (ej_dense_plan.hip): the join
// covers rhs dims 0 .. n_keys-1 once each, their lhs dims (ldim[i] for rhs
// dim i) increasing; the output is lhs dims 0 .. nlo-1 followed by the rhs
// dims after the join dims; every lhs dim from nlo on is joined.  Otherwise
// EJ_E_UNSUPPORTED with a message naming `who`.
int run_plan_structure(const char *who, int n_keys, const int32_t *lhs_dims,
                       const int32_t *rhs_dims, int lhs_ncols, int rhs_ncols, int n_out,
                       const int32_t *agg_src, const int32_t *agg_dim, int32_t *ldim, int *nlo);

// Zeroes n bytes (a multiple of 4, 4-byte aligned) with a kernel rather than
// hipMemsetAsync, which misbehaves when a caller records the call into a
// HIP graph.
int zero_async(void *p, size_t bytes, hipStream_t stream);

// ---- device helpers --------------------------------------------------------
__device__ inline uint64_t pack_key(const int32_t *row, const KeySpec &ks, int *bad) {
  uint64_t key = 0;
  for (int i = 0; i < ks.n; ++i) {
    int64_t c = row[ks.dims[i]];
    if (c < 0 || c >= ks.radix[i]) {
      *bad = 1;
      c = 0;
    }
    key = key * static_cast<uint64_t>(ks.radix[i]) + static_cast<uint64_t>(c);
  }
  return key;
}

constexpr int kBlock = 256;   // threads per block for the integer kernels

// Live length of a sequence with host-side bound cap whose device-side count,
// if dev is non-null, is *dev: min(cap, max(*dev, 0)).  Kernels launched on a
// bound before the exact count reaches the host clip their work with it.
__device__ inline int64_t live_count(int64_t cap, const int64_t *dev) {
  if (!dev) return cap;
  const int64_t v = *dev;
  return v < 0 ? 0 : (v < cap ? v : cap);
}

// ---- block-level scans ------------------------------------------------------
// A workgroup barrier that orders LDS only: each wave's LDS operations are
// complete, its global stores stay in flight (__syncthreads would wait for
// them as well, a round trip to memory after every phase that writes).
__device__ inline void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// One DPP move of a 64-bit value (its two halves, DPP control CTRL, rows
// ROWS); lanes the move does not reach take 0.
template <int CTRL, int ROWS>
__device__ inline int64_t dpp_move64(int64_t v) {
  const int lo = __builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, ROWS, 0xf, false);
  const int hi = __builtin_amdgcn_update_dpp(0, static_cast<int>(v >> 32), CTRL, ROWS, 0xf, false);
  return static_cast<int64_t>((static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) |
                              static_cast<uint32_t>(lo));
}

// Inclusive prefix sum across the 64 lanes of a wave, with DPP moves (row
// shifts by 1, 2, 4 and 8 within 16 lanes, then the broadcasts of lanes 15
// and 31 into the rows after them) rather than LDS-routed shuffles.
__device__ inline int64_t wave_inclusive_sum(int64_t v) {
  v += dpp_move64<0x111, 0xf>(v);  // row_shr:1
  v += dpp_move64<0x112, 0xf>(v);  // row_shr:2
  v += dpp_move64<0x114, 0xf>(v);  // row_shr:4
  v += dpp_move64<0x118, 0xf>(v);  // row_shr:8
  v += dpp_move64<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
  v += dpp_move64<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3
  return v;
}

// Exclusive prefix of v across a block of NT threads; *block_total receives
// the sum.  Every thread of the block must call it.
template <int NT>
__device__ inline int64_t block_exclusive_sum(int64_t v, int64_t *block_total) {
  __shared__ int64_t wave_tot[NT / 64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int64_t inc = wave_inclusive_sum(v);
  if (lane == 63) wave_tot[wave] = inc;
  __syncthreads();
  int64_t wave_off = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < NT / 64; ++w) {
    int64_t t = wave_tot[w];
    if (w < wave) wave_off += t;
    tot += t;
  }
  __syncthreads();
  *block_total = tot;
  return wave_off + inc - v;
}

// ---- two-launch exclusive scan ---------------------------------------------
// Sequences of up to kFastScanBlocks tiles of kScanTile values are scanned by
// two launches: scan_reduce (each block sums its tile) and scan_apply (each
// block adds up the sums of the blocks before it, scans its tile and writes
// the prefixes).  Values come from a functor load(i) -> int64 so callers can
// generate them (flags from sorted keys, say) instead of materialising them;
// emit(i, value, prefix, n) runs once per index i < n in scan_apply, with the
// exclusive prefix of i.  out (may be null) receives the prefixes.
constexpr int kScanItems = 8;
constexpr int kScanTile = kBlock * kScanItems;
constexpr int64_t kFastScanBlocks = kBlock;
constexpr int64_t kFastScanMax = kFastScanBlocks * kScanTile;

template <class Load>
__global__ __launch_bounds__(kBlock) void scan_reduce_kernel(Load load, int64_t n,
                                                             const int64_t *n_dev,
                                                             int64_t *block_sums) {
  n = live_count(n, n_dev);
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile;
  int64_t s = 0;
#pragma unroll
  for (int r = 0; r < kScanItems; ++r) {
    const int64_t i = base + r * kBlock + threadIdx.x;
    s += i < n ? load(i) : 0;
  }
  int64_t tot;
  block_exclusive_sum<kBlock>(s, &tot);
  if (threadIdx.x == 0) block_sums[blockIdx.x] = tot;
}

template <class Load, class Emit>
__global__ __launch_bounds__(kBlock) void scan_apply_kernel(Load load, Emit emit, int64_t n,
                                                            const int64_t *n_dev,
                                                            const int64_t *block_sums,
                                                            int64_t nblocks, int64_t *out,
                                                            int64_t *total) {
  n = live_count(n, n_dev);
  // Offset of this block: sum of the block sums before it (nblocks <= kBlock).
  const int64_t bs = threadIdx.x < nblocks ? block_sums[threadIdx.x] : 0;
  int64_t offset;
  block_exclusive_sum<kBlock>(threadIdx.x < blockIdx.x ? bs : 0, &offset);
  if (blockIdx.x == 0 && total) {
    int64_t grand;
    block_exclusive_sum<kBlock>(bs, &grand);
    if (threadIdx.x == 0) *total = grand;
  }
  // Blocked layout inside the tile: thread t owns kScanItems consecutive values.
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile +
                       static_cast<int64_t>(threadIdx.x) * kScanItems;
  int64_t v[kScanItems];
  int64_t s = 0;
#pragma unroll
  for (int r = 0; r < kScanItems; ++r) {
    v[r] = base + r < n ? load(base + r) : 0;
    s += v[r];
  }
  int64_t tile_tot;
  int64_t run = offset + block_exclusive_sum<kBlock>(s, &tile_tot);
#pragma unroll
  for (int r = 0; r < kScanItems; ++r) {
    if (base + r < n) {
      if (out) out[base + r] = run;
      emit(base + r, v[r], run, n);
    }
    run += v[r];
  }
}

struct LoadI64 {
  const int64_t *in;
  __device__ int64_t operator()(int64_t i) const { return in[i]; }
};

struct NoEmit {
  __device__ void operator()(int64_t, int64_t, int64_t, int64_t) const {}
};

// Launches the two kernels for n in [1, kFastScanMax] (n_dev: optional
// device-side count clipping n); block_sums holds ceil(n / kScanTile) values.
template <class Load, class Emit>
inline void launch_fast_scan(Load load, Emit emit, int64_t n, const int64_t *n_dev,
                             int64_t *block_sums, int64_t *out, int64_t *total,
                             hipStream_t stream) {
  const int64_t nblocks = (n + kScanTile - 1) / kScanTile;
  hipLaunchKernelGGL(scan_reduce_kernel<Load>, dim3(static_cast<unsigned>(nblocks)),
                     dim3(kBlock), 0, stream, load, n, n_dev, block_sums);
  hipLaunchKernelGGL((scan_apply_kernel<Load, Emit>), dim3(static_cast<unsigned>(nblocks)),
                     dim3(kBlock), 0, stream, load, emit, n, n_dev, block_sums, nblocks, out,
                     total);
}

inline unsigned grid_for(int64_t n, int per_block = kBlock) {
  int64_t g = ceil_div(n, per_block);
  if (g < 1) g = 1;
  return static_cast<unsigned>(g);
}

}  // namespace ej
