// Backward of the per-pair tile einsum.
//
// Reference: sparse_einsum_raw._bwd (autodiff/custom_vjp.py:254-275).  For
// the forward out[p] = einsum("A,B->C", lhs[li[p]], rhs[ri[p]]) and the
// cotangent g[p] of out[p]:
//   grad_lhs[l] = sum over pairs p with li[p] == l of einsum("C,B->A", g[p], rhs[ri[p]])
//   grad_rhs[r] = sum over pairs p with ri[p] == r of einsum("A,C->B", lhs[li[p]], g[p])
// (the reversed strings of _reverse_einsum_string, custom_vjp.py:31-62; the
// sums are the reference's .at[idx].add scatter, :271-272).
//
// The scatter becomes a segment sum keyed by operand tile: ej_index_plan
// groups the pairs by target tile with a stable radix sort (positions
// ascending inside a target), and the fused segment einsum computes every
// gradient tile in one workgroup pass, written once, in a fixed order, with
// no atomics.  Tiles that no pair touches get zeros.
#include "ej_internal.h"

#include <string.h>

#include <string>
#include <vector>

namespace ej {
namespace {

__global__ __launch_bounds__(256) void plan_keys_kernel(const int64_t *__restrict__ idx, int64_t n,
                                                        int64_t n_targets,
                                                        uint64_t *__restrict__ keys,
                                                        int32_t *__restrict__ pos) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int64_t t = idx[i];
  keys[i] = t >= 0 && t < n_targets ? static_cast<uint64_t>(t) : static_cast<uint64_t>(n_targets);
  pos[i] = static_cast<int32_t>(i);
}

// offsets[t] = number of sorted keys below t, for t in [0, n_targets].
__global__ __launch_bounds__(256) void plan_offsets_kernel(const uint64_t *__restrict__ keys,
                                                           int64_t n, int64_t n_targets,
                                                           int32_t *__restrict__ offsets) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t > n_targets) return;
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (keys[mid] < static_cast<uint64_t>(t)) lo = mid + 1;
    else hi = mid;
  }
  offsets[t] = static_cast<int32_t>(lo);
}

// ---- counting plan ---------------------------------------------------------
// For target counts whose histogram fits LDS, the plan is a stable counting
// sort in three launches (the radix sort takes two passes of a histogram and
// a scatter for 13 bits, plus keys and offsets: six launches).  Bins are the
// targets [0, n_targets) plus one bin for invalid indices, which sorts last.
// Blocks take kPlanChunk consecutive pairs each.
//   plan_count:   hist[b][t] = pairs of block b with bin t;
//   plan_colscan: hist[b][t] <- pairs of blocks before b with bin t, and per
//                 group of 256 bins the exclusive prefix of the bin totals
//                 (tpref) and the group's total (tsum);
//   plan_scatter: a pair's position is the bins before its own (the groups'
//                 totals before its group plus tpref), the pairs of its bin
//                 in earlier blocks, and its rank among the pairs of its bin
//                 earlier in the block (wave ballots on the bin's bits, then
//                 the waves of a round in order through an LDS count per bin).
constexpr int kPlanChunk = 1024;
constexpr int64_t kPlanMaxBins = 63 * 256;  // LDS counts within 64 KB with the carries
constexpr int kPlanMaxGroups = 64;

__device__ inline uint32_t plan_bin(const int64_t *idx, int64_t i, int64_t n_targets) {
  const int64_t t = idx[i];
  return t >= 0 && t < n_targets ? static_cast<uint32_t>(t) : static_cast<uint32_t>(n_targets);
}

__global__ __launch_bounds__(256) void plan_count_kernel(const int64_t *__restrict__ idx,
                                                         int64_t n, int64_t n_targets,
                                                         uint32_t *__restrict__ hist) {
  extern __shared__ uint32_t cnt[];
  const int64_t bins = n_targets + 1;
  for (int64_t t = threadIdx.x; t < bins; t += 256) cnt[t] = 0;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kPlanChunk;
  uint32_t bin[kPlanChunk / 256];
#pragma unroll
  for (int r = 0; r < kPlanChunk / 256; ++r) {
    const int64_t i = base + r * 256 + threadIdx.x;
    bin[r] = i < n ? plan_bin(idx, i, n_targets) : 0xFFFFFFFFu;
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < kPlanChunk / 256; ++r)
    if (bin[r] != 0xFFFFFFFFu) atomicAdd(&cnt[bin[r]], 1u);
  __syncthreads();
  uint32_t *h = hist + static_cast<int64_t>(blockIdx.x) * bins;
  for (int64_t t = threadIdx.x; t < bins; t += 256) h[t] = cnt[t];
}

__global__ __launch_bounds__(256) void plan_colscan_kernel(uint32_t *__restrict__ hist,
                                                           int64_t nb, int64_t bins,
                                                           uint32_t *__restrict__ tpref,
                                                           uint32_t *__restrict__ tsum) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  uint32_t s = 0;
  if (t < bins) {
#pragma unroll 8
    for (int64_t b = 0; b < nb; ++b) {
      const uint32_t v = hist[b * bins + t];
      hist[b * bins + t] = s;
      s += v;
    }
  }
  int64_t total;
  const int64_t ex = block_exclusive_sum<256>(static_cast<int64_t>(s), &total);
  if (t < bins) tpref[t] = static_cast<uint32_t>(ex);
  if (threadIdx.x == 0) tsum[blockIdx.x] = static_cast<uint32_t>(total);
}

__global__ __launch_bounds__(256) void plan_scatter_kernel(
    const int64_t *__restrict__ idx, int64_t n, int64_t n_targets, int key_bits,
    const uint32_t *__restrict__ hist, const uint32_t *__restrict__ tpref,
    const uint32_t *__restrict__ tsum, int32_t *__restrict__ perm, int32_t *__restrict__ offsets) {
  extern __shared__ uint32_t run[];
  __shared__ uint32_t carry[kPlanMaxGroups];
  constexpr int R = kPlanChunk / 256;
  const int64_t bins = n_targets + 1;
  const int ngroups = static_cast<int>((bins + 255) / 256);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kPlanChunk;
  const uint32_t *h = hist + static_cast<int64_t>(blockIdx.x) * bins;
  // Every load that does not depend on the counts first: the pairs' bins,
  // then the bins' prefixes (tpref, h) and the group totals.
  uint32_t bin[R], pre[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t i = base + r * 256 + tid;
    bin[r] = i < n ? plan_bin(idx, i, n_targets) : 0xFFFFFFFFu;
  }
#pragma unroll
  for (int r = 0; r < R; ++r) pre[r] = bin[r] != 0xFFFFFFFFu ? tpref[bin[r]] + h[bin[r]] : 0u;
  const uint32_t gsum = tid < ngroups ? tsum[tid] : 0u;
  for (int64_t t = tid; t < bins; t += 256) run[t] = 0;
  if (wave == 0) {  // exclusive prefix of the group totals
    const uint32_t inc = static_cast<uint32_t>(wave_inclusive_sum(static_cast<int64_t>(gsum)));
    if (lane < ngroups) carry[lane] = inc - gsum;
  }
  __syncthreads();
  // Offsets, spread over the blocks: offsets[t] = pairs with a bin below t.
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + tid; t < bins;
       t += static_cast<int64_t>(gridDim.x) * 256)
    offsets[t] = static_cast<int32_t>(carry[t >> 8] + tpref[t]);
  const uint64_t lt_mask = lane == 0 ? 0ull : (~0ull >> (64 - lane));
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const bool valid = bin[r] != 0xFFFFFFFFu;
    const uint32_t k = valid ? bin[r] : 0u;
    uint64_t peers = __ballot(valid);
    for (int b = 0; b < key_bits; ++b) {
      const bool bit = (k >> b) & 1u;
      const uint64_t m = __ballot(bit);
      peers &= bit ? m : ~m;
    }
    const uint32_t rank = static_cast<uint32_t>(__popcll(peers & lt_mask));
    uint32_t before = 0;
    // The waves of this round in order: each reads the count of its bins so
    // far, then the first lane of each bin adds the wave's pairs of it.
    for (int w = 0; w < 4; ++w) {
      if (wave == w && valid) {
        before = run[k];
        if (rank == 0) run[k] = before + static_cast<uint32_t>(__popcll(peers));
      }
      __syncthreads();
    }
    if (valid) perm[carry[k >> 8] + pre[r] + before + rank] = static_cast<int32_t>(base + r * 256 + tid);
  }
}

__global__ __launch_bounds__(256) void bf16_to_f32_kernel(const uint16_t *__restrict__ in,
                                                          float *__restrict__ out, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    out[i] = __uint_as_float(static_cast<uint32_t>(in[i]) << 16);
}

template <typename T>
__global__ void zero_kernel(T *p, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    p[i] = T(0);
}

// Run order of the lhs gradient's segments: keys[s] = the rhs tile of
// segment s's first pair (n_rhs for a segment without pairs), vals[s] = s.
// Sorted stably, segments that contract the same rhs tiles become
// neighbours, which the fused einsum places on one XCD at the same time, so
// each rhs tile is fetched into that XCD's L2 once for all of them.
__global__ __launch_bounds__(256) void seg_first_rhs_kernel(const int64_t *__restrict__ ridx,
                                                            const int32_t *__restrict__ perm,
                                                            const int32_t *__restrict__ off,
                                                            int64_t n_seg, int64_t n_rhs,
                                                            uint64_t *__restrict__ keys,
                                                            int32_t *__restrict__ vals) {
  const int64_t s = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (s >= n_seg) return;
  uint64_t k = static_cast<uint64_t>(n_rhs);
  if (off[s] < off[s + 1]) {
    const int64_t r = ridx[perm[off[s]]];
    if (r >= 0 && r < n_rhs) k = static_cast<uint64_t>(r);
  }
  keys[s] = k;
  vals[s] = static_cast<int32_t>(s);
}

__global__ __launch_bounds__(256) void write_order_kernel(const int32_t *__restrict__ vals,
                                                          int64_t n, int32_t *__restrict__ order) {
  const int64_t b = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (b == 0) order[0] = static_cast<int32_t>(n);
  if (b < n) order[1 + b] = vals[b];
}

unsigned grid_capped(int64_t n) {
  const int64_t g = ceil_div(n > 0 ? n : 1, kBlock);
  return static_cast<unsigned>(g < 4096 ? g : 4096);
}

struct PlanWs {
  uint64_t *keys, *keys_alt;
  int32_t *pos_alt;
  void *sort_ws;
  size_t bytes;  // carved, alignment included
  size_t span;   // from keys to the end
};

PlanWs carve_plan(Carver &c, int64_t n) {
  PlanWs w;
  const size_t start = c.off;
  w.keys = c.take<uint64_t>(n);
  const size_t at_keys = c.off - sizeof(uint64_t) * static_cast<size_t>(n > 0 ? n : 1);
  w.keys_alt = c.take<uint64_t>(n);
  w.pos_alt = c.take<int32_t>(n);
  w.sort_ws = c.take<char>(static_cast<int64_t>(sort_workspace_bytes(n)));
  w.bytes = c.off - start;
  w.span = c.off - at_keys;
  return w;
}

// Workspace of the counting plan (hist, tpref, tsum).
size_t counting_plan_bytes(int64_t n, int64_t bins) {
  return align_up(sizeof(uint32_t) * ceil_div(n, kPlanChunk) * bins, 256) +
         align_up(sizeof(uint32_t) * bins, 256) + sizeof(uint32_t) * kPlanMaxGroups;
}

int index_plan(const int64_t *idx, int64_t n, int64_t n_targets, int32_t *perm, int32_t *offsets,
               const PlanWs &w, hipStream_t stream) {
  const int bits = [&] {
    int b = 0;
    while (b < 63 && (int64_t(1) << b) < n_targets + 1) ++b;
    return b;
  }();
  const int64_t bins = n_targets + 1;
  // The counting plan runs in the plan workspace carved for the radix sort
  // (which depends on n only) when its histograms fit there.
  if (n > 0 && bins <= kPlanMaxBins && counting_plan_bytes(n, bins) <= w.span) {
    const int64_t nb = ceil_div(n, kPlanChunk);
    char *c = static_cast<char *>(static_cast<void *>(w.keys));
    uint32_t *hist = reinterpret_cast<uint32_t *>(c);
    c += align_up(sizeof(uint32_t) * nb * bins, 256);
    uint32_t *tpref = reinterpret_cast<uint32_t *>(c);
    uint32_t *tsum = reinterpret_cast<uint32_t *>(c + align_up(sizeof(uint32_t) * bins, 256));
    const size_t lds = sizeof(uint32_t) * static_cast<size_t>(bins);
    hipLaunchKernelGGL(plan_count_kernel, dim3(static_cast<unsigned>(nb)), dim3(256), lds, stream,
                       idx, n, n_targets, hist);
    EJ_LAUNCH_CHECK();
    hipLaunchKernelGGL(plan_colscan_kernel, dim3(static_cast<unsigned>(ceil_div(bins, 256))),
                       dim3(256), 0, stream, hist, nb, bins, tpref, tsum);
    EJ_LAUNCH_CHECK();
    hipLaunchKernelGGL(plan_scatter_kernel, dim3(static_cast<unsigned>(nb)), dim3(256), lds,
                       stream, idx, n, n_targets, bits, hist, tpref, tsum, perm, offsets);
    EJ_LAUNCH_CHECK();
    return EJ_OK;
  }
  if (n > 0) {
    const bool alt = radix_passes(bits) % 2 == 1;
    hipLaunchKernelGGL(plan_keys_kernel, dim3(grid_for(n)), dim3(kBlock), 0, stream, idx, n,
                       n_targets, alt ? w.keys_alt : w.keys, alt ? w.pos_alt : perm);
    EJ_LAUNCH_CHECK();
    EJ_TRY(sort_pairs_u64(w.keys, perm, w.keys_alt, w.pos_alt, n, bits, w.sort_ws, stream, alt));
  }
  hipLaunchKernelGGL(plan_offsets_kernel, dim3(grid_for(n_targets + 1)), dim3(kBlock), 0, stream,
                     w.keys, n, n_targets, offsets);
  EJ_LAUNCH_CHECK();
  return EJ_OK;
}

// "A,B->C" -> terms A, B, C (no validation beyond the separators; the
// descriptor parser checks the labels).
int split_terms(const char *ks, std::string *a, std::string *b, std::string *c) {
  EJ_CHECK_ARG(ks, "kernel_string is null");
  const char *arrow = strstr(ks, "->");
  EJ_CHECK_ARG(arrow, "kernel_string must contain '->': %s", ks);
  const char *comma = static_cast<const char *>(memchr(ks, ',', arrow - ks));
  EJ_CHECK_ARG(comma, "kernel_string must have exactly two operands: %s", ks);
  a->assign(ks, comma - ks);
  b->assign(comma + 1, arrow - comma - 1);
  c->assign(arrow + 2);
  return EJ_OK;
}

int check_dtypes(int32_t dtype, int32_t grad_dtype) {
  EJ_CHECK_ARG(dtype == EJ_F32 || dtype == EJ_BF16, "unknown dtype %d", dtype);
  EJ_CHECK_ARG(grad_dtype == EJ_F32 || (grad_dtype == EJ_BF16 && dtype == EJ_BF16),
               "gradient dtype %d with operand dtype %d: gradients are fp32, or bf16 for bf16 "
               "operands", grad_dtype, dtype);
  return EJ_OK;
}

struct VjpWs {
  int32_t *perm_l, *off_l, *perm_r, *off_r;
  float *lhs32, *rhs32;
  PlanWs plan, plan_r;  // the lhs and rhs gradients' sorts (they may run concurrently)
  // run order of the lhs gradient's segments and its sort
  int32_t *order, *ovals, *ovals_alt;
  uint64_t *okeys, *okeys_alt;
  void *osort_ws;
  size_t bytes;
};

// Widened operands are needed for bf16 operands under an fp32 cotangent.
VjpWs carve_vjp(void *base, int64_t n_pairs, int64_t n_lhs, int64_t n_rhs, int64_t lhs_elems,
                int64_t rhs_elems, int32_t dtype, int32_t grad_dtype) {
  Carver c(base);
  VjpWs w{};
  w.perm_l = c.take<int32_t>(n_pairs);
  w.off_l = c.take<int32_t>(n_lhs + 1);
  w.perm_r = c.take<int32_t>(n_pairs);
  w.off_r = c.take<int32_t>(n_rhs + 1);
  if (dtype == EJ_BF16 && grad_dtype == EJ_F32) {
    w.lhs32 = c.take<float>(n_lhs * lhs_elems);
    w.rhs32 = c.take<float>(n_rhs * rhs_elems);
  }
  w.plan = carve_plan(c, n_pairs);
  w.plan_r = carve_plan(c, n_pairs);
  w.order = c.take<int32_t>(n_lhs + 1);
  w.ovals = c.take<int32_t>(n_lhs);
  w.ovals_alt = c.take<int32_t>(n_lhs);
  w.okeys = c.take<uint64_t>(n_lhs);
  w.okeys_alt = c.take<uint64_t>(n_lhs);
  w.osort_ws = c.take<char>(static_cast<int64_t>(sort_workspace_bytes(n_lhs)));
  w.bytes = c.off;
  return w;
}

// Sorts the lhs gradient's segments by the rhs tile of their first pair into
// w.order (the fused einsum's run order for groups of one segment).
int lhs_grad_order(const int64_t *ridx, const int32_t *perm, const int32_t *off, int64_t n_seg,
                   int64_t n_rhs, const VjpWs &w, hipStream_t stream) {
  int bits = 1;
  while (bits < 63 && (int64_t(1) << bits) < n_rhs + 1) ++bits;
  const bool alt = radix_passes(bits) % 2 == 1;
  hipLaunchKernelGGL(seg_first_rhs_kernel, dim3(grid_for(n_seg)), dim3(kBlock), 0, stream, ridx,
                     perm, off, n_seg, n_rhs, alt ? w.okeys_alt : w.okeys,
                     alt ? w.ovals_alt : w.ovals);
  EJ_LAUNCH_CHECK();
  EJ_TRY(sort_pairs_u64(w.okeys, w.ovals, w.okeys_alt, w.ovals_alt, n_seg, bits, w.osort_ws,
                        stream, alt));
  hipLaunchKernelGGL(write_order_kernel, dim3(grid_for(n_seg)), dim3(kBlock), 0, stream, w.ovals,
                     n_seg, w.order);
  EJ_LAUNCH_CHECK();
  return EJ_OK;
}

// A second stream of the calling thread on the current device, with the two
// events that fork work onto it from a caller's stream and join it back
// (created once per thread and device, default priority, never destroyed).
struct SideStream {
  hipStream_t stream = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
};

bool side_stream(SideStream *out) {
  thread_local std::vector<SideStream> per_device;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return false;
  if (static_cast<int>(per_device.size()) <= dev) per_device.resize(dev + 1);
  SideStream &ss = per_device[dev];
  if (!ss.stream) {
    SideStream n;
    if (hipStreamCreateWithFlags(&n.stream, hipStreamNonBlocking) != hipSuccess) return false;
    if (hipEventCreateWithFlags(&n.fork, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&n.join, hipEventDisableTiming) != hipSuccess) {
      if (n.fork) (void)hipEventDestroy(n.fork);
      (void)hipStreamDestroy(n.stream);
      return false;
    }
    ss = n;
  }
  *out = ss;
  return true;
}

}  // namespace
}  // namespace ej

using namespace ej;

extern "C" int ej_index_plan_workspace_size(int64_t n, size_t *bytes) {
  clear_error();
  EJ_CHECK_ARG(bytes, "bytes is null");
  EJ_CHECK_ARG(n >= 0 && n <= INT32_MAX, "n=%lld outside [0, 2^31)", (long long)n);
  Carver c(nullptr);
  *bytes = carve_plan(c, n).bytes;
  return EJ_OK;
}

extern "C" int ej_index_plan(const int64_t *idx, int64_t n, int64_t n_targets, int32_t *perm,
                             int32_t *offsets, void *workspace, size_t workspace_bytes,
                             ej_stream_t stream) {
  clear_error();
  EJ_CHECK_ARG(n >= 0 && n <= INT32_MAX, "n=%lld outside [0, 2^31)", (long long)n);
  EJ_CHECK_ARG(n_targets >= 0 && n_targets < INT32_MAX, "n_targets out of range");
  EJ_CHECK_ARG(offsets && (n == 0 || (idx && perm)), "null pointer argument");
  Carver c(workspace);
  PlanWs w = carve_plan(c, n);
  EJ_CHECK_ARG(workspace && workspace_bytes >= w.bytes, "workspace too small: %zu < %zu bytes",
               workspace_bytes, w.bytes);
  return index_plan(idx, n, n_targets, perm, offsets, w, as_stream(stream));
}

extern "C" int ej_pair_einsum_vjp_workspace_size(int64_t n_pairs, int64_t n_lhs_tiles,
                                                 int64_t n_rhs_tiles, int64_t lhs_elems,
                                                 int64_t rhs_elems, int32_t dtype,
                                                 int32_t grad_dtype, size_t *bytes) {
  clear_error();
  EJ_CHECK_ARG(bytes, "bytes is null");
  EJ_TRY(check_dtypes(dtype, grad_dtype));
  EJ_CHECK_ARG(n_pairs >= 0 && n_pairs <= INT32_MAX, "n_pairs outside [0, 2^31)");
  EJ_CHECK_ARG(n_lhs_tiles >= 0 && n_lhs_tiles < INT32_MAX && n_rhs_tiles >= 0 &&
                   n_rhs_tiles < INT32_MAX && lhs_elems >= 1 && rhs_elems >= 1,
               "bad sizes");
  *bytes = carve_vjp(nullptr, n_pairs, n_lhs_tiles, n_rhs_tiles, lhs_elems, rhs_elems, dtype,
                     grad_dtype).bytes;
  return EJ_OK;
}

extern "C" int ej_pair_einsum_vjp(const char *kernel_string, const int64_t *lhs_tile,
                                  int32_t lhs_ndim, const int64_t *rhs_tile, int32_t rhs_ndim,
                                  int32_t dtype, const void *lhs_values, int64_t n_lhs_tiles,
                                  const void *rhs_values, int64_t n_rhs_tiles,
                                  const int64_t *lhs_idx, const int64_t *rhs_idx,
                                  int64_t n_pairs, int32_t grad_dtype, const void *grad_out,
                                  void *grad_lhs, void *grad_rhs, void *workspace,
                                  size_t workspace_bytes, ej_stream_t stream_) {
  clear_error();
  hipStream_t stream = as_stream(stream_);
  EJ_TRY(check_dtypes(dtype, grad_dtype));
  EJ_CHECK_ARG(n_pairs >= 0 && n_pairs <= INT32_MAX, "n_pairs outside [0, 2^31)");
  EJ_CHECK_ARG(n_lhs_tiles >= 0 && n_lhs_tiles < INT32_MAX && n_rhs_tiles >= 0 &&
                   n_rhs_tiles < INT32_MAX,
               "tile counts out of range");
  std::string ta, tb, tc;
  EJ_TRY(split_terms(kernel_string, &ta, &tb, &tc));
  // Forward descriptor: validates the string against the tiles and gives
  // the output tile extents (label order of the output term).
  ej_einsum_desc fwd;
  EJ_TRY(ej_einsum_describe(kernel_string, lhs_tile, lhs_ndim, rhs_tile, rhs_ndim, &fwd));
  int64_t out_tile[EJ_MAX_LABELS];
  for (int i = 0; i < fwd.n_out; ++i) out_tile[i] = fwd.out_ext[i];
  int64_t lhs_elems = 1, rhs_elems = 1;
  for (int i = 0; i < lhs_ndim; ++i) lhs_elems *= lhs_tile[i];
  for (int i = 0; i < rhs_ndim; ++i) rhs_elems *= rhs_tile[i];
  const std::string s_lhs = tc + "," + tb + "->" + ta;  // grad_lhs: "C,B->A"
  const std::string s_rhs = ta + "," + tc + "->" + tb;  // grad_rhs: "A,C->B"
  ej_einsum_desc dl, dr;
  if (grad_lhs) {
    const int st = ej_einsum_describe(s_lhs.c_str(), out_tile, fwd.n_out, rhs_tile, rhs_ndim, &dl);
    if (st != EJ_OK) {
      set_error("gradient string %s for the lhs is not a valid einsum of the output and rhs "
                "tiles: %s", s_lhs.c_str(), ej_last_error());
      return st;
    }
  }
  if (grad_rhs) {
    const int st = ej_einsum_describe(s_rhs.c_str(), lhs_tile, lhs_ndim, out_tile, fwd.n_out, &dr);
    if (st != EJ_OK) {
      set_error("gradient string %s for the rhs is not a valid einsum of the lhs and output "
                "tiles: %s", s_rhs.c_str(), ej_last_error());
      return st;
    }
  }
  if (!grad_lhs && !grad_rhs) return EJ_OK;
  dl.out_dtype = dr.out_dtype = grad_dtype;
  // The rhs gradient's segments are rhs tiles in index order.  Rhs tiles
  // with equal join key pair with the same lhs tiles in the same order, and
  // tiles sorted by coordinates keep equal keys adjacent when the key
  // dimensions lead (every join of a matmul-shaped einsum): mark the segments
  // as sharing their lhs tiles, so the fused kernel runs them grouped.  The
  // kernel checks the property on each group's pairs and runs a group
  // without it pair by pair, with the same results.
  dr.seg_group = 4;
  VjpWs w = carve_vjp(workspace, n_pairs, n_lhs_tiles, n_rhs_tiles, lhs_elems, rhs_elems, dtype,
                      grad_dtype);
  EJ_CHECK_ARG(workspace && workspace_bytes >= w.bytes, "workspace too small: %zu < %zu bytes",
               workspace_bytes, w.bytes);
  EJ_CHECK_ARG(n_pairs == 0 || (grad_out && lhs_idx && rhs_idx), "null pointer argument");
  EJ_CHECK_ARG((!grad_lhs || n_rhs_tiles == 0 || rhs_values) &&
                   (!grad_rhs || n_lhs_tiles == 0 || lhs_values),
               "null operand values");
  const void *lhs_v = lhs_values, *rhs_v = rhs_values;
  // An fp32 cotangent with bf16 operands, the lhs gradient on k-contiguous
  // 128 x 128 blocks: the cotangent is split into three bf16 terms in the
  // kernel and the rhs stays bf16 (segment_einsum_split), so the rhs is not
  // widened.
  const bool split = dtype == EJ_BF16 && grad_dtype == EJ_F32 && grad_lhs && n_lhs_tiles > 0 &&
                     n_rhs_tiles > 0 && n_pairs > 0 &&
                     segment_einsum_split_ok(&dl, grad_out, rhs_values);
  // The same for the rhs gradient on [k][m] lhs blocks against the fp32
  // cotangent (segment_einsum_split_b): the lhs is not widened.
  const bool split_b = dtype == EJ_BF16 && grad_dtype == EJ_F32 && grad_rhs && n_rhs_tiles > 0 &&
                       n_lhs_tiles > 0 && n_pairs > 0 &&
                       segment_einsum_split_b_ok(&dr, lhs_values, grad_out);
  if (dtype == EJ_BF16 && grad_dtype == EJ_F32) {
    // Otherwise, with an fp32 cotangent and bf16 operands, the operands are
    // widened to fp32 once so the gradient einsums run in fp32 throughout.
    // (A bf16 cotangent runs them on bf16 operands with fp32 sums.)
    if (grad_rhs && n_lhs_tiles > 0 && !split_b) {
      hipLaunchKernelGGL(bf16_to_f32_kernel, dim3(grid_capped(n_lhs_tiles * lhs_elems)),
                         dim3(kBlock), 0, stream, static_cast<const uint16_t *>(lhs_values),
                         w.lhs32, n_lhs_tiles * lhs_elems);
      EJ_LAUNCH_CHECK();
      lhs_v = w.lhs32;
    }
    if (grad_lhs && n_rhs_tiles > 0 && !split) {
      hipLaunchKernelGGL(bf16_to_f32_kernel, dim3(grid_capped(n_rhs_tiles * rhs_elems)),
                         dim3(kBlock), 0, stream, static_cast<const uint16_t *>(rhs_values),
                         w.rhs32, n_rhs_tiles * rhs_elems);
      EJ_LAUNCH_CHECK();
      rhs_v = w.rhs32;
    }
  }
  // Operand dtype of the gradient einsums: the cotangent's.
  const int32_t edt = grad_dtype;
  auto zero = [&](void *p, int64_t n, hipStream_t st) -> int {
    if (grad_dtype == EJ_BF16)
      hipLaunchKernelGGL(zero_kernel<uint16_t>, dim3(grid_capped(n)), dim3(kBlock), 0, st,
                         static_cast<uint16_t *>(p), n);
    else
      hipLaunchKernelGGL(zero_kernel<float>, dim3(grid_capped(n)), dim3(kBlock), 0, st,
                         static_cast<float *>(p), n);
    EJ_LAUNCH_CHECK();
    return EJ_OK;
  };
  // The two gradients' einsums run one after the other on the caller's
  // stream (run side by side they slow each other down more than they fill
  // each other's idle CUs).  With both gradients, the lhs gradient's plan and
  // run order are computed on a second stream while the rhs gradient's plan
  // and einsum run; the lhs einsum waits for both.  Each plan has its own
  // sort workspace.
  const bool lhs_live = grad_lhs && n_lhs_tiles > 0 && n_pairs > 0 && n_rhs_tiles > 0;
  const int og = split ? 1
                 : lhs_live ? segment_einsum_order_group(&dl, edt, n_lhs_tiles, grad_out, rhs_v)
                            : 0;
  auto lhs_prep = [&](hipStream_t st) -> int {
    EJ_TRY(index_plan(lhs_idx, n_pairs, n_lhs_tiles, w.perm_l, w.off_l, w.plan, st));
    // One lhs tile per workgroup on the LDS ring: run the tiles that
    // contract the same rhs tiles side by side (see seg_first_rhs_kernel).
    if (og == 1) EJ_TRY(lhs_grad_order(rhs_idx, w.perm_l, w.off_l, n_lhs_tiles, n_rhs_tiles, w, st));
    return EJ_OK;
  };
  auto rhs_grad = [&](hipStream_t st) -> int {
    if (!grad_rhs || n_rhs_tiles == 0) return EJ_OK;
    if (n_pairs == 0 || n_lhs_tiles == 0) return zero(grad_rhs, n_rhs_tiles * rhs_elems, st);
    EJ_TRY(index_plan(rhs_idx, n_pairs, n_rhs_tiles, w.perm_r, w.off_r, w.plan_r, st));
    if (split_b)
      return segment_einsum_split_b(&dr, static_cast<const uint16_t *>(lhs_values),
                                    static_cast<const float *>(grad_out), n_lhs_tiles, n_pairs,
                                    lhs_idx, nullptr, w.perm_r, w.off_r, n_rhs_tiles, grad_rhs,
                                    st);
    return ej_segment_einsum(&dr, edt, lhs_v, grad_out, n_lhs_tiles, n_pairs, lhs_idx, nullptr,
                             w.perm_r, w.off_r, n_rhs_tiles, grad_rhs,
                             reinterpret_cast<ej_stream_t>(st));
  };
  SideStream side;
  const bool fork = lhs_live && grad_rhs && n_rhs_tiles > 0 && side_stream(&side);
  if (fork) {
    EJ_HIP(hipEventRecord(side.fork, stream));
    EJ_HIP(hipStreamWaitEvent(side.stream, side.fork, 0));
    const int sl = lhs_prep(side.stream);
    EJ_HIP(hipEventRecord(side.join, side.stream));
    const int sr = rhs_grad(stream);
    EJ_HIP(hipStreamWaitEvent(stream, side.join, 0));
    EJ_TRY(sl);
    EJ_TRY(sr);
  } else {
    if (lhs_live) EJ_TRY(lhs_prep(stream));
    EJ_TRY(rhs_grad(stream));
  }
  if (grad_lhs && n_lhs_tiles > 0) {
    if (!lhs_live) {
      EJ_TRY(zero(grad_lhs, n_lhs_tiles * lhs_elems, stream));
    } else {
      if (split)
        EJ_TRY(segment_einsum_split(&dl, static_cast<const float *>(grad_out),
                                    static_cast<const uint16_t *>(rhs_values), n_pairs,
                                    n_rhs_tiles, nullptr, rhs_idx, w.perm_l, w.off_l,
                                    n_lhs_tiles, w.order, 1, grad_lhs, stream));
      else
        EJ_TRY(segment_einsum_ordered(&dl, edt, grad_out, rhs_v, n_pairs, n_rhs_tiles, nullptr,
                                      rhs_idx, w.perm_l, w.off_l, n_lhs_tiles,
                                      og == 1 ? w.order : nullptr, 1, grad_lhs, stream));
    }
  }
  return EJ_OK;
}
