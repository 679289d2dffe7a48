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
#include <mutex>
#include "ej_internal.h"

#include <type_traits>

namespace ej {

namespace {

// Packs the join keys of both relations in one launch: threads [0, n_lhs)
// take lhs rows, the rest rhs rows.  A non-null perm gets the identity
// permutation the stable sort starts from.
__global__ void pack_keys_kernel(const int32_t *lc, int64_t n_lhs, KeySpec lks, uint64_t *lkeys,
                                 int32_t *lperm, const int32_t *rc, int64_t n_rhs, KeySpec rks,
                                 uint64_t *rkeys, int32_t *rperm, int *bad) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  int b = 0;
  if (i < n_lhs) {
    lkeys[i] = pack_key(lc + i * lks.ncols, lks, &b);
    if (lperm) lperm[i] = static_cast<int32_t>(i);
  } else if (i - n_lhs < n_rhs) {
    const int64_t j = i - n_lhs;
    rkeys[j] = pack_key(rc + j * rks.ncols, rks, &b);
    if (rperm) rperm[j] = static_cast<int32_t>(j);
  }
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

// Probe count and scan in one workgroup, for build sides that fit in LDS:
// lo_out[j] = first build position equal to probe key j, offs = exclusive
// scan of the equal-range sizes, *total = P.  The build keys are staged in
// LDS and each thread runs kProbeBatch branch-free equal-range searches side
// by side (fixed trip count ceil(log2 n_build)), so their LDS reads overlap.
constexpr int kProbeThreads = 1024;
constexpr int kProbeLdsKeys = 8192;
constexpr int64_t kProbeSmallMax = 8192;
constexpr int kProbeBatch = 4;

__global__ __launch_bounds__(kProbeThreads) void probe_scan_small_kernel(
    const uint64_t *__restrict__ probe_keys, int64_t n_probe,
    const uint64_t *__restrict__ build_sorted, int n_build, int64_t *__restrict__ lo_out,
    int64_t *__restrict__ offs, int64_t *__restrict__ total) {
  __shared__ uint64_t bk[kProbeLdsKeys];
  for (int i = threadIdx.x; i < n_build; i += kProbeThreads) bk[i] = build_sorted[i];
  __syncthreads();
  const int64_t c = (n_probe + kProbeThreads - 1) / kProbeThreads;
  const int64_t lo = min(n_probe, static_cast<int64_t>(threadIdx.x) * c);
  const int64_t hi = min(n_probe, lo + c);
  int64_t s = 0;
  for (int64_t j0 = lo; j0 < hi; j0 += kProbeBatch) {
    uint64_t k[kProbeBatch];
    int lb[kProbeBatch], ub[kProbeBatch];
#pragma unroll
    for (int u = 0; u < kProbeBatch; ++u) {
      k[u] = j0 + u < hi ? probe_keys[j0 + u] : 0;
      lb[u] = 0;
      ub[u] = 0;
    }
    // Invariant: the answer lies in [base, base + len]; base + len <= n_build.
    for (int len = n_build; len > 1;) {
      const int half = len >> 1;
#pragma unroll
      for (int u = 0; u < kProbeBatch; ++u) {
        lb[u] += bk[lb[u] + half] < k[u] ? half : 0;
        ub[u] += bk[ub[u] + half] <= k[u] ? half : 0;
      }
      len -= half;
    }
#pragma unroll
    for (int u = 0; u < kProbeBatch; ++u) {
      lb[u] += bk[lb[u]] < k[u] ? 1 : 0;
      ub[u] += bk[ub[u]] <= k[u] ? 1 : 0;
      if (j0 + u < hi) {
        lo_out[j0 + u] = lb[u];
        offs[j0 + u] = ub[u] - lb[u];
        s += ub[u] - lb[u];
      }
    }
  }
  int64_t tot;
  int64_t run = block_exclusive_sum<kProbeThreads>(s, &tot);
  for (int64_t j = lo; j < hi; ++j) {
    const int64_t v = offs[j];
    offs[j] = run;
    run += v;
  }
  if (threadIdx.x == 0) *total = tot;
}

// The whole EJ_ORDER_PROBE count in one workgroup, for a build side (lhs) of
// at most kJoinSmallBuild rows and a probe side of at most kProbeSmallMax:
// the lhs keys are packed and stably radix-sorted in LDS (8-bit digits;
// ranks inside a wave from ballot peer masks, across waves from per-digit
// counts), the sorted permutation is written to lperm, every rhs row's equal
// range is found by side-by-side branch-free searches, and the counts are
// scanned into offs.  scalars[0] = P and scalars[1] = the out-of-range flag
// are written outright, so nothing needs clearing first; the n_clear int64s
// at `clear` and the n_clear2 at `clear2` (a later phase's counters) are
// zeroed on the way.  One launch replaces the clear, pack, sort and probe
// launches of the general path.  With join keys of at most 32 bits (PACK)
// each LDS entry is (key << 32 | row) and the build side may have up to
// kJoinSmallBuildPacked rows.
constexpr int kJoinSmallThreads = 1024;
constexpr int kJoinSmallBuild = 4096;
constexpr int kJoinSmallBuildPacked = 8192;

template <bool PACK>
__global__ __launch_bounds__(kJoinSmallThreads) void join_probe_small_kernel(
    const int32_t *__restrict__ lc, int n_build, KeySpec lks, const int32_t *__restrict__ rc,
    int64_t n_probe, KeySpec rks, int bits, int32_t *__restrict__ lperm,
    int64_t *__restrict__ lo_out, int64_t *__restrict__ offs, int64_t *__restrict__ scalars,
    int64_t *__restrict__ clear, int n_clear, int64_t *__restrict__ clear2, int n_clear2) {
  constexpr int NW = kJoinSmallThreads / 64;
  constexpr int NB = PACK ? kJoinSmallBuildPacked : kJoinSmallBuild;
  constexpr int KS = PACK ? 32 : 0;  // key position inside an entry
  // entries: PACK: (key << 32 | row); otherwise the key, its row in sidx
  __shared__ uint64_t skey[2][NB];
  __shared__ int32_t sidx[PACK ? 1 : 2][PACK ? 1 : NB];
  // digits: 9 bits with packed entries (fewer passes for 9-bit keys), else 8
  constexpr int DB = PACK ? 9 : 8, NBIN = 1 << DB;
  using cnt_t = typename std::conditional<PACK, uint16_t, int32_t>::type;
  __shared__ cnt_t wcnt[NW][NBIN];  // per wave and digit: count, then prefix over waves
  __shared__ int32_t dbase[NBIN];
  __shared__ int bad_any;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint64_t lt_mask = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  // This thread's probe rows [plo, phi), at most PPT, packed first so that
  // their loads overlap the build side's.
  constexpr int PPT = static_cast<int>(kProbeSmallMax / kJoinSmallThreads);
  const int64_t pc = (n_probe + kJoinSmallThreads - 1) / kJoinSmallThreads;
  const int64_t plo = min(n_probe, static_cast<int64_t>(tid) * pc);
  const int64_t phi = min(n_probe, plo + pc);
  int bad = 0;
  uint64_t pk[PPT];
#pragma unroll
  for (int u = 0; u < PPT; ++u)
    pk[u] = plo + u < phi ? pack_key(rc + (plo + u) * rks.ncols, rks, &bad) : 0;
  if (tid == 0) bad_any = 0;
  if (tid < n_clear) clear[tid] = 0;
  for (int i = tid; i < n_clear2; i += kJoinSmallThreads) clear2[i] = 0;
  __syncthreads();
  for (int i = tid; i < n_build; i += kJoinSmallThreads) {
    const uint64_t k = pack_key(lc + static_cast<int64_t>(i) * lks.ncols, lks, &bad);
    if constexpr (PACK) {
      skey[0][i] = (k << 32) | static_cast<uint32_t>(i);
    } else {
      skey[0][i] = k;
      sidx[0][i] = i;
    }
  }
  if (bad) bad_any = 1;
  int cur = 0;
  for (int shift = 0; shift < bits; shift += DB) {
    for (int x = tid; x < NBIN; x += kJoinSmallThreads) dbase[x] = 0;
    __syncthreads();
    for (int i = tid; i < n_build; i += kJoinSmallThreads)
      atomicAdd(&dbase[(skey[cur][i] >> (KS + shift)) & (NBIN - 1)], 1);
    __syncthreads();
    if (wave == 0) {  // exclusive scan of the digit counts, NBIN / 64 per lane
      constexpr int PL = NBIN / 64;
      int v[PL], sum = 0;
#pragma unroll
      for (int u = 0; u < PL; ++u) {
        v[u] = dbase[lane * PL + u];
        sum += v[u];
      }
      int inc = sum;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(inc, o);
        if (lane >= o) inc += t;
      }
      int run = inc - sum;
#pragma unroll
      for (int u = 0; u < PL; ++u) {
        dbase[lane * PL + u] = run;
        run += v[u];
      }
    }
    // Stable scatter, kJoinSmallThreads keys per round in index order.
    for (int r0 = 0; r0 < n_build; r0 += kJoinSmallThreads) {
      for (int x = tid; x < NW * NBIN; x += kJoinSmallThreads) (&wcnt[0][0])[x] = 0;
      __syncthreads();
      const int i = r0 + tid;
      const bool valid = i < n_build;
      const uint64_t k = valid ? skey[cur][i] : 0;
      const int d = static_cast<int>((k >> (KS + shift)) & (NBIN - 1));
      uint64_t peers = __ballot(valid);
#pragma unroll
      for (int b = 0; b < DB; ++b) {
        const int bit = (d >> b) & 1;
        const uint64_t m = __ballot(bit);
        peers &= bit ? m : ~m;
      }
      const int rank = __popcll(peers & lt_mask);
      if (valid && rank == 0) wcnt[wave][d] = static_cast<cnt_t>(__popcll(peers));
      __syncthreads();
      int total = 0;
      if (tid < NBIN) {  // per digit: exclusive prefix over the waves, in place
#pragma unroll
        for (int w = 0; w < NW; ++w) {
          const int c = wcnt[w][tid];
          wcnt[w][tid] = static_cast<cnt_t>(total);
          total += c;
        }
      }
      __syncthreads();
      if (valid) {
        const int pos = dbase[d] + wcnt[wave][d] + rank;
        skey[cur ^ 1][pos] = k;
        if constexpr (!PACK) sidx[cur ^ 1][pos] = sidx[cur][i];
      }
      __syncthreads();
      if (tid < NBIN) dbase[tid] += total;
    }
    cur ^= 1;
  }
  __syncthreads();
  for (int i = tid; i < n_build; i += kJoinSmallThreads)
    lperm[i] = PACK ? static_cast<int32_t>(skey[cur][i] & 0xFFFFFFFFu) : sidx[cur][i];
  const uint64_t *bk = skey[cur];
  auto bkey = [&](int i) -> uint64_t { return bk[i] >> KS; };
  // Equal ranges of the PPT probe keys, searched side by side (branch-free,
  // fixed trip count); the counts stay in registers for the scan.
  int lb[PPT], ub[PPT];
#pragma unroll
  for (int u = 0; u < PPT; ++u) lb[u] = ub[u] = 0;
  // Invariant: the answer lies in [base, base + len]; base + len <= n_build.
  for (int len = n_build; len > 1;) {
    const int half = len >> 1;
#pragma unroll
    for (int u = 0; u < PPT; ++u) {
      if (u < pc) {  // pc is the same for every thread
        lb[u] += bkey(lb[u] + half) < pk[u] ? half : 0;
        ub[u] += bkey(ub[u] + half) <= pk[u] ? half : 0;
      }
    }
    len -= half;
  }
  int64_t s = 0;
#pragma unroll
  for (int u = 0; u < PPT; ++u) {
    lb[u] += bkey(lb[u]) < pk[u] ? 1 : 0;
    ub[u] += bkey(ub[u]) <= pk[u] ? 1 : 0;
    if (plo + u < phi) {
      lo_out[plo + u] = lb[u];
      s += ub[u] - lb[u];
    }
  }
  if (bad) bad_any = 1;
  int64_t tot;
  int64_t run = block_exclusive_sum<kJoinSmallThreads>(s, &tot);
#pragma unroll
  for (int u = 0; u < PPT; ++u) {
    if (plo + u < phi) {
      offs[plo + u] = run;
      run += ub[u] - lb[u];
    }
  }
  if (tid == 0) {
    scalars[0] = tot;
    scalars[1] = bad_any;
  }
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

namespace ej {
namespace {

// Enqueues the join count.  *host_known >= 0 on return: the pair count is
// known on the host (cross product or an empty side) and nothing was
// enqueued; otherwise (-1) the count and a range flag land in w.scalars[0..1].
// clear (optional): kClearScalars int64s of a later phase, zeroed in stream
// order before the count finishes; clear2 (optional, one-workgroup count
// only): n_clear2 more.
constexpr int kClearScalars = 8;

// Whether the one-workgroup join count takes these sides (bits: the join
// key's width; wider than 32 bits allows kJoinSmallBuild build rows).
bool join_small_ok(int32_t order, int64_t n_lhs, int64_t n_rhs, int bits) {
  const int64_t nb = bits <= 32 ? kJoinSmallBuildPacked : kJoinSmallBuild;
  return order == EJ_ORDER_PROBE && n_lhs <= nb && n_rhs <= kProbeSmallMax;
}

int join_count_enqueue(const int32_t *lhs_coords, int64_t n_lhs, int32_t lhs_ncols,
                       const int32_t *rhs_coords, int64_t n_rhs, int32_t rhs_ncols,
                       int32_t n_keys, const int32_t *lhs_dims, const int32_t *rhs_dims,
                       const int64_t *radices, int32_t order, void *workspace,
                       size_t workspace_bytes, int64_t *host_known, int64_t **dev_scalars,
                       hipStream_t stream, int64_t *clear = nullptr, int64_t *clear2 = nullptr,
                       int n_clear2 = 0) {
  *host_known = -1;
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
    *host_known = static_cast<int64_t>(p);
    return EJ_OK;
  }
  EJ_CHECK_ARG(lhs_coords && rhs_coords, "coordinate pointer is null");
  int bits = 0;
  EJ_TRY(key_bits(radices, n_keys, &bits));
  JoinWs w = carve_join(workspace, n_lhs, n_rhs, order);
  EJ_CHECK_ARG(workspace && workspace_bytes >= w.bytes, "workspace too small: %zu < %zu bytes",
               workspace_bytes, w.bytes);
  *dev_scalars = w.scalars;
  if (join_small_ok(order, n_lhs, n_rhs, bits)) {
    if (bits <= 32)
      hipLaunchKernelGGL(join_probe_small_kernel<true>, dim3(1), dim3(kJoinSmallThreads), 0,
                         stream, lhs_coords, static_cast<int>(n_lhs), lks, rhs_coords, n_rhs, rks,
                         bits, w.lperm, w.lo, w.offs, w.scalars, clear,
                         clear ? kClearScalars : 0, clear2, clear2 ? n_clear2 : 0);
    else
      hipLaunchKernelGGL(join_probe_small_kernel<false>, dim3(1), dim3(kJoinSmallThreads), 0,
                         stream, lhs_coords, static_cast<int>(n_lhs), lks, rhs_coords, n_rhs, rks,
                         bits, w.lperm, w.lo, w.offs, w.scalars, clear,
                         clear ? kClearScalars : 0, clear2, clear2 ? n_clear2 : 0);
    EJ_LAUNCH_CHECK();
    return EJ_OK;
  }

  EJ_TRY(zero_async(w.scalars, 4 * sizeof(int64_t), stream));
  if (clear) EJ_TRY(zero_async(clear, kClearScalars * sizeof(int64_t), stream));
  if (clear2) EJ_TRY(zero_async(clear2, n_clear2 * sizeof(int64_t), stream));
  int *bad = reinterpret_cast<int *>(w.scalars + 1);
  // Sorted sides are packed where an odd number of radix passes leaves them
  // in the primary buffers.
  const bool sort_rhs = order == EJ_ORDER_SORTED;
  const bool l_alt = n_lhs > 1 && (radix_passes(bits) & 1);
  const bool r_alt = sort_rhs && n_rhs > 1 && (radix_passes(bits) & 1);
  hipLaunchKernelGGL(pack_keys_kernel, dim3(grid_for(n_lhs + n_rhs)), dim3(kBlock), 0, stream,
                     lhs_coords, n_lhs, lks, l_alt ? w.lkeys_alt : w.lkeys,
                     l_alt ? w.lperm_alt : w.lperm, rhs_coords, n_rhs, rks,
                     r_alt ? w.rkeys_alt : w.rkeys,
                     sort_rhs ? (r_alt ? w.rperm_alt : w.rperm) : nullptr, bad);
  EJ_LAUNCH_CHECK();
  EJ_TRY(sort_pairs_u64(w.lkeys, w.lperm, w.lkeys_alt, w.lperm_alt, n_lhs, bits, w.sort_ws,
                        stream, l_alt));
  if (sort_rhs)
    EJ_TRY(sort_pairs_u64(w.rkeys, w.rperm, w.rkeys_alt, w.rperm_alt, n_rhs, bits, w.sort_ws,
                          stream, r_alt));
  const int64_t n_probe = sort_rhs ? n_lhs : n_rhs;
  const int64_t n_build = sort_rhs ? n_rhs : n_lhs;
  const uint64_t *probe = sort_rhs ? w.lkeys : w.rkeys;
  const uint64_t *build = sort_rhs ? w.rkeys : w.lkeys;
  if (n_probe <= kProbeSmallMax && n_build <= kProbeLdsKeys) {
    hipLaunchKernelGGL(probe_scan_small_kernel, dim3(1), dim3(kProbeThreads), 0, stream, probe,
                       n_probe, build, static_cast<int>(n_build), w.lo, w.offs, w.scalars);
    EJ_LAUNCH_CHECK();
  } else {
    hipLaunchKernelGGL(probe_count_kernel, dim3(grid_for(n_probe)), dim3(kBlock), 0, stream,
                       probe, n_probe, build, n_build, w.lo, w.cnt);
    EJ_LAUNCH_CHECK();
    EJ_TRY(scan_exclusive_i64(w.cnt, w.offs, n_probe, w.scalars, w.scan_ws, stream));
  }
  return EJ_OK;
}

}  // namespace
}  // namespace ej

extern "C" int ej_join_count(const int32_t *lhs_coords, int64_t n_lhs, int32_t lhs_ncols,
                             const int32_t *rhs_coords, int64_t n_rhs, int32_t rhs_ncols,
                             int32_t n_keys, const int32_t *lhs_dims, const int32_t *rhs_dims,
                             const int64_t *radices, int32_t order, void *workspace,
                             size_t workspace_bytes, int64_t *n_pairs, ej_stream_t stream_) {
  clear_error();
  hipStream_t stream = as_stream(stream_);
  EJ_CHECK_ARG(n_pairs, "n_pairs is null");
  int64_t known = -1;
  int64_t *scal = nullptr;
  EJ_TRY(join_count_enqueue(lhs_coords, n_lhs, lhs_ncols, rhs_coords, n_rhs, rhs_ncols, n_keys,
                            lhs_dims, rhs_dims, radices, order, workspace, workspace_bytes,
                            &known, &scal, stream));
  if (known >= 0) {
    *n_pairs = known;
    return EJ_OK;
  }
  int64_t host[2] = {0, 0};
  EJ_HIP(hipMemcpyAsync(host, scal, 2 * sizeof(int64_t), hipMemcpyDeviceToHost, stream));
  EJ_HIP(hipStreamSynchronize(stream));
  if (host[1] != 0) {
    set_error("a join-key coordinate lies outside [0, radix)");
    return EJ_E_RANGE;
  }
  *n_pairs = host[0];
  return EJ_OK;
}

extern "C" int ej_join_count_async(const int32_t *lhs_coords, int64_t n_lhs, int32_t lhs_ncols,
                                   const int32_t *rhs_coords, int64_t n_rhs, int32_t rhs_ncols,
                                   int32_t n_keys, const int32_t *lhs_dims,
                                   const int32_t *rhs_dims, const int64_t *radices,
                                   int32_t order, void *workspace, size_t workspace_bytes,
                                   int64_t *counts, ej_stream_t stream_) {
  clear_error();
  hipStream_t stream = as_stream(stream_);
  EJ_CHECK_ARG(counts, "counts is null");
  int64_t known = -1;
  int64_t *scal = nullptr;
  EJ_TRY(join_count_enqueue(lhs_coords, n_lhs, lhs_ncols, rhs_coords, n_rhs, rhs_ncols, n_keys,
                            lhs_dims, rhs_dims, radices, order, workspace, workspace_bytes,
                            &known, &scal, stream));
  if (known >= 0) {
    // Nothing was enqueued: hand the host-known count over in stream order
    // through the workspace so that device-side consumers see it too.
    JoinWs w = carve_join(workspace, n_lhs, n_rhs, order);
    EJ_CHECK_ARG(workspace && workspace_bytes >= w.bytes, "workspace too small");
    const int64_t v[2] = {known, 0};
    EJ_HIP(hipMemcpyAsync(w.scalars, v, sizeof(v), hipMemcpyHostToDevice, stream));
    scal = w.scalars;
  }
  EJ_HIP(hipMemcpyAsync(counts, scal, 2 * sizeof(int64_t), hipMemcpyDeviceToHost, stream));
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

// scal[2] receives the live pair count (n clipped by *n_dev).
__global__ void pair_keys_kernel(const int32_t *lc, const int32_t *rc, const int64_t *li,
                                 const int64_t *ri, int64_t n, const int64_t *n_dev, AggSpec a,
                                 uint64_t *keys, int32_t *perm, int64_t *scal) {
  n = live_count(n, n_dev);
  int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (p == 0) scal[2] = n;
  int *bad = reinterpret_cast<int *>(scal + 1);
  if (p >= n) return;
  perm[p] = static_cast<int32_t>(p);
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

// EJ_ORDER_PROBE fill that also forms each pair's output key for the segment
// sort (what pair_keys_kernel does for caller-supplied pairs): writes li, ri,
// keys and perm = q for q < n = min(P, cap).  Thread 0 stores n as the plan's
// live pair count (sscal[2]) and copies P and the join's range flag to
// sscal[4..5], next to the plan's counts, so that one copy returns them all.
// hist (optional, zeroed): the sort's first-pass digit histogram, block-major
// over sort blocks of `tile` keys (a multiple of the block size, so each
// block's pairs fall in one sort block), counted here in LDS and added once
// per digit.  WIDE: instead, whist (zeroed, int32) counts every key value
// (keys below wk = 2^bits <= kOnePassMaxKeys) per block of kOnePassTile
// pairs, for the one-pass plan, and perm is not written (the plan uses the
// pair index itself).
constexpr int kOnePassMaxBits = 12;
constexpr int kOnePassMaxKeys = 1 << kOnePassMaxBits;
constexpr int kOnePassThreads = 512;
constexpr int kOnePassItems = 8;  // rounds of 64 pairs per wave
constexpr int64_t kOnePassTile = static_cast<int64_t>(kOnePassThreads) * kOnePassItems;
constexpr int64_t kOnePassMaxBlocks = 8;

template <bool WIDE>
__global__ __launch_bounds__(kBlock) void fill_probe_keys_kernel(
    const int64_t *offs, int64_t n_rhs, const int64_t *lo, const int32_t *lhs_perm, int64_t cap,
    const int64_t *jscal, const int32_t *lc, const int32_t *rc, AggSpec a, int64_t *lhs_idx,
    int64_t *rhs_idx, uint64_t *keys, int32_t *perm, int64_t *sscal, int64_t *hist,
    int64_t tile, int32_t *whist, int wk) {
  __shared__ int digit_count[WIDE ? kOnePassMaxKeys : 256];
  const int64_t P = jscal[0];
  const int64_t n = P < cap ? P : cap;
  const int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (q == 0) {
    sscal[2] = n;
    sscal[4] = P;
    sscal[5] = jscal[1];
  }
  if constexpr (WIDE) {
    for (int d = threadIdx.x; d < wk; d += kBlock) digit_count[d] = 0;
    __syncthreads();
  } else if (hist) {
    digit_count[threadIdx.x] = 0;
    __syncthreads();
  }
  if (q < n) {
    const int64_t j = owner_of(offs, n_rhs, q);
    const int64_t l = lhs_perm[lo[j] + (q - offs[j])];
    lhs_idx[q] = l;
    rhs_idx[q] = j;
    if constexpr (!WIDE) perm[q] = static_cast<int32_t>(q);
    const int32_t *lrow = lc + l * a.lncols;
    const int32_t *rrow = rc + j * a.rncols;
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
    keys[q] = key;
    if (b) atomicOr(reinterpret_cast<int *>(sscal + 1), 1);
    if constexpr (WIDE) atomicAdd(&digit_count[key], 1);
    else if (hist) atomicAdd(&digit_count[key & 255], 1);
  }
  if constexpr (WIDE) {
    __syncthreads();
    const int64_t sb = static_cast<int64_t>(blockIdx.x) * kBlock / kOnePassTile;
    for (int d = threadIdx.x; d < wk; d += kBlock) {
      const int c = digit_count[d];
      if (c) atomicAdd(whist + sb * wk + d, c);
    }
  } else if (hist) {
    __syncthreads();
    const int c = digit_count[threadIdx.x];
    if (c) {
      const int64_t sb = static_cast<int64_t>(blockIdx.x) * blockDim.x / tile;
      atomicAdd(reinterpret_cast<unsigned long long *>(hist + sb * 256 + threadIdx.x),
                static_cast<unsigned long long>(c));
    }
  }
}

// One-pass segment plan for output keys of at most kOnePassMaxBits bits and
// at most kOnePassMaxBlocks * kOnePassTile pairs: the key is a single radix
// digit, so one stable counting sort orders the pairs, and the key histogram
// (whist, per block of kOnePassTile pairs, from the pair fill) also gives the
// segments: segment u is the u-th key value that occurs, starting at that
// value's first sorted position.  Every block derives the sorted start of
// each key value for its own pairs: counts of the earlier blocks (all
// histogram rows read at once, each thread's loads independent) plus an
// exclusive scan of the totals.  Each wave then ranks its own contiguous
// eighth of the block's pairs (keys loaded up front) in rounds of 64 with
// ballot peer masks and a wave-private count per key value in LDS, with no
// workgroup barrier; the waves' totals give their offsets, and every pair
// lands at key start + earlier waves' counts + its rank.  The blocks share
// writing the segments (seg_offsets, out_coords decoded by the radices);
// block 0 stores U = sscal[0] and the end offset, and, given host_counts
// (coherent host memory), the six counts there, then the caller's ticket in
// host_counts[6], each step fenced at system scope, so that a host that sees
// the ticket sees the counts.  perm receives the pair indices in sorted order.
// Given run_order, the blocks also write the order in which a grouped einsum
// (groups of `group` consecutive segments, one workgroup each) should run
// the ngroups = ceil(min(U, seg_cap) / group) live groups, into
// run_order[1 .. ngroups], with ngroups in run_order[0]: the workgroups of each XCD
// (the contiguous chunks that the einsum's XCD mapping assigns to the live
// workgroups) take their chunk's groups in descending pair count (counts
// above 255 tie), ties by index, so that the longest groups start first.  Chunk x is ordered by wave x of block x % nblocks: a counting
// sort over the 256 count classes, ranked in index order with ballots.
__global__ __launch_bounds__(kOnePassThreads) void plan_one_pass_kernel(
    const uint64_t *__restrict__ keys, const int32_t *__restrict__ whist, int64_t nblocks,
    int wk, int bits, AggSpec a, int64_t seg_cap, int32_t *__restrict__ perm,
    int32_t *__restrict__ seg_offsets, int32_t *__restrict__ out_coords,
    int64_t *__restrict__ sscal, int64_t *__restrict__ host_counts, int64_t ticket,
    int group, int32_t *__restrict__ run_order) {
  constexpr int NT = kOnePassThreads, NW = NT / 64;
  constexpr int DPT = kOnePassMaxKeys / NT;          // key values per thread
  constexpr int RPW = kOnePassItems;                  // rounds of 64 per wave
  constexpr int64_t WSPAN = static_cast<int64_t>(RPW) * 64;  // pairs per wave
  __shared__ int32_t base_off[kOnePassMaxKeys];
  __shared__ int32_t seg_rank[kOnePassMaxKeys];
  __shared__ uint16_t wcnt[NW][kOnePassMaxKeys];
  __shared__ int32_t seglen[kOnePassMaxKeys];  // pairs of segment u (run order only)
  __shared__ int32_t cls_base[NW][256];         // per-wave count-class offsets (run order)
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  (void)bits;  // ranks compare all kOnePassMaxBits bits (the keys lie below 2^bits)
  const int64_t n = sscal[2];
  const int64_t blk = blockIdx.x;
  const int64_t wbase = blk * kOnePassTile + wave * WSPAN;
  uint32_t kk[RPW];  // this lane's keys, loaded before anything waits
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const int64_t i = wbase + r * 64 + lane;
    kk[r] = i < n ? static_cast<uint32_t>(keys[i]) : 0u;
  }
  int32_t c[kOnePassMaxBlocks][DPT];
#pragma unroll
  for (int b = 0; b < kOnePassMaxBlocks; ++b)
#pragma unroll
    for (int j = 0; j < DPT; ++j) {
      const int d = tid + j * NT;
      c[b][j] = b < nblocks && d < wk ? whist[b * wk + d] : 0;
    }
  for (int x = tid; x < NW * kOnePassMaxKeys / 2; x += NT)
    reinterpret_cast<uint32_t *>(&wcnt[0][0])[x] = 0u;
#pragma unroll
  for (int j = 0; j < DPT; ++j) {
    int32_t tot = 0, before = 0;
#pragma unroll
    for (int b = 0; b < kOnePassMaxBlocks; ++b) {
      tot += c[b][j];
      before += b < blk ? c[b][j] : 0;
    }
    const int d = tid + j * NT;
    if (d < wk) {
      base_off[d] = tot;
      seg_rank[d] = before;
    }
  }
  __syncthreads();
  // Exclusive scans over the key values, each thread a contiguous run:
  // sorted start (from totals) and segment rank (from totals > 0).
  const int per = (wk + NT - 1) / NT;
  const int d0 = min(wk, tid * per), d1 = min(wk, d0 + per);
  // Both prefixes in one scan: pair count (< 2^31) high, segment count low.
  int64_t sum_tf = 0;
  for (int d = d0; d < d1; ++d) sum_tf += (int64_t(base_off[d]) << 20) + (base_off[d] > 0 ? 1 : 0);
  int64_t all_tf;
  const int64_t run_tf = block_exclusive_sum<NT>(sum_tf, &all_tf);
  int64_t run_t = run_tf >> 20, run_f = run_tf & ((int64_t(1) << 20) - 1);
  const int64_t all_f = all_tf & ((int64_t(1) << 20) - 1);
  const bool order = run_order && group > 0;
  for (int d = d0; d < d1; ++d) {
    const int32_t t = base_off[d], bf = seg_rank[d];
    if (order && t > 0) seglen[run_f] = t;
    if (t > 0 && run_f < seg_cap && (static_cast<int64_t>(d) * nblocks) / wk == blk) {
      seg_offsets[run_f] = static_cast<int32_t>(run_t);
      uint32_t key = static_cast<uint32_t>(d);
      for (int cc = a.n - 1; cc >= 0; --cc) {
        const uint32_t rad = static_cast<uint32_t>(a.radix[cc]);
        out_coords[run_f * a.n + cc] = static_cast<int32_t>(key % rad);
        key /= rad;
      }
    }
    base_off[d] = static_cast<int32_t>(run_t) + bf;
    run_t += t;
    run_f += t > 0 ? 1 : 0;
  }
  if (blk == 0 && tid == 0) {
    sscal[0] = all_f;
    if (all_f <= seg_cap) seg_offsets[all_f] = static_cast<int32_t>(n);
    if (host_counts) {
      host_counts[0] = all_f;
      host_counts[1] = sscal[1];
      host_counts[2] = n;
      host_counts[3] = 0;
      host_counts[4] = sscal[4];
      host_counts[5] = sscal[5];
      __threadfence_system();
      host_counts[6] = ticket;
      __threadfence_system();
    }
  }
  if (order) {
    // Group pair counts (segments beyond U count 0), then per XCD chunk a
    // stable counting sort of its groups by descending count class.
    __syncthreads();
    const int64_t live_segs = all_f < seg_cap ? all_f : seg_cap;
    const int64_t ngroups = (live_segs + group - 1) / group;  // <= kOnePassMaxKeys
    int32_t *glen = seg_rank;  // reused: no longer read
    for (int64_t g = tid; g < ngroups; g += NT) {
      int32_t sum = 0;
      for (int u = 0; u < group; ++u) {
        const int64_t seg = g * group + u;
        sum += seg < all_f ? seglen[seg] : 0;
      }
      glen[g] = sum;
    }
    for (int x = lane; x < 256; x += 64) cls_base[wave][x] = 0;
    if (blk == 0 && tid == 0) run_order[0] = static_cast<int32_t>(ngroups);  // the header
    __syncthreads();
    const int64_t x = wave;
    if (x % nblocks == blk) {
      const int64_t per = ngroups / 8, rem = ngroups % 8;
      const int64_t start = x < rem ? x * (per + 1) : rem * (per + 1) + (x - rem) * per;
      const int64_t cnt = per + (x < rem ? 1 : 0);
      auto cls = [&](int64_t i) { return 255 - min(glen[start + i], 255); };
      for (int64_t i = lane; i < cnt; i += 64) atomicAdd(&cls_base[wave][cls(i)], 1);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      // exclusive prefix over the 256 classes, 4 per lane
      int v[4], sum = 0;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        v[u] = cls_base[wave][lane * 4 + u];
        sum += v[u];
      }
      int inc = sum;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(inc, o);
        if (lane >= o) inc += t;
      }
      int run = inc - sum;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        cls_base[wave][lane * 4 + u] = run;
        run += v[u];
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      const uint64_t lt = lane == 0 ? 0ull : (~0ull >> (64 - lane));
      for (int64_t i0 = 0; i0 < cnt; i0 += 64) {
        const int64_t i = i0 + lane;
        const bool valid = i < cnt;
        const int c = valid ? cls(i) : 0;
        uint64_t peers = __ballot(valid);
#pragma unroll
        for (int b = 0; b < 8; ++b) {
          const int bit = (c >> b) & 1;
          const uint64_t m = __ballot(bit);
          peers &= bit ? m : ~m;
        }
        asm volatile("" ::: "memory");
        const int base = valid ? cls_base[wave][c] : 0;
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (valid)
          run_order[1 + start + base + __popcll(peers & lt)] = static_cast<int32_t>(start + i);
        if (valid && (peers & lt) == 0) cls_base[wave][c] = base + __popcll(peers);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      }
    }
  }
  // Wave-local stable ranks: rounds of 64 consecutive pairs; the lanes of a
  // key value read its running count, then its first lane adds the round's
  // count.  LDS operations of one wave execute in order; the waits and
  // compiler barriers keep them in program order.
  const uint64_t lt_mask = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  uint16_t rank[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const bool valid = wbase + r * 64 + lane < n;
    const int d = static_cast<int>(kk[r]);
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int b = 0; b < kOnePassMaxBits; ++b) {  // keys lie below 2^bits <= 2^kOnePassMaxBits
      const int bit = (d >> b) & 1;
      const uint64_t m = __ballot(bit);
      peers &= bit ? m : ~m;
    }
    asm volatile("" ::: "memory");
    const int run = valid ? wcnt[wave][d] : 0;
    rank[r] = static_cast<uint16_t>(run + __popcll(peers & lt_mask));
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if (valid && (peers & lt_mask) == 0)
      wcnt[wave][d] = static_cast<uint16_t>(run + __popcll(peers));
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const int64_t i = wbase + r * 64 + lane;
    if (i < n) {
      const int d = static_cast<int>(kk[r]);
      int pos = base_off[d] + rank[r];
      for (int w = 0; w < wave; ++w) pos += wcnt[w][d];
      if (pos < n) perm[pos] = static_cast<int32_t>(i);
    }
  }
}

// Copies the plan's six counts into coherent host memory and then stores the
// caller's ticket after them, fenced at system scope (one launch in place of
// a copy and the ticket kernel).
__global__ void publish_counts_kernel(const int64_t *__restrict__ scalars,
                                      int64_t *__restrict__ host_counts, int64_t ticket) {
  if (threadIdx.x < 6) host_counts[threadIdx.x] = scalars[threadIdx.x];
  __threadfence_system();
  __syncthreads();
  if (threadIdx.x == 0) {
    host_counts[6] = ticket;
    __threadfence_system();
  }
}

__global__ void seg_flags_kernel(const uint64_t *skeys, int64_t n, const int64_t *n_dev,
                                 int64_t *flags) {
  n = live_count(n, n_dev);
  int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (q >= n) return;
  flags[q] = (q == 0 || skeys[q] != skeys[q - 1]) ? 1 : 0;
}

// Segment-start flag of sorted position q, generated inside the scan.
struct SegFlagLoad {
  const uint64_t *skeys;
  __device__ int64_t operator()(int64_t q) const {
    return (q == 0 || skeys[q] != skeys[q - 1]) ? 1 : 0;
  }
};

struct StoreFlag {
  int64_t *flags;
  __device__ void operator()(int64_t q, int64_t f, int64_t, int64_t) const { flags[q] = f; }
};

// The segment fill done inside the flag scan (seg_fill_kernel's writes for
// sorted position q, whose segment is prefix + flag - 1): perm, the start
// offset and the coordinates of each segment below the capacity, and the
// end offset after the last segment.
struct SegFillEmit {
  const uint64_t *skeys;
  const int32_t *sperm;
  AggSpec a;
  int64_t cap;
  int32_t *out_coords, *seg_offsets, *perm;
  __device__ void operator()(int64_t q, int64_t f, int64_t prefix, int64_t n) const {
    perm[q] = sperm[q];
    const int64_t seg = prefix + f - 1;
    if (f && seg < cap) {
      seg_offsets[seg] = static_cast<int32_t>(q);
      uint64_t key = skeys[q];
      for (int d = a.n - 1; d >= 0; --d) {
        const uint64_t r = static_cast<uint64_t>(a.radix[d]);
        out_coords[seg * a.n + d] = static_cast<int32_t>(key % r);
        key /= r;
      }
    }
    if (q == n - 1 && seg < cap) seg_offsets[seg + 1] = static_cast<int32_t>(n);
  }
};

// dev_counts (optional): the workspace scalars; the live pair count is
// dev_counts[2] and the segment count dev_counts[0] (then n_seg is the
// capacity of out_coords / seg_offsets).
__global__ void seg_fill_kernel(const uint64_t *skeys, const int32_t *sperm, const int64_t *flags,
                                const int64_t *excl, int64_t n, int64_t n_seg,
                                const int64_t *dev_counts, AggSpec a, int32_t *out_coords,
                                int32_t *seg_offsets, int32_t *perm, int32_t *seg_ids) {
  if (dev_counts) {
    n = live_count(n, dev_counts + 2);
    const int64_t u = dev_counts[0];
    if (u > n_seg) return;  // capacity exceeded: the host sees the count and rejects
    n_seg = u;
  }
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
  int64_t *scalars;  // [0] = U, [1] = bad flag, [2] = live pairs; 8 slots
  uint64_t *keys, *keys_alt;
  int32_t *perm, *perm_alt;
  int64_t *flags, *excl;
  int32_t *whist;  // one-pass plan key histogram (pair counts up to the one-pass limit)
  void *sort_ws, *scan_ws;
  size_t bytes;
};

int64_t one_pass_blocks(int64_t n) { return ceil_div(n, kOnePassTile); }

SegWs carve_seg(void *base, int64_t n) {
  Carver c(base);
  SegWs w;
  w.scalars = c.take<int64_t>(kClearScalars);
  w.keys = c.take<uint64_t>(n);
  w.keys_alt = c.take<uint64_t>(n);
  w.perm = c.take<int32_t>(n);
  w.perm_alt = c.take<int32_t>(n);
  w.flags = c.take<int64_t>(n);
  w.excl = c.take<int64_t>(n);
  const int64_t nb = one_pass_blocks(n);
  w.whist = c.take<int32_t>(nb <= kOnePassMaxBlocks ? nb * kOnePassMaxKeys : 0);
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

namespace ej {
namespace {

// Segment flags of the sorted keys and their exclusive scan (w.flags, w.excl);
// U lands in w.scalars[0].
int segment_scan_enqueue(const SegWs &w, int64_t n_pairs, const int64_t *live,
                         hipStream_t stream) {
  if (n_pairs <= kFastScanMax) {
    launch_fast_scan(SegFlagLoad{w.keys}, StoreFlag{w.flags}, n_pairs, live,
                     static_cast<int64_t *>(w.scan_ws), w.excl, w.scalars, stream);
    EJ_LAUNCH_CHECK();
  } else {
    hipLaunchKernelGGL(seg_flags_kernel, dim3(grid_for(n_pairs)), dim3(kBlock), 0, stream, w.keys,
                       n_pairs, live, w.flags);
    EJ_LAUNCH_CHECK();
    EJ_TRY(scan_exclusive_i64(w.flags, w.excl, n_pairs, w.scalars, w.scan_ws, stream, live));
  }
  return EJ_OK;
}

// Enqueues the segment count; *known_empty on return: no pairs, nothing
// enqueued.  Otherwise U and a range flag land in w.scalars[0..1] and the
// live pair count in w.scalars[2].
int segment_count_enqueue(const int32_t *lhs_coords, int64_t n_lhs, int32_t lhs_ncols,
                          const int32_t *rhs_coords, int64_t n_rhs, int32_t rhs_ncols,
                          const int64_t *lhs_idx, const int64_t *rhs_idx, int64_t n_pairs,
                          const int64_t *n_pairs_dev, int32_t n_out, const int32_t *agg_src,
                          const int32_t *agg_dim, const int64_t *radices, void *workspace,
                          size_t workspace_bytes, bool *known_empty, int64_t **dev_scalars,
                          hipStream_t stream) {
  *known_empty = false;
  EJ_CHECK_ARG(n_pairs >= 0 && n_pairs < (int64_t(1) << 31), "n_pairs must lie in [0, 2^31)");
  EJ_CHECK_ARG(radices || n_out == 0, "radices is null");
  AggSpec a;
  EJ_TRY(check_agg(n_out, agg_src, agg_dim, n_lhs, lhs_ncols, n_rhs, rhs_ncols, radices, &a));
  if (n_pairs == 0) {
    *known_empty = true;
    return EJ_OK;
  }
  EJ_CHECK_ARG(lhs_coords && rhs_coords && lhs_idx && rhs_idx, "null pointer argument");
  int bits = 0;
  EJ_TRY(key_bits(a.radix, n_out, &bits));
  SegWs w = carve_seg(workspace, n_pairs);
  EJ_CHECK_ARG(workspace && workspace_bytes >= w.bytes, "workspace too small: %zu < %zu bytes",
               workspace_bytes, w.bytes);
  *dev_scalars = w.scalars;
  EJ_TRY(zero_async(w.scalars, 4 * sizeof(int64_t), stream));
  const bool alt = n_pairs > 1 && (radix_passes(bits) & 1);
  hipLaunchKernelGGL(pair_keys_kernel, dim3(grid_for(n_pairs)), dim3(kBlock), 0, stream,
                     lhs_coords, rhs_coords, lhs_idx, rhs_idx, n_pairs, n_pairs_dev, a,
                     alt ? w.keys_alt : w.keys, alt ? w.perm_alt : w.perm, w.scalars);
  EJ_LAUNCH_CHECK();
  // From here on the live pair count is w.scalars[2] (n_pairs clipped).
  const int64_t *live = n_pairs_dev ? w.scalars + 2 : nullptr;
  EJ_TRY(sort_pairs_u64(w.keys, w.perm, w.keys_alt, w.perm_alt, n_pairs, bits, w.sort_ws, stream,
                        alt, live));
  return segment_scan_enqueue(w, n_pairs, live, stream);
}

}  // namespace
}  // namespace ej

extern "C" int ej_segment_count(const int32_t *lhs_coords, int64_t n_lhs, int32_t lhs_ncols,
                                const int32_t *rhs_coords, int64_t n_rhs, int32_t rhs_ncols,
                                const int64_t *lhs_idx, const int64_t *rhs_idx, int64_t n_pairs,
                                int32_t n_out, const int32_t *agg_src, const int32_t *agg_dim,
                                const int64_t *radices, void *workspace, size_t workspace_bytes,
                                int64_t *n_segments, ej_stream_t stream_) {
  clear_error();
  hipStream_t stream = as_stream(stream_);
  EJ_CHECK_ARG(n_segments, "n_segments is null");
  bool empty = false;
  int64_t *scal = nullptr;
  EJ_TRY(segment_count_enqueue(lhs_coords, n_lhs, lhs_ncols, rhs_coords, n_rhs, rhs_ncols,
                               lhs_idx, rhs_idx, n_pairs, nullptr, n_out, agg_src, agg_dim,
                               radices, workspace, workspace_bytes, &empty, &scal, stream));
  if (empty) {
    *n_segments = 0;
    return EJ_OK;
  }
  int64_t host[2] = {0, 0};
  EJ_HIP(hipMemcpyAsync(host, scal, 2 * sizeof(int64_t), hipMemcpyDeviceToHost, stream));
  EJ_HIP(hipStreamSynchronize(stream));
  if (host[1] != 0) {
    set_error("a pair index or an output coordinate lies outside [0, radix)");
    return EJ_E_RANGE;
  }
  *n_segments = host[0];
  return EJ_OK;
}

extern "C" int ej_segment_count_async(const int32_t *lhs_coords, int64_t n_lhs,
                                      int32_t lhs_ncols, const int32_t *rhs_coords,
                                      int64_t n_rhs, int32_t rhs_ncols, const int64_t *lhs_idx,
                                      const int64_t *rhs_idx, int64_t n_pairs,
                                      const int64_t *n_pairs_dev, int32_t n_out,
                                      const int32_t *agg_src, const int32_t *agg_dim,
                                      const int64_t *radices, void *workspace,
                                      size_t workspace_bytes, int64_t *counts,
                                      ej_stream_t stream_) {
  clear_error();
  hipStream_t stream = as_stream(stream_);
  EJ_CHECK_ARG(counts, "counts is null");
  bool empty = false;
  int64_t *scal = nullptr;
  EJ_TRY(segment_count_enqueue(lhs_coords, n_lhs, lhs_ncols, rhs_coords, n_rhs, rhs_ncols,
                               lhs_idx, rhs_idx, n_pairs, n_pairs_dev, n_out, agg_src, agg_dim,
                               radices, workspace, workspace_bytes, &empty, &scal, stream));
  if (empty) {
    SegWs w = carve_seg(workspace, 0);
    EJ_CHECK_ARG(workspace && workspace_bytes >= w.bytes, "workspace too small");
    EJ_TRY(zero_async(w.scalars, 4 * sizeof(int64_t), stream));
    scal = w.scalars;
  }
  EJ_HIP(hipMemcpyAsync(counts, scal, 2 * sizeof(int64_t), hipMemcpyDeviceToHost, stream));
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
    if (seg_offsets) EJ_TRY(zero_async(seg_offsets, sizeof(int32_t), stream));
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
                     w.perm, w.flags, w.excl, n_pairs, n_segments, nullptr, a, out_coords,
                     seg_offsets, perm, seg_ids);
  EJ_LAUNCH_CHECK();
  return EJ_OK;
}

extern "C" int ej_segment_fill_async(int64_t n_pairs, int32_t n_out, const int64_t *radices,
                                     const void *workspace, size_t workspace_bytes,
                                     int32_t *out_coords, int32_t *seg_offsets, int32_t *perm,
                                     int32_t *seg_ids, int64_t capacity, ej_stream_t stream_) {
  clear_error();
  hipStream_t stream = as_stream(stream_);
  EJ_CHECK_ARG(n_pairs >= 0 && capacity >= 0, "bad sizes");
  if (n_pairs == 0) return EJ_OK;
  EJ_CHECK_ARG(seg_offsets && perm && (out_coords || n_out == 0), "null output pointer");
  EJ_CHECK_ARG(n_out >= 0 && n_out <= EJ_MAX_KEYS && (radices || n_out == 0), "bad n_out");
  AggSpec a;
  a.n = n_out;
  for (int d = 0; d < n_out; ++d) a.radix[d] = radices[d];
  SegWs w = carve_seg(const_cast<void *>(workspace), n_pairs);
  EJ_CHECK_ARG(workspace && workspace_bytes >= w.bytes, "workspace too small");
  hipLaunchKernelGGL(seg_fill_kernel, dim3(grid_for(n_pairs)), dim3(kBlock), 0, stream, w.keys,
                     w.perm, w.flags, w.excl, n_pairs, capacity, w.scalars, a, out_coords,
                     seg_offsets, perm, seg_ids);
  EJ_LAUNCH_CHECK();
  return EJ_OK;
}

namespace ej {
namespace {

// The queued pair plan on caller-supplied workspaces (ej_pair_plan_async) or
// on the library's static scratch (ej_pair_plan_async_noalloc).
int pair_plan_impl(const int32_t *lhs_coords, int64_t n_lhs, int32_t lhs_ncols,
                   const int32_t *rhs_coords, int64_t n_rhs, int32_t rhs_ncols, int32_t n_keys,
                   const int32_t *lhs_dims, const int32_t *rhs_dims, const int64_t *join_radices,
                   int32_t n_out, const int32_t *agg_src, const int32_t *agg_dim,
                   const int64_t *agg_radices, int64_t pair_capacity, void *join_workspace,
                   size_t join_workspace_bytes, void *seg_workspace, size_t seg_workspace_bytes,
                   int64_t *lhs_idx, int64_t *rhs_idx, int32_t *out_coords,
                   int32_t *seg_offsets, int32_t *perm, int64_t seg_capacity, int32_t group,
                   int32_t *run_order, int32_t *run_order_written, int64_t *counts,
                   int32_t counts_direct, hipStream_t stream) {
  EJ_CHECK_ARG(counts && lhs_idx && rhs_idx && seg_offsets && perm &&
                   (out_coords || n_out == 0),
               "null pointer argument");
  EJ_CHECK_ARG(seg_capacity >= 0, "negative seg_capacity");
  EJ_CHECK_ARG(group >= 0, "negative group");
  EJ_CHECK_ARG(n_keys >= 1 && n_lhs >= 1 && n_rhs >= 1,
               "the queued pair plan needs join keys and two non-empty relations");
  EJ_CHECK_ARG(pair_capacity >= 1 && pair_capacity < (int64_t(1) << 31),
               "pair_capacity must lie in [1, 2^31)");
  EJ_CHECK_ARG(agg_radices || n_out == 0, "agg_radices is null");
  AggSpec a;
  EJ_TRY(check_agg(n_out, agg_src, agg_dim, n_lhs, lhs_ncols, n_rhs, rhs_ncols, agg_radices, &a));
  int sbits = 0;
  EJ_TRY(key_bits(a.radix, n_out, &sbits));
  SegWs sw = carve_seg(seg_workspace, pair_capacity);
  EJ_CHECK_ARG(seg_workspace && seg_workspace_bytes >= sw.bytes,
               "segment workspace too small: %zu < %zu bytes", seg_workspace_bytes, sw.bytes);
  int jbits = 0;
  EJ_TRY(key_bits(join_radices, n_keys, &jbits));
  const bool small_join = join_small_ok(EJ_ORDER_PROBE, n_lhs, n_rhs, jbits);
  JoinWs jw = carve_join(join_workspace, n_lhs, n_rhs, EJ_ORDER_PROBE);
  EJ_CHECK_ARG(counts_direct >= 0, "negative counts_direct");
  int64_t *direct = nullptr;  // device address of counts when the kernels store them
  if (counts_direct)
    EJ_HIP(hipHostGetDevicePointer(reinterpret_cast<void **>(&direct), counts, 0));
  int64_t known = -1;
  int64_t *jscal = nullptr;
  // Output keys of at most kOnePassMaxBits bits: one counting-sort pass that
  // also yields the segments (the join count clears its histogram).
  const int64_t nb1 = one_pass_blocks(pair_capacity);
  if (small_join && sbits >= 1 && sbits <= kOnePassMaxBits && nb1 <= kOnePassMaxBlocks) {
    const int wk = 1 << sbits;
    EJ_TRY(join_count_enqueue(lhs_coords, n_lhs, lhs_ncols, rhs_coords, n_rhs, rhs_ncols, n_keys,
                              lhs_dims, rhs_dims, join_radices, EJ_ORDER_PROBE, join_workspace,
                              join_workspace_bytes, &known, &jscal, stream, sw.scalars,
                              reinterpret_cast<int64_t *>(sw.whist),
                              static_cast<int>(nb1 * wk / 2)));
    EJ_CHECK_ARG(known < 0, "internal: join size known on the host");
    hipLaunchKernelGGL(fill_probe_keys_kernel<true>, dim3(grid_for(pair_capacity)), dim3(kBlock),
                       0, stream, jw.offs, n_rhs, jw.lo, jw.lperm, pair_capacity, jw.scalars,
                       lhs_coords, rhs_coords, a, lhs_idx, rhs_idx, sw.keys, nullptr, sw.scalars,
                       nullptr, int64_t(0), sw.whist, wk);
    EJ_LAUNCH_CHECK();
    // Run order for grouped einsums: groups of up to kOnePassMaxKeys segments.
    const bool order = run_order && group > 0 && seg_capacity <= kOnePassMaxKeys;
    hipLaunchKernelGGL(plan_one_pass_kernel, dim3(static_cast<unsigned>(nb1)),
                       dim3(kOnePassThreads), 0,
                       stream, sw.keys, sw.whist, nb1, wk, sbits, a, seg_capacity, perm,
                       seg_offsets, out_coords, sw.scalars, direct, int64_t(counts_direct),
                       order ? group : 0, order ? run_order : nullptr);
    EJ_LAUNCH_CHECK();
    if (order && run_order_written) *run_order_written = 1;
    if (!direct)
      EJ_HIP(hipMemcpyAsync(counts, sw.scalars, 6 * sizeof(int64_t), hipMemcpyDeviceToHost,
                            stream));
    return EJ_OK;
  }
  // The fill also counts the sort's first-pass digits when the join count
  // (one workgroup) can clear that histogram and the sort reads it inline.
  const SortTiling st = sort_tiling(pair_capacity);
  const bool fill_hist = pair_capacity > 1 && sbits > 0 && st.inline_offsets && small_join;
  int64_t *hist = fill_hist ? static_cast<int64_t *>(sw.sort_ws) : nullptr;
  EJ_TRY(join_count_enqueue(lhs_coords, n_lhs, lhs_ncols, rhs_coords, n_rhs, rhs_ncols, n_keys,
                            lhs_dims, rhs_dims, join_radices, EJ_ORDER_PROBE, join_workspace,
                            join_workspace_bytes, &known, &jscal, stream, sw.scalars, hist,
                            static_cast<int>(st.nblocks * 256)));
  EJ_CHECK_ARG(known < 0, "internal: join size known on the host");
  const bool alt = pair_capacity > 1 && (radix_passes(sbits) & 1);
  hipLaunchKernelGGL(fill_probe_keys_kernel<false>, dim3(grid_for(pair_capacity)), dim3(kBlock),
                     0, stream, jw.offs, n_rhs, jw.lo, jw.lperm, pair_capacity, jw.scalars,
                     lhs_coords, rhs_coords, a, lhs_idx, rhs_idx, alt ? sw.keys_alt : sw.keys,
                     alt ? sw.perm_alt : sw.perm, sw.scalars, hist, st.tile, nullptr, 0);
  EJ_LAUNCH_CHECK();
  const int64_t *live = sw.scalars + 2;
  EJ_TRY(sort_pairs_u64(sw.keys, sw.perm, sw.keys_alt, sw.perm_alt, pair_capacity, sbits,
                        sw.sort_ws, stream, alt, live, fill_hist));
  // Segment flags, their scan and the segment fill: one pass inside the scan
  // for up to kFastScanMax pairs.
  if (pair_capacity <= kFastScanMax) {
    launch_fast_scan(SegFlagLoad{sw.keys},
                     SegFillEmit{sw.keys, sw.perm, a, seg_capacity, out_coords, seg_offsets, perm},
                     pair_capacity, live, static_cast<int64_t *>(sw.scan_ws), nullptr,
                     sw.scalars, stream);
    EJ_LAUNCH_CHECK();
  } else {
    EJ_TRY(segment_scan_enqueue(sw, pair_capacity, live, stream));
    hipLaunchKernelGGL(seg_fill_kernel, dim3(grid_for(pair_capacity)), dim3(kBlock), 0, stream,
                       sw.keys, sw.perm, sw.flags, sw.excl, pair_capacity, seg_capacity,
                       sw.scalars, a, out_coords, seg_offsets, perm, nullptr);
    EJ_LAUNCH_CHECK();
  }
  if (direct) {  // counts and then the ticket, stored by the device
    hipLaunchKernelGGL(publish_counts_kernel, dim3(1), dim3(64), 0, stream, sw.scalars, direct,
                       int64_t(counts_direct));
    EJ_LAUNCH_CHECK();
  } else {
    EJ_HIP(hipMemcpyAsync(counts, sw.scalars, 6 * sizeof(int64_t), hipMemcpyDeviceToHost,
                          stream));
  }
  return EJ_OK;
}

// Static scratch of the allocation-free plan: the join workspace and the
// segment workspace of one call, carved from one device array that every
// GPU holds (its own copy) from the library's load to the end of the
// process.  The array's name is a host-side stand-in: kernels receive its
// device address, looked up once per device with hipGetSymbolAddress.
constexpr size_t kNoAllocScratchBytes = size_t(64) << 20;
constexpr int kNoAllocMaxDevices = 64;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

std::mutex g_scratch_mu;
void *g_scratch_ptr[kNoAllocMaxDevices];  // device address of scratch, per device

int scratch_base(void **base) {
  int dev = -1;
  EJ_HIP(hipGetDevice(&dev));
  EJ_CHECK_ARG(dev >= 0 && dev < kNoAllocMaxDevices, "device %d beyond the %d supported", dev,
               kNoAllocMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      set_error("hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                hipGetErrorString(e));
      return EJ_E_HIP;
    }
    g_scratch_ptr[dev] = p;
  }
  *base = g_scratch_ptr[dev];
  return EJ_OK;
}

}  // namespace
}  // namespace ej

extern "C" int ej_pair_plan_async(const int32_t *lhs_coords, int64_t n_lhs, int32_t lhs_ncols,
                                  const int32_t *rhs_coords, int64_t n_rhs, int32_t rhs_ncols,
                                  int32_t n_keys, const int32_t *lhs_dims,
                                  const int32_t *rhs_dims, const int64_t *join_radices,
                                  int32_t n_out, const int32_t *agg_src, const int32_t *agg_dim,
                                  const int64_t *agg_radices, int64_t pair_capacity,
                                  void *join_workspace, size_t join_workspace_bytes,
                                  void *seg_workspace, size_t seg_workspace_bytes,
                                  int64_t *lhs_idx, int64_t *rhs_idx, int32_t *out_coords,
                                  int32_t *seg_offsets, int32_t *perm, int64_t seg_capacity,
                                  int32_t group, int32_t *run_order, int32_t *run_order_written,
                                  int64_t *counts, int32_t counts_direct, ej_stream_t stream_) {
  clear_error();
  if (run_order_written) *run_order_written = 0;
  return pair_plan_impl(lhs_coords, n_lhs, lhs_ncols, rhs_coords, n_rhs, rhs_ncols, n_keys,
                        lhs_dims, rhs_dims, join_radices, n_out, agg_src, agg_dim, agg_radices,
                        pair_capacity, join_workspace, join_workspace_bytes, seg_workspace,
                        seg_workspace_bytes, lhs_idx, rhs_idx, out_coords, seg_offsets, perm,
                        seg_capacity, group, run_order, run_order_written, counts,
                        counts_direct, as_stream(stream_));
}

extern "C" int ej_pair_plan_async_noalloc(
    const int32_t *lhs_coords, int64_t n_lhs, int32_t lhs_ncols, const int32_t *rhs_coords,
    int64_t n_rhs, int32_t rhs_ncols, int32_t n_keys, const int32_t *lhs_dims,
    const int32_t *rhs_dims, const int64_t *join_radices, int32_t n_out, const int32_t *agg_src,
    const int32_t *agg_dim, const int64_t *agg_radices, int64_t pair_capacity, int64_t *lhs_idx,
    int64_t *rhs_idx, int32_t *out_coords, int32_t *seg_offsets, int32_t *perm,
    int64_t seg_capacity, int32_t group, int32_t *run_order, int32_t *run_order_written,
    int64_t *counts, int32_t counts_direct, ej_stream_t stream_) {
  clear_error();
  if (run_order_written) *run_order_written = 0;
  EJ_CHECK_ARG(n_lhs >= 1 && n_rhs >= 1 && n_lhs < (int64_t(1) << 31) &&
                   n_rhs < (int64_t(1) << 31),
               "the queued pair plan needs two non-empty relations below 2^31 tiles");
  EJ_CHECK_ARG(pair_capacity >= 1 && pair_capacity < (int64_t(1) << 31),
               "pair_capacity must lie in [1, 2^31)");
  const size_t jb = carve_join(nullptr, n_lhs, n_rhs, EJ_ORDER_PROBE).bytes;
  const size_t sb = carve_seg(nullptr, pair_capacity).bytes;
  const size_t joff = 0, soff = (jb + 255) & ~size_t(255);
  if (soff + sb > kNoAllocScratchBytes) {
    set_error("the allocation-free plan needs %zu bytes of scratch for %lld x %lld tiles and "
              "%lld pairs; its static scratch holds %zu (use ej_pair_plan_async with "
              "caller workspaces)",
              soff + sb, (long long)n_lhs, (long long)n_rhs, (long long)pair_capacity,
              kNoAllocScratchBytes);
    return EJ_E_CAPACITY;
  }
  void *base = nullptr;
  EJ_TRY(scratch_base(&base));
  unsigned char *b = static_cast<unsigned char *>(base);
  return pair_plan_impl(lhs_coords, n_lhs, lhs_ncols, rhs_coords, n_rhs, rhs_ncols, n_keys,
                        lhs_dims, rhs_dims, join_radices, n_out, agg_src, agg_dim, agg_radices,
                        pair_capacity, b + joff, jb, b + soff, sb, lhs_idx, rhs_idx, out_coords,
                        seg_offsets, perm, seg_capacity, group, run_order, run_order_written,
                        counts, counts_direct, as_stream(stream_));
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
