// Join and segment plan of a sparse einsum whose rhs holds every tile of its
// grid, in one launch and without sorting.
//
// The reference joins with a dict and groups the pairs by output coordinate
// with a second dict and a sort (execution/sparse_dispatch.py:29-82,
// :129-171).  When the rhs relation is the full tile grid in lexicographic
// order (a dense operand), its join dimensions lead, and the lhs coordinates
// are strictly increasing, both results have a closed form: every lhs tile
// meets exactly one rhs tile per combination of the rhs's free dimensions,
// and the lhs tiles that share their leading (output) coordinates form a
// contiguous run.  Output segment (run r, free index k) sums the pairs
// (lhs tile t, rhs tile jrow(t) * NK + k) for t in run r, in lhs order; the
// reference accumulates them in the same order (ascending rhs index, which
// within a run is ascending lhs index).  Segments come in run order, then k:
// the reference's sorted output coordinates.
//
// The kernel checks those properties on the device; where they fail it
// reports it (counts[1] = 1) and leaves the segment count at 0, so that an
// einsum queued behind it does no work and the caller takes the general
// join and plan.
#include <algorithm>

#include "ej_internal.h"

namespace ej {
namespace {

constexpr int kDenseThreads = 1024;
constexpr int kDenseTilesPerThread = 16;  // lhs tiles each thread scans
constexpr int kDenseMaxLhs = kDenseThreads * kDenseTilesPerThread;  // bits and join rows in LDS
constexpr int kDenseMaxRuns = 8192;       // run starts held in LDS (rank_of is 16-bit)
constexpr int kDenseMinPairsPerBlock = 2 * kDenseThreads;
// Every block rescans the lhs coordinates for run starts: at most one block
// per CU.
constexpr int kDenseMaxBlocks = 256;

// Every count and grid extent is below 2^31 (checked on the host), so the
// kernel's index arithmetic and divisions are 32-bit.
struct DenseSpec {
  int32_t lncols, rncols;
  int32_t nk;     // join keys; rhs dims 0 .. nk-1 are the join dims
  int32_t nlo;    // lhs dims 0 .. nlo-1 are the output dims taken from the lhs
  int32_t n_out;  // nlo + (rncols - nk)
  int32_t ldim[EJ_MAX_KEYS];   // lhs dim joined with rhs dim i
  int32_t lgrid[EJ_MAX_DIMS];  // lhs tile grid
  int32_t rgrid[EJ_MAX_DIMS];  // rhs tile grid
  int32_t NK;                  // rhs tiles per join value: prod rgrid[nk .. rncols)
  int32_t n_lhs, n_rhs, P;     // P = n_lhs * NK
  int32_t ppb;                 // pairs per block
};

// Blocks of kDenseThreads threads; LN and RN are the lhs and rhs coordinate
// ranks (0: read from the spec, up to EJ_MAX_DIMS).  Every block finds the
// run starts among all lhs tiles (one bit per tile in LDS, ranked by a scan
// of the words' counts, and the table of run starts) and each lhs tile's rhs
// join row (LDS), and in the same pass checks its own slice of the lhs tiles
// (range, join bounds, order).  Block b then writes its share of the
// segments, the pairs at
// positions [b * ppb, (b + 1) * ppb) of the segment-ordered pair list, its
// share of the rhs check (the first row loaded with the lhs scan's first
// pass, so that the latencies overlap) and (run_order) the order of the XCD chunks
// assigned to it.  The last block to finish publishes the counts: scal[0] =
// U (0 when a check failed), scal[1] = not-applicable flag, scal[2] = scal[4]
// = P, scal[3] = scal[5] = 0, and, given host_counts, the single word
// host_counts[6] = ticket << 33 | flag << 32 | U.  Blocks meet through one
// atomic word, scal[7]: each adds 1 plus its check failure in the upper
// half, so the block that sees nblk - 1 finished blocks before it also sees
// every failure; no fence is needed (a fence here would write back the L2,
// which the einsum before this kernel left full of output tiles).  scal[7]
// must be zero at launch; the last block returns it to zero.
template <int LN, int RN>
__global__ __launch_bounds__(kDenseThreads) void dense_plan_kernel(
    const int32_t *__restrict__ lc, const int32_t *__restrict__ rc, DenseSpec s,
    int64_t *__restrict__ lidx, int64_t *__restrict__ ridx, int32_t *__restrict__ out_coords,
    int32_t *__restrict__ seg_offsets, int64_t seg_cap, int group,
    int32_t *__restrict__ run_order, int64_t *__restrict__ scal,
    int64_t *__restrict__ host_counts, int64_t ticket) {
  constexpr int LD = LN ? LN : EJ_MAX_DIMS, RD = RN ? RN : EJ_MAX_DIMS;
  constexpr int NW = kDenseThreads / 64;
  __shared__ int32_t run_start[kDenseMaxRuns + 1];
  __shared__ int32_t jrow[kDenseMaxLhs];  // the rhs join row of each lhs tile
  __shared__ unsigned long long start_bits[kDenseMaxLhs / 64];  // bit: the tile starts a run
  __shared__ int32_t word_base[kDenseMaxLhs / 64];              // runs started before the word
  __shared__ int32_t cls_base[NW][256];
  const int lncols = LN ? LN : s.lncols, rncols = RN ? RN : s.rncols;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int blk = blockIdx.x, nblk = gridDim.x;
  const uint32_t nk32 = static_cast<uint32_t>(s.NK);
  int bad = 0;

  // ---- rhs check, first row: issued before the lhs loads -------------------
  const int64_t rpb = (static_cast<uint32_t>(s.n_rhs) - 1u) / static_cast<uint32_t>(nblk) + 1u;
  const int64_t r0 = blk * rpb, r1 = min(static_cast<int64_t>(s.n_rhs), r0 + rpb);
  const int64_t rfirst = r0 + tid;
  int32_t rv[RD];
  auto load_r = [&](int64_t r) {
#pragma unroll
    for (int d = 0; d < RD; ++d) rv[d] = d < rncols ? rc[r * rncols + d] : 0;
  };
  auto rhs_ok = [&](int64_t r) {  // row r holds the coordinates of grid position r
    uint32_t rem = static_cast<uint32_t>(r);
    bool ok = true;
#pragma unroll
    for (int d = RD - 1; d >= 0; --d)
      if (d < rncols) {
        const uint32_t g = static_cast<uint32_t>(s.rgrid[d]), q = rem / g;
        ok = ok && rv[d] == static_cast<int32_t>(rem - q * g);
        rem = q;
      }
    return ok;
  };

  // ---- run starts: one bit per lhs tile, every block over every tile -------
  // Tile t starts a run when one of its output dims (0 .. nlo-1) differs from
  // tile t - 1's.  Thread tid takes tiles tid, tid + kDenseThreads, ... (each
  // wave's loads coalesced), eight tiles per pass with their loads (clamped,
  // always valid indices) issued before any is used.
  const int nm = (s.n_lhs + kDenseThreads - 1) / kDenseThreads;  // <= kDenseTilesPerThread
  constexpr int kScanBatch = 8;
  // This block's slice of the tiles, checked in the same pass: coordinates
  // inside the lhs grid, join coordinates inside the rhs grid, strictly
  // increasing rows; the blocks' failures meet in the publish.
  const int tpb = (s.n_lhs + nblk - 1) / nblk;
  const int c0 = min(s.n_lhs, blk * tpb), c1 = min(s.n_lhs, c0 + tpb);
  for (int m0 = 0; m0 < nm; m0 += kScanBatch) {
    int32_t cvb[kScanBatch][LD], pvb[kScanBatch][LD];
#pragma unroll
    for (int k = 0; k < kScanBatch; ++k) {
      if (m0 + k >= nm) break;  // uniform: no loads for passes past the tiles
      const int tc = min((m0 + k) * kDenseThreads + tid, s.n_lhs - 1), tp = max(tc - 1, 0);
#pragma unroll
      for (int d = 0; d < LD; ++d) cvb[k][d] = d < lncols ? lc[tc * lncols + d] : 0;
#pragma unroll
      for (int d = 0; d < LD; ++d) pvb[k][d] = d < lncols ? lc[tp * lncols + d] : 0;
    }
    // the rhs check's first row, loaded behind the first pass's lhs loads so
    // that the latencies overlap
    if (m0 == 0 && rfirst < r1) load_r(rfirst);
#pragma unroll
    for (int k = 0; k < kScanBatch; ++k) {
      const int m = m0 + k;
      if (m >= nm) break;  // uniform
      const int t = m * kDenseThreads + tid;
      bool newrun = t == 0;
#pragma unroll
      for (int d = 0; d < LD; ++d) newrun = newrun || (d < s.nlo && cvb[k][d] != pvb[k][d]);
      const unsigned long long bits = __ballot(t < s.n_lhs && newrun);
      if (lane == 0) start_bits[m * NW + wave] = bits;
      if (t < s.n_lhs) {
        uint32_t j = 0;  // the rhs join row: the tile's join coordinates over the join grid
#pragma unroll
        for (int i = 0; i < RD; ++i)
          if (i < s.nk) {
            int32_t c = 0;
#pragma unroll
            for (int d = 0; d < LD; ++d) c = d == s.ldim[i] ? cvb[k][d] : c;
            j = j * static_cast<uint32_t>(s.rgrid[i]) + static_cast<uint32_t>(c);
          }
        jrow[t] = static_cast<int32_t>(j);
      }
      if (t >= c0 && t < c1) {
        const int32_t *cv = cvb[k], *pv = pvb[k];
#pragma unroll
        for (int d = 0; d < LD; ++d)
          if (d < lncols && (cv[d] < 0 || cv[d] >= s.lgrid[d])) bad = 1;
#pragma unroll
        for (int i = 0; i < RD; ++i)
          if (i < s.nk) {
            int32_t c = 0;
#pragma unroll
            for (int d = 0; d < LD; ++d) c = d == s.ldim[i] ? cv[d] : c;
            if (c >= s.rgrid[i]) bad = 1;  // no rhs tile to meet
          }
        if (t > 0) {
          int cmp = 0;
#pragma unroll
          for (int d = 0; d < LD; ++d)
            if (d < lncols && cmp == 0 && cv[d] != pv[d]) cmp = cv[d] < pv[d] ? -1 : 1;
          if (cmp <= 0) bad = 1;  // coordinates must be strictly increasing
        }
      }
    }
  }
  if (rfirst < r1 && !rhs_ok(rfirst)) bad = 1;
  __syncthreads();

  // ---- run table: run r starts at tile run_start[r] ------------------------
  const int nwords = nm * NW;
  int64_t nruns64 = 0;
  const int64_t wb = block_exclusive_sum<kDenseThreads>(
      tid < nwords ? __popcll(start_bits[tid]) : 0, &nruns64);
  if (tid < nwords) word_base[tid] = static_cast<int32_t>(wb);
  const int nruns = static_cast<int>(nruns64);
  const bool fits = nruns <= kDenseMaxRuns;
  if (fits && tid < nwords) {
    unsigned long long bits = start_bits[tid];
    for (int r = static_cast<int>(wb); bits; ++r, bits &= bits - 1ull)
      run_start[r] = tid * 64 + __builtin_ctzll(bits);
  }
  if (fits && tid == 0) run_start[nruns] = s.n_lhs;
  if (!fits) bad = 1;
  __syncthreads();
  // Run of tile t: the run starts at or before it, less one (tile 0 starts run 0).
  auto run_of = [&](uint32_t t) {
    const unsigned long long bits = start_bits[t >> 6];
    const uint32_t b = t & 63u;
    const unsigned long long upto = b == 63u ? bits : bits & ((2ull << b) - 1ull);
    return word_base[t >> 6] + __popcll(upto) - 1;
  };
  const int64_t U = fits ? static_cast<int64_t>(nruns) * s.NK : 0;
  const int live_u = static_cast<int>(U < seg_cap ? U : seg_cap);
  if (U > seg_cap) bad = 1;

  if (fits) {
    // ---- segments: this block's share of [0, live_u) ----------------------
    // Run r (tiles rs .. rs + len - 1) owns pairs [rs * NK, (rs + len) * NK):
    // segment (r, k) is pairs rs * NK + k * len + (t - rs), t ascending.
    const int64_t upb = live_u ? (static_cast<uint32_t>(live_u) - 1u) / nblk + 1u : 0;
    const int64_t u0 = blk * upb, u1 = min(static_cast<int64_t>(live_u), u0 + upb);
    for (int64_t u = u0 + tid; u < u1; u += kDenseThreads) {
      const uint32_t uu = static_cast<uint32_t>(u);
      const uint32_t r = uu / nk32, kk = uu - r * nk32;
      const int rs = run_start[r], len = run_start[r + 1] - rs;
      seg_offsets[u] = rs * s.NK + static_cast<int>(kk) * len;
      int32_t *oc = out_coords + u * s.n_out;
#pragma unroll
      for (int d = 0; d < LD; ++d)
        if (d < s.nlo) oc[d] = lc[rs * lncols + d];
      uint32_t rem = kk;
#pragma unroll
      for (int d = RD - 1; d >= 0; --d)
        if (d >= s.nk && d < rncols) {
          const uint32_t g = static_cast<uint32_t>(s.rgrid[d]), qd = rem / g;
          oc[s.nlo + (d - s.nk)] = static_cast<int32_t>(rem - qd * g);
          rem = qd;
        }
    }
    if (blk == 0 && tid == 0 && U <= seg_cap) seg_offsets[U] = s.P;
    // ---- pairs: positions [q0, q1) of the segment-ordered pair list ---------
    // Run r owns positions [rs * NK, (rs + len) * NK), so position q lies in
    // the run of lhs tile q / NK; there q - rs * NK = kk * len + p, the pair of
    // lhs tile rs + p and free index kk.  Consecutive threads write
    // consecutive positions.
    const int64_t q0 = static_cast<int64_t>(blk) * s.ppb;
    const int64_t q1 = min(static_cast<int64_t>(s.P), q0 + s.ppb);
    for (int64_t q = q0 + tid; q < q1; q += kDenseThreads) {
      const uint32_t uq = static_cast<uint32_t>(q);
      const int r = run_of(uq / nk32);
      const int rs = run_start[r], len = run_start[r + 1] - rs;
      const uint32_t off = uq - static_cast<uint32_t>(rs) * nk32;
      const uint32_t kk = off / static_cast<uint32_t>(len), p = off - kk * static_cast<uint32_t>(len);
      const int t = rs + static_cast<int>(p);
      lidx[q] = t;
      ridx[q] = static_cast<int64_t>(jrow[t]) * s.NK + kk;
    }
  }

  // ---- rhs check, remaining rows ------------------------------------------
  for (int64_t r = rfirst + kDenseThreads; r < r1; r += kDenseThreads) {
    load_r(r);
    if (!rhs_ok(r)) bad = 1;
  }

  // ---- run order, whole runs: balanced over the XCDs, longest first --------
  // When every run holds gpr = NK / group whole groups (which share the
  // run's lhs tiles) and the einsum's equal shares of consecutive groups
  // would leave one XCD more than 5% above the mean pair total, the runs are
  // ranked longest first (a stable counting sort over 256 pair-count
  // classes, counts above 255 tying) and dealt to the eight XCDs in snake
  // order (ranks 0-7 to XCDs 0-7, ranks 8-15 to XCDs 7-0, ...), which evens
  // out the XCDs' pair totals while keeping each run's groups on one XCD.
  // The order lists XCD 0's runs, then XCD 1's, ..., each XCD's longest
  // first and each run's groups in order; the einsum's XCD mapping cuts it
  // into the XCDs' equal shares of groups.  Balanced consecutive shares are
  // left in plan order instead (below): neighbouring runs often read the
  // same rhs tiles (a banded lhs), which their XCD's L2 then serves.
  const bool whole_runs = s.NK % (group > 0 ? group : 1) == 0;
  bool snake = false;
  if (fits && group > 0 && run_order && U <= seg_cap && whole_runs) {
    __shared__ unsigned long long share_load[8];
    const int ngroups = live_u / group, gpr = s.NK / group;
    const int sper = ngroups / 8, srem = ngroups % 8;
    auto share_end = [&](int x) {  // end of XCD x's share of the groups
      return x < srem ? (x + 1) * (sper + 1) : srem * (sper + 1) + (x + 1 - srem) * sper;
    };
    if (tid < 8) share_load[tid] = 0;
    lds_barrier();
    // pair totals of the consecutive shares: thread tid walks runs [ra, rb)
    const int rpt = (nruns + kDenseThreads - 1) / kDenseThreads;
    const int ra = min(nruns, tid * rpt), rb = min(nruns, ra + rpt);
    if (ra < rb) {
      int g = ra * gpr;
      int x = g < srem * (sper + 1) ? g / (sper + 1)
                                    : srem + (sper ? (g - srem * (sper + 1)) / sper : 0);
      x = min(x, 7);
      int end = share_end(x);
      unsigned long long acc = 0;
      for (int r = ra; r < rb; ++r) {
        const unsigned long long w = static_cast<unsigned long long>(group) *
                                     static_cast<unsigned>(run_start[r + 1] - run_start[r]);
        int left = gpr;
        while (left > 0) {
          while (g >= end && x < 7) {
            atomicAdd(&share_load[x], acc);
            acc = 0;
            end = share_end(++x);
          }
          const int take = x < 7 ? min(left, end - g) : left;
          acc += w * static_cast<unsigned>(take);
          g += take;
          left -= take;
        }
      }
      atomicAdd(&share_load[x], acc);
    }
    lds_barrier();
    unsigned long long mx = 0, tot = 0;
#pragma unroll
    for (int y = 0; y < 8; ++y) {
      mx = share_load[y] > mx ? share_load[y] : mx;
      tot += share_load[y];
    }
    snake = mx * 8 * 100 > tot * 105;
  }
  if (snake) {
    const int ngroups = live_u / group;
    if (blk == 0 && tid == 0) run_order[0] = ngroups;
    __shared__ uint16_t rank_of[kDenseMaxRuns];  // rank of run r
    const int rpw = ((nruns + NW - 1) / NW + 63) & ~63;  // runs per wave, whole 64-run steps
    const int w0 = min(nruns, wave * rpw), w1 = min(nruns, w0 + rpw);
    auto run_cls = [&](int r) {
      const int len = run_start[r + 1] - run_start[r];
      return 255 - (len < 255 ? len : 255);
    };
    for (int c = lane; c < 256; c += 64) cls_base[wave][c] = 0;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    for (int r = w0 + lane; r < w1; r += 64) atomicAdd(&cls_base[wave][run_cls(r)], 1);
    lds_barrier();
    // Exclusive scan of the class counts in (class, wave) order: thread tid
    // holds entries 4 tid .. 4 tid + 3 of the 256 x NW.
    int hv[4], hs = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int e = 4 * tid + k;
      hv[k] = cls_base[e % NW][e / NW];
      hs += hv[k];
    }
    int64_t htot = 0;
    int hrun = static_cast<int>(block_exclusive_sum<kDenseThreads>(hs, &htot));
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int e = 4 * tid + k;
      cls_base[e % NW][e / NW] = hrun;
      hrun += hv[k];
    }
    lds_barrier();
    const uint64_t lt = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    for (int rb = w0; rb < w1; rb += 64) {
      const int r = rb + lane;
      const bool valid = r < w1;
      const int c = valid ? run_cls(r) : 0;
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
      if (valid) rank_of[r] = static_cast<uint16_t>(base + __popcll(peers & lt));
      if (valid && (peers & lt) == 0) cls_base[wave][c] = base + __popcll(peers);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    lds_barrier();
    // Rank p goes to XCD snake(p) as its (p / 8)-th run; XCD x holds n(x)
    // runs: one per full round of eight and one more if the last round
    // reaches it.
    const int gpr = s.NK / group;
    const int rounds = (nruns + 7) / 8, last = nruns - 8 * (rounds - 1);
    const bool last_fwd = ((rounds - 1) & 1) == 0;
    auto n_of = [&](int x) {
      return rounds - 1 + ((last_fwd ? x < last : x >= 8 - last) ? 1 : 0);
    };
    const int gpb = (ngroups + nblk - 1) / nblk;
    const int g0 = min(ngroups, blk * gpb), g1 = min(ngroups, g0 + gpb);
    for (int gi = g0 + tid; gi < g1; gi += kDenseThreads) {
      const int r = gi / gpr, kg = gi - r * gpr;
      const int p = rank_of[r];
      const int q = p & 7, x = (p >> 3) & 1 ? 7 - q : q;
      int before = 0;  // runs of the XCDs before x
#pragma unroll
      for (int y = 0; y < 7; ++y) before += y < x ? n_of(y) : 0;
      run_order[1 + (before + (p >> 3)) * gpr + kg] = gi;
    }
  }

  // ---- run order, otherwise: none ------------------------------------------
  // A header of 0 matches no launch, so the einsum takes its groups in plan
  // order (consecutive runs on each XCD).  Measured on a banded lhs, that
  // beats both the same order read through the table and each share sorted
  // longest first.
  if (fits && group > 0 && run_order && !snake && blk == 0 && tid == 0) run_order[0] = 0;

  // ---- publish: the last block to finish writes the counts ----------------
  const int blk_bad = __syncthreads_or(bad);
  if (tid == 0) {
    unsigned long long *meet = reinterpret_cast<unsigned long long *>(scal + 7);
    const unsigned long long prev =
        atomicAdd(meet, 1ull + (blk_bad ? (1ull << 32) : 0ull));
    if ((prev & 0xffffffffull) == static_cast<unsigned long long>(nblk - 1)) {
      const int64_t any_bad = (prev >> 32) != 0 || blk_bad ? 1 : 0;
      const int64_t u_out = any_bad ? 0 : U;
      scal[0] = u_out;
      scal[1] = any_bad;
      scal[2] = s.P;
      scal[3] = 0;
      scal[4] = s.P;
      scal[5] = 0;
      scal[6] = 0;
      scal[7] = 0;  // ready for the next call
      if (host_counts)
        __hip_atomic_store(reinterpret_cast<unsigned long long *>(host_counts + 6),
                           (static_cast<unsigned long long>(ticket) << 33) |
                               (static_cast<unsigned long long>(any_bad) << 32) |
                               static_cast<unsigned long long>(u_out),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
  }
}

using DenseKernel = void (*)(const int32_t *, const int32_t *, DenseSpec, int64_t *, int64_t *,
                             int32_t *, int32_t *, int64_t, int, int32_t *, int64_t *,
                             int64_t *, int64_t);

template <int LN>
DenseKernel dense_kernel_for_rhs(int rn) {
  switch (rn) {
    case 1: return dense_plan_kernel<LN, 1>;
    case 2: return dense_plan_kernel<LN, 2>;
    case 3: return dense_plan_kernel<LN, 3>;
    case 4: return dense_plan_kernel<LN, 4>;
    default: return dense_plan_kernel<0, 0>;
  }
}

// The kernel specialised for the coordinate ranks (both up to 4), else the
// general one.
DenseKernel dense_kernel_for(int ln, int rn) {
  switch (ln) {
    case 1: return dense_kernel_for_rhs<1>(rn);
    case 2: return dense_kernel_for_rhs<2>(rn);
    case 3: return dense_kernel_for_rhs<3>(rn);
    case 4: return dense_kernel_for_rhs<4>(rn);
    default: return dense_plan_kernel<0, 0>;
  }
}

}  // namespace

int run_plan_structure(const char *who, int n_keys, const int32_t *lhs_dims,
                       const int32_t *rhs_dims, int lhs_ncols, int rhs_ncols, int n_out,
                       const int32_t *agg_src, const int32_t *agg_dim, int32_t *ldim, int *nlo_out) {
  // Join dims: rhs dims 0 .. nk-1, each once, their lhs dims increasing in
  // rhs-dim order (so that lhs order within a run is rhs order).
  for (int i = 0; i < n_keys; ++i) ldim[i] = -1;
  for (int k = 0; k < n_keys; ++k) {
    const int r = rhs_dims[k], l = lhs_dims[k];
    if (r < 0 || r >= n_keys || ldim[r] >= 0 || l < 0 || l >= lhs_ncols) {
      set_error("%s needs the join to cover rhs dims 0 .. %d once each", who, n_keys - 1);
      return EJ_E_UNSUPPORTED;
    }
    ldim[r] = l;
  }
  for (int i = 1; i < n_keys; ++i)
    if (ldim[i] <= ldim[i - 1]) {
      set_error("%s needs the join's lhs dims in the rhs dims' order", who);
      return EJ_E_UNSUPPORTED;
    }
  // Output: lhs dims 0 .. nlo-1, then every rhs dim from nk on, in order.
  int nlo = 0;
  while (nlo < n_out && agg_src[nlo] == 0 && agg_dim[nlo] == nlo) ++nlo;
  bool agg_ok = nlo >= 1 && n_out == nlo + (rhs_ncols - n_keys);
  for (int d = nlo; agg_ok && d < n_out; ++d)
    agg_ok = agg_src[d] == 1 && agg_dim[d] == n_keys + (d - nlo);
  // Every lhs dim from nlo on is a join dim (it varies within a run).
  for (int d = nlo; agg_ok && d < lhs_ncols; ++d) {
    bool joined = false;
    for (int i = 0; i < n_keys; ++i) joined = joined || ldim[i] == d;
    agg_ok = joined;
  }
  if (!agg_ok) {
    set_error("%s needs output dims = a prefix of the lhs dims, then the rhs dims after its "
              "join dims", who);
    return EJ_E_UNSUPPORTED;
  }
  *nlo_out = nlo;
  return EJ_OK;
}

}  // namespace ej

using namespace ej;

extern "C" int ej_dense_plan_async(const int32_t *lhs_coords, int64_t n_lhs, int32_t lhs_ncols,
                                   const int32_t *rhs_coords, int64_t n_rhs, int32_t rhs_ncols,
                                   int32_t n_keys, const int32_t *lhs_dims,
                                   const int32_t *rhs_dims, const int64_t *lhs_grid,
                                   const int64_t *rhs_grid, int32_t n_out,
                                   const int32_t *agg_src, const int32_t *agg_dim,
                                   int64_t *lhs_idx, int64_t *rhs_idx, int64_t pair_capacity,
                                   int32_t *out_coords, int32_t *seg_offsets,
                                   int64_t seg_capacity, int32_t group, int32_t *run_order,
                                   int32_t *run_order_written, int64_t *dev_counts,
                                   int64_t *counts, int32_t counts_direct,
                                   ej_stream_t stream_) {
  clear_error();
  hipStream_t stream = as_stream(stream_);
  if (run_order_written) *run_order_written = 0;
  EJ_CHECK_ARG(lhs_coords && rhs_coords && lhs_idx && rhs_idx && out_coords && seg_offsets &&
                   dev_counts && counts && lhs_grid && rhs_grid,
               "null pointer argument");
  EJ_CHECK_ARG(group >= 0 && counts_direct >= 0, "negative group or counts_direct");
  EJ_CHECK_ARG(lhs_ncols >= 1 && lhs_ncols <= EJ_MAX_DIMS && rhs_ncols >= 1 &&
                   rhs_ncols <= EJ_MAX_DIMS,
               "coordinate rank outside [1, %d]", EJ_MAX_DIMS);
  EJ_CHECK_ARG(n_keys >= 1 && n_keys <= rhs_ncols && n_keys <= EJ_MAX_KEYS,
               "the dense plan needs 1 .. rhs rank join keys");
  EJ_CHECK_ARG(lhs_dims && rhs_dims && (agg_src || n_out == 0) && (agg_dim || n_out == 0),
               "null key arrays");
  DenseSpec s{};
  s.lncols = lhs_ncols;
  s.rncols = rhs_ncols;
  s.nk = n_keys;
  int nlo = 0;
  EJ_TRY(run_plan_structure("the dense plan", n_keys, lhs_dims, rhs_dims, lhs_ncols, rhs_ncols,
                            n_out, agg_src, agg_dim, s.ldim, &nlo));
  s.nlo = nlo;
  s.n_out = n_out;
  // The grid product stops growing past 2^31 (no overflow); such a grid is
  // beyond the kernel's 32-bit indices.
  int64_t grid_r = 1, NK = 1;
  for (int d = 0; d < rhs_ncols; ++d) {
    EJ_CHECK_ARG(rhs_grid[d] >= 1 && rhs_grid[d] < (int64_t(1) << 31), "bad rhs grid");
    s.rgrid[d] = static_cast<int32_t>(rhs_grid[d]);
    grid_r = std::min(grid_r * rhs_grid[d], int64_t(1) << 31);
    if (d >= n_keys) NK = std::min(NK * rhs_grid[d], int64_t(1) << 31);
  }
  for (int d = 0; d < lhs_ncols; ++d) {
    EJ_CHECK_ARG(lhs_grid[d] >= 1 && lhs_grid[d] < (int64_t(1) << 31), "bad lhs grid");
    s.lgrid[d] = static_cast<int32_t>(lhs_grid[d]);
  }
  if (grid_r >= (int64_t(1) << 31) || n_rhs != grid_r || n_lhs < 1 || n_lhs > kDenseMaxLhs) {
    set_error("the dense plan needs a full rhs grid of under 2^31 tiles and 1 .. %d lhs tiles",
              kDenseMaxLhs);
    return EJ_E_UNSUPPORTED;
  }
  const int64_t P = n_lhs * NK;
  if (P >= (int64_t(1) << 30)) {
    set_error("the dense plan needs under 2^30 pairs (%lld)", (long long)P);
    return EJ_E_UNSUPPORTED;
  }
  if (pair_capacity < P) {
    set_error("pair capacity %lld < %lld pairs", (long long)pair_capacity, (long long)P);
    return EJ_E_CAPACITY;
  }
  s.n_lhs = static_cast<int32_t>(n_lhs);
  s.n_rhs = static_cast<int32_t>(n_rhs);
  s.NK = static_cast<int32_t>(NK);
  s.P = static_cast<int32_t>(P);
  EJ_CHECK_ARG(seg_capacity >= 1, "seg_capacity must be positive");
  EJ_CHECK_ARG(counts_direct < (int64_t(1) << 30), "counts_direct (the ticket) beyond 2^30");
  int64_t *direct = nullptr;
  if (counts_direct) EJ_HIP(hipHostGetDevicePointer(reinterpret_cast<void **>(&direct), counts, 0));
  s.ppb = static_cast<int32_t>(std::max<int64_t>(kDenseMinPairsPerBlock, ceil_div(P, kDenseMaxBlocks)));
  const int64_t nblk = ceil_div(P, s.ppb);
  const bool order = run_order && group > 0;
  hipLaunchKernelGGL(dense_kernel_for(lhs_ncols, rhs_ncols), dim3(static_cast<unsigned>(nblk)), dim3(kDenseThreads), 0,
                     stream, lhs_coords, rhs_coords, s, lhs_idx, rhs_idx, out_coords,
                     seg_offsets, seg_capacity, order ? group : 0,
                     order ? run_order : nullptr, dev_counts, direct, int64_t(counts_direct));
  EJ_LAUNCH_CHECK();
  if (order && run_order_written) *run_order_written = 1;
  if (!direct)
    EJ_HIP(hipMemcpyAsync(counts, dev_counts, 6 * sizeof(int64_t), hipMemcpyDeviceToHost, stream));
  return EJ_OK;
}
