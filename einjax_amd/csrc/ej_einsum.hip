// Tile einsum over matched pairs: description of the kernel string, the
// MFMA grouped GEMM (per-pair and fused segmented modes), a generic
// strided einsum for strings that are not GEMM-shaped, the deterministic
// segment sum and the tile gather.
//
// Reference: kernel_einsum (execution/sparse_dispatch.py:85-126) gathers the
// matched tiles (:118-119) and calls jnp.einsum on "z"+kernel_string
// (:121-126); segment_sum (:129-171) adds the per-pair results of equal
// output coordinate in pair order in float32.
#include <ctype.h>
#include <string.h>

#include "ej_internal.h"

namespace ej {
namespace {

// ---------------------------------------------------------------------------
// Kernel-string description.

struct LabelInfo {
  char c;
  int64_t ext = -1;
  int64_t sa = 0, sb = 0, sc = 0;  // strides (summed over repeats)
  int in_a = 0, in_b = 0, in_c = 0;
};

int parse_term(const char *s, size_t len, char *out, int *n) {
  int k = 0;
  for (size_t i = 0; i < len; ++i) {
    char ch = s[i];
    if (isspace(static_cast<unsigned char>(ch))) continue;
    if (ch == '.') {
      set_error("ellipsis in a tile einsum is not supported");
      return EJ_E_UNSUPPORTED;
    }
    EJ_CHECK_ARG(isalpha(static_cast<unsigned char>(ch)), "invalid label '%c' in kernel string",
                 ch);
    EJ_CHECK_ARG(k < EJ_MAX_DIMS, "a term of the kernel string has more than %d labels",
                 EJ_MAX_DIMS);
    out[k++] = ch;
  }
  *n = k;
  return EJ_OK;
}

void row_major_strides(const int64_t *shape, int nd, int64_t *st) {
  int64_t s = 1;
  for (int d = nd - 1; d >= 0; --d) {
    st[d] = s;
    s *= shape[d];
  }
}

// Flattens a group of labels (in the given order) into one (extent, stride)
// for one operand; extent-1 labels are ignored.  Fails if the group is not
// a single uniformly strided run in that operand.
bool flatten(const LabelInfo *const *grp, int n, int which, int64_t *ext, int64_t *stride) {
  int64_t e = 1, s = 0;
  bool have = false;
  int64_t prev_stride = 0;
  for (int i = 0; i < n; ++i) {
    const LabelInfo *L = grp[i];
    if (L->ext == 1) continue;
    int64_t st = which == 0 ? L->sa : which == 1 ? L->sb : L->sc;
    if (have && prev_stride != st * L->ext) return false;
    prev_stride = st;
    s = st;
    e *= L->ext;
    have = true;
  }
  *ext = e;
  *stride = have ? s : 0;
  return true;
}

}  // namespace
}  // namespace ej

using namespace ej;

extern "C" int ej_einsum_describe(const char *ks, const int64_t *lhs_tile, int32_t lhs_ndim,
                                  const int64_t *rhs_tile, int32_t rhs_ndim,
                                  ej_einsum_desc *d) {
  clear_error();
  EJ_CHECK_ARG(ks && d, "null argument");
  EJ_CHECK_ARG(lhs_ndim >= 0 && lhs_ndim <= EJ_MAX_DIMS && rhs_ndim >= 0 &&
                   rhs_ndim <= EJ_MAX_DIMS,
               "tile rank outside [0, %d]", EJ_MAX_DIMS);
  const char *arrow = strstr(ks, "->");
  EJ_CHECK_ARG(arrow, "kernel_string must contain '->': %s", ks);
  EJ_CHECK_ARG(!strstr(arrow + 2, "->"), "kernel_string has more than one '->': %s", ks);
  const char *comma = static_cast<const char *>(memchr(ks, ',', arrow - ks));
  EJ_CHECK_ARG(comma, "kernel_string must have exactly two operands: %s", ks);
  EJ_CHECK_ARG(!memchr(comma + 1, ',', arrow - comma - 1),
               "kernel_string must have exactly two operands: %s", ks);
  char ta[EJ_MAX_DIMS], tb[EJ_MAX_DIMS], tc[EJ_MAX_DIMS];
  int na, nb, nc;
  EJ_TRY(parse_term(ks, comma - ks, ta, &na));
  EJ_TRY(parse_term(comma + 1, arrow - comma - 1, tb, &nb));
  EJ_TRY(parse_term(arrow + 2, strlen(arrow + 2), tc, &nc));
  EJ_CHECK_ARG(na == lhs_ndim, "lhs term has %d labels but the lhs tile has rank %d", na, lhs_ndim);
  EJ_CHECK_ARG(nb == rhs_ndim, "rhs term has %d labels but the rhs tile has rank %d", nb, rhs_ndim);

  LabelInfo labels[3 * EJ_MAX_DIMS];
  int nl = 0;
  auto find = [&](char c) -> LabelInfo * {
    for (int i = 0; i < nl; ++i)
      if (labels[i].c == c) return &labels[i];
    labels[nl] = LabelInfo();
    labels[nl].c = c;
    return &labels[nl++];
  };
  int64_t sa[EJ_MAX_DIMS], sb[EJ_MAX_DIMS];
  row_major_strides(lhs_tile, na, sa);
  row_major_strides(rhs_tile, nb, sb);
  for (int i = 0; i < na; ++i) {
    LabelInfo *L = find(ta[i]);
    EJ_CHECK_ARG(lhs_tile[i] >= 1, "tile extents must be positive");
    EJ_CHECK_ARG(L->ext < 0 || L->ext == lhs_tile[i], "label '%c' has inconsistent extents",
                 ta[i]);
    L->ext = lhs_tile[i];
    L->sa += sa[i];
    L->in_a++;
  }
  for (int i = 0; i < nb; ++i) {
    LabelInfo *L = find(tb[i]);
    EJ_CHECK_ARG(rhs_tile[i] >= 1, "tile extents must be positive");
    EJ_CHECK_ARG(L->ext < 0 || L->ext == rhs_tile[i], "label '%c' has extent %lld in lhs and %lld in rhs",
                 tb[i], (long long)L->ext, (long long)rhs_tile[i]);
    L->ext = rhs_tile[i];
    L->sb += sb[i];
    L->in_b++;
  }
  int64_t cshape[EJ_MAX_DIMS];
  for (int i = 0; i < nc; ++i) {
    LabelInfo *L = nullptr;
    for (int j = 0; j < nl; ++j)
      if (labels[j].c == tc[i]) L = &labels[j];
    EJ_CHECK_ARG(L, "output label '%c' does not appear in the inputs", tc[i]);
    EJ_CHECK_ARG(L->in_c == 0, "output label '%c' is repeated", tc[i]);
    L->in_c = 1;
    cshape[i] = L->ext;
  }
  int64_t sc[EJ_MAX_DIMS];
  row_major_strides(cshape, nc, sc);

  memset(d, 0, sizeof(*d));
  d->n_out = nc;
  const LabelInfo *outl[EJ_MAX_DIMS];
  for (int i = 0; i < nc; ++i) {
    LabelInfo *L = nullptr;
    for (int j = 0; j < nl; ++j)
      if (labels[j].c == tc[i]) L = &labels[j];
    L->sc = sc[i];
    outl[i] = L;
    d->out_ext[i] = L->ext;
    d->out_a[i] = L->sa;
    d->out_b[i] = L->sb;
  }
  const LabelInfo *redl[3 * EJ_MAX_DIMS];
  int nr = 0;
  for (int j = 0; j < nl; ++j) {
    if (labels[j].in_c) continue;
    redl[nr++] = &labels[j];
  }
  if (nr > EJ_MAX_LABELS) {
    set_error("more than %d contracted labels", EJ_MAX_LABELS);
    return EJ_E_UNSUPPORTED;
  }
  d->n_red = nr;
  for (int i = 0; i < nr; ++i) {
    d->red_ext[i] = redl[i]->ext;
    d->red_a[i] = redl[i]->sa;
    d->red_b[i] = redl[i]->sb;
  }
  d->a_elems = 1;
  for (int i = 0; i < na; ++i) d->a_elems *= lhs_tile[i];
  d->b_elems = 1;
  for (int i = 0; i < nb; ++i) d->b_elems *= rhs_tile[i];
  d->c_elems = 1;
  for (int i = 0; i < nc; ++i) d->c_elems *= cshape[i];

  // GEMM form: batch = output labels in both operands, M = output labels of
  // lhs only, N = output labels of rhs only, K = contracted labels present
  // in both operands.  A contracted label present in one operand only, a
  // repeated input label or a group that does not flatten into one strided
  // run keeps the generic strided kernel.
  const LabelInfo *gb[EJ_MAX_DIMS], *gm[EJ_MAX_DIMS], *gn[EJ_MAX_DIMS], *gk[3 * EJ_MAX_DIMS];
  int nbt = 0, nm = 0, nn = 0, nk = 0;
  bool gemm = true;
  for (int j = 0; j < nl; ++j)
    if (labels[j].in_a > 1 || labels[j].in_b > 1) gemm = false;
  for (int i = 0; i < nc; ++i) {
    const LabelInfo *L = outl[i];
    if (L->in_a && L->in_b) gb[nbt++] = L;
    else if (L->in_a) gm[nm++] = L;
    else gn[nn++] = L;
  }
  for (int i = 0; i < na; ++i) {  // K in lhs order
    for (int j = 0; j < nl; ++j) {
      const LabelInfo *L = &labels[j];
      if (L->c != ta[i] || L->in_c) continue;
      if (!L->in_b) gemm = false;
      gk[nk++] = L;
    }
  }
  for (int j = 0; j < nl; ++j)
    if (!labels[j].in_c && !labels[j].in_a) gemm = false;
  if (gemm) {
    int64_t e, s_a, s_b, s_c;
    bool ok = true;
    ok = ok && flatten(gb, nbt, 0, &e, &s_a) && flatten(gb, nbt, 1, &e, &s_b) &&
         flatten(gb, nbt, 2, &e, &s_c);
    d->batch = e; d->a_sb = s_a; d->b_sb = s_b; d->c_sb = s_c;
    ok = ok && flatten(gm, nm, 0, &e, &s_a) && flatten(gm, nm, 2, &e, &s_c);
    d->m = e; d->a_sm = s_a; d->c_sm = s_c;
    ok = ok && flatten(gn, nn, 1, &e, &s_b) && flatten(gn, nn, 2, &e, &s_c);
    d->n = e; d->b_sn = s_b; d->c_sn = s_c;
    ok = ok && flatten(gk, nk, 0, &e, &s_a) && flatten(gk, nk, 1, &e, &s_b);
    d->k = e; d->a_sk = s_a; d->b_sk = s_b;
    d->is_gemm = ok ? 1 : 0;
  }
  return EJ_OK;
}

namespace ej {
namespace {

// ---------------------------------------------------------------------------
// Shared pair addressing.

struct PairSrc {
  const int64_t *lidx, *ridx;  // null: identity
  const int32_t *perm;         // null: identity
  const int32_t *seg_off;      // null: one pair per segment
  int64_t n_a_tiles, n_b_tiles;
  const int64_t *n_live;       // non-null: segments >= *n_live are skipped (grid is a bound)
  const int32_t *run_order;    // non-null: grouped launches run group run_order[b] as block b
  int32_t order_group;         // segments per group that run_order was made for
};

// Whether the workgroup's segment lies beyond the device-side segment count.
__device__ inline bool seg_dead(const PairSrc &s, int64_t seg) {
  return s.n_live && seg >= *s.n_live;
}

__device__ inline void seg_range(const PairSrc &s, int64_t seg, int64_t *q0, int64_t *q1) {
  if (s.seg_off) {
    *q0 = s.seg_off[seg];
    *q1 = s.seg_off[seg + 1];
  } else {
    *q0 = seg;
    *q1 = seg + 1;
  }
}

// Tiles of the q-th pair in plan order; false if an index is out of range.
__device__ inline bool pair_tiles(const PairSrc &s, int64_t q, int64_t *at, int64_t *bt) {
  int64_t p = s.perm ? s.perm[q] : q;
  *at = s.lidx ? s.lidx[p] : p;
  *bt = s.ridx ? s.ridx[p] : p;
  return *at >= 0 && *at < s.n_a_tiles && *bt >= 0 && *bt < s.n_b_tiles;
}

__device__ inline float to_f32(float x) { return x; }
__device__ inline float to_f32(uint16_t x) { return __uint_as_float(static_cast<uint32_t>(x) << 16); }

// Output element stores: fp32 as is, bf16 rounded to nearest even
// (v_cvt_pk_bf16_f32).  Sums are always formed in fp32; a bf16 output is
// rounded once, when the finished tile is written.
__device__ inline void put_out(float *p, float v) { *p = v; }
__device__ inline void put_out(uint16_t *p, float v) {
  *p = __builtin_bit_cast(uint16_t, static_cast<__bf16>(v));
}

// Reads a workgroup-uniform element of a read-only index array through the
// scalar cache, so the load does not occupy the vector memory counter that
// paces the LDS ring.
template <typename T>
__device__ inline T ld_uniform(const T *p, int64_t i) {
  return ((const __attribute__((address_space(4))) T *)(p))[i];
}

// Maps the first `live` block ids onto logical blocks (block id b runs on XCD
// b % 8).  run == 0: the logical range is split into 8 contiguous parts, one
// per XCD, so that neighbouring logical blocks (sharing operand tiles) share
// an L2 over the widest window.  run > 0: runs of `run` consecutive logical
// blocks go to one XCD, the runs dealt to the XCDs in turn, so that every XCD
// gets a share of each region of the logical range (work that is heavier in
// one region, as for skewed sparsity, stays balanced); the last, partial
// round of runs is split into 8 contiguous parts.  Block ids from `live` on
// keep their id: they lie beyond the work of a grid sized for a bound.
__device__ inline int64_t xcd_logical_block(int64_t live, int64_t run = 0) {
  const int64_t bid = blockIdx.x;
  if (bid >= live) return bid;
  const int64_t full = run > 0 ? live / (8 * run) * (8 * run) : 0;
  const int64_t xcd = bid % 8;
  if (bid < full) {
    const int64_t local = bid / 8;
    return ((local / run) * 8 + xcd) * run + local % run;
  }
  const int64_t rest = live - full, local = (bid - full) / 8;
  const int64_t per = rest / 8, rem = rest % 8;
  const int64_t start = xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per;
  return full + start + local;
}

// Run length of the dealt mapping for one-segment workgroups taken in plan
// order (no run order): their neighbours share few tiles, and skewed
// sparsity makes whole regions of the plan heavier.
constexpr int64_t kXcdRun = 16;

// Blocks that carry work when each segment takes blocks_per_seg of them: the
// whole grid, or, given a device-side segment count, that many segments' blocks
// (so that a grid sized for a bound still spreads its live work over every XCD).
__device__ inline int64_t live_blocks(const PairSrc &s, int64_t blocks_per_seg) {
  const int64_t total = gridDim.x;
  if (!s.n_live) return total;
  const int64_t live = ld_uniform(s.n_live, 0) * blocks_per_seg;
  return live < total ? live : total;
}

// ---------------------------------------------------------------------------
// MFMA grouped GEMM.
//
// One workgroup (4 waves, 2x2) computes a BM x BN block of one output tile
// (segment) for one batch index, iterating the segment's pairs and the K
// dimension in BK chunks ("stages").  Operands are staged through LDS as
// [rows][k] (k contiguous, the layout both MFMA operands read); an operand
// whose free dimension is contiguous in HBM is transposed in registers
// before its LDS store.  LDS is double-buffered: the global loads of stage
// s+1 are issued before the MFMAs of stage s and written to the other buffer
// after them, so one barrier per stage suffices and HBM/L2 latency overlaps
// the math.  The tile indices of the next pair are fetched one pair ahead.
// Accumulation is fp32 in registers; each output block is written once.

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

struct GemmGeom {
  int64_t m, n, k, batch;
  int64_t a_sb, a_sm, a_sk, b_sb, b_sk, b_sn, c_sb, c_sm, c_sn;
  int64_t a_elems, b_elems, c_elems;
  int64_t mblocks, nblocks;
  int32_t out_bf16;  // output tiles in bf16 (else fp32)
};

// LDS placement of a [rows][BK] operand chunk in 16-byte chunks of VEC
// elements.  With 128-byte rows (8 chunks) the chunk index is XOR-swizzled
// by (row & 7) ^ ((row >> 3) & 7): the MFMA operand reads (16 consecutive
// rows, one chunk) and the transposed stores (rows 8 apart, one chunk) then
// touch distinct bank groups.  Other row widths use a 16-byte pad.
template <typename T, int BK>
struct LdsLayout {
  static constexpr int VEC = 16 / sizeof(T);
  static constexpr int CH = BK / VEC;
  static constexpr bool SWZ = CH == 8;
  static constexpr int LDK = SWZ ? BK : BK + VEC;
  __device__ static inline int off(int row, int chunk) {
    const int p = SWZ ? (chunk ^ ((row & 7) ^ ((row >> 3) & 7))) : chunk;
    return row * LDK + p * VEC;
  }
};

template <typename T, int ROWS, int BK, bool DIRECT>
struct OperandStage {
  using L = LdsLayout<T, BK>;
  static constexpr int VEC = L::VEC;
  // DIRECT: k contiguous in HBM; one 16-byte vector per (row, chunk).
  static constexpr int NVEC_D = ROWS * BK / VEC;
  static constexpr int PER_D = (NVEC_D + 255) / 256;
  // Transposed: rows contiguous in HBM; each thread owns KV k-rows x VEC rows.
  static constexpr int KV0 = ROWS * BK / (256 * VEC);
  static constexpr int KV = KV0 > 0 ? KV0 : 1;
  static constexpr int NBLK_T = (BK / KV) * (ROWS / VEC);
  static constexpr int NREG = DIRECT ? PER_D : KV;
  static_assert(KV <= VEC, "a thread's k run must fit in one 16-byte chunk");
  uint4 r[NREG];

  // base points at element (row 0, k 0) of the chunk.
  __device__ inline void load(const T *base, int64_t s_row, int64_t s_k, bool valid, int tid) {
    if (DIRECT) {
#pragma unroll
      for (int v = 0; v < PER_D; ++v) {
        const int id = v * 256 + tid;
        if (id < NVEC_D && valid) {
          const int row = id / (BK / VEC), kv = id % (BK / VEC);
          r[v] = *reinterpret_cast<const uint4 *>(base + row * s_row + kv * VEC);
        } else {
          r[v] = make_uint4(0, 0, 0, 0);
        }
      }
    } else {
      const bool own = tid < NBLK_T;
      const int rb = tid % (ROWS / VEC), kb = tid / (ROWS / VEC);
#pragma unroll
      for (int j = 0; j < KV; ++j) {
        if (own && valid)
          r[j] = *reinterpret_cast<const uint4 *>(base + (kb * KV + j) * s_k + rb * VEC);
        else
          r[j] = make_uint4(0, 0, 0, 0);
      }
    }
  }

  __device__ inline void store(T *lds, int tid) const {
    if (DIRECT) {
#pragma unroll
      for (int v = 0; v < PER_D; ++v) {
        const int id = v * 256 + tid;
        if (id < NVEC_D) {
          const int row = id / (BK / VEC), kv = id % (BK / VEC);
          *reinterpret_cast<uint4 *>(lds + L::off(row, kv)) = r[v];
        }
      }
    } else {
      if (tid >= NBLK_T) return;
      const int rb = tid % (ROWS / VEC), kb = tid / (ROWS / VEC);
      const int chunk = (kb * KV) / VEC, within = (kb * KV) % VEC;
      const uint32_t *w = reinterpret_cast<const uint32_t *>(r);
      if (sizeof(T) == 2) {
        // r[j] holds 8 bf16 of k-row j; emit, per row c, the KV values of k.
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          uint16_t vals[KV];
#pragma unroll
          for (int j = 0; j < KV; ++j) {
            uint32_t word = w[j * 4 + c / 2];
            vals[j] = static_cast<uint16_t>((c & 1) ? (word >> 16) : (word & 0xffffu));
          }
          T *dst = lds + L::off(rb * VEC + c, chunk) + within;
          if (KV == 8) {
            uint4 o;
            o.x = vals[0] | (static_cast<uint32_t>(vals[1 % KV]) << 16);
            o.y = vals[2 % KV] | (static_cast<uint32_t>(vals[3 % KV]) << 16);
            o.z = vals[4 % KV] | (static_cast<uint32_t>(vals[5 % KV]) << 16);
            o.w = vals[6 % KV] | (static_cast<uint32_t>(vals[7 % KV]) << 16);
            *reinterpret_cast<uint4 *>(dst) = o;
          } else if (KV == 4) {
            uint2 o;
            o.x = vals[0] | (static_cast<uint32_t>(vals[1 % KV]) << 16);
            o.y = vals[2 % KV] | (static_cast<uint32_t>(vals[3 % KV]) << 16);
            *reinterpret_cast<uint2 *>(dst) = o;
          } else if (KV == 2) {
            *reinterpret_cast<uint32_t *>(dst) = vals[0] | (static_cast<uint32_t>(vals[1 % KV]) << 16);
          } else {
#pragma unroll
            for (int j = 0; j < KV; ++j) reinterpret_cast<uint16_t *>(dst)[j] = vals[j];
          }
        }
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          T *dst = lds + L::off(rb * VEC + c, chunk) + within;
          if (KV == 4) {
            *reinterpret_cast<uint4 *>(dst) = make_uint4(w[c], w[4 + c], w[8 + c], w[12 + c]);
          } else {
#pragma unroll
            for (int j = 0; j < KV; ++j) reinterpret_cast<uint32_t *>(dst)[j] = w[j * 4 + c];
          }
        }
      }
    }
  }
};

struct PairTiles {
  int64_t at, bt;
  bool ok;
};

__device__ inline PairTiles load_pair(const PairSrc &s, int64_t q) {
  PairTiles t;
  t.ok = pair_tiles(s, q, &t.at, &t.bt);
  if (!t.ok) t.at = t.bt = 0;
  return t;
}

// Three workgroups per CU for bf16 (40 KB of LDS each with the padded rows);
// fp32 tiles need more registers and keep two.
template <typename T, int BM, int BN, int BK, bool A_DIRECT, bool B_DIRECT>
__global__ __launch_bounds__(256, sizeof(T) == 2 ? 3 : 2) void tile_gemm_kernel(const T *__restrict__ A,
                                                        const T *__restrict__ B,
                                                        void *__restrict__ C, PairSrc src,
                                                        GemmGeom g) {
  using SA = OperandStage<T, BM, BK, A_DIRECT>;
  using SB = OperandStage<T, BN, BK, B_DIRECT>;
  using L = LdsLayout<T, BK>;
  constexpr int LDK = L::LDK;
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int FM = WM / 16, FN = WN / 16;
  constexpr bool BF16 = sizeof(T) == 2;
  constexpr int KSTEP = BF16 ? 32 : 16;  // k consumed per inner step (4 chunks)
  __shared__ __align__(16) T As[2][BM * LDK];
  __shared__ __align__(16) T Bs[2][BN * LDK];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  int64_t lb = xcd_logical_block(live_blocks(src, g.nblocks * g.mblocks * g.batch));
  const int64_t nb = lb % g.nblocks;
  lb /= g.nblocks;
  const int64_t mb = lb % g.mblocks;
  lb /= g.mblocks;
  const int64_t bi = lb % g.batch;
  const int64_t seg = lb / g.batch;
  if (seg_dead(src, seg)) return;

  int64_t q0, q1;
  seg_range(src, seg, &q0, &q1);
  const int nkc = static_cast<int>(g.k / BK);
  const int64_t stages = (q1 - q0) * nkc;

  f32x4_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  SA sa;
  SB sb;
  const int64_t a_off0 = bi * g.a_sb + mb * BM * g.a_sm;
  const int64_t b_off0 = bi * g.b_sb + nb * BN * g.b_sn;
  auto issue = [&](const PairTiles &p, int kc) {
    const T *ab = A + p.at * g.a_elems + a_off0 + kc * BK * g.a_sk;
    const T *bb = B + p.bt * g.b_elems + b_off0 + kc * BK * g.b_sk;
    sa.load(ab, g.a_sm, g.a_sk, p.ok, tid);
    sb.load(bb, g.b_sn, g.b_sk, p.ok, tid);
  };

  PairTiles cur{0, 0, false}, nxt{0, 0, false};
  if (stages > 0) {
    cur = load_pair(src, q0);
    nxt = q0 + 1 < q1 ? load_pair(src, q0 + 1) : cur;
    issue(cur, 0);
    sa.store(As[0], tid);
    sb.store(Bs[0], tid);
  }
  __syncthreads();
  int kc = 0;
  int64_t q = q0;
  for (int64_t st = 0; st < stages; ++st) {
    const int buf = static_cast<int>(st & 1);
    const bool more = st + 1 < stages;
    if (more) {
      if (kc + 1 < nkc) issue(cur, kc + 1);
      else issue(nxt, 0);
    }
    const T *as = As[buf];
    const T *bs = Bs[buf];
#pragma unroll
    for (int ks = 0; ks < BK / KSTEP; ++ks) {
      const int ch = ks * 4 + (lane >> 4);
      if constexpr (BF16) {
        bf16x8_t af[FM], bfr[FN];
#pragma unroll
        for (int i = 0; i < FM; ++i)
          af[i] = *reinterpret_cast<const bf16x8_t *>(as + L::off(wm * WM + i * 16 + (lane & 15), ch));
#pragma unroll
        for (int j = 0; j < FN; ++j)
          bfr[j] = *reinterpret_cast<const bf16x8_t *>(bs + L::off(wn * WN + j * 16 + (lane & 15), ch));
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
      } else {
        f32x4_t af[FM], bfr[FN];
#pragma unroll
        for (int i = 0; i < FM; ++i)
          af[i] = *reinterpret_cast<const f32x4_t *>(as + L::off(wm * WM + i * 16 + (lane & 15), ch));
#pragma unroll
        for (int j = 0; j < FN; ++j)
          bfr[j] = *reinterpret_cast<const f32x4_t *>(bs + L::off(wn * WN + j * 16 + (lane & 15), ch));
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
          for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i][s4], bfr[j][s4], acc[i][j], 0, 0, 0);
      }
    }
    if (++kc == nkc) {  // the stage just issued starts pair q + 1
      kc = 0;
      ++q;
      cur = nxt;
      if (q + 1 < q1) nxt = load_pair(src, q + 1);
    }
    if (more) {
      sa.store(As[buf ^ 1], tid);
      sb.store(Bs[buf ^ 1], tid);
    }
    __syncthreads();
  }

  const int64_t c0 = seg * g.c_elems + bi * g.c_sb + mb * BM * g.c_sm + nb * BN * g.c_sn;
  auto store = [&](auto *cb) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = wm * WM + i * 16 + (lane >> 4) * 4 + r;
          const int col = wn * WN + j * 16 + (lane & 15);
          put_out(cb + row * g.c_sm + col * g.c_sn, acc[i][j][r]);
        }
  };
  if (g.out_bf16) store(static_cast<uint16_t *>(C) + c0);
  else store(static_cast<float *>(C) + c0);
}

// ---------------------------------------------------------------------------
// MFMA grouped GEMM, bf16, streaming operands straight into an LDS ring.
//
// Used for the common layout: lhs tiles k-contiguous ([m][k]) and rhs tiles
// n-contiguous ([k][n]), bf16.  Each stage (one pair's K-chunk of 64) is
// copied HBM -> LDS with 16-byte direct loads (global_load_lds_dwordx4, no
// register staging) into an NS-deep ring, so NS-1 stages are in flight while
// the MFMAs of the current one run.  Both operands keep their HBM layout in
// LDS; the per-lane source addresses are permuted so that 16-byte chunks
// land XOR-swizzled:
//   A [row][k]:  chunk c of row r at c ^ ((r & 7) ^ ((r >> 3) & 7)) (rows of
//                128 B; the 16-row operand reads hit distinct bank groups);
//   B [k][n]:    chunk j of k-row r at j ^ (2 * (r & 3)) (the 4-row reads of
//                the transpose load hit distinct bank groups).
// The B operand of v_mfma_f32_16x16x32_bf16 (8 consecutive k of one column
// per lane) comes from two ds_read_b64_tr_b16: within each 16-lane group,
// lane i receives element i % 4 of the 8 bytes read by lane 4t + i / 4
// (t = 0..3), so lanes 4t..4t+3 read k-row t, columns 4q..4q+3.
// The waits are explicit: s_waitcnt vmcnt(loads per stage x stages issued
// later) then s_barrier (no fence), one barrier per stage.

#define EJ_LDS(p) ((__attribute__((address_space(3))) void *)(p))
typedef int i32x2_t __attribute__((ext_vector_type(2)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));

// ds_read_b64_tr_b16 at LDS byte address `addr`.  Issued as inline asm: the
// compiler would otherwise order it behind every LDS DMA in flight
// (s_waitcnt vmcnt(0)), which defeats the ring.  Its completion is awaited
// by lgkm_wait_all.
__device__ inline i32x2_t ds_read_tr16_b64(uint32_t addr) {
  i32x2_t v;
  asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(v) : "v"(addr));
  return v;
}

// The same at LDS byte address addr + OFF (the instruction's offset field).
template <int OFF>
__device__ inline i32x2_t ds_read_tr16_b64_at(uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536, "LDS offset field");
  i32x2_t v;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "n"(OFF));
  return v;
}

// s_waitcnt lgkmcnt(0), threaded through the values it guards so that their
// consumers cannot be scheduled ahead of it.
template <int N>
__device__ inline void lgkm_wait_all(i32x4_t (&v)[N]) {
  asm volatile("s_waitcnt lgkmcnt(0)");
#pragma unroll
  for (int i = 0; i < N; ++i) asm volatile("" : "+v"(v[i]));
}

// Ring depth (stages) of the LDS-ring kernel per block shape.
#ifndef EJ_DMA_STAGES_128
#define EJ_DMA_STAGES_128 2
#endif
#ifndef EJ_DMA_STAGES_64
#define EJ_DMA_STAGES_64 4
#endif
#ifndef EJ_DMA_BK_128
#define EJ_DMA_BK_128 64
#endif
#ifndef EJ_USE_DMA_GEMM
#define EJ_USE_DMA_GEMM 1
#endif

__device__ inline PairTiles load_pair_uniform(const PairSrc &s, int64_t q) {
  const int32_t qq = __builtin_amdgcn_readfirstlane(static_cast<int32_t>(q));
  const int32_t p = s.perm ? ld_uniform(s.perm, qq) : qq;
  PairTiles t;
  t.at = s.lidx ? ld_uniform(s.lidx, p) : p;
  t.bt = s.ridx ? ld_uniform(s.ridx, p) : p;
  t.ok = t.at >= 0 && t.at < s.n_a_tiles && t.bt >= 0 && t.bt < s.n_b_tiles;
  if (!t.ok) t.at = t.bt = 0;
  return t;
}

template <int N>
__device__ inline void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

template <int NS, int LPS>
__device__ inline void wait_stage(int later) {
  // later = number of stages issued after the one about to be consumed;
  // each stage is LPS load instructions per wave.
  static_assert(NS >= 2 && NS <= 6, "ring depth");
  if constexpr (NS >= 6) {
    if (later >= 4) { wait_vmcnt<4 * LPS>(); return; }
  }
  if constexpr (NS >= 5) {
    if (later >= 3) { wait_vmcnt<3 * LPS>(); return; }
  }
  if constexpr (NS >= 4) {
    if (later >= 2) { wait_vmcnt<2 * LPS>(); return; }
  }
  if constexpr (NS >= 3) {
    if (later >= 1) { wait_vmcnt<LPS>(); return; }
  }
  wait_vmcnt<0>();
}

// The same when the stages issued after the one about to be consumed may
// number up to NS - 1 (the next stage is issued before the wait).
template <int NS, int LPS>
__device__ inline void wait_stage_in(int later) {
  static_assert(NS >= 2 && NS <= 5, "ring depth");
  if constexpr (NS >= 5) {
    if (later >= 4) { wait_vmcnt<4 * LPS>(); return; }
  }
  if constexpr (NS >= 4) {
    if (later >= 3) { wait_vmcnt<3 * LPS>(); return; }
  }
  if constexpr (NS >= 3) {
    if (later >= 2) { wait_vmcnt<2 * LPS>(); return; }
  }
  if (later >= 1) { wait_vmcnt<LPS>(); return; }
  wait_vmcnt<0>();
}

// XOR swizzles of 16-byte chunks (see the kernel comment).
template <int CHA>
__device__ inline int swz_a(int row) {
  if constexpr (CHA == 8) return (row & 7) ^ ((row >> 3) & 7);
  else return (row >> 2) & 3;
}
template <int CHB>
__device__ inline int swz_b(int krow) {
  if constexpr (CHB == 16) return (2 * (krow & 3)) ^ (8 * ((krow >> 3) & 1));
  else return 2 * (krow & 3);
}

template <int BM, int BN, int BK, int NS>
__global__ __launch_bounds__(256) void tile_gemm_dma_kernel(const uint16_t *__restrict__ A,
                                                            const uint16_t *__restrict__ B,
                                                            void *__restrict__ C, PairSrc src,
                                                            GemmGeom g) {
#if defined(__HIP_DEVICE_COMPILE__)  // device-only body (LDS address-space casts, gfx950 asm)
  constexpr int A_ROWB = BK * 2;               // bytes per A row of a stage
  constexpr int CHA = A_ROWB / 16;             // 16-byte chunks per A row
  constexpr int A_BYTES = BM * A_ROWB;         // [BM][BK] bf16
  constexpr int B_ROWB = BN * 2;               // bytes per k-row of B
  constexpr int CHB = B_ROWB / 16;             // 16-byte chunks per B k-row
  constexpr int B_BYTES = BK * B_ROWB;
  constexpr int SLOT = A_BYTES + B_BYTES;
  constexpr int A_BLOCKS = A_BYTES / 1024;     // 1 KB per wave-wide load
  constexpr int B_BLOCKS = B_BYTES / 1024;
  static_assert(A_BLOCKS % 4 == 0 && B_BLOCKS % 4 == 0, "blocks split over 4 waves");
  constexpr int LPS = A_BLOCKS / 4 + B_BLOCKS / 4;  // load instructions per wave per stage
  static_assert(NS >= 2 && NS <= 6 && (NS - 2) * LPS < 64, "ring depth / vmcnt range");
  static_assert(BK == 32 || BK == 64, "stage depth");
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int FM = WM / 16, FN = WN / 16;
  __shared__ __align__(1024) unsigned char ring[NS * SLOT];
  const uint32_t ring_lds = static_cast<uint32_t>(
      reinterpret_cast<size_t>((__attribute__((address_space(3))) unsigned char *)ring));

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  int64_t lb = xcd_logical_block(live_blocks(src, g.nblocks * g.mblocks * g.batch));
  const int64_t nb = lb % g.nblocks;
  lb /= g.nblocks;
  const int64_t mb = lb % g.mblocks;
  lb /= g.mblocks;
  const int64_t bi = lb % g.batch;
  const int64_t seg = lb / g.batch;
  if (seg_dead(src, seg)) return;
  int64_t q0, q1;
  seg_range(src, seg, &q0, &q1);
  const int nkc = static_cast<int>(g.k / BK);
  const int64_t stages = (q1 - q0) * nkc;

  // Per-lane source offsets inside a stage (elements), fixed for the kernel.
  int64_t a_src[A_BLOCKS / 4], b_src[B_BLOCKS / 4];
#pragma unroll
  for (int v = 0; v < A_BLOCKS / 4; ++v) {
    const int blk = v * 4 + wave;
    const int row = blk * (1024 / A_ROWB) + lane / CHA;
    const int c = (lane % CHA) ^ swz_a<CHA>(row);
    a_src[v] = row * g.a_sm + c * 8;
  }
#pragma unroll
  for (int v = 0; v < B_BLOCKS / 4; ++v) {
    const int blk = v * 4 + wave;
    const int krow = blk * (64 / CHB) + lane / CHB;
    const int j = (lane % CHB) ^ swz_b<CHB>(krow);
    b_src[v] = krow * g.b_sk + j * 8;
  }
  const int64_t a_off0 = bi * g.a_sb + mb * BM * g.a_sm;
  const int64_t b_off0 = bi * g.b_sb + nb * BN;

  // issue cursor (runs NS-1 stages ahead of the compute cursor)
  int64_t iq = q0;
  int ikc = 0;
  PairTiles icur = stages > 0 ? load_pair_uniform(src, q0) : PairTiles{0, 0, false};
  uint32_t okmask = 0;  // bit s % 32: stage s holds a valid pair
  auto issue = [&](int64_t st) {
    unsigned char *slot = ring + (st % NS) * SLOT;
    const uint16_t *ab = A + icur.at * g.a_elems + a_off0 + ikc * BK;
    const uint16_t *bb = B + icur.bt * g.b_elems + b_off0 + ikc * BK * g.b_sk;
#pragma unroll
    for (int v = 0; v < A_BLOCKS / 4; ++v)
      __builtin_amdgcn_global_load_lds(ab + a_src[v], EJ_LDS(slot + (v * 4 + wave) * 1024), 16, 0,
                                       0);
#pragma unroll
    for (int v = 0; v < B_BLOCKS / 4; ++v)
      __builtin_amdgcn_global_load_lds(bb + b_src[v],
                                       EJ_LDS(slot + A_BYTES + (v * 4 + wave) * 1024), 16, 0, 0);
    okmask = (okmask & ~(1u << (st & 31))) | ((icur.ok ? 1u : 0u) << (st & 31));
    if (++ikc == nkc) {
      ikc = 0;
      ++iq;
      if (iq < q1) icur = load_pair_uniform(src, iq);
    }
  };

  f32x4_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int s0 = 0; s0 < NS - 1; ++s0)
    if (s0 < stages) issue(s0);

  for (int64_t st = 0; st < stages; ++st) {
    const int64_t later = stages - 1 - st < NS - 2 ? stages - 1 - st : NS - 2;
    wait_stage<NS, LPS>(static_cast<int>(later));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (st + NS - 1 < stages) issue(st + NS - 1);
    if (!((okmask >> (st & 31)) & 1u)) continue;  // uniform: the pair's index is invalid
    const unsigned char *as = ring + (st % NS) * SLOT;
    const uint32_t bs_lds = ring_lds + static_cast<uint32_t>((st % NS) * SLOT + A_BYTES);
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks) {
      bf16x8_t af[FM];
      i32x4_t bq[FN];
      const int ch = ks * 4 + (lane >> 4);
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int row = wm * WM + i * 16 + (lane & 15);
        const int phys = ch ^ swz_a<CHA>(row);
        af[i] = *reinterpret_cast<const bf16x8_t *>(as + row * A_ROWB + phys * 16);
      }
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int n0 = wn * WN + j * 16;
        const int t = (lane & 15) >> 2, qq = lane & 3;
        const int jc = (n0 >> 3) + (qq >> 1);
        i32x2_t h[2];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const int krow = ks * 32 + (lane >> 4) * 8 + hh * 4 + t;
          const int phys = jc ^ swz_b<CHB>(krow);
          h[hh] = ds_read_tr16_b64(bs_lds + krow * B_ROWB + phys * 16 + (qq & 1) * 8);
        }
        bq[j] = i32x4_t{h[0][0], h[0][1], h[1][0], h[1][1]};
      }
      lgkm_wait_all<FN>(bq);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              af[i], __builtin_bit_cast(bf16x8_t, bq[j]), acc[i][j], 0, 0, 0);
    }
  }

  const int64_t c0 = seg * g.c_elems + bi * g.c_sb + mb * BM * g.c_sm + nb * BN * g.c_sn;
  auto store = [&](auto *cb) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = wm * WM + i * 16 + (lane >> 4) * 4 + r;
          const int col = wn * WN + j * 16 + (lane & 15);
          put_out(cb + row * g.c_sm + col * g.c_sn, acc[i][j][r]);
        }
  };
  if (g.out_bf16) store(static_cast<uint16_t *>(C) + c0);
  else store(static_cast<float *>(C) + c0);
#endif
}

// ---------------------------------------------------------------------------
// Grouped segment GEMM: G consecutive output segments per workgroup,
// operands streamed HBM -> LDS ring (bf16 or fp32).
//
// Consecutive segments often contract the same sequence of lhs tiles: an
// lhs row against a dense rhs gives segments (i, k), (i, k+1), ... that all
// pair A(i, j) with B(j, k), B(j, k+1), ... over the same j.  One workgroup
// then computes G of them at once: every stage streams one lhs K-chunk and
// G rhs K-chunks into the LDS ring, so an lhs chunk is fetched once per G
// output tiles, and the workgroup holds G output tiles of accumulators.
// The workgroup checks that property on its own pairs.  A group without it
// (different lengths or lhs tiles, fewer than G live segments, an invalid
// index) runs pair by pair in plan order, each stage feeding only the waves
// of that pair's segment, so every plan gives the results of G = 1.
//
// The tile indices of the group's pairs are read once, one pair per lane,
// and passed to the issue loop with readlane, so issuing a stage waits on
// nothing but the ring.  Every stage is one K-chunk of 32 of both operands,
// copied with 16-byte direct loads (global_load_lds_dwordx4) whose per-lane
// source addresses are permuted so that the chunks land swizzled in LDS.
// NW waves tile the group's BM x (G * BN) output as WGM x (NW / WGM); each
// wave's columns lie in one segment.  The operand policy (SegOpBf16,
// SegOpF32) fixes the LDS layout, the swizzles and the MFMA loop.

__device__ inline void pair_tile_idx(const PairSrc &s, int64_t q, int32_t *a, int32_t *b) {
  const int64_t p = s.perm ? s.perm[q] : q;
  const int64_t at = s.lidx ? s.lidx[p] : p;
  const int64_t bt = s.ridx ? s.ridx[p] : p;
  const bool ok = at >= 0 && at < s.n_a_tiles && bt >= 0 && bt < s.n_b_tiles;
  *a = ok ? static_cast<int32_t>(at) : -1;
  *b = ok ? static_cast<int32_t>(bt) : -1;
}

__device__ inline int32_t lane_value(int32_t v, int lane) {
  return __builtin_amdgcn_readlane(v, lane);
}

typedef float f32x2_t __attribute__((ext_vector_type(2)));

// bf16 operands, v_mfma_f32_16x16x32_bf16, in either layout per operand.
// The MFMA takes, per lane l, 8 consecutive k of row m = l % 16 (lhs) or of
// column n = l % 16 (rhs).  An operand whose contraction dimension is
// contiguous in its tile ("k-rows": lhs [m][k], or rhs [n][k] when AT / BT
// say so) is staged as [rows][32] (64-byte rows, 16-byte chunk c of row r at
// c ^ ((r >> 2) & 3)) and read with one 16-byte LDS read per fragment.  An
// operand whose free dimension is contiguous ("k-major": rhs [k][n], or lhs
// [k][m]) is staged as [32][cols] as tile_gemm_dma_kernel lays it out and
// read with two ds_read_b64_tr_b16 per fragment, which transpose 16-bit
// elements across the lanes of a group.  The forward 'ij,jk->ik' uses
// k-rows lhs and k-major rhs (AT = BT = false); the backward's 'ik,jk->ij'
// reads its rhs as k-rows (BT) and 'ij,ik->jk' its lhs as k-major (AT).
template <int BM_, int BN_, bool AT_ = false, bool BT_ = false>
struct SegOpBf16 {
  using elem = uint16_t;
  using a_elem = uint16_t;
  using b_elem = uint16_t;
  static constexpr bool kBf16 = true, kSplit = false, kSplitB = false, AT = AT_, BT = BT_;
  static constexpr int BM = BM_, BN = BN_, BK = 32;
  static constexpr int A_ROWB = AT ? BM * 2 : BK * 2, CHA = A_ROWB / 16, A_BYTES = BM * BK * 2;
  static constexpr int B_ROWB = BT ? BK * 2 : BN * 2, CHB = B_ROWB / 16, B_BYTES = BK * BN * 2;
  static_assert((AT ? (CHA == 8 || CHA == 16) : CHA == 4) &&
                    (BT ? CHB == 4 : (CHB == 8 || CHB == 16)),
                "row widths");

  // Element offset (inside a stage) of the 16 bytes that `lane` copies into
  // LDS block `blk` (1 KB) of a k-rows chunk (rows of 64 bytes; `stride` =
  // the tile's row stride) or of a k-major chunk with CH 16-byte chunks per
  // k-row (`stride` = the tile's k stride).
  __device__ static uint32_t krows_src(int blk, int lane, int64_t stride) {
    const int row = blk * 16 + lane / 4;
    const int c = (lane % 4) ^ swz_a<4>(row);
    return static_cast<uint32_t>(row * stride + c * 8);
  }
  template <int CH>
  __device__ static uint32_t kmajor_src(int blk, int lane, int64_t stride) {
    const int krow = blk * (64 / CH) + lane / CH;
    const int j = (lane % CH) ^ swz_b<CH>(krow);
    return static_cast<uint32_t>(krow * stride + j * 8);
  }
  __device__ static uint32_t a_src(int blk, int lane, const GemmGeom &g) {
    if constexpr (AT) return kmajor_src<CHA>(blk, lane, g.a_sk);
    else return krows_src(blk, lane, g.a_sm);
  }
  __device__ static uint32_t b_src(int blk, int lane, const GemmGeom &g) {
    if constexpr (BT) return krows_src(blk, lane, g.b_sn);
    else return kmajor_src<CHB>(blk, lane, g.b_sk);
  }

  // Per-lane LDS read offsets (bytes inside a slot).  A k-rows operand needs
  // one: its swizzle depends on the row inside 16 only, so fragment f sits
  // f * 16 rows further.  A k-major operand needs one per fragment (the
  // swizzle moves 16-byte chunks); of its two transpose reads (k rows t and
  // 4 + t of the lane group's 8) the second has the same swizzle, 4 rows
  // further: an immediate offset.  Order: lhs offsets, then rhs offsets.
  template <int FM>
  static constexpr int n_ra = AT ? FM : 1;
  template <int FN>
  static constexpr int n_rb = BT ? 1 : FN;
  template <int FM, int FN>
  static constexpr int n_rd = n_ra<FM> + n_rb<FN>;

  __device__ static uint32_t krows_rd(int row0, int rowb, int lane) {
    return static_cast<uint32_t>((row0 + (lane & 15)) * rowb +
                                 (((lane >> 4) ^ swz_a<4>(lane & 15)) * 16));
  }
  template <int CH>
  __device__ static uint32_t kmajor_rd(int col0, int rowb, int lane) {
    const int t = (lane & 15) >> 2, qq = lane & 3;
    const int jc = (col0 >> 3) + (qq >> 1);
    const int krow = (lane >> 4) * 8 + t;
    const int phys = jc ^ swz_b<CH>(krow);
    return static_cast<uint32_t>(krow * rowb + phys * 16 + (qq & 1) * 8);
  }

  template <int FM, int FN>
  __device__ static void read_offsets(uint32_t (&rd)[n_rd<FM, FN>], int row0, int wcol,
                                      uint32_t b_region, int lane) {
    if constexpr (AT) {
#pragma unroll
      for (int i = 0; i < FM; ++i) rd[i] = kmajor_rd<CHA>(row0 + i * 16, A_ROWB, lane);
    } else {
      rd[0] = krows_rd(row0, A_ROWB, lane);
    }
    constexpr int o = n_ra<FM>;
    if constexpr (BT) {
      rd[o] = b_region + krows_rd(wcol, B_ROWB, lane);
    } else {
#pragma unroll
      for (int j = 0; j < FN; ++j) rd[o + j] = b_region + kmajor_rd<CHB>(wcol + j * 16, B_ROWB, lane);
    }
  }
};

// fp32 operands, lhs [m][k] and rhs [k][n] tiles, v_mfma_f32_16x16x4f32.
// The 32 k of a stage are split over 8 MFMAs so that lane group g = lane / 16
// of MFMA 4h + c takes k = 16h + 4g + c: each lane then reads its lhs values
// of four MFMAs with one 16-byte read (chunk 4h + g of its row), and its rhs
// values as four 4-byte reads of rows 16h + 4g + c.  The order of the k terms
// inside the fp32 sum differs from k-major by construction; the contraction
// is the same.
// LDS: lhs chunk [BM][32] (128-byte rows, chunk c of row r at
// c ^ (r & 7) ^ ((r >> 3) & 1)); rhs chunk [32][BN] (chunk c of k-row r at
// c ^ 4 ((r >> 2) & 3), so the four lane groups of a read hit four bank
// quarters).
template <int BM_, int BN_>
struct SegOpF32 {
  using elem = float;
  using a_elem = float;
  using b_elem = float;
  static constexpr bool kBf16 = false, kSplit = false, kSplitB = false, AT = false, BT = false;
  static constexpr int BM = BM_, BN = BN_, BK = 32;
  static constexpr int A_ROWB = BK * 4, CHA = A_ROWB / 16, A_BYTES = BM * A_ROWB;
  static constexpr int B_ROWB = BN * 4, CHB = B_ROWB / 16, B_BYTES = BK * B_ROWB;
  static_assert(CHA == 8 && CHB >= 8, "row widths");

  __device__ static int swa(int row) { return (row & 7) ^ ((row >> 3) & 1); }
  __device__ static int swb(int krow) { return CHB >= 16 ? 4 * ((krow >> 2) & 3) : 4 * ((krow >> 2) & 1); }

  __device__ static uint32_t a_src(int blk, int lane, const GemmGeom &g) {
    const int row = blk * (1024 / A_ROWB) + lane / CHA;
    const int c = (lane % CHA) ^ swa(row);
    return static_cast<uint32_t>(row * g.a_sm + c * 4);
  }
  __device__ static uint32_t b_src(int blk, int lane, const GemmGeom &g) {
    const int krow = blk * (1024 / B_ROWB) + lane / CHB;
    const int c = (lane % CHB) ^ swb(krow);
    return static_cast<uint32_t>(krow * g.b_sk + c * 4);
  }

  // Per-lane LDS read offsets (rd[h], h = 0, 1: lhs chunk 4h + g of row
  // row0 + (lane & 15); rd[2 + j]: column wcol + 16j + (lane & 15) of k-row
  // 4g).  The MFMA loop is seg_gemm_kernel's.
  template <int FM, int FN>
  static constexpr int n_rd = 2 + FN;

  template <int FM, int FN>
  __device__ static void read_offsets(uint32_t (&rd)[n_rd<FM, FN>], int row0, int wcol,
                                      uint32_t b_region, int lane) {
    const int row = row0 + (lane & 15), g = lane >> 4;
#pragma unroll
    for (int h = 0; h < 2; ++h)
      rd[h] = static_cast<uint32_t>(row * A_ROWB + (((4 * h + g) ^ swa(row)) * 16));
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int col = wcol + j * 16 + (lane & 15);
      const int krow = 4 * g;  // rows 16h + 4g + c share this swizzle
      rd[2 + j] = b_region + static_cast<uint32_t>(krow * B_ROWB +
                                                   (((col >> 2) ^ swb(krow)) * 16) + (col & 3) * 4);
    }
  }
};

// An fp32 lhs [m][k] against an exactly-bf16 rhs [n][k] (the backward's lhs
// gradient 'ik,jk->ij' under an fp32 cotangent with bf16 operands).  The
// lhs stage is fp32 in LDS, laid out as SegOpF32's ([BM][32], 128-byte rows,
// chunk c of row r at c ^ (r & 7) ^ ((r >> 3) & 1)); the rhs stage is bf16
// k-rows as SegOpBf16's.  At read time each lane's 8 fp32 lhs values (k
// 8g .. 8g + 7 of its row, chunks 2g and 2g + 1) are split into three bf16
// terms whose sum is the value exactly (split3), and each product runs as
// three v_mfma_f32_16x16x32_bf16 into one fp32 accumulator: with the rhs
// exact in bf16, every partial product is exact and the sums are fp32, as
// in an fp32 product.
template <int BM_, int BN_>
struct SegOpSplit {
  using elem = void;
  using a_elem = float;
  using b_elem = uint16_t;
  static constexpr bool kBf16 = false, kSplit = true, kSplitB = false, AT = false, BT = true;
  static constexpr int BM = BM_, BN = BN_, BK = 32;
  static constexpr int A_ROWB = BK * 4, CHA = A_ROWB / 16, A_BYTES = BM * A_ROWB;
  static constexpr int B_ROWB = BK * 2, CHB = B_ROWB / 16, B_BYTES = BN * B_ROWB;
  static_assert(CHA == 8 && CHB == 4, "row widths");

  __device__ static int swa(int row) { return (row & 7) ^ ((row >> 3) & 1); }
  __device__ static uint32_t a_src(int blk, int lane, const GemmGeom &g) {
    const int row = blk * (1024 / A_ROWB) + lane / CHA;
    const int c = (lane % CHA) ^ swa(row);
    return static_cast<uint32_t>(row * g.a_sm + c * 4);
  }
  __device__ static uint32_t b_src(int blk, int lane, const GemmGeom &g) {
    return SegOpBf16<BM_, BN_, false, true>::krows_src(blk, lane, g.b_sn);
  }

  // rd[0], rd[1]: lhs chunks 2g and 2g + 1 of row row0 + (lane & 15) (the
  // swizzle depends on the row inside 16 only, so fragment i is 16 rows
  // further); rd[2]: the rhs k-row read of SegOpBf16 (fragment j 16 columns
  // further).
  template <int FM, int FN>
  static constexpr int n_rd = 3;

  template <int FM, int FN>
  __device__ static void read_offsets(uint32_t (&rd)[n_rd<FM, FN>], int row0, int wcol,
                                      uint32_t b_region, int lane) {
    const int row = row0 + (lane & 15), g = lane >> 4;
    rd[0] = static_cast<uint32_t>(row * A_ROWB + (((2 * g) ^ swa(row)) * 16));
    rd[1] = static_cast<uint32_t>(row * A_ROWB + (((2 * g + 1) ^ swa(row)) * 16));
    rd[2] = b_region + SegOpBf16<BM_, BN_, false, true>::krows_rd(wcol, B_ROWB, lane);
  }
};

// x = hi + mid + lo exactly, each a bf16: hi keeps the top 8 significand bits
// of x (truncation), mid the next 8 of the remainder, lo the rest (x - hi and
// its remainder are exact in fp32).  A non-finite x goes to hi alone (a NaN
// keeps a quiet bit).  Packed two values per 32-bit word, element 0 low.
__device__ inline void split3_pair(float x0, float x1, uint32_t &hi, uint32_t &mid,
                                   uint32_t &lo) {
  auto one = [](float x, uint32_t &h, uint32_t &m, uint32_t &l) {
    const uint32_t b = __builtin_bit_cast(uint32_t, x);
    if ((b & 0x7F800000u) == 0x7F800000u) {
      h = (b >> 16) | ((b & 0x007FFFFFu) ? 0x0040u : 0u);
      m = 0;
      l = 0;
      return;
    }
    const float fh = __builtin_bit_cast(float, b & 0xFFFF0000u);
    const float r = x - fh;
    const uint32_t rb = __builtin_bit_cast(uint32_t, r);
    const float fm = __builtin_bit_cast(float, rb & 0xFFFF0000u);
    const float q = r - fm;
    h = b >> 16;
    m = rb >> 16;
    l = __builtin_bit_cast(uint32_t, q) >> 16;
  };
  uint32_t h0, m0, l0, h1, m1, l1;
  one(x0, h0, m0, l0);
  one(x1, h1, m1, l1);
  hi = h0 | (h1 << 16);
  mid = m0 | (m1 << 16);
  lo = l0 | (l1 << 16);
}

// An exactly-bf16 lhs [k][m] against an fp32 rhs [k][n] (the backward's rhs
// gradient 'ij,ik->jk' under an fp32 cotangent with bf16 operands).  The lhs
// stage is SegOpBf16's k-major one (transpose reads); the rhs stage is fp32
// [32][BN] (512-byte k-rows for BN = 128) with 16-byte chunk c of k-row r at
// c ^ 4 ((r >> 3) & 3), so that the four lane groups of a read (k-rows 8g + t)
// hit four different bank quarters.  Each lane reads its 8 fp32 rhs values
// (k 8g .. 8g + 7 of its column) with eight 4-byte reads, splits them into
// three bf16 terms (split3_pair) and each product runs as three
// v_mfma_f32_16x16x32_bf16.
template <int BM_, int BN_>
struct SegOpSplitB {
  using elem = void;
  using a_elem = uint16_t;
  using b_elem = float;
  static constexpr bool kBf16 = false, kSplit = false, kSplitB = true, AT = true, BT = false;
  static constexpr int BM = BM_, BN = BN_, BK = 32;
  static constexpr int A_ROWB = BM * 2, CHA = A_ROWB / 16, A_BYTES = BM * BK * 2;
  static constexpr int B_ROWB = BN * 4, CHB = B_ROWB / 16, B_BYTES = BK * B_ROWB;
  static_assert(BN == 128 && (CHA == 8 || CHA == 16), "row widths");
  using BfOp = SegOpBf16<BM_, BN_, true, false>;

  __device__ static int swb(int krow) { return 4 * ((krow >> 3) & 3); }
  __device__ static uint32_t a_src(int blk, int lane, const GemmGeom &g) {
    return BfOp::a_src(blk, lane, g);
  }
  __device__ static uint32_t b_src(int blk, int lane, const GemmGeom &g) {
    const int krow = blk * (1024 / B_ROWB) + lane / CHB;
    const int c = (lane % CHB) ^ swb(krow);
    return static_cast<uint32_t>(krow * g.b_sk + c * 4);
  }

  // rd[i] (i < FM): the lhs transpose reads of SegOpBf16 (fragment i);
  // rd[FM + j]: k-row 8g of column wcol + 16 j + (lane & 15) (the swizzle is
  // the same for its 8 k-rows, which follow at 512-byte steps).
  template <int FM, int FN>
  static constexpr int n_rd = FM + FN;

  template <int FM, int FN>
  __device__ static void read_offsets(uint32_t (&rd)[n_rd<FM, FN>], int row0, int wcol,
                                      uint32_t b_region, int lane) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
      rd[i] = BfOp::template kmajor_rd<CHA>(row0 + i * 16, A_ROWB, lane);
    const int g = lane >> 4;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int n = wcol + 16 * j + (lane & 15);
      const int c = (n >> 2) ^ swb(8 * g);
      rd[FM + j] = b_region + static_cast<uint32_t>(8 * g * B_ROWB + c * 16 + (n & 3) * 4);
    }
  }
};

template <class Op, int NS, int G, int WGM, int NW, bool MULTI>
__global__ __launch_bounds__(NW * 64, 2) void seg_gemm_kernel(const typename Op::a_elem *__restrict__ A,
                                                           const typename Op::b_elem *__restrict__ B,
                                                           void *__restrict__ C, PairSrc src,
                                                           GemmGeom g, int64_t n_seg, int spw,
                                                           int mb_loop) {
#if defined(__HIP_DEVICE_COMPILE__)
  using TA = typename Op::a_elem;
  using TB = typename Op::b_elem;
  constexpr int BM = Op::BM, BN = Op::BN, BK = Op::BK;
  constexpr int WGN = NW / WGM;
  constexpr int WM = BM / WGM, WN = G * BN / WGN;
  static_assert(WGM * WGN == NW && WM % 16 == 0 && WN % 16 == 0 && BN % WN == 0, "wave tiling");
  constexpr int FM = WM / 16, FN = WN / 16;
  constexpr int A_BYTES = Op::A_BYTES, B_BYTES = Op::B_BYTES;
  constexpr int SLOT = A_BYTES + G * B_BYTES;
  constexpr int LPA = A_BYTES / (1024 * NW), LPB = B_BYTES / (1024 * NW);  // 1 KB loads per wave
  static_assert(LPA * 1024 * NW == A_BYTES && LPB * 1024 * NW == B_BYTES, "chunks split over waves");
  constexpr int LPS = LPA + G * LPB;
  static_assert(NS >= 2 && NS <= 5 && (NS - 1) * LPS < 64, "ring depth / vmcnt range");
  static_assert(G == 1 || G == 2 || G == 4, "group size");
  // Segments one workgroup covers: a group of G, or (G == 1) up to SMAX
  // consecutive segments computed one after another.
  constexpr int SMAX = G > 1 || !MULTI ? G : 8;
  // Stage codes, 8 bits per ring slot: the segment (inside the workgroup's
  // range) the stage feeds, kAll for a stage shared by the whole group, or
  // with kSkip set for a pair whose tile index is invalid.
  constexpr uint32_t kAll = 0x20, kSkip = 0x10;
  __shared__ __align__(1024) unsigned char ring[NS * SLOT];
  const uint32_t ring_lds = static_cast<uint32_t>(
      reinterpret_cast<size_t>((__attribute__((address_space(3))) unsigned char *)ring));

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WGN, wn = wave % WGN;
  const int wseg = (wn * WN) / BN;  // segment (inside a group) of this wave's columns
  const int wcol = (wn * WN) % BN;  // its first column inside that segment's tile
  // Work of this workgroup: m-blocks [mb0, mb0 + nmb) of segments
  // [seg0, seg0 + nls) for one n-block and one batch index.
  const int segs = G > 1 || !MULTI ? G : spw;
  int64_t nseg = n_seg;
  int64_t live = gridDim.x;  // blocks with work
  if (src.n_live) {
    const int64_t nl = ld_uniform(src.n_live, 0);
    nseg = nl < nseg ? nl : nseg;
    const int64_t per_grp = g.nblocks * (MULTI && mb_loop ? 1 : g.mblocks) * g.batch;
    const int64_t lg = (nseg + segs - 1) / segs * per_grp;
    live = lg < live ? lg : live;
  }
  int64_t lb = xcd_logical_block(live, G == 1 && !src.run_order ? kXcdRun : 0);
  const int64_t nb = lb % g.nblocks;
  lb /= g.nblocks;
  int64_t mb0 = 0, nmb = g.mblocks;
  if (!MULTI || !mb_loop) {
    mb0 = lb % g.mblocks;
    lb /= g.mblocks;
    nmb = 1;
  }
  const int64_t bi = lb % g.batch;
  int64_t grp = lb / g.batch;
  if (grp * segs >= nseg) return;
  // A run order (for instance heaviest groups first on each XCD) replaces
  // the block's group (its n-, m- and batch blocks stay together).  Its header, run_order[0], is the number of live groups it
  // permutes (the launcher passes only an order made for groups of G): only
  // an order made for exactly ceil(nseg / G) live groups is followed, by
  // every block alike, so each live group runs once; any other order is
  // ignored as a whole.
  if (!MULTI && src.run_order) {
    const int64_t ngroups = (nseg + segs - 1) / segs;
    if (ld_uniform(src.run_order, 0) == ngroups) {
      const int64_t o = ld_uniform(src.run_order, grp + 1);
      if (o >= 0 && o < ngroups) grp = o;
    }
  }
  const int64_t seg0 = grp * segs;
  if (seg0 >= nseg) return;
  const int nls = nseg - seg0 < segs ? static_cast<int>(nseg - seg0) : segs;  // live segments
  int32_t off[SMAX + 1];  // off[s] = off[nls] for s > nls
#pragma unroll
  for (int s = 0; s <= SMAX; ++s) {
    const int64_t ss = seg0 + (s <= nls ? s : nls);
    off[s] = src.seg_off ? ld_uniform(src.seg_off, ss) : static_cast<int32_t>(ss);
  }
  const int32_t len = off[1] - off[0];
  bool uni = G > 1 && nls == G;
#pragma unroll
  for (int s = 1; s < G; ++s) uni = uni && off[s + 1] - off[s] == len;

  // Pair table, one pair per lane, 64 pairs per chunk.  Shared mode: lane t
  // holds pair t of every segment (ta = its lhs tile, tb[s] = segment s's rhs
  // tile).  Sequential mode: lane r holds the r-th pair of the workgroup's plan
  // range (ta, tb[0]) and its segment in tsg.
  // (The pair arrays are copied out of src so that no lambda refers to the
  // kernel argument itself, which would keep it in scratch memory.)
  const int32_t *const s_perm = src.perm;
  const int64_t *const s_lidx = src.lidx, *const s_ridx = src.ridx;
  const int64_t n_at = src.n_a_tiles, n_bt = src.n_b_tiles;
  int32_t ta = -1, tb[G], tsg = 0;
#pragma unroll
  for (int s = 0; s < G; ++s) tb[s] = -1;
  int chunk = -1;
  // Both loaders assign every table variable, in the same order, whatever
  // the lane holds (the compiler otherwise merges their stores through a
  // selected pointer and moves the table to scratch memory).
  auto load_shared = [&](int c) -> bool {  // whether the chunk's pairs share their lhs tiles
    const int t = c * 64 + lane;
    bool bad = false;
    int32_t na = -1, nb[G];
#pragma unroll
    for (int s = 0; s < G; ++s) nb[s] = -1;
    if (t < len) {  // loads batched per level: plan -> pair -> tiles
      int64_t p[G], a[G], b[G];
#pragma unroll
      for (int s = 0; s < G; ++s) p[s] = off[s] + t;
      if (s_perm) {
#pragma unroll
        for (int s = 0; s < G; ++s) p[s] = s_perm[p[s]];
      }
#pragma unroll
      for (int s = 0; s < G; ++s) a[s] = s_lidx ? s_lidx[p[s]] : p[s];
#pragma unroll
      for (int s = 0; s < G; ++s) b[s] = s_ridx ? s_ridx[p[s]] : p[s];
#pragma unroll
      for (int s = 0; s < G; ++s) {
        const bool ok = a[s] >= 0 && a[s] < n_at && b[s] >= 0 && b[s] < n_bt;
        bad = bad || !ok || a[s] != a[0];
        nb[s] = ok ? static_cast<int32_t>(b[s]) : -1;
      }
      na = static_cast<int32_t>(a[0]);
    }
    ta = na;
#pragma unroll
    for (int s = 0; s < G; ++s) tb[s] = nb[s];
    tsg = 0;
    chunk = c;
    return __builtin_amdgcn_ballot_w64(bad) == 0;
  };
  auto load_seq = [&](int c) {
    const int r = c * 64 + lane;
    int32_t na = -1, nb = -1, ns = 0;
    if (off[0] + r < off[SMAX]) {
      const int64_t q = off[0] + r;
      const int64_t p = s_perm ? s_perm[q] : q;
      const int64_t a = s_lidx ? s_lidx[p] : p;
      const int64_t b = s_ridx ? s_ridx[p] : p;
      const bool ok = a >= 0 && a < n_at && b >= 0 && b < n_bt;
      na = ok ? static_cast<int32_t>(a) : -1;
      nb = ok ? static_cast<int32_t>(b) : -1;
#pragma unroll
      for (int u = 1; u < SMAX; ++u) ns += q >= off[u] ? 1 : 0;
    }
    ta = na;
    tb[0] = nb;
#pragma unroll
    for (int s = 1; s < G; ++s) tb[s] = -1;
    tsg = ns;
    chunk = c;
  };
  if (uni) {
    for (int c = (len + 63) / 64 - 1; c >= 0 && uni; --c) uni = load_shared(c);
  }
  if (!uni) load_seq(0);
  const int nkc = static_cast<int>(g.k / BK);
  const int64_t npos = uni ? len : off[SMAX] - off[0];  // pairs per m-block
  const int64_t per_mb = npos * nkc;                    // stages per m-block
  const int64_t stages = per_mb * nmb;

  // Per-lane source offsets inside a stage (elements), fixed for the kernel;
  // 32-bit so that the loads take a scalar base plus a vector offset.
  uint32_t a_src[LPA], b_src[LPB];
#pragma unroll
  for (int v = 0; v < LPA; ++v) a_src[v] = Op::a_src(v * NW + wave, lane, g);
#pragma unroll
  for (int v = 0; v < LPB; ++v) b_src[v] = Op::b_src(v * NW + wave, lane, g);
  const int64_t b_off0 = bi * g.b_sb + nb * BN * g.b_sn;

  // Issue cursor: m-block imb, pair ipos, K-chunk ikc.
  int64_t imb = mb0, ipos = 0;
  int ikc = 0;
  uint64_t codes = 0;  // 8 bits per ring slot
  auto issue = [&](int64_t st) {
    if ((ipos >> 6) != chunk) {  // more than 64 pairs per m-block only
      if (uni) load_shared(static_cast<int>(ipos >> 6));
      else load_seq(static_cast<int>(ipos >> 6));
    }
    const int li = static_cast<int>(ipos & 63);
    const int32_t at = lane_value(ta, li);
    int32_t bt[G];
    uint32_t code;
    if (uni) {
#pragma unroll
      for (int s = 0; s < G; ++s) bt[s] = lane_value(tb[s], li);
      code = kAll;
    } else {
      const int32_t b0 = lane_value(tb[0], li);
#pragma unroll
      for (int s = 0; s < G; ++s) bt[s] = b0;
      code = static_cast<uint32_t>(lane_value(tsg, li)) | (at < 0 ? kSkip : 0u);
    }
    const int64_t a_tile = at < 0 ? 0 : at;
    unsigned char *slot = ring + (st % NS) * SLOT;
    const TA *ab = A + a_tile * g.a_elems + bi * g.a_sb + imb * BM * g.a_sm + ikc * BK * g.a_sk;
#pragma unroll
    for (int v = 0; v < LPA; ++v)
      __builtin_amdgcn_global_load_lds(ab + a_src[v], EJ_LDS(slot + (v * NW + wave) * 1024), 16,
                                       0, 0);
#pragma unroll
    for (int s = 0; s < G; ++s) {
      const int64_t b_tile = bt[s] < 0 ? 0 : bt[s];
      const TB *bb = B + b_tile * g.b_elems + b_off0 + ikc * BK * g.b_sk;
#pragma unroll
      for (int v = 0; v < LPB; ++v)
        __builtin_amdgcn_global_load_lds(
            bb + b_src[v], EJ_LDS(slot + A_BYTES + s * B_BYTES + (v * NW + wave) * 1024), 16, 0,
            0);
    }
    const int sh = static_cast<int>(st % NS) * 8;
    codes = (codes & ~(uint64_t(0xFF) << sh)) | (uint64_t(code) << sh);
    if (++ikc == nkc) {
      ikc = 0;
      if (++ipos == npos) {
        ipos = 0;
        ++imb;
      }
    }
  };

  f32x4_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // This wave's part of output block (segment seg0 + sseg, m-block mb):
  // the accumulators, or zeros.  (Stores issued mid-loop count in vmcnt and
  // retire in order with the ring's loads, so the next stage wait also
  // covers them; measured, that beats both an exact allowance for them and
  // fewer, wider stores after an in-quad transpose.)
  const uint32_t row0 = static_cast<uint32_t>(wm * WM + (lane >> 4) * 4);
  const uint32_t col0 = static_cast<uint32_t>(wcol + (lane & 15));
  auto block_off = [&](int sseg, int64_t mb) -> int64_t {  // in elements
    return (seg0 + sseg) * g.c_elems + bi * g.c_sb + mb * BM * g.c_sm + nb * BN * g.c_sn;
  };
  auto store_zero = [&](int sseg, int64_t mb) {
    if (sseg >= nls) return;
    auto zero = [&](auto *cb) {
      for (int i = 0; i < FM; ++i)
        for (int j = 0; j < FN; ++j)
          for (int r = 0; r < 4; ++r)
            put_out(cb + (row0 + i * 16 + r) * g.c_sm + (col0 + j * 16) * g.c_sn, 0.f);
    };
    const int64_t c0 = block_off(sseg, mb);
    if (g.out_bf16) zero(static_cast<uint16_t *>(C) + c0);
    else zero(static_cast<float *>(C) + c0);
  };

#pragma unroll
  for (int s0 = 0; s0 < NS - 1; ++s0)
    if (s0 < stages) issue(s0);

  uint32_t rd[Op::template n_rd<FM, FN>];
  Op::template read_offsets<FM, FN>(rd, wm * WM, wcol,
                                    static_cast<uint32_t>(A_BYTES + wseg * B_BYTES), lane);
  int64_t cmb = mb0;      // compute cursor's m-block
  int64_t cleft = per_mb;  // stages left in it
  for (int64_t st = 0; st < stages; ++st) {
    const int slot = static_cast<int>(st % NS);
    // The next stage goes into the slot of stage st - 1 as soon as every
    // wave is done with it, before this stage's data is waited for, so NS - 1
    // stages are in flight while the waves wait and NS - 2 while they compute.
    if (st > 0) {
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
    }
    if (st + NS - 1 < stages) issue(st + NS - 1);
    const int64_t later = stages - 1 - st < NS - 1 ? stages - 1 - st : NS - 1;
    wait_stage_in<NS, LPS>(static_cast<int>(later));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    const uint32_t code = static_cast<uint32_t>(codes >> (slot * 8)) & 0xFFu;
    // Whether this wave takes part: every wave for a shared stage or (one
    // segment per wave column group) any valid stage of a lone segment;
    // with G > 1, only the waves of the stage's segment.  Wave-uniform.
    const bool feed = !(code & kSkip) && (code == kAll || G == 1 ||
                                          (code & 0xFu) == static_cast<uint32_t>(wseg));
    if (feed) {
      uint32_t base = ring_lds + static_cast<uint32_t>(slot * SLOT);
      asm volatile("" : "+s"(base));  // keeps the read addresses per stage, not per slot
      // The stage's MFMAs (written out here: as a separate function taking the
      // accumulators by reference the compiler kept extra copies of them).
      typedef const __attribute__((address_space(3))) unsigned char *lds_ptr;
      if constexpr (Op::kSplit) {
        constexpr int A_ROWB = Op::A_ROWB, B_ROWB = Op::B_ROWB;
        i32x4_t bq[FN];
#pragma unroll
        for (int j = 0; j < FN; ++j)
          bq[j] = *reinterpret_cast<const i32x4_t *>((lds_ptr)(size_t)(base + rd[2]) +
                                                    j * 16 * B_ROWB);
        // terms[0] = lo, [1] = mid, [2] = hi of each lhs fragment
        i32x4_t terms[3][FM];
#pragma unroll
        for (int i = 0; i < FM; ++i) {
          const f32x4_t x0 = *reinterpret_cast<const f32x4_t *>((lds_ptr)(size_t)(base + rd[0]) +
                                                                i * 16 * A_ROWB);
          const f32x4_t x1 = *reinterpret_cast<const f32x4_t *>((lds_ptr)(size_t)(base + rd[1]) +
                                                                i * 16 * A_ROWB);
          uint32_t h, m, l;
          split3_pair(x0[0], x0[1], h, m, l);
          terms[2][i][0] = h; terms[1][i][0] = m; terms[0][i][0] = l;
          split3_pair(x0[2], x0[3], h, m, l);
          terms[2][i][1] = h; terms[1][i][1] = m; terms[0][i][1] = l;
          split3_pair(x1[0], x1[1], h, m, l);
          terms[2][i][2] = h; terms[1][i][2] = m; terms[0][i][2] = l;
          split3_pair(x1[2], x1[3], h, m, l);
          terms[2][i][3] = h; terms[1][i][3] = m; terms[0][i][3] = l;
        }
        // lo, then mid, then hi into each accumulator; consecutive MFMAs
        // go to different accumulators
#pragma unroll
        for (int t = 0; t < 3; ++t)
#pragma unroll
          for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                  __builtin_bit_cast(bf16x8_t, terms[t][i]), __builtin_bit_cast(bf16x8_t, bq[j]),
                  acc[i][j], 0, 0, 0);
      } else if constexpr (Op::kSplitB) {
        constexpr int A_ROWB = Op::A_ROWB, B_ROWB = Op::B_ROWB;
        i32x4_t aq[FM];
#pragma unroll
        for (int i = 0; i < FM; ++i) {
          const i32x2_t h0 = ds_read_tr16_b64(base + rd[i]);
          const i32x2_t h1 = ds_read_tr16_b64_at<4 * A_ROWB>(base + rd[i]);
          aq[i] = i32x4_t{h0[0], h0[1], h1[0], h1[1]};
        }
        lgkm_wait_all<FM>(aq);
        // terms[0] = lo, [1] = mid, [2] = hi of each rhs fragment
        i32x4_t terms[3][FN];
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          float x[8];
#pragma unroll
          for (int t = 0; t < 8; ++t)
            x[t] = *reinterpret_cast<const float *>((lds_ptr)(size_t)(base + rd[FM + j]) +
                                                    t * B_ROWB);
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            uint32_t h, m, l;
            split3_pair(x[2 * q], x[2 * q + 1], h, m, l);
            terms[2][j][q] = h; terms[1][j][q] = m; terms[0][j][q] = l;
          }
        }
#pragma unroll
        for (int t = 0; t < 3; ++t)
#pragma unroll
          for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                  __builtin_bit_cast(bf16x8_t, aq[i]), __builtin_bit_cast(bf16x8_t, terms[t][j]),
                  acc[i][j], 0, 0, 0);
      } else if constexpr (Op::kBf16) {
        constexpr int A_ROWB = Op::A_ROWB, B_ROWB = Op::B_ROWB;
        constexpr int RA = Op::template n_ra<FM>;
        i32x4_t aq[FM], bq[FN];
        if constexpr (Op::AT) {
#pragma unroll
          for (int i = 0; i < FM; ++i) {
            const i32x2_t h0 = ds_read_tr16_b64(base + rd[i]);
            const i32x2_t h1 = ds_read_tr16_b64_at<4 * A_ROWB>(base + rd[i]);
            aq[i] = i32x4_t{h0[0], h0[1], h1[0], h1[1]};
          }
        } else {
#pragma unroll
          for (int i = 0; i < FM; ++i)
            aq[i] = *reinterpret_cast<const i32x4_t *>((lds_ptr)(size_t)(base + rd[0]) +
                                                      i * 16 * A_ROWB);
        }
        if constexpr (Op::BT) {
#pragma unroll
          for (int j = 0; j < FN; ++j)
            bq[j] = *reinterpret_cast<const i32x4_t *>((lds_ptr)(size_t)(base + rd[RA]) +
                                                      j * 16 * B_ROWB);
        } else {
#pragma unroll
          for (int j = 0; j < FN; ++j) {
            const i32x2_t h0 = ds_read_tr16_b64(base + rd[RA + j]);
            const i32x2_t h1 = ds_read_tr16_b64_at<4 * B_ROWB>(base + rd[RA + j]);
            bq[j] = i32x4_t{h0[0], h0[1], h1[0], h1[1]};
          }
        }
        if constexpr (Op::AT) lgkm_wait_all<FM>(aq);
        if constexpr (!Op::BT) lgkm_wait_all<FN>(bq);
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                __builtin_bit_cast(bf16x8_t, aq[i]), __builtin_bit_cast(bf16x8_t, bq[j]),
                acc[i][j], 0, 0, 0);
      } else {
        constexpr int A_ROWB = Op::A_ROWB, B_ROWB = Op::B_ROWB;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          f32x4_t af[FM];
          float bv[FN][4];
#pragma unroll
          for (int i = 0; i < FM; ++i)
            af[i] = *reinterpret_cast<const f32x4_t *>((lds_ptr)(size_t)(base + rd[h]) +
                                                      i * 16 * A_ROWB);
#pragma unroll
          for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int c = 0; c < 4; ++c)
              bv[j][c] = *reinterpret_cast<const float *>((lds_ptr)(size_t)(base + rd[2 + j]) +
                                                         (16 * h + c) * B_ROWB);
#pragma unroll
          for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
              for (int j = 0; j < FN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i][c], bv[j][c], acc[i][j],
                                                                 0, 0, 0);
        }
      }
    }
    // Output after the last stage of an output block: the end of an m-block,
    // or (one segment per wave column group) the end of a segment's stages.
    // A single-unit workgroup (!MULTI) writes once, after the loop.
    if constexpr (!MULTI) continue;
    bool done = --cleft == 0;
    if constexpr (G == 1) {
      if (!done && !uni) {
        const uint32_t nxt = static_cast<uint32_t>(codes >> (((st + 1) % NS) * 8)) & 0xFu;
        done = nxt != (code & 0xFu);
      }
    }
    if (done) {
      const int sseg = G > 1 ? wseg : static_cast<int>(code & 0xFu);
      if (sseg < nls) {
        // Strides made opaque here, so that the store offsets are formed at
        // the store and not hoisted out of the stage loop into registers.
        int32_t csm = static_cast<int32_t>(g.c_sm), csn = static_cast<int32_t>(g.c_sn);
        asm volatile("" : "+s"(csm), "+s"(csn));
        const uint32_t o0 = row0 * csm + col0 * csn;
        auto store = [&](auto *cb) {
#pragma unroll
          for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
              for (int r = 0; r < 4; ++r)
                put_out(cb + o0 + (i * 16 + r) * csm + j * 16 * csn, acc[i][j][r]);
        };
        const int64_t c0 = block_off(sseg, cmb);
        if (g.out_bf16) store(static_cast<uint16_t *>(C) + c0);
        else store(static_cast<float *>(C) + c0);
      }
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      if (cleft == 0) {
        ++cmb;
        cleft = per_mb;
      }
    }
  }
  if constexpr (!MULTI) {
    if (wseg < nls) {
      auto store = [&](auto *cb) {
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const uint32_t o = static_cast<uint32_t>((row0 + i * 16 + r) * g.c_sm +
                                                       (col0 + j * 16) * g.c_sn);
              put_out(cb + o, acc[i][j][r]);
            }
      };
      const int64_t c0 = block_off(wseg, mb0);
      if (g.out_bf16) store(static_cast<uint16_t *>(C) + c0);
      else store(static_cast<float *>(C) + c0);
    }
    return;
  }
  // Every output block is written once, also where no stage fed it: a
  // segment without pairs (a caller's plan may hold one) or a workgroup with
  // no stages at all gets zeros.
  if constexpr (G == 1) {
#pragma unroll
    for (int s = 0; s < SMAX; ++s)
      if (s < nls && off[s + 1] == off[s])
        for (int64_t mb = mb0; mb < mb0 + nmb; ++mb) store_zero(s, mb);
  } else {
    if (stages == 0)
      for (int64_t mb = mb0; mb < mb0 + nmb; ++mb) store_zero(wseg, mb);
  }
#endif
}

// ---------------------------------------------------------------------------
// Generic strided tile einsum (any binary string the describer accepts).
// One thread per output element; the per-pair sum is formed in fp32 and
// added to the segment total in plan order.

struct GenDesc {
  int32_t n_out, n_red;
  int64_t out_ext[EJ_MAX_LABELS], out_a[EJ_MAX_LABELS], out_b[EJ_MAX_LABELS];
  int64_t red_ext[EJ_MAX_LABELS], red_a[EJ_MAX_LABELS], red_b[EJ_MAX_LABELS];
  int64_t red_total, a_elems, b_elems, c_elems, eblocks;
  int32_t out_bf16;
};

// Arithmetic of the generic kernel.  Floating tiles (fp32, bf16): products
// and sums in fp32, the result stored as fp32 or rounded once to bf16.
// Integer tiles (int32): products and sums in two's-complement 32-bit
// arithmetic, wrapping on overflow as an integer dot in XLA does (formed in
// uint32_t, where wrapping is defined; the order of the terms then cannot
// change the result).
struct GenFloat {
  using acc = float;
  template <typename T>
  __device__ static float load(const T *p) { return to_f32(*p); }
  __device__ static void store(void *C, int64_t i, float v, bool bf16) {
    if (bf16) put_out(static_cast<uint16_t *>(C) + i, v);
    else put_out(static_cast<float *>(C) + i, v);
  }
};
struct GenInt32 {
  using acc = uint32_t;
  __device__ static uint32_t load(const int32_t *p) { return static_cast<uint32_t>(*p); }
  __device__ static void store(void *C, int64_t i, uint32_t v, bool) {
    static_cast<int32_t *>(C)[i] = static_cast<int32_t>(v);
  }
};

template <typename T, class Ar = GenFloat>
__global__ __launch_bounds__(256) void generic_einsum_kernel(const T *__restrict__ A,
                                                             const T *__restrict__ B,
                                                             void *__restrict__ C, PairSrc src,
                                                             GenDesc d) {
  using Acc = typename Ar::acc;
  const int64_t seg = blockIdx.x / d.eblocks;
  const int64_t e = (blockIdx.x % d.eblocks) * 256 + threadIdx.x;
  if (e >= d.c_elems || seg_dead(src, seg)) return;
  int64_t rem = e, aoff = 0, boff = 0;
  for (int i = d.n_out - 1; i >= 0; --i) {
    int64_t x = rem % d.out_ext[i];
    rem /= d.out_ext[i];
    aoff += x * d.out_a[i];
    boff += x * d.out_b[i];
  }
  int64_t q0, q1;
  seg_range(src, seg, &q0, &q1);
  Acc acc = 0;
  for (int64_t q = q0; q < q1; ++q) {
    int64_t at, bt;
    if (!pair_tiles(src, q, &at, &bt)) continue;
    const T *a = A + at * d.a_elems + aoff;
    const T *b = B + bt * d.b_elems + boff;
    Acc pacc = 0;
    int64_t idx[EJ_MAX_LABELS] = {0};
    int64_t ra = 0, rb = 0;
    for (int64_t r = 0; r < d.red_total; ++r) {
      pacc += Ar::load(a + ra) * Ar::load(b + rb);
      // odometer increment over the contracted labels (last fastest)
      for (int i = d.n_red - 1; i >= 0; --i) {
        idx[i]++;
        ra += d.red_a[i];
        rb += d.red_b[i];
        if (idx[i] < d.red_ext[i]) break;
        ra -= d.red_a[i] * d.red_ext[i];
        rb -= d.red_b[i] * d.red_ext[i];
        idx[i] = 0;
      }
    }
    acc += pacc;
  }
  Ar::store(C, seg * d.c_elems + e, acc, d.out_bf16 != 0);
}

// ---------------------------------------------------------------------------
// Dispatch.

template <typename T, int BM, int BN, int BK>
int launch_gemm_layout(bool a_direct, bool b_direct, const void *A, const void *B, void *C,
                       const PairSrc &src, const GemmGeom &g, int64_t nblk, hipStream_t stream) {
  const T *a = static_cast<const T *>(A);
  const T *b = static_cast<const T *>(B);
  dim3 grid(static_cast<unsigned>(nblk)), block(256);
  if (a_direct && b_direct)
    hipLaunchKernelGGL((tile_gemm_kernel<T, BM, BN, BK, true, true>), grid, block, 0, stream, a, b, C, src, g);
  else if (a_direct)
    hipLaunchKernelGGL((tile_gemm_kernel<T, BM, BN, BK, true, false>), grid, block, 0, stream, a, b, C, src, g);
  else if (b_direct)
    hipLaunchKernelGGL((tile_gemm_kernel<T, BM, BN, BK, false, true>), grid, block, 0, stream, a, b, C, src, g);
  else
    hipLaunchKernelGGL((tile_gemm_kernel<T, BM, BN, BK, false, false>), grid, block, 0, stream, a, b, C, src, g);
  EJ_LAUNCH_CHECK();
  return EJ_OK;
}

template <typename T, int BK>
int launch_gemm_bk(int bm, int bn, bool ad, bool bd, const void *A, const void *B, void *C,
                   const PairSrc &src, const GemmGeom &g, int64_t nblk, hipStream_t s) {
#define EJ_GEMM_CASE(M_, N_) \
  if (bm == M_ && bn == N_) return launch_gemm_layout<T, M_, N_, BK>(ad, bd, A, B, C, src, g, nblk, s);
  EJ_GEMM_CASE(128, 128) EJ_GEMM_CASE(128, 64) EJ_GEMM_CASE(128, 32)
  EJ_GEMM_CASE(64, 128) EJ_GEMM_CASE(64, 64) EJ_GEMM_CASE(64, 32)
  EJ_GEMM_CASE(32, 128) EJ_GEMM_CASE(32, 64) EJ_GEMM_CASE(32, 32)
#undef EJ_GEMM_CASE
  set_error("no GEMM tile configuration for %dx%d", bm, bn);
  return EJ_E_UNSUPPORTED;
}

// Ring depth of the grouped kernels: NS stages of (BM + G * BN) x 32 operand
// elements, capped by the 160 KB of LDS.  Two stages by default: a small ring
// lets several workgroups share a CU, which hides the memory latency better
// than a deep ring in one workgroup (block-sparse fp32 and banded bf16 einsums
// ran 12-21% faster with 2 stages than with 4).
constexpr int seg_ring_depth(int slot_bytes, int want) {
  return want * slot_bytes <= 163840 ? want : 163840 / slot_bytes;
}
#ifndef EJ_SEG_NS
#define EJ_SEG_NS 2
#endif

// Work per workgroup.  Short work items leave a workgroup mostly filling and
// draining its ring, so a workgroup takes every m-block of its segments, and
// (G == 1) several consecutive segments, as long as the grid keeps at least
// kSegMinBlocks workgroups.
constexpr int64_t kSegMinBlocks = 1024;
constexpr int kSegMaxRun = 8;  // segments per workgroup when G == 1 (SMAX)

// Work split of a segment GEMM launch: whether each workgroup loops over the
// m-blocks (mb_loop), how many consecutive segments it runs when G == 1
// (spw), and the workgroups per group.
struct SegSplit {
  int mb_loop, spw;
  int64_t per_group;
  bool multi() const { return mb_loop || spw > 1; }
};
SegSplit seg_split(int G, int64_t n_seg, int64_t batch, int64_t nblocks, int64_t mblocks,
                   bool has_offsets) {
  SegSplit r;
  const int64_t groups = ceil_div(n_seg, G);
  r.per_group = batch * nblocks;  // workgroups per group, m-blocks looped inside
  r.mb_loop = mblocks > 1 && groups * r.per_group >= kSegMinBlocks ? 1 : 0;
  if (!r.mb_loop) r.per_group *= mblocks;
  r.spw = 1;
  if (G == 1 && has_offsets)
    while (r.spw < kSegMaxRun && ceil_div(n_seg, 2 * r.spw) * r.per_group >= kSegMinBlocks)
      r.spw *= 2;
  return r;
}

template <class Op, int G, int WGM, int NW, int NSW = EJ_SEG_NS>
int launch_seg_gemm_t(const void *A, const void *B, void *C, const PairSrc &src_in,
                      const GemmGeom &g, int64_t n_seg, hipStream_t stream) {
  constexpr int NS = seg_ring_depth(Op::A_BYTES + G * Op::B_BYTES, NSW);
  PairSrc src = src_in;
  if (src.order_group != G) src.run_order = nullptr;  // an order for other groups
  const int64_t groups = ceil_div(n_seg, G);
  const SegSplit sp = seg_split(G, n_seg, g.batch, g.nblocks, g.mblocks, src.seg_off != nullptr);
  const int mb_loop = sp.mb_loop, spw = sp.spw;
  const int64_t per_group = sp.per_group;
  const int64_t nblk = ceil_div(groups, spw) * per_group;
  if (nblk >= (int64_t(1) << 32)) {
    set_error("einsum launch too large");
    return EJ_E_UNSUPPORTED;
  }
  using TA = typename Op::a_elem;
  using TB = typename Op::b_elem;
  if (mb_loop || spw > 1)
    hipLaunchKernelGGL((seg_gemm_kernel<Op, NS, G, WGM, NW, true>),
                       dim3(static_cast<unsigned>(nblk)), dim3(NW * 64), 0, stream,
                       static_cast<const TA *>(A), static_cast<const TB *>(B), C, src, g, n_seg,
                       spw, mb_loop);
  else
    hipLaunchKernelGGL((seg_gemm_kernel<Op, NS, G, WGM, NW, false>),
                       dim3(static_cast<unsigned>(nblk)), dim3(NW * 64), 0, stream,
                       static_cast<const TA *>(A), static_cast<const TB *>(B), C, src, g, n_seg, 1,
                       0);
  EJ_LAUNCH_CHECK();
  return EJ_OK;
}

// bf16: 128 x 128 tiles, a group of 2 on 4 waves (2 x 2, one segment per wave
// column) with a 3-stage ring (72 KB of LDS, so two workgroups share a CU and
// one's prologue and epilogue overlap the other's stream), or one segment on
// 4 waves (2 x 2); 64 x 64 tiles on 4 waves.  One segment with a k-rows rhs
// (the lhs gradient of the backward: long segments whose lhs tiles are each
// read once) gets a 4-stage ring: 48 KB in flight per workgroup, two
// workgroups per CU.
template <bool AT, bool BT>
int launch_seg_gemm_bf16_l(int bm, int grp, const void *A, const void *B, void *C,
                           const PairSrc &src, const GemmGeom &g, int64_t n_seg,
                           hipStream_t stream) {
  if (bm == 128) {
    if (grp == 4)
      return launch_seg_gemm_t<SegOpBf16<128, 128, AT, BT>, 2, 2, 4, 3>(A, B, C, src, g, n_seg, stream);
    return launch_seg_gemm_t<SegOpBf16<128, 128, AT, BT>, 1, 2, 4, BT && !AT ? 4 : EJ_SEG_NS>(
        A, B, C, src, g, n_seg, stream);
  }
  if (grp == 4) return launch_seg_gemm_t<SegOpBf16<64, 64, AT, BT>, 4, 1, 4>(A, B, C, src, g, n_seg, stream);
  return launch_seg_gemm_t<SegOpBf16<64, 64, AT, BT>, 1, 2, 4>(A, B, C, src, g, n_seg, stream);
}

// Operand layouts: a_rows = lhs k-contiguous ([m][k]), b_rows = rhs
// k-contiguous ([n][k]).  Both operands free-dimension-contiguous is not
// instantiated (no einsum of this path produces it).
int launch_seg_gemm_bf16(int bm, int grp, bool a_rows, bool b_rows, const void *A, const void *B,
                         void *C, const PairSrc &src, const GemmGeom &g, int64_t n_seg,
                         hipStream_t stream) {
  if (a_rows && !b_rows) return launch_seg_gemm_bf16_l<false, false>(bm, grp, A, B, C, src, g, n_seg, stream);
  if (a_rows && b_rows) return launch_seg_gemm_bf16_l<false, true>(bm, grp, A, B, C, src, g, n_seg, stream);
  if (!a_rows && !b_rows) return launch_seg_gemm_bf16_l<true, false>(bm, grp, A, B, C, src, g, n_seg, stream);
  set_error("no bf16 segment GEMM for a [k][m] lhs with an [n][k] rhs");
  return EJ_E_UNSUPPORTED;
}

// fp32 on 4 waves: a group of 4 puts one segment on each wave (WGM = 1);
// one segment splits the tile into wave tiles of at least 16 x 16.
int launch_seg_gemm_f32(int bm, int bn, int grp, const void *A, const void *B, void *C,
                        const PairSrc &src, const GemmGeom &g, int64_t n_seg,
                        hipStream_t stream) {
#define EJ_F32_CASE(M_, N_, WGM1_)                                                             \
  if (bm == M_ && bn == N_)                                                                    \
    return grp == 4                                                                            \
               ? launch_seg_gemm_t<SegOpF32<M_, N_>, 4, 1, 4>(A, B, C, src, g, n_seg, stream)  \
               : launch_seg_gemm_t<SegOpF32<M_, N_>, 1, WGM1_, 4>(A, B, C, src, g, n_seg, stream);
  EJ_F32_CASE(32, 32, 2) EJ_F32_CASE(32, 64, 2) EJ_F32_CASE(64, 32, 2)
  EJ_F32_CASE(64, 64, 2) EJ_F32_CASE(128, 32, 4) EJ_F32_CASE(128, 64, 2)
#undef EJ_F32_CASE
  set_error("no fp32 segment GEMM configuration for %dx%d", bm, bn);
  return EJ_E_UNSUPPORTED;
}

int pick_block(int64_t x) { return x % 128 == 0 ? 128 : x % 64 == 0 ? 64 : x % 32 == 0 ? 32 : 0; }

// Segments per workgroup of the fused kernel that try_gemm picks for a
// descriptor with the seg_group hint, given 16-byte aligned operands: the
// group size a run order must be made for (1: the einsum does not run
// grouped).  The launcher checks the order's group size again, so an order
// made for another size is ignored, never misapplied.
int fused_group(const ej_einsum_desc *d, int32_t dtype) {
  if (!d->is_gemm || d->seg_group <= 0 || d->seg_group % 4 != 0) return 1;
  const int vec = dtype == EJ_BF16 ? 8 : 4;
  const int bm = pick_block(d->m), bn = pick_block(d->n);
  if (!bm || !bn || d->k % 32 != 0) return 1;
  if (dtype == EJ_BF16) {
    const bool a_rows = d->a_sk == 1 && d->a_sm % vec == 0;
    const bool a_cols = d->a_sm == 1 && d->a_sk % vec == 0;
    const bool b_rows = d->b_sk == 1 && d->b_sn % vec == 0;
    const bool b_cols = d->b_sn == 1 && d->b_sk % vec == 0;
    if (!((a_rows && (b_rows || b_cols)) || (a_cols && b_cols))) return 1;
    return bm == bn && bm == 128 ? 2 : bm == bn && bm == 64 ? 4 : 1;
  }
  if (d->a_sk != 1 || d->a_sm % vec != 0 || d->b_sn != 1 || d->b_sk % vec != 0) return 1;
  return (bm == 32 || bm == 64 || bm == 128) && d->n % 32 == 0 ? 4 : 1;
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }



// Chooses the MFMA path when the einsum is GEMM-shaped with tile-friendly
// extents and 16-byte aligned operand rows; returns false to fall back.
bool try_gemm(const ej_einsum_desc *d, int32_t dtype, const void *A, const void *B, void *C,
              const PairSrc &src, int64_t n_seg, hipStream_t stream, int *status) {
  if (!d->is_gemm) return false;
  const int esz = dtype == EJ_BF16 ? 2 : 4;
  const int vec = 16 / esz;
  const int bm = pick_block(d->m), bn = pick_block(d->n);
  if (!bm || !bn) return false;
  int bk;
  if (dtype == EJ_BF16) bk = d->k % 64 == 0 ? 64 : d->k % 32 == 0 ? 32 : 0;
  else bk = d->k % 32 == 0 ? 32 : d->k % 16 == 0 ? 16 : 0;
  if (!bk) return false;
  // Operand layouts: "direct" = contraction dim contiguous.
  bool ad, bd;
  if (d->a_sk == 1 && d->a_sm % vec == 0) ad = true;
  else if (d->a_sm == 1 && d->a_sk % vec == 0) ad = false;
  else return false;
  if (d->b_sk == 1 && d->b_sn % vec == 0) bd = true;
  else if (d->b_sn == 1 && d->b_sk % vec == 0) bd = false;
  else return false;
  if (d->a_elems % vec || d->b_elems % vec || d->a_sb % vec || d->b_sb % vec) return false;
  if (!aligned16(A) || !aligned16(B)) return false;
  GemmGeom g;
  g.m = d->m; g.n = d->n; g.k = d->k; g.batch = d->batch;
  g.a_sb = d->a_sb; g.a_sm = d->a_sm; g.a_sk = d->a_sk;
  g.b_sb = d->b_sb; g.b_sk = d->b_sk; g.b_sn = d->b_sn;
  g.c_sb = d->c_sb; g.c_sm = d->c_sm; g.c_sn = d->c_sn;
  g.a_elems = d->a_elems; g.b_elems = d->b_elems; g.c_elems = d->c_elems;
  g.mblocks = d->m / bm;
  g.nblocks = d->n / bn;
  g.out_bf16 = d->out_dtype == EJ_BF16;
  const int64_t nblk = n_seg * g.batch * g.mblocks * g.nblocks;
  if (nblk >= (int64_t(1) << 32)) return false;
  // bf16 with at least one operand k-contiguous: the LDS-ring kernels
  // (direct HBM -> LDS loads, transpose reads for a free-dimension-contiguous
  // operand).  Segments the caller marks as sharing their lhs tiles in runs
  // of 4 go several to a workgroup.  Otherwise a k-contiguous lhs with an
  // n-contiguous rhs runs one segment per workgroup with 64-deep K stages
  // (tile_gemm_dma_kernel), and the transposed layouts of the backward run
  // one segment per workgroup on the ring.
  if (dtype == EJ_BF16 && (ad || !bd) && d->k % 32 == 0 && bm == bn && (bm == 128 || bm == 64) &&
      src.n_a_tiles < (int64_t(1) << 31) && src.n_b_tiles < (int64_t(1) << 31)) {
    const uint16_t *a = static_cast<const uint16_t *>(A);
    const uint16_t *b = static_cast<const uint16_t *>(B);
    const bool grouped = src.seg_off && d->seg_group > 0 && d->seg_group % 4 == 0;
    if (grouped || d->k % 64 != 0 || !ad || bd) {
      *status = launch_seg_gemm_bf16(bm, grouped ? 4 : 1, ad, bd, a, b, C, src, g, n_seg, stream);
      return true;
    }
    if (bm == 128)
      hipLaunchKernelGGL((tile_gemm_dma_kernel<128, 128, EJ_DMA_BK_128, EJ_DMA_STAGES_128>),
                         dim3(static_cast<unsigned>(nblk)), dim3(256), 0, stream, a, b, C, src, g);
    else
      hipLaunchKernelGGL((tile_gemm_dma_kernel<64, 64, 64, EJ_DMA_STAGES_64>),
                         dim3(static_cast<unsigned>(nblk)), dim3(256), 0, stream, a, b, C, src, g);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
      set_error("tile_gemm_dma_kernel launch failed: %s", hipGetErrorString(e));
      *status = EJ_E_HIP;
    } else {
      *status = EJ_OK;
    }
    return true;
  }
  // fp32, k-contiguous lhs, n-contiguous rhs, K a multiple of 32, 16-byte
  // rows: the LDS-ring kernel with fp32 MFMAs (grouped like the bf16 one).
  if (dtype == EJ_F32 && ad && !bd && d->k % 32 == 0 && d->b_sn == 1 && d->b_sk % 4 == 0 &&
      (bm == 32 || bm == 64 || bm == 128) && src.n_a_tiles < (int64_t(1) << 31) &&
      src.n_b_tiles < (int64_t(1) << 31)) {
    const int fbn = d->n % 64 == 0 ? 64 : 32;
    if (d->n % fbn == 0) {
      g.nblocks = d->n / fbn;
      const bool grouped = src.seg_off && d->seg_group > 0 && d->seg_group % 4 == 0;
      *status = launch_seg_gemm_f32(bm, fbn, grouped ? 4 : 1, A, B, C, src, g, n_seg, stream);
      return true;
    }
  }
  if (dtype == EJ_BF16) {
    // 32-deep K stages for bf16 too: 32 KB of LDS, so three workgroups share
    // a CU (the backward's transposed-operand GEMMs ran 4% faster than with
    // 64-deep stages and two per CU).
    *status = launch_gemm_bk<uint16_t, 32>(bm, bn, ad, bd, A, B, C, src, g, nblk, stream);
  } else {
    *status = bk == 32 ? launch_gemm_bk<float, 32>(bm, bn, ad, bd, A, B, C, src, g, nblk, stream)
                       : launch_gemm_bk<float, 16>(bm, bn, ad, bd, A, B, C, src, g, nblk, stream);
  }
  return true;
}

int run_generic(const ej_einsum_desc *d, int32_t dtype, const void *A, const void *B, void *C,
                const PairSrc &src, int64_t n_seg, hipStream_t stream) {
  GenDesc g;
  memset(&g, 0, sizeof(g));
  g.n_out = d->n_out;
  g.n_red = d->n_red;
  g.red_total = 1;
  for (int i = 0; i < d->n_out; ++i) {
    g.out_ext[i] = d->out_ext[i];
    g.out_a[i] = d->out_a[i];
    g.out_b[i] = d->out_b[i];
  }
  for (int i = 0; i < d->n_red; ++i) {
    g.red_ext[i] = d->red_ext[i];
    g.red_a[i] = d->red_a[i];
    g.red_b[i] = d->red_b[i];
    g.red_total *= d->red_ext[i];
  }
  g.a_elems = d->a_elems;
  g.b_elems = d->b_elems;
  g.c_elems = d->c_elems;
  g.eblocks = ceil_div(d->c_elems, 256);
  g.out_bf16 = d->out_dtype == EJ_BF16;
  const int64_t nblk = n_seg * g.eblocks;
  if (nblk >= (int64_t(1) << 32)) {
    set_error("einsum launch too large");
    return EJ_E_UNSUPPORTED;
  }
  if (dtype == EJ_I32)
    hipLaunchKernelGGL((generic_einsum_kernel<int32_t, GenInt32>),
                       dim3(static_cast<unsigned>(nblk)), dim3(256), 0, stream,
                       static_cast<const int32_t *>(A), static_cast<const int32_t *>(B), C, src,
                       g);
  else if (dtype == EJ_BF16)
    hipLaunchKernelGGL(generic_einsum_kernel<uint16_t>, dim3(static_cast<unsigned>(nblk)), dim3(256),
                       0, stream, static_cast<const uint16_t *>(A),
                       static_cast<const uint16_t *>(B), C, src, g);
  else
    hipLaunchKernelGGL(generic_einsum_kernel<float>, dim3(static_cast<unsigned>(nblk)), dim3(256), 0,
                       stream, static_cast<const float *>(A), static_cast<const float *>(B), C,
                       src, g);
  EJ_LAUNCH_CHECK();
  return EJ_OK;
}

// Every element a descriptor can address must lie inside its tile: the
// kernels index tiles with these strides and no further checks.
int check_desc(const ej_einsum_desc *d) {
  int64_t a = 0, b = 0, c = 0, c_expect = 1;
  for (int i = 0; i < d->n_out; ++i) {
    EJ_CHECK_ARG(d->out_ext[i] >= 1 && d->out_a[i] >= 0 && d->out_b[i] >= 0,
                 "malformed einsum descriptor");
    a += (d->out_ext[i] - 1) * d->out_a[i];
    b += (d->out_ext[i] - 1) * d->out_b[i];
    c_expect *= d->out_ext[i];
  }
  for (int i = 0; i < d->n_red; ++i) {
    EJ_CHECK_ARG(d->red_ext[i] >= 1 && d->red_a[i] >= 0 && d->red_b[i] >= 0,
                 "malformed einsum descriptor");
    a += (d->red_ext[i] - 1) * d->red_a[i];
    b += (d->red_ext[i] - 1) * d->red_b[i];
  }
  EJ_CHECK_ARG(a < d->a_elems && b < d->b_elems && c_expect == d->c_elems,
               "einsum descriptor addresses elements outside its tiles");
  if (d->is_gemm) {
    EJ_CHECK_ARG(d->batch >= 1 && d->m >= 1 && d->n >= 1 && d->k >= 1 && d->a_sb >= 0 &&
                     d->a_sm >= 0 && d->a_sk >= 0 && d->b_sb >= 0 && d->b_sk >= 0 &&
                     d->b_sn >= 0 && d->c_sb >= 0 && d->c_sm >= 0 && d->c_sn >= 0,
                 "malformed GEMM descriptor");
    a = (d->batch - 1) * d->a_sb + (d->m - 1) * d->a_sm + (d->k - 1) * d->a_sk;
    b = (d->batch - 1) * d->b_sb + (d->k - 1) * d->b_sk + (d->n - 1) * d->b_sn;
    c = (d->batch - 1) * d->c_sb + (d->m - 1) * d->c_sm + (d->n - 1) * d->c_sn;
    EJ_CHECK_ARG(a < d->a_elems && b < d->b_elems && c < d->c_elems,
                 "GEMM descriptor addresses elements outside its tiles");
  }
  return EJ_OK;
}

// The group size of the LDS-ring launch try_gemm makes for this descriptor
// when it follows a run order (one workgroup per group: no m-block loop, no
// run of segments, one n-block, batch 1), else 0.
int ring_order_group(const ej_einsum_desc *d, int32_t dtype, int64_t n_seg, const void *A,
                     const void *B) {
  if (!d->is_gemm || dtype != EJ_BF16 || d->k % 32 != 0 || d->batch != 1) return 0;
  const int bm = pick_block(d->m), bn = pick_block(d->n);
  if (!bm || bm != bn || (bm != 128 && bm != 64) || d->m != bm || d->n != bn) return 0;
  const bool ad = d->a_sk == 1 && d->a_sm % 8 == 0, acol = d->a_sm == 1 && d->a_sk % 8 == 0;
  const bool bd = d->b_sk == 1 && d->b_sn % 8 == 0, bcol = d->b_sn == 1 && d->b_sk % 8 == 0;
  if (!(ad || acol) || !(bd || bcol) || (!ad && bd)) return 0;
  if (d->a_elems % 8 || d->b_elems % 8 || !aligned16(A) || !aligned16(B)) return 0;
  const bool grouped = d->seg_group > 0 && d->seg_group % 4 == 0;
  // the one-segment-per-workgroup DMA kernel takes no order
  if (!grouped && d->k % 64 == 0 && ad && !bd) return 0;
  const int G = grouped ? (bm == 128 ? 2 : 4) : 1;
  return seg_split(G, n_seg, 1, 1, 1, true).multi() ? 0 : G;
}

int einsum_common(const ej_einsum_desc *d, int32_t dtype, const void *A, const void *B,
                  const PairSrc &src, int64_t n_seg, void *C, hipStream_t stream) {
  EJ_CHECK_ARG(d, "desc is null");
  EJ_CHECK_ARG(dtype == EJ_F32 || dtype == EJ_BF16 || dtype == EJ_I32, "unknown dtype %d", dtype);
  EJ_CHECK_ARG((dtype == EJ_I32) == (d->out_dtype == EJ_I32) &&
                   (d->out_dtype == EJ_F32 || d->out_dtype == EJ_I32 ||
                    (d->out_dtype == EJ_BF16 && dtype == EJ_BF16)),
               "output dtype %d with operand dtype %d: outputs are fp32, bf16 for bf16 "
               "operands, int32 for int32 operands", d->out_dtype, dtype);
  EJ_CHECK_ARG(n_seg >= 0, "negative count");
  EJ_CHECK_ARG(d->n_out >= 0 && d->n_out <= EJ_MAX_LABELS && d->n_red >= 0 &&
                   d->n_red <= EJ_MAX_LABELS && d->c_elems >= 1 && d->a_elems >= 1 &&
                   d->b_elems >= 1,
               "malformed einsum descriptor");
  if (n_seg == 0) return EJ_OK;
  EJ_CHECK_ARG(A && B && C, "null pointer argument");
  EJ_TRY(check_desc(d));
  int status = EJ_OK;
  if (dtype != EJ_I32 && try_gemm(d, dtype, A, B, C, src, n_seg, stream, &status)) return status;
  return run_generic(d, dtype, A, B, C, src, n_seg, stream);
}

// ---------------------------------------------------------------------------
// Segment sum and gather.

__global__ __launch_bounds__(256) void segment_sum_vec4_kernel(const float4 *__restrict__ vals,
                                                               int64_t tile_vecs,
                                                               const int32_t *perm,
                                                               const int32_t *off, int64_t eblocks,
                                                               float4 *__restrict__ out) {
  const int64_t seg = blockIdx.x / eblocks;
  const int64_t e = (blockIdx.x % eblocks) * 256 + threadIdx.x;
  if (e >= tile_vecs) return;
  const int32_t q0 = off[seg], q1 = off[seg + 1];
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int32_t q = q0; q < q1; ++q) {
    const float4 v = vals[static_cast<int64_t>(perm[q]) * tile_vecs + e];
    acc.x += v.x;
    acc.y += v.y;
    acc.z += v.z;
    acc.w += v.w;
  }
  out[seg * tile_vecs + e] = acc;
}

// bf16 pair values, 8 per thread (one 16-byte load); fp32 sums, rounded
// to bf16 once.
__global__ __launch_bounds__(256) void segment_sum_bf16x8_kernel(const uint4 *__restrict__ vals,
                                                                 int64_t tile_vecs,
                                                                 const int32_t *perm,
                                                                 const int32_t *off,
                                                                 int64_t eblocks,
                                                                 uint4 *__restrict__ out) {
  const int64_t seg = blockIdx.x / eblocks;
  const int64_t e = (blockIdx.x % eblocks) * 256 + threadIdx.x;
  if (e >= tile_vecs) return;
  const int32_t q0 = off[seg], q1 = off[seg + 1];
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int32_t q = q0; q < q1; ++q) {
    const uint4 v = vals[static_cast<int64_t>(perm[q]) * tile_vecs + e];
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      acc[2 * h] += __uint_as_float(w[h] << 16);
      acc[2 * h + 1] += __uint_as_float(w[h] & 0xFFFF0000u);
    }
  }
  uint32_t w[4];
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    uint16_t lo, hi;
    put_out(&lo, acc[2 * h]);
    put_out(&hi, acc[2 * h + 1]);
    w[h] = static_cast<uint32_t>(lo) | (static_cast<uint32_t>(hi) << 16);
  }
  out[seg * tile_vecs + e] = make_uint4(w[0], w[1], w[2], w[3]);
}

template <typename T>
__global__ __launch_bounds__(256) void segment_sum_scalar_kernel(const T *__restrict__ vals,
                                                                 int64_t tile_elems,
                                                                 const int32_t *perm,
                                                                 const int32_t *off,
                                                                 int64_t eblocks,
                                                                 T *__restrict__ out) {
  const int64_t seg = blockIdx.x / eblocks;
  const int64_t e = (blockIdx.x % eblocks) * 256 + threadIdx.x;
  if (e >= tile_elems) return;
  float acc = 0.f;
  for (int32_t q = off[seg]; q < off[seg + 1]; ++q)
    acc += to_f32(vals[static_cast<int64_t>(perm[q]) * tile_elems + e]);
  put_out(out + seg * tile_elems + e, acc);
}

// Segment sums kept in the values' own type, one element per thread, the
// pair tiles added one after another in plan order: float64 (double sums,
// so each element's sum is formed exactly as a sequential float64 loop
// forms it) and int32 / int64 (two's-complement wrapping, formed unsigned).
template <typename T, typename Acc>
__global__ __launch_bounds__(256) void segment_sum_exact_kernel(const T *__restrict__ vals,
                                                                int64_t tile_elems,
                                                                const int32_t *perm,
                                                                const int32_t *off,
                                                                int64_t eblocks,
                                                                T *__restrict__ out) {
  const int64_t seg = blockIdx.x / eblocks;
  const int64_t e = (blockIdx.x % eblocks) * 256 + threadIdx.x;
  if (e >= tile_elems) return;
  Acc acc = 0;
  for (int32_t q = off[seg]; q < off[seg + 1]; ++q)
    acc += static_cast<Acc>(vals[static_cast<int64_t>(perm[q]) * tile_elems + e]);
  out[seg * tile_elems + e] = static_cast<T>(acc);
}

// float16 values: each addition formed in fp32 and rounded to float16, as
// numpy adds float16 arrays (so each element's sum matches the reference's
// sequential float16 additions bit for bit).
__global__ __launch_bounds__(256) void segment_sum_f16_kernel(const _Float16 *__restrict__ vals,
                                                              int64_t tile_elems,
                                                              const int32_t *perm,
                                                              const int32_t *off, int64_t eblocks,
                                                              _Float16 *__restrict__ out) {
  const int64_t seg = blockIdx.x / eblocks;
  const int64_t e = (blockIdx.x % eblocks) * 256 + threadIdx.x;
  if (e >= tile_elems) return;
  _Float16 acc = 0;
  for (int32_t q = off[seg]; q < off[seg + 1]; ++q)
    acc = static_cast<_Float16>(static_cast<float>(acc) +
                                static_cast<float>(vals[static_cast<int64_t>(perm[q]) * tile_elems + e]));
  out[seg * tile_elems + e] = acc;
}

template <typename V>
__global__ __launch_bounds__(256) void gather_kernel(const V *__restrict__ vals, int64_t n_tiles,
                                                     int64_t tile_vecs, const int64_t *idx,
                                                     int64_t eblocks, V *__restrict__ out) {
  const int64_t i = blockIdx.x / eblocks;
  const int64_t e0 = (blockIdx.x % eblocks) * (256 * 4);
  const int64_t t = idx[i];
  const bool ok = t >= 0 && t < n_tiles;
  const V *src = vals + (ok ? t : 0) * tile_vecs;
  V *dst = out + i * tile_vecs;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int64_t e = e0 + u * 256 + threadIdx.x;
    if (e < tile_vecs) {
      V v;
      if (ok) v = src[e];
      else memset(&v, 0, sizeof(V));
      dst[e] = v;
    }
  }
}

}  // namespace
}  // namespace ej

extern "C" int ej_pair_einsum(const ej_einsum_desc *desc, int32_t dtype, const void *lhs_values,
                              const void *rhs_values, int64_t n_lhs_tiles, int64_t n_rhs_tiles,
                              const int64_t *lhs_idx, const int64_t *rhs_idx, int64_t n_pairs,
                              void *out, ej_stream_t stream) {
  clear_error();
  PairSrc src{lhs_idx, rhs_idx, nullptr, nullptr, n_lhs_tiles, n_rhs_tiles, nullptr, nullptr, 0};
  return einsum_common(desc, dtype, lhs_values, rhs_values, src, n_pairs, out, as_stream(stream));
}

extern "C" int ej_segment_einsum(const ej_einsum_desc *desc, int32_t dtype, const void *lhs_values,
                                 const void *rhs_values, int64_t n_lhs_tiles,
                                 int64_t n_rhs_tiles, const int64_t *lhs_idx,
                                 const int64_t *rhs_idx, const int32_t *perm,
                                 const int32_t *seg_offsets, int64_t n_segments, void *out,
                                 ej_stream_t stream) {
  clear_error();
  EJ_CHECK_ARG(seg_offsets || n_segments == 0, "seg_offsets is null");
  PairSrc src{lhs_idx, rhs_idx, perm, seg_offsets, n_lhs_tiles, n_rhs_tiles, nullptr, nullptr, 0};
  return einsum_common(desc, dtype, lhs_values, rhs_values, src, n_segments, out,
                       as_stream(stream));
}

extern "C" int ej_segment_einsum_async(const ej_einsum_desc *desc, int32_t dtype,
                                       const void *lhs_values, const void *rhs_values,
                                       int64_t n_lhs_tiles, int64_t n_rhs_tiles,
                                       const int64_t *lhs_idx, const int64_t *rhs_idx,
                                       const int32_t *perm, const int32_t *seg_offsets,
                                       int64_t max_segments, const int64_t *n_segments_dev,
                                       const int32_t *run_order, int32_t run_order_group,
                                       void *out, ej_stream_t stream) {
  clear_error();
  EJ_CHECK_ARG(seg_offsets || max_segments == 0, "seg_offsets is null");
  EJ_CHECK_ARG(n_segments_dev, "n_segments_dev is null");
  PairSrc src{lhs_idx,     rhs_idx,     perm,           seg_offsets,
              n_lhs_tiles, n_rhs_tiles, n_segments_dev, run_order,
              run_order_group};
  return einsum_common(desc, dtype, lhs_values, rhs_values, src, max_segments, out,
                       as_stream(stream));
}

int ej::segment_einsum_order_group(const ej_einsum_desc *d, int32_t dtype, int64_t n_seg,
                                   const void *A, const void *B) {
  return ring_order_group(d, dtype, n_seg, A, B);
}

int ej::segment_einsum_ordered(const ej_einsum_desc *d, int32_t dtype, const void *A,
                               const void *B, int64_t n_a_tiles, int64_t n_b_tiles,
                               const int64_t *lidx, const int64_t *ridx, const int32_t *perm,
                               const int32_t *seg_off, int64_t n_seg, const int32_t *run_order,
                               int32_t order_group, void *out, hipStream_t stream) {
  PairSrc src{lidx, ridx, perm, seg_off, n_a_tiles, n_b_tiles, nullptr, run_order, order_group};
  return einsum_common(d, dtype, A, B, src, n_seg, out, stream);
}

bool ej::segment_einsum_split_ok(const ej_einsum_desc *d, const void *A, const void *B) {
  // fp32 k-rows lhs, bf16 k-rows rhs, 128 x 128 output blocks
  return d && d->is_gemm && d->m % 128 == 0 && d->n % 128 == 0 && d->k % 32 == 0 &&
         d->a_sk == 1 && d->a_sm % 4 == 0 && d->b_sk == 1 && d->b_sn % 8 == 0 &&
         d->a_elems % 4 == 0 && d->b_elems % 8 == 0 && d->a_sb % 4 == 0 && d->b_sb % 8 == 0 &&
         aligned16(A) && aligned16(B);
}

int ej::segment_einsum_split(const ej_einsum_desc *d, const float *A, const uint16_t *B,
                             int64_t n_a_tiles, int64_t n_b_tiles, const int64_t *lidx,
                             const int64_t *ridx, const int32_t *perm, const int32_t *seg_off,
                             int64_t n_seg, const int32_t *run_order, int32_t order_group,
                             void *out, hipStream_t stream) {
  if (!segment_einsum_split_ok(d, A, B) || !seg_off || n_a_tiles >= (int64_t(1) << 31) ||
      n_b_tiles >= (int64_t(1) << 31))
    return EJ_E_UNSUPPORTED;
  if (n_seg == 0) return EJ_OK;
  GemmGeom g;
  g.m = d->m; g.n = d->n; g.k = d->k; g.batch = d->batch;
  g.a_sb = d->a_sb; g.a_sm = d->a_sm; g.a_sk = d->a_sk;
  g.b_sb = d->b_sb; g.b_sk = d->b_sk; g.b_sn = d->b_sn;
  g.c_sb = d->c_sb; g.c_sm = d->c_sm; g.c_sn = d->c_sn;
  g.a_elems = d->a_elems; g.b_elems = d->b_elems; g.c_elems = d->c_elems;
  g.mblocks = d->m / 128;
  g.nblocks = d->n / 128;
  g.out_bf16 = d->out_dtype == EJ_BF16;
  PairSrc src{lidx, ridx, perm, seg_off, n_a_tiles, n_b_tiles, nullptr, run_order, order_group};
  return launch_seg_gemm_t<SegOpSplit<128, 128>, 1, 2, 4, 3>(A, B, out, src, g, n_seg, stream);
}

bool ej::segment_einsum_split_b_ok(const ej_einsum_desc *d, const void *A, const void *B) {
  // bf16 k-major lhs ([k][m]), fp32 k-major rhs ([k][n]), 128 x 128 blocks
  return d && d->is_gemm && d->m % 128 == 0 && d->n % 128 == 0 && d->k % 32 == 0 &&
         d->a_sm == 1 && d->a_sk % 8 == 0 && d->b_sn == 1 && d->b_sk % 4 == 0 &&
         d->a_elems % 8 == 0 && d->b_elems % 4 == 0 && d->a_sb % 8 == 0 && d->b_sb % 4 == 0 &&
         aligned16(A) && aligned16(B);
}

int ej::segment_einsum_split_b(const ej_einsum_desc *d, const uint16_t *A, const float *B,
                               int64_t n_a_tiles, int64_t n_b_tiles, const int64_t *lidx,
                               const int64_t *ridx, const int32_t *perm, const int32_t *seg_off,
                               int64_t n_seg, void *out, hipStream_t stream) {
  if (!segment_einsum_split_b_ok(d, A, B) || !seg_off || n_a_tiles >= (int64_t(1) << 31) ||
      n_b_tiles >= (int64_t(1) << 31))
    return EJ_E_UNSUPPORTED;
  if (n_seg == 0) return EJ_OK;
  GemmGeom g;
  g.m = d->m; g.n = d->n; g.k = d->k; g.batch = d->batch;
  g.a_sb = d->a_sb; g.a_sm = d->a_sm; g.a_sk = d->a_sk;
  g.b_sb = d->b_sb; g.b_sk = d->b_sk; g.b_sn = d->b_sn;
  g.c_sb = d->c_sb; g.c_sm = d->c_sm; g.c_sn = d->c_sn;
  g.a_elems = d->a_elems; g.b_elems = d->b_elems; g.c_elems = d->c_elems;
  g.mblocks = d->m / 128;
  g.nblocks = d->n / 128;
  g.out_bf16 = d->out_dtype == EJ_BF16;
  PairSrc src{lidx, ridx, perm, seg_off, n_a_tiles, n_b_tiles, nullptr, nullptr, 0};
  return launch_seg_gemm_t<SegOpSplitB<128, 128>, 1, 2, 4, 3>(A, B, out, src, g, n_seg, stream);
}

extern "C" int ej_segment_einsum_group(const ej_einsum_desc *desc, int32_t dtype,
                                       int32_t *group) {
  clear_error();
  EJ_CHECK_ARG(desc && group, "null pointer argument");
  EJ_CHECK_ARG(dtype == EJ_F32 || dtype == EJ_BF16 || dtype == EJ_I32, "unknown dtype %d", dtype);
  *group = dtype == EJ_I32 ? 1 : fused_group(desc, dtype);
  return EJ_OK;
}

extern "C" int ej_segment_sum(const void *pair_values, int32_t dtype, int64_t tile_elems,
                              const int32_t *perm, const int32_t *seg_offsets,
                              int64_t n_segments, void *out, ej_stream_t stream_) {
  clear_error();
  hipStream_t stream = as_stream(stream_);
  EJ_CHECK_ARG(dtype == EJ_F32 || dtype == EJ_BF16 || dtype == EJ_F64 || dtype == EJ_F16 ||
                   dtype == EJ_I32 || dtype == EJ_I64,
               "unknown dtype %d", dtype);
  EJ_CHECK_ARG(tile_elems >= 1 && n_segments >= 0, "bad sizes");
  if (n_segments == 0) return EJ_OK;
  EJ_CHECK_ARG(pair_values && perm && seg_offsets && out, "null pointer argument");
  if (n_segments * ceil_div(tile_elems, 256) >= (int64_t(1) << 32)) {
    set_error("segment sum launch too large");
    return EJ_E_UNSUPPORTED;
  }
  const bool vec = aligned16(pair_values) && aligned16(out);
  if (dtype == EJ_F64 || dtype == EJ_F16 || dtype == EJ_I32 || dtype == EJ_I64) {
    const int64_t eb = ceil_div(tile_elems, 256);
    const dim3 grid(static_cast<unsigned>(n_segments * eb));
    if (dtype == EJ_F16)
      hipLaunchKernelGGL(segment_sum_f16_kernel, grid, dim3(256), 0, stream,
                         static_cast<const _Float16 *>(pair_values), tile_elems, perm, seg_offsets,
                         eb, static_cast<_Float16 *>(out));
    else if (dtype == EJ_F64)
      hipLaunchKernelGGL((segment_sum_exact_kernel<double, double>), grid, dim3(256), 0, stream,
                         static_cast<const double *>(pair_values), tile_elems, perm, seg_offsets,
                         eb, static_cast<double *>(out));
    else if (dtype == EJ_I32)
      hipLaunchKernelGGL((segment_sum_exact_kernel<int32_t, uint32_t>), grid, dim3(256), 0,
                         stream, static_cast<const int32_t *>(pair_values), tile_elems, perm,
                         seg_offsets, eb, static_cast<int32_t *>(out));
    else
      hipLaunchKernelGGL((segment_sum_exact_kernel<int64_t, uint64_t>), grid, dim3(256), 0,
                         stream, static_cast<const int64_t *>(pair_values), tile_elems, perm,
                         seg_offsets, eb, static_cast<int64_t *>(out));
  } else if (dtype == EJ_F32 && vec && tile_elems % 4 == 0) {
    const int64_t tv = tile_elems / 4, eb = ceil_div(tv, 256);
    hipLaunchKernelGGL(segment_sum_vec4_kernel, dim3(static_cast<unsigned>(n_segments * eb)),
                       dim3(256), 0, stream, static_cast<const float4 *>(pair_values), tv,
                       perm, seg_offsets, eb, static_cast<float4 *>(out));
  } else if (dtype == EJ_BF16 && vec && tile_elems % 8 == 0) {
    const int64_t tv = tile_elems / 8, eb = ceil_div(tv, 256);
    hipLaunchKernelGGL(segment_sum_bf16x8_kernel, dim3(static_cast<unsigned>(n_segments * eb)),
                       dim3(256), 0, stream, static_cast<const uint4 *>(pair_values), tv,
                       perm, seg_offsets, eb, static_cast<uint4 *>(out));
  } else {
    const int64_t eb = ceil_div(tile_elems, 256);
    if (dtype == EJ_F32)
      hipLaunchKernelGGL(segment_sum_scalar_kernel<float>,
                         dim3(static_cast<unsigned>(n_segments * eb)), dim3(256), 0, stream,
                         static_cast<const float *>(pair_values), tile_elems, perm, seg_offsets,
                         eb, static_cast<float *>(out));
    else
      hipLaunchKernelGGL(segment_sum_scalar_kernel<uint16_t>,
                         dim3(static_cast<unsigned>(n_segments * eb)), dim3(256), 0, stream,
                         static_cast<const uint16_t *>(pair_values), tile_elems, perm,
                         seg_offsets, eb, static_cast<uint16_t *>(out));
  }
  EJ_LAUNCH_CHECK();
  return EJ_OK;
}

extern "C" int ej_gather_tiles(const void *values, int64_t n_tiles, int64_t tile_bytes,
                               const int64_t *idx, int64_t n, void *out, ej_stream_t stream_) {
  clear_error();
  hipStream_t stream = as_stream(stream_);
  EJ_CHECK_ARG(tile_bytes >= 1 && n >= 0 && n_tiles >= 0, "bad sizes");
  if (n == 0) return EJ_OK;
  EJ_CHECK_ARG(values && idx && out, "null pointer argument");
  if (tile_bytes % 16 == 0 && aligned16(values) && aligned16(out)) {
    const int64_t tv = tile_bytes / 16, eb = ceil_div(tv, 1024);
    hipLaunchKernelGGL(gather_kernel<uint4>, dim3(static_cast<unsigned>(n * eb)), dim3(256), 0,
                       stream, static_cast<const uint4 *>(values), n_tiles, tv, idx, eb,
                       static_cast<uint4 *>(out));
  } else if (tile_bytes % 4 == 0) {
    const int64_t tv = tile_bytes / 4, eb = ceil_div(tv, 1024);
    hipLaunchKernelGGL(gather_kernel<uint32_t>, dim3(static_cast<unsigned>(n * eb)), dim3(256), 0,
                       stream, static_cast<const uint32_t *>(values), n_tiles, tv, idx, eb,
                       static_cast<uint32_t *>(out));
  } else {
    const int64_t tv = tile_bytes, eb = ceil_div(tv, 1024);
    hipLaunchKernelGGL(gather_kernel<uint8_t>, dim3(static_cast<unsigned>(n * eb)), dim3(256), 0,
                       stream, static_cast<const uint8_t *>(values), n_tiles, tv, idx, eb,
                       static_cast<uint8_t *>(out));
  }
  EJ_LAUNCH_CHECK();
  return EJ_OK;
}
