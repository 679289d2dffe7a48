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
};

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

// Spreads consecutive block ids over the 8 XCDs in contiguous chunks, so
// that neighbouring logical blocks (sharing operand tiles) share an L2.
__device__ inline int64_t xcd_logical_block() {
  const int64_t bid = blockIdx.x, total = gridDim.x;
  const int64_t per = total / 8, rem = total % 8;
  const int64_t xcd = bid % 8, local = bid / 8;
  const int64_t start = xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per;
  return start + local;
}

// ---------------------------------------------------------------------------
// MFMA grouped GEMM.
//
// One workgroup (4 waves, 2x2) computes a BM x BN block of one output tile
// (segment) for one batch index, iterating the segment's pairs and the K
// dimension in BK chunks.  Operands are staged through LDS as [rows][k]
// (k contiguous, the layout both MFMA operands read); an operand whose free
// dimension is contiguous in HBM is transposed in registers before the LDS
// store.  The next chunk's global loads are issued before the current
// chunk's MFMAs, so HBM/L2 latency overlaps the math.  Accumulation is fp32
// in registers; each output block is written once.

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

struct GemmGeom {
  int64_t m, n, k, batch;
  int64_t a_sb, a_sm, a_sk, b_sb, b_sk, b_sn, c_sb, c_sm, c_sn;
  int64_t a_elems, b_elems, c_elems;
  int64_t mblocks, nblocks;
};

template <typename T, int ROWS, int BK, bool DIRECT>
struct OperandStage {
  static constexpr int VEC = 16 / sizeof(T);
  static constexpr int LDK = BK + VEC;  // row pitch in LDS (elements)
  // DIRECT: k contiguous in HBM; vectors along k.
  static constexpr int NVEC_D = ROWS * BK / VEC;
  static constexpr int PER_D = (NVEC_D + 255) / 256;
  // Transposed: rows contiguous in HBM; each thread owns KV k-rows x VEC rows.
  static constexpr int KV0 = ROWS * BK / (256 * VEC);
  static constexpr int KV = KV0 > 0 ? KV0 : 1;
  static constexpr int NBLK_T = (BK / KV) * (ROWS / VEC);
  static constexpr int NREG = DIRECT ? PER_D : KV;
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
          *reinterpret_cast<uint4 *>(lds + row * LDK + kv * VEC) = r[v];
        }
      }
    } else {
      if (tid >= NBLK_T) return;
      const int rb = tid % (ROWS / VEC), kb = tid / (ROWS / VEC);
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
          T *dst = lds + (rb * VEC + c) * LDK + kb * KV;
          if (KV == 4) {
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
          T *dst = lds + (rb * VEC + c) * LDK + kb * KV;
#pragma unroll
          for (int j = 0; j < KV; ++j) reinterpret_cast<uint32_t *>(dst)[j] = w[j * 4 + c];
        }
      }
    }
  }
};

template <typename T, int BM, int BN, int BK, bool A_DIRECT, bool B_DIRECT>
__global__ __launch_bounds__(256) void tile_gemm_kernel(const T *__restrict__ A,
                                                        const T *__restrict__ B,
                                                        float *__restrict__ C, PairSrc src,
                                                        GemmGeom g) {
  using SA = OperandStage<T, BM, BK, A_DIRECT>;
  using SB = OperandStage<T, BN, BK, B_DIRECT>;
  constexpr int LDK = SA::LDK;
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int FM = WM / 16, FN = WN / 16;
  constexpr bool BF16 = sizeof(T) == 2;
  constexpr int KSTEP = BF16 ? 32 : 16;  // k consumed per inner step
  __shared__ __align__(16) T As[BM * LDK];
  __shared__ __align__(16) T Bs[BN * LDK];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  int64_t lb = xcd_logical_block();
  const int64_t nb = lb % g.nblocks;
  lb /= g.nblocks;
  const int64_t mb = lb % g.mblocks;
  lb /= g.mblocks;
  const int64_t bi = lb % g.batch;
  const int64_t seg = lb / g.batch;

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
  // A chunk rows advance by a_sm (direct) and k by a_sk; see OperandStage.
  auto issue = [&](int64_t st) {
    const int64_t q = q0 + st / nkc;
    const int kc = static_cast<int>(st % nkc);
    int64_t at, bt;
    const bool ok = pair_tiles(src, q, &at, &bt);
    const T *ab = A + (ok ? at : 0) * g.a_elems + a_off0 + kc * BK * g.a_sk;
    const T *bb = B + (ok ? bt : 0) * g.b_elems + b_off0 + kc * BK * g.b_sk;
    sa.load(ab, g.a_sm, g.a_sk, ok, tid);
    sb.load(bb, g.b_sn, g.b_sk, ok, tid);
  };

  if (stages > 0) issue(0);
  for (int64_t st = 0; st < stages; ++st) {
    __syncthreads();
    sa.store(As, tid);
    sb.store(Bs, tid);
    __syncthreads();
    if (st + 1 < stages) issue(st + 1);
#pragma unroll
    for (int ks = 0; ks < BK / KSTEP; ++ks) {
      if constexpr (BF16) {
        bf16x8_t af[FM], bfr[FN];
#pragma unroll
        for (int i = 0; i < FM; ++i)
          af[i] = *reinterpret_cast<const bf16x8_t *>(
              As + (wm * WM + i * 16 + (lane & 15)) * LDK + ks * 32 + (lane >> 4) * 8);
#pragma unroll
        for (int j = 0; j < FN; ++j)
          bfr[j] = *reinterpret_cast<const bf16x8_t *>(
              Bs + (wn * WN + j * 16 + (lane & 15)) * LDK + ks * 32 + (lane >> 4) * 8);
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
      } else {
        f32x4_t af[FM], bfr[FN];
#pragma unroll
        for (int i = 0; i < FM; ++i)
          af[i] = *reinterpret_cast<const f32x4_t *>(
              As + (wm * WM + i * 16 + (lane & 15)) * LDK + ks * 16 + (lane >> 4) * 4);
#pragma unroll
        for (int j = 0; j < FN; ++j)
          bfr[j] = *reinterpret_cast<const f32x4_t *>(
              Bs + (wn * WN + j * 16 + (lane & 15)) * LDK + ks * 16 + (lane >> 4) * 4);
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
          for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i][s], bfr[j][s], acc[i][j], 0, 0, 0);
      }
    }
  }

  float *cb = C + seg * g.c_elems + bi * g.c_sb + mb * BM * g.c_sm + nb * BN * g.c_sn;
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = wm * WM + i * 16 + (lane >> 4) * 4 + r;
        const int col = wn * WN + j * 16 + (lane & 15);
        cb[row * g.c_sm + col * g.c_sn] = acc[i][j][r];
      }
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
};

template <typename T>
__global__ __launch_bounds__(256) void generic_einsum_kernel(const T *__restrict__ A,
                                                             const T *__restrict__ B,
                                                             float *__restrict__ C, PairSrc src,
                                                             GenDesc d) {
  const int64_t seg = blockIdx.x / d.eblocks;
  const int64_t e = (blockIdx.x % d.eblocks) * 256 + threadIdx.x;
  if (e >= d.c_elems) return;
  int64_t rem = e, aoff = 0, boff = 0;
  for (int i = d.n_out - 1; i >= 0; --i) {
    int64_t x = rem % d.out_ext[i];
    rem /= d.out_ext[i];
    aoff += x * d.out_a[i];
    boff += x * d.out_b[i];
  }
  int64_t q0, q1;
  seg_range(src, seg, &q0, &q1);
  float acc = 0.f;
  for (int64_t q = q0; q < q1; ++q) {
    int64_t at, bt;
    if (!pair_tiles(src, q, &at, &bt)) continue;
    const T *a = A + at * d.a_elems + aoff;
    const T *b = B + bt * d.b_elems + boff;
    float pacc = 0.f;
    int64_t idx[EJ_MAX_LABELS] = {0};
    int64_t ra = 0, rb = 0;
    for (int64_t r = 0; r < d.red_total; ++r) {
      pacc += to_f32(a[ra]) * to_f32(b[rb]);
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
  C[seg * d.c_elems + e] = acc;
}

// ---------------------------------------------------------------------------
// Dispatch.

template <typename T, int BM, int BN, int BK>
int launch_gemm_layout(bool a_direct, bool b_direct, const void *A, const void *B, float *C,
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
int launch_gemm_bk(int bm, int bn, bool ad, bool bd, const void *A, const void *B, float *C,
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

int pick_block(int64_t x) { return x % 128 == 0 ? 128 : x % 64 == 0 ? 64 : x % 32 == 0 ? 32 : 0; }

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Chooses the MFMA path when the einsum is GEMM-shaped with tile-friendly
// extents and 16-byte aligned operand rows; returns false to fall back.
bool try_gemm(const ej_einsum_desc *d, int32_t dtype, const void *A, const void *B, float *C,
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
  const int64_t nblk = n_seg * g.batch * g.mblocks * g.nblocks;
  if (nblk >= (int64_t(1) << 32)) return false;
  if (dtype == EJ_BF16) {
    *status = bk == 64 ? launch_gemm_bk<uint16_t, 64>(bm, bn, ad, bd, A, B, C, src, g, nblk, stream)
                       : launch_gemm_bk<uint16_t, 32>(bm, bn, ad, bd, A, B, C, src, g, nblk, stream);
  } else {
    *status = bk == 32 ? launch_gemm_bk<float, 32>(bm, bn, ad, bd, A, B, C, src, g, nblk, stream)
                       : launch_gemm_bk<float, 16>(bm, bn, ad, bd, A, B, C, src, g, nblk, stream);
  }
  return true;
}

int run_generic(const ej_einsum_desc *d, int32_t dtype, const void *A, const void *B, float *C,
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
  const int64_t nblk = n_seg * g.eblocks;
  if (nblk >= (int64_t(1) << 32)) {
    set_error("einsum launch too large");
    return EJ_E_UNSUPPORTED;
  }
  if (dtype == EJ_BF16)
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

int einsum_common(const ej_einsum_desc *d, int32_t dtype, const void *A, const void *B,
                  const PairSrc &src, int64_t n_seg, float *C, hipStream_t stream) {
  EJ_CHECK_ARG(d, "desc is null");
  EJ_CHECK_ARG(dtype == EJ_F32 || dtype == EJ_BF16, "unknown dtype %d", dtype);
  EJ_CHECK_ARG(n_seg >= 0, "negative count");
  EJ_CHECK_ARG(d->n_out >= 0 && d->n_out <= EJ_MAX_LABELS && d->n_red >= 0 &&
                   d->n_red <= EJ_MAX_LABELS && d->c_elems >= 1 && d->a_elems >= 1 &&
                   d->b_elems >= 1,
               "malformed einsum descriptor");
  if (n_seg == 0) return EJ_OK;
  EJ_CHECK_ARG(A && B && C, "null pointer argument");
  int status = EJ_OK;
  if (try_gemm(d, dtype, A, B, C, src, n_seg, stream, &status)) return status;
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

__global__ __launch_bounds__(256) void segment_sum_scalar_kernel(const float *__restrict__ vals,
                                                                 int64_t tile_elems,
                                                                 const int32_t *perm,
                                                                 const int32_t *off,
                                                                 int64_t eblocks,
                                                                 float *__restrict__ out) {
  const int64_t seg = blockIdx.x / eblocks;
  const int64_t e = (blockIdx.x % eblocks) * 256 + threadIdx.x;
  if (e >= tile_elems) return;
  float acc = 0.f;
  for (int32_t q = off[seg]; q < off[seg + 1]; ++q)
    acc += vals[static_cast<int64_t>(perm[q]) * tile_elems + e];
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
                              float *out, ej_stream_t stream) {
  clear_error();
  PairSrc src{lhs_idx, rhs_idx, nullptr, nullptr, n_lhs_tiles, n_rhs_tiles};
  return einsum_common(desc, dtype, lhs_values, rhs_values, src, n_pairs, out, as_stream(stream));
}

extern "C" int ej_segment_einsum(const ej_einsum_desc *desc, int32_t dtype, const void *lhs_values,
                                 const void *rhs_values, int64_t n_lhs_tiles,
                                 int64_t n_rhs_tiles, const int64_t *lhs_idx,
                                 const int64_t *rhs_idx, const int32_t *perm,
                                 const int32_t *seg_offsets, int64_t n_segments, float *out,
                                 ej_stream_t stream) {
  clear_error();
  EJ_CHECK_ARG(seg_offsets || n_segments == 0, "seg_offsets is null");
  PairSrc src{lhs_idx, rhs_idx, perm, seg_offsets, n_lhs_tiles, n_rhs_tiles};
  return einsum_common(desc, dtype, lhs_values, rhs_values, src, n_segments, out,
                       as_stream(stream));
}

extern "C" int ej_segment_sum(const float *pair_values, int64_t tile_elems, const int32_t *perm,
                              const int32_t *seg_offsets, int64_t n_segments, float *out,
                              ej_stream_t stream_) {
  clear_error();
  hipStream_t stream = as_stream(stream_);
  EJ_CHECK_ARG(tile_elems >= 1 && n_segments >= 0, "bad sizes");
  if (n_segments == 0) return EJ_OK;
  EJ_CHECK_ARG(pair_values && perm && seg_offsets && out, "null pointer argument");
  if (tile_elems % 4 == 0 && aligned16(pair_values) && aligned16(out)) {
    const int64_t tv = tile_elems / 4, eb = ceil_div(tv, 256);
    hipLaunchKernelGGL(segment_sum_vec4_kernel, dim3(static_cast<unsigned>(n_segments * eb)),
                       dim3(256), 0, stream, reinterpret_cast<const float4 *>(pair_values), tv,
                       perm, seg_offsets, eb, reinterpret_cast<float4 *>(out));
  } else {
    const int64_t eb = ceil_div(tile_elems, 256);
    hipLaunchKernelGGL(segment_sum_scalar_kernel, dim3(static_cast<unsigned>(n_segments * eb)),
                       dim3(256), 0, stream, pair_values, tile_elems, perm, seg_offsets, eb, out);
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
