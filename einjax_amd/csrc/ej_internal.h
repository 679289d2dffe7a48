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

#define EJ_LAUNCH_CHECK() EJ_HIP(hipGetLastError())

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
size_t scan_workspace_bytes(int64_t n);
int scan_exclusive_i64(const int64_t *in, int64_t *out, int64_t n, int64_t *total,
                       void *ws, hipStream_t stream);

// Stable LSD radix sort of (key, value) pairs on the low `bits` key bits.
// The result ends in keys/vals; keys_alt/vals_alt are scratch of length n.
size_t sort_workspace_bytes(int64_t n);
int sort_pairs_u64(uint64_t *keys, int32_t *vals, uint64_t *keys_alt, int32_t *vals_alt,
                   int64_t n, int bits, void *ws, hipStream_t stream);

int fill_iota_i32(int32_t *v, int64_t n, hipStream_t stream);

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

inline unsigned grid_for(int64_t n, int per_block = kBlock) {
  int64_t g = ceil_div(n, per_block);
  if (g < 1) g = 1;
  return static_cast<unsigned>(g);
}

}  // namespace ej
