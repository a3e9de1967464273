// Host-side helpers shared by the launchers: descriptor predicates and
// attribute-blob readers.  HIP-free so that the registry compiles as plain C++.
#pragma once

#include <cstdint>
#include <cstring>

#include "registry.hpp"

namespace aicf::hip {

// Thread-local message of the last failing HIP runtime call.
const char* last_error_message();
void set_last_error(const char* what, const char* detail);

inline DType dt(const TensorDesc& t) { return static_cast<DType>(t.dtype); }

inline int64_t numel_of(const TensorDesc& t) {
  if (t.rank < 0 || t.rank > AICF_MAX_RANK) return 0;
  int64_t n = 1;
  for (int i = 0; i < t.rank; ++i) n *= t.shape[i];
  return n;
}

// numel with every dim > 0 required and rank >= 1 (reference compute_numel,
// e.g. mse_grad/launcher.cu:140-155).
inline bool numel_pos(const TensorDesc& t, int64_t* out) {
  if (t.rank < 1 || t.rank > AICF_MAX_RANK) return false;
  int64_t n = 1;
  for (int i = 0; i < t.rank; ++i) {
    if (t.shape[i] <= 0) return false;
    n *= t.shape[i];
  }
  *out = n;
  return n > 0;
}

inline bool same_shape(const TensorDesc& a, const TensorDesc& b) {
  if (a.rank != b.rank) return false;
  for (int i = 0; i < a.rank; ++i)
    if (a.shape[i] != b.shape[i]) return false;
  return true;
}

// Row-major contiguity computed from strides (reference relu/launcher.cu:90-98).
inline bool strides_rowmajor(const TensorDesc& t) {
  if (t.rank <= 0) return false;
  if (t.stride[t.rank - 1] != 1) return false;
  for (int i = t.rank - 2; i >= 0; --i)
    if (t.stride[i] != t.shape[i + 1] * t.stride[i + 1]) return false;
  return true;
}

inline bool is_contig_2d_rowmajor(const TensorDesc& t) {
  return t.rank == 2 && t.stride[1] == 1 && t.stride[0] == t.shape[1];
}

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

// Byte range [lo, hi) that a view with non-negative strides can touch.
struct Span {
  uintptr_t lo, hi;
};
inline Span span_of(const TensorDesc& t) {
  const int64_t es = dt(t) == DType::kF32 || dt(t) == DType::kI32 ? 4 : 2;
  int64_t last = 0;
  for (int i = 0; i < t.rank && i < AICF_MAX_RANK; ++i) {
    if (t.shape[i] <= 0) return {0, 0};  // touches nothing
    last += (t.shape[i] - 1) * t.stride[i];
  }
  const uintptr_t lo = reinterpret_cast<uintptr_t>(t.data);
  return {lo, lo + (uintptr_t)((last + 1) * es)};
}
inline bool overlap(const Span& a, const Span& b) { return a.lo < b.hi && b.lo < a.hi; }
// Whether two views can touch a common byte (a written view against one the
// same kernel reads or writes).
inline bool views_overlap(const TensorDesc& a, const TensorDesc& b) { return overlap(span_of(a), span_of(b)); }

// Flatten leading dims into M, keep the last dim as N (rank >= 2).
inline bool rows_cols(const TensorDesc& t, int64_t* M, int64_t* N) {
  if (t.rank < 2 || t.rank > AICF_MAX_RANK) return false;
  const int64_t n = t.shape[t.rank - 1];
  if (n <= 0) return false;
  int64_t m = 1;
  for (int i = 0; i < t.rank - 1; ++i) {
    if (t.shape[i] <= 0) return false;
    m *= t.shape[i];
  }
  *M = m;
  *N = n;
  return m > 0;
}

inline const AttrBlob& blob(const void* attr) {
  static const AttrBlob kEmpty{0u, 0u, nullptr};
  return attr ? *static_cast<const AttrBlob*>(attr) : kEmpty;
}

// Reads the i-th 4-byte field of the payload when the schema is one of the
// accepted ids and the payload is at least `need` bytes long.
template <typename T>
inline T field(const AttrBlob& a, int byte_off) {
  T v;
  std::memcpy(&v, static_cast<const uint8_t*>(a.data) + byte_off, sizeof(T));
  return v;
}

inline bool payload_ok(const AttrBlob& a, uint32_t need) { return a.data && a.bytes >= need; }

}  // namespace aicf::hip
