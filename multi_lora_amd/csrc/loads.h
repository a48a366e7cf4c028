// Masked 16-byte chunk loads/stores used where an operand row may be
// unaligned or end inside a chunk.  `aligned` is a launch-uniform flag
// computed on the host (base address, strides and row width all multiples of
// the chunk), so the branch costs nothing on the fast path.
#pragma once

#include "common.h"

namespace mlora {

// Load up to VEC elements starting at p; elements at or past `valid` read as 0.
template <class T>
__device__ __forceinline__ u32x4 load_chunk(const typename T::raw_t* p, int valid, bool aligned) {
  if (valid <= 0) return zero_chunk();
  if (aligned) {
    u32x4 v = ld_chunk(p);
    return valid >= T::VEC ? v : chunk_keep<T>(v, valid);
  }
  u32x4 v = zero_chunk();
  if constexpr (sizeof(typename T::raw_t) == 2) {
#pragma unroll
    for (int e = 0; e < T::VEC; ++e) {
      if (e < valid) {
        uint32_t h = static_cast<uint32_t>(p[e]);
        v[e >> 1] |= (e & 1) ? (h << 16) : h;
      }
    }
  } else {
#pragma unroll
    for (int e = 0; e < T::VEC; ++e)
      if (e < valid) v[e] = __float_as_uint(p[e]);
  }
  return v;
}

// Store the first `valid` elements of a chunk at p.
template <class T>
__device__ __forceinline__ void store_chunk(typename T::raw_t* p, u32x4 v, int valid, bool aligned) {
  if (valid <= 0) return;
  if (aligned && valid >= T::VEC) {
    st_chunk(p, v);
    return;
  }
  if constexpr (sizeof(typename T::raw_t) == 2) {
#pragma unroll
    for (int e = 0; e < T::VEC; ++e)
      if (e < valid) p[e] = static_cast<uint16_t>((e & 1) ? (v[e >> 1] >> 16) : (v[e >> 1] & 0xffffu));
  } else {
#pragma unroll
    for (int e = 0; e < T::VEC; ++e)
      if (e < valid) p[e] = __uint_as_float(v[e]);
  }
}

}  // namespace mlora
