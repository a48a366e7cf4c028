// Chunk loads/stores for the kernels' operand rows.
//
// Fast path (`AL` true: base, strides and row width are multiples of the
// 16-byte chunk): every load is unconditional.  Callers clamp row indices to
// a row that exists and pass the number of valid elements; an invalid chunk
// is read from the row start (always in bounds) and zeroed by a select.  No
// branch surrounds a load, so a wave keeps many loads in flight.
//
// Slow path (`AL` false): element-wise loads/stores of the valid elements.
#pragma once

#include "common.h"

namespace mlora {

// Word masks keeping the first `valid` elements of a chunk (computed without
// touching the loaded data, so the AND can sit at the point of use).
template <class T>
__device__ __forceinline__ u32x4 keep_mask(int valid) {
  u32x4 m;
  if constexpr (sizeof(typename T::raw_t) == 2) {
#pragma unroll
    for (int w = 0; w < 4; ++w)
      m[w] = (2 * w < valid ? 0x0000ffffu : 0u) | (2 * w + 1 < valid ? 0xffff0000u : 0u);
  } else {
#pragma unroll
    for (int w = 0; w < 4; ++w) m[w] = (w < valid) ? 0xffffffffu : 0u;
  }
  return m;
}

template <class T, bool AL>
__device__ __forceinline__ u32x4 load_row_chunk(const typename T::raw_t* row, int kk, int valid) {
  if constexpr (AL) {
    const u32x4 v = ld_chunk(row + (valid > 0 ? kk : 0));
    return v & keep_mask<T>(valid);
  } else {
    u32x4 v = zero_chunk();
    const typename T::raw_t* p = row + kk;
    if constexpr (sizeof(typename T::raw_t) == 2) {
#pragma unroll
      for (int e = 0; e < T::VEC; ++e) {
        if (e < valid) {
          const uint32_t h = static_cast<uint32_t>(p[e]);
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
}

// Store the first `valid` elements of a chunk at p (p must be in bounds when valid > 0).
template <class T, bool AL>
__device__ __forceinline__ void store_row_chunk(typename T::raw_t* p, u32x4 v, int valid) {
  if (valid <= 0) return;
  if (AL && valid >= T::VEC) {
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

// An empty asm that takes the registers of `r` in and out: instructions
// that use them cannot move above it, and neither can the wait for their
// loads.  It costs no instruction.
template <class V, int A>
__device__ __forceinline__ void fence_regs(V (&r)[A]) {
#pragma unroll
  for (int i = 0; i < A; ++i) asm volatile("" : "+v"(r[i]));
}
template <class V, int A, int B>
__device__ __forceinline__ void fence_regs(V (&r)[A][B]) {
#pragma unroll
  for (int i = 0; i < A; ++i) fence_regs(r[i]);
}

// s_waitcnt with vmcnt <= N and the other counters unconstrained (gfx9
// encoding: vmcnt bits [3:0] and [15:14], expcnt [6:4], lgkmcnt [11:8]).
// Vector memory loads, direct-to-LDS ones included, complete in issue order,
// so this waits for every load but the N most recent.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Workgroup barrier that orders LDS accesses only: the fences are scoped to
// the local address space, so the wait before s_barrier is lgkmcnt(0) and
// global loads and stores still in flight stay in flight.  __syncthreads()
// would also wait for vmcnt(0), i.e. for every outstanding global access.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Exclusive prefix sum of `v` over a workgroup of NW wave64s; `*total` gets
// the sum.  `tmp` is NW ints of LDS.  Every thread of the workgroup must call
// it.  Loads the caller has in flight are not waited for.
template <int NW>
__device__ __forceinline__ int block_exclusive_scan(int v, int* tmp, int* total) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int y = __shfl_up(x, off, kWave);
    if (lane >= off) x += y;
  }
  if (lane == kWave - 1) tmp[wave] = x;
  lds_barrier();
  int before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const int t = tmp[w];
    before += (w < wave) ? t : 0;
    all += t;
  }
  lds_barrier();
  *total = all;
  return before + x - v;
}

}  // namespace mlora
