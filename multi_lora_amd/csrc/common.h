// Device-side building blocks shared by the gfx950 segment-LoRA kernels:
// element traits (bf16 / fp16 / fp32 storage, fp32 math), 128-bit fragment
// loads, and one K-step of a 16x16 MFMA tile.
//
// MFMA fragment convention used by every kernel here (wave64):
//   lane l owns row (l & 15) of a 16-row operand and the 16-byte chunk
//   k = k0 + (l >> 4) * VEC .. + VEC of that row, so one K-step covers
//   KSTEP = 4 * VEC reduction elements.  Both operands of an MFMA are loaded
//   with this same mapping, which makes the product independent of the order
//   in which the hardware walks k inside a step.
//   The 16x16 fp32 result lives as lane l -> column (l & 15),
//   rows 4 * (l >> 4) + q for q = 0..3.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mlora_hip.h"

namespace mlora {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int kWave = 64;

// ---------------------------------------------------------------- traits
struct BF16 {
  using raw_t = uint16_t;
  static constexpr int VEC = 8;  // elements per 16-byte chunk
  static constexpr int KSTEP = 32;
  __device__ static __forceinline__ float to_f32(raw_t v) {
    return __uint_as_float(static_cast<uint32_t>(v) << 16);
  }
  __device__ static __forceinline__ raw_t from_f32(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
  }
  // from_f32(lo) | from_f32(hi) << 16, in one conversion instruction.
  __device__ static __forceinline__ uint32_t pack2(float lo, float hi) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t));
  }
  __device__ static __forceinline__ f32x4 mma(f32x4 acc, u32x4 a, u32x4 b) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
  }
};

struct F16 {
  using raw_t = uint16_t;
  static constexpr int VEC = 8;
  static constexpr int KSTEP = 32;
  __device__ static __forceinline__ float to_f32(raw_t v) {
    return static_cast<float>(__builtin_bit_cast(_Float16, v));
  }
  __device__ static __forceinline__ raw_t from_f32(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
  }
  __device__ static __forceinline__ uint32_t pack2(float lo, float hi) {
    return static_cast<uint32_t>(from_f32(lo)) | (static_cast<uint32_t>(from_f32(hi)) << 16);
  }
  __device__ static __forceinline__ f32x4 mma(f32x4 acc, u32x4 a, u32x4 b) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), acc, 0, 0, 0);
  }
};

struct F32 {
  using raw_t = float;
  static constexpr int VEC = 4;
  static constexpr int KSTEP = 16;
  __device__ static __forceinline__ float to_f32(raw_t v) { return v; }
  __device__ static __forceinline__ raw_t from_f32(float f) { return f; }
  __device__ static __forceinline__ f32x4 mma(f32x4 acc, u32x4 a, u32x4 b) {
    // Four 16x16x4 steps; element e of every lane's chunk feeds step e.
#pragma unroll
    for (int e = 0; e < 4; ++e)
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a[e]), __uint_as_float(b[e]),
                                                  acc, 0, 0, 0);
    return acc;
  }
};

// Element e (0..VEC-1) of a 16-byte chunk, as fp32.
template <class T>
__device__ __forceinline__ float chunk_elem(const u32x4& v, int e) {
  if constexpr (sizeof(typename T::raw_t) == 2) {
    uint32_t w = v[e >> 1];
    return T::to_f32(static_cast<uint16_t>((e & 1) ? (w >> 16) : (w & 0xffffu)));
  } else {
    return __uint_as_float(v[e]);
  }
}

// Keep the first `valid` elements of a chunk, zero the rest.
template <class T>
__device__ __forceinline__ u32x4 chunk_keep(u32x4 v, int valid) {
  if (valid >= T::VEC) return v;
  if constexpr (sizeof(typename T::raw_t) == 2) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const int e0 = 2 * w;
      uint32_t keep = (e0 < valid ? 0x0000ffffu : 0u) | (e0 + 1 < valid ? 0xffff0000u : 0u);
      v[w] &= keep;
    }
  } else {
#pragma unroll
    for (int w = 0; w < 4; ++w) v[w] = (w < valid) ? v[w] : 0u;
  }
  return v;
}

__device__ __forceinline__ u32x4 zero_chunk() { return u32x4{0u, 0u, 0u, 0u}; }

// 16-byte aligned global load / store of one chunk.
template <class R>
__device__ __forceinline__ u32x4 ld_chunk(const R* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
template <class R>
__device__ __forceinline__ void st_chunk(R* p, u32x4 v) {
  *reinterpret_cast<u32x4*>(p) = v;
}
// Cache-policy operand of a load builtin (global_load_lds): non-temporal.
constexpr int kCpolNt = 2;
// The same with the non-temporal hint (nt), for data a kernel reads or
// writes once: an output row's read-modify-write.  Keep these apart from the
// plain forms at the source level; a branch choosing between a hinted and a
// plain store of the same value is merged by the compiler into the plain one.
template <class R>
__device__ __forceinline__ u32x4 ld_chunk_nt(const R* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
template <class R>
__device__ __forceinline__ void st_chunk_nt(R* p, u32x4 v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}

// Pack VEC fp32 values into one chunk of T.
template <class T>
__device__ __forceinline__ u32x4 pack_chunk(const float* f) {
  u32x4 v;
  if constexpr (sizeof(typename T::raw_t) == 2) {
#pragma unroll
    for (int w = 0; w < 4; ++w)
      v[w] = static_cast<uint32_t>(T::from_f32(f[2 * w])) |
             (static_cast<uint32_t>(T::from_f32(f[2 * w + 1])) << 16);
  } else {
#pragma unroll
    for (int w = 0; w < 4; ++w) v[w] = __float_as_uint(f[w]);
  }
  return v;
}

__device__ __forceinline__ float load_scaling(const void* p, int idx, int dtype) {
  if (dtype == MLORA_BF16) return BF16::to_f32(static_cast<const uint16_t*>(p)[idx]);
  if (dtype == MLORA_F16) return F16::to_f32(static_cast<const uint16_t*>(p)[idx]);
  return static_cast<const float*>(p)[idx];
}

// load_scaling for a wave-uniform index, as a scalar load: a 16-bit value is
// taken from the 4-byte aligned word that holds it (that word lies in the
// aligned 4-byte window of a valid element, so it never crosses a page), so
// waiting for it waits for the scalar queue only, not for vector loads the
// wave has in flight.
__device__ __forceinline__ float load_scaling_uniform(const void* p, int idx, int dtype) {
  if (dtype != MLORA_BF16 && dtype != MLORA_F16) return static_cast<const float*>(p)[idx];
  const char* v = static_cast<const char*>(p) + 2 * static_cast<int64_t>(idx);
  const int mis = static_cast<int>(reinterpret_cast<uintptr_t>(v) & 3);
  const uint32_t w = *reinterpret_cast<const uint32_t*>(v - mis);
  const uint16_t h = static_cast<uint16_t>(mis ? (w >> 16) : (w & 0xffffu));
  return dtype == MLORA_BF16 ? BF16::to_f32(h) : F16::to_f32(h);
}

// Kernel-side view of the per-step segment table.
struct SegView {
  const int32_t* indptr;
  const int32_t* widx;
  const int32_t* ranks;
  const void* scalings;
  int bs;
  int num_slots;
  int scal_dtype;
};

// Slot and live rank of segment `seg`; rank 0 for a slot outside the pool.
__device__ __forceinline__ void seg_slot_rank(const SegView& m, int seg, int r_max, int rank_mult,
                                              int* slot, int* rank) {
  int s = m.widx[seg];
  int r = 0;
  if (s >= 0 && s < m.num_slots) r = m.ranks[s] * rank_mult;
  if (r < 0) r = 0;
  if (r > r_max) r = r_max;
  *slot = s;
  *rank = r;
}

// Inclusive prefix sum over the 64 lanes of a wave.
__device__ __forceinline__ int wave_incl_sum(int v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int o = __shfl_up(v, d, kWave);
    if (lane >= d) v += o;
  }
  return v;
}

// The tile's segment, its tile number within the segment, the segment's
// clamped row range [start, end) and its slot (weight_indices, unchecked).
struct TileRef {
  int seg, mt, start, end, slot;
};

// Dense row tiles: tile `tile` of the batch, counting ceil(len / bm) tiles
// per segment in segment order (len = rows of the segment inside [0, rows)),
// as a TileRef.  Launching about rows / bm + bs workgroups instead of
// bs * ceil(max_len / bm) keeps a mixed batch (a few long segments among
// many one-row ones) from dispatching mostly empty workgroups.
// The table is scanned 64 segments at a time, one segment per lane: the
// lane's bounds and slot are loaded together (one round trip per chunk),
// a wave prefix sum counts the tiles, and a ballot finds the segment.
// Every wave computes the same result on its own (no LDS, no barrier); the
// result is wave-uniform.
struct SegChunk {
  int s, e, w;  // this lane's segment: clamped bounds and slot
  int n, incl;  // its tile count and the inclusive prefix over the chunk
  int total;    // tiles in the chunk
};

// Segments of at most `short_max` rows count no tiles (-1: every segment
// counts).
__device__ __forceinline__ SegChunk load_chunk(const SegView& m, int rows, int c0, int bm, int short_max = -1) {
  const int i = c0 + (threadIdx.x & 63);
  SegChunk c{0, 0, 0, 0, 0, 0};
  if (i < m.bs) {
    c.s = max(m.indptr[i], 0);
    c.e = min(m.indptr[i + 1], rows);
    c.w = m.widx[i];
    c.n = c.e - c.s > short_max && c.e > c.s ? (c.e - c.s + bm - 1) / bm : 0;
  }
  c.incl = wave_incl_sum(c.n);
  c.total = __builtin_amdgcn_readlane(c.incl, kWave - 1);
  return c;
}

// Tile `tile` if it lies in chunk `c` (which starts at segment c0, after
// `before` tiles); no memory access.
__device__ __forceinline__ bool pick_tile(const SegChunk& c, int c0, int before, int tile, TileRef* t) {
  if (tile >= before + c.total) return false;
  const uint64_t hit = __ballot(before + c.incl > tile);
  const int l = __builtin_amdgcn_readfirstlane(static_cast<int>(__ffsll(static_cast<unsigned long long>(hit))) - 1);
  t->seg = c0 + l;
  t->mt = tile - before - (__builtin_amdgcn_readlane(c.incl, l) - __builtin_amdgcn_readlane(c.n, l));
  t->start = __builtin_amdgcn_readlane(c.s, l);
  t->end = __builtin_amdgcn_readlane(c.e, l);
  t->slot = __builtin_amdgcn_readlane(c.w, l);
  return true;
}

// Chunks from segment c0 on (`before` tiles ahead of it); false when the
// batch has fewer tiles.
__device__ __forceinline__ bool dense_tile_from(const SegView& m, int rows, int tile, int bm, int c0, int before,
                                                TileRef* t) {
  for (; c0 < m.bs; c0 += kWave) {
    const SegChunk c = load_chunk(m, rows, c0, bm);
    if (pick_tile(c, c0, before, tile, t)) return true;
    before += c.total;
  }
  return false;
}

__device__ __forceinline__ bool dense_tile(const SegView& m, int rows, int tile, int bm, TileRef* t) {
  return dense_tile_from(m, rows, tile, bm, 0, 0, t);
}

// Dense tiles over the segments of more than `short_max` rows only.  Scans
// the whole table and returns the number of such tiles; *found tells
// whether tile `tile` exists (then *t holds it).
__device__ __forceinline__ int long_tile(const SegView& m, int rows, int tile, int bm, int short_max, TileRef* t,
                                         bool* found) {
  int before = 0;
  *found = false;
  for (int c0 = 0; c0 < m.bs; c0 += kWave) {
    const SegChunk c = load_chunk(m, rows, c0, bm, short_max);
    if (!*found && pick_tile(c, c0, before, tile, t)) *found = true;
    before += c.total;
  }
  return before;
}

// Rank of a slot read from the table (slot already loaded): 0 outside the
// pool, clamped to [0, r_max].
__device__ __forceinline__ int slot_rank_of(const SegView& m, int slot, int r_max, int rank_mult) {
  if (slot < 0 || slot >= m.num_slots) return 0;
  return min(max(m.ranks[slot] * rank_mult, 0), r_max);
}

struct SliceView {
  const void* a;
  int64_t a_slot_stride, a_row_stride;
  const void* b;
  int64_t b_slot_stride, b_row_stride;
  int out_dim;
  int out_col;
};

constexpr int kMaxSlices = MLORA_MAX_SLICES;

}  // namespace mlora
