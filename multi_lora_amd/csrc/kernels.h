// Launch-side contracts between the C ABI layer (api.hip) and the kernel
// translation units.  Every struct here is passed to a kernel by value.
#pragma once

#include "common.h"

namespace mlora {

// Flags for operands whose rows can be read/written as 16-byte chunks.
enum AlignBits : int {
  kAlX = 1,
  kAlA = 2,
  kAlB = 4,
  kAlMid = 8,
  kAlOut = 16,
};

struct ShrinkArgs {
  const void* x;
  int64_t x_stride;
  int rows;         // rows of x / mid; segment bounds are clamped to it
  int in_dim;
  SliceView slices[kMaxSlices];
  int n_slices;
  int r_max;
  int rank_mult;
  void* mid;
  int64_t mid_stride;
  SegView meta;
  int m_tiles;      // row tiles per segment
  int ks;           // K splits per row tile
  int k_per_split;  // reduction elements per split (multiple of KSTEP)
  int* counters;    // [bs * m_tiles] arrival counters (ks > 1), zero between calls
  float* partials;  // [bs * m_tiles][ks][WM][n_slices * nb_slice][64] f32x4
  int nb_slice;     // 16-wide n-blocks per slice = cdiv(r_max, 16)
  int align;        // AlignBits
};

struct ShrinkPlan {
  int bm;        // 16 or 64 token rows per tile
  int m_tiles;
  int ks;
  int k_per_split;
  int nbs;       // compiled n-blocks per slice (1, 4 or 8)
  int maxs;      // compiled slice count (1 or 4)
  size_t ws_bytes;
};

// Chooses the tile shape for a shrink launch; returns false if unsupported.
bool plan_shrink(int in_dim, int r_max, int n_slices, int bs, int max_len, int dtype, int num_cus,
                 ShrinkPlan* plan);
hipError_t launch_shrink(const ShrinkPlan& plan, ShrinkArgs args, int dtype, hipStream_t stream);

constexpr int kExpandBN = 256;  // output columns per tile

struct ExpandArgs {
  const void* mid;
  int64_t mid_stride;
  int rows;         // rows of mid / out; segment bounds are clamped to it
  SliceView slices[kMaxSlices];
  int n_slices;
  int r_max;
  void* out;
  int64_t out_stride;
  SegView meta;
  int m_tiles;
  int n_tiles;                     // n-tiles over all slices
  int tile_base[kMaxSlices + 1];   // first n-tile of each slice
  int align;
};

hipError_t launch_expand(int bm, ExpandArgs args, int dtype, hipStream_t stream);

struct RmsArgs {
  const void* x;
  int64_t x_stride_outer;
  int64_t x_stride_inner;
  int64_t inner;
  const void* w;
  int w_dtype;
  void* y;
  int64_t y_stride;
  int64_t rows;
  int hidden;
  float eps;
  int tpr;      // threads per row (power of two, 16..256)
  int aligned;  // x rows, y rows and w readable as 16-byte chunks
};

hipError_t launch_rmsnorm(RmsArgs args, int dtype, hipStream_t stream);

inline int cdiv(int a, int b) { return (a + b - 1) / b; }

}  // namespace mlora
