// Segment shrink on gfx950: mid[t, s*r_max + n] = sum_k x[t,k] * A_s[slot,n,k].
//
// Behaviour follows the reference's segment GEMM for LoRA A
// (multi_lora/kernels/sgemm_lora_a.py:10-115 tiled form, :118-183 decode
// form): segment -> slot -> rank lookup from device metadata, fp32
// accumulation, one rounding to the storage type, columns at or past the rank
// are zero.  Unlike the reference, rank-0 segments write zeros (the
// per-segment PyTorch path returns a zero-initialised tensor,
// multi_lora/backend/torch_backend.py:30-48), so `mid` is fully defined.
//
// Work decomposition (one 256-thread workgroup = 4 wave64s); the MFMA tile
// is 16 rank rows x 16 tokens, D[n][t] += A[n][k] * x[t][k]:
//   short segments (<= 16 rows, shrink_kernel): workgroup = (segment, K
//     split); the 4 waves take alternate K-steps of the same 16 rows and are
//     summed through LDS in wave order.
//   long segments: workgroup = (dense 64-row tile, K split); each wave owns
//     16 rows of the tile and every rank block.  16-bit aligned data with K
//     splits in multiples of 64 stream x and A straight into LDS three
//     stages deep (shrink_dma_kernel); other 16-bit aligned data stage them
//     through registers (shrink_lds_kernel); the rest load MFMA fragments
//     directly (shrink_rows_kernel).
// When K is split over workgroups each split stores fp32 sums and a second
// launch adds them in split order, so the result is deterministic and no
// workgroup ever waits on another.
//
// Loads in the K loop are unconditional: rows past the segment end or the
// rank are clamped to a row that exists (their products are discarded), so a
// wave keeps several 16-byte loads of x and A in flight.
#include "kernels.h"
#include "loads.h"

namespace mlora {

namespace {

// 16-row blocks per wave of the long-segment kernels, by the number of
// 16-row A blocks (keeps the LDS tiles of shrink_lds_kernel within 70 KB).
template <int NBT>
constexpr int kShrinkRb = 1;

template <class T>
__device__ __forceinline__ void zero_mid_cols(const ShrinkArgs& a, int row0, int rows_here, int col_from) {
  using raw = typename T::raw_t;
  const int width = a.r_max - col_from;
  if (width <= 0) return;
  raw* mid = static_cast<raw*>(a.mid);
  const int per_row = a.n_slices * width;
  for (int i = threadIdx.x; i < rows_here * per_row; i += blockDim.x) {
    const int r = i / per_row;
    const int c = i - r * per_row;
    const int s = c / width;
    const int col = s * a.r_max + col_from + (c - s * width);
    mid[static_cast<int64_t>(row0 + r) * a.mid_stride + col] = T::from_f32(0.f);
  }
}

template <class T, int WM, int NBT, bool AL>
__global__ __launch_bounds__(256) void shrink_kernel(ShrinkArgs a) {
  using raw = typename T::raw_t;
  constexpr int WK = 4 / WM;
  constexpr int BM = 16 * WM;
  constexpr int VEC = T::VEC;
  constexpr int KSTEP = T::KSTEP;
  __shared__ f32x4 red[WK > 1 ? (WK - 1) * NBT : 1][kWave];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave % WM;
  const int wk = wave / WM;
  const int r16 = lane & 15;
  const int g = lane >> 4;

  const int bid = blockIdx.x;
  const int kz = bid % a.ks;
  const int tile = bid / a.ks;
  const int seg = tile / a.m_tiles;
  const int mt = tile - seg * a.m_tiles;

  const int start = max(a.meta.indptr[seg], 0);
  const int end = min(a.meta.indptr[seg + 1], a.rows);
  const int row0 = start + mt * BM;
  if (row0 >= end) return;
  const int rows_here = min(BM, end - row0);

  int slot, rank;
  seg_slot_rank(a.meta, seg, a.r_max, a.rank_mult, &slot, &rank);
  if (rank == 0) {
    if (kz == 0) zero_mid_cols<T>(a, row0, rows_here, 0);
    return;
  }
  const int nb_act = (rank + 15) >> 4;
  const int nbt = a.n_slices * nb_act;

  // One A row pointer per 16-row block (slice-major), rows clamped to the rank.
  const raw* arow[NBT];
#pragma unroll
  for (int j = 0; j < NBT; ++j) {
    const int jj = j < nbt ? j : 0;
    const int s = jj / nb_act;
    const int n = min((jj - s * nb_act) * 16 + r16, rank - 1);
    arow[j] = slice_a<raw>(a.slices, s, slot, n);
  }
  const raw* xrow =
      static_cast<const raw*>(a.x) + static_cast<int64_t>(min(row0 + wm * 16 + r16, end - 1)) * a.x_stride;

  f32x4 acc[NBT];
#pragma unroll
  for (int j = 0; j < NBT; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int kbeg = kz * a.k_per_split;
  const int kend = min(a.in_dim, kbeg + a.k_per_split);
  const int nfull = (kend - kbeg) / KSTEP;
  for (int i = wk; i < nfull; i += WK) {
    const int kk = kbeg + i * KSTEP + g * VEC;
    const u32x4 xv = load_row_chunk<T, AL>(xrow, kk, VEC);
#pragma unroll
    for (int j = 0; j < NBT; ++j)
      if (j < nbt) acc[j] = T::mma(acc[j], load_row_chunk<T, AL>(arow[j], kk, VEC), xv);
  }
  if (kbeg + nfull * KSTEP < kend && (nfull % WK) == wk) {
    // Last, partial step of the reduction (in_dim not a multiple of KSTEP).
    const int kk = kbeg + nfull * KSTEP + g * VEC;
    const int valid = a.in_dim - kk;
    const u32x4 xv = load_row_chunk<T, AL>(xrow, kk, valid);
#pragma unroll
    for (int j = 0; j < NBT; ++j)
      if (j < nbt) acc[j] = T::mma(acc[j], load_row_chunk<T, AL>(arow[j], kk, valid), xv);
  }

  if constexpr (WK > 1) {
    if (wk > 0) {
#pragma unroll
      for (int j = 0; j < NBT; ++j)
        if (j < nbt) red[(wk - 1) * NBT + j][lane] = acc[j];
    }
    __syncthreads();
    if (wk == 0) {
#pragma unroll
      for (int w2 = 1; w2 < WK; ++w2)
#pragma unroll
        for (int j = 0; j < NBT; ++j)
          if (j < nbt) acc[j] += red[(w2 - 1) * NBT + j][lane];
    }
  }

  const int t = row0 + wm * 16 + r16;
  if (wk == 0 && t < end) {
    const int ncols = a.part_cols;
    raw* mrow = static_cast<raw*>(a.mid) + static_cast<int64_t>(t) * a.mid_stride;
    float* prow = a.partials + (static_cast<int64_t>(kz) * a.rows + t) * ncols;
#pragma unroll
    for (int j = 0; j < NBT; ++j) {
      if (j >= nbt) continue;
      const int s = j / nb_act;
      const int n = (j - s * nb_act) * 16 + 4 * g;
      const int col = s * a.r_max + n;
      f32x4 v = acc[j];
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] = (n + q < rank) ? v[q] : 0.f;
      if (a.ks == 1) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (n + q < a.r_max) mrow[col + q] = T::from_f32(v[q]);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (n + q < a.r_max) prow[col + q] = v[q];
      }
    }
  }
  if (kz == 0) zero_mid_cols<T>(a, row0, rows_here, nb_act * 16);
}

template <class T, int RB, int NBT, bool AL>
__device__ __forceinline__ void load_step(const typename T::raw_t* const (&xrow)[RB],
                                          const typename T::raw_t* const (&arow)[NBT], int kk, u32x4 (&xv)[RB],
                                          u32x4 (&av)[NBT]) {
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) xv[rb] = load_row_chunk<T, AL>(xrow[rb], kk, T::VEC);
#pragma unroll
  for (int j = 0; j < NBT; ++j) av[j] = load_row_chunk<T, AL>(arow[j], kk, T::VEC);
}

template <class T, int RB, int NBT>
__device__ __forceinline__ void mma_step(f32x4 (&acc)[RB][NBT], const u32x4 (&xv)[RB], const u32x4 (&av)[NBT]) {
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int j = 0; j < NBT; ++j) acc[rb][j] = T::mma(acc[rb][j], av[j], xv[rb]);
}

// Long segments (prefill): workgroup = (segment, 64*RB-row tile, K split);
// each wave owns RB 16-row blocks of the tile and every rank block, so x is
// read once per workgroup and the A fragments, the same for all four waves,
// come from L1.  No LDS and no barriers: waves run independently.
template <class T, int NBT, int RB, bool AL>
__global__ __launch_bounds__(256) void shrink_rows_kernel(ShrinkArgs a) {
  using raw = typename T::raw_t;
  constexpr int BM = 64 * RB;
  constexpr int VEC = T::VEC;
  constexpr int KSTEP = T::KSTEP;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r16 = lane & 15;
  const int g = lane >> 4;

  const int bid = blockIdx.x;
  const int kz = bid % a.ks;
  TileRef tr;
  if (!dense_tile(a.meta, a.rows, bid / a.ks, BM, &tr)) return;
  const int end = tr.end;
  const int row0 = tr.start + tr.mt * BM;
  const int rows_here = min(BM, end - row0);
  const int slot = tr.slot;
  const int rank = slot_rank_of(a.meta, slot, a.r_max, a.rank_mult);
  if (rank == 0) {
    if (kz == 0) zero_mid_cols<T>(a, row0, rows_here, 0);
    return;
  }
  const int nb_act = (rank + 15) >> 4;
  const int nbt = a.n_slices * nb_act;

  const raw* arow[NBT];
#pragma unroll
  for (int j = 0; j < NBT; ++j) {
    const int jj = j < nbt ? j : 0;
    const int s = jj / nb_act;
    arow[j] = slice_a<raw>(a.slices, s, slot, min((jj - s * nb_act) * 16 + r16, rank - 1));
  }
  const int wrow0 = row0 + wave * RB * 16;
  const raw* xrow[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
    xrow[rb] = static_cast<const raw*>(a.x) + static_cast<int64_t>(min(wrow0 + rb * 16 + r16, end - 1)) * a.x_stride;

  f32x4 acc[RB][NBT];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int j = 0; j < NBT; ++j) acc[rb][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int kbeg = kz * a.k_per_split;
  const int kend = min(a.in_dim, kbeg + a.k_per_split);
  const int nfull = (kend - kbeg) / KSTEP;
  // A wave whose row blocks all lie past the segment end has nothing to add.
  // Two K-steps in flight per wave: step i+1's loads are issued before step
  // i's MFMAs.  Every MFMA runs (blocks past the rank read a clamped row and
  // are dropped at the store), so the loop body has no branches.
  if (wrow0 < end && nfull > 0) {
    u32x4 xv0[RB], av0[NBT], xv1[RB], av1[NBT];
    load_step<T, RB, NBT, AL>(xrow, arow, kbeg + g * VEC, xv0, av0);
    int i = 0;
    // The scheduling barriers keep the compiler from sinking the next step's
    // loads down to their first use, which would leave one step in flight.
    for (; i + 2 <= nfull; i += 2) {
      load_step<T, RB, NBT, AL>(xrow, arow, kbeg + (i + 1) * KSTEP + g * VEC, xv1, av1);
      __builtin_amdgcn_sched_barrier(0);
      mma_step<T, RB, NBT>(acc, xv0, av0);
      __builtin_amdgcn_sched_barrier(0);
      load_step<T, RB, NBT, AL>(xrow, arow, kbeg + min(i + 2, nfull - 1) * KSTEP + g * VEC, xv0, av0);
      __builtin_amdgcn_sched_barrier(0);
      mma_step<T, RB, NBT>(acc, xv1, av1);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (i < nfull) mma_step<T, RB, NBT>(acc, xv0, av0);
  }
  if (wrow0 < end && kbeg + nfull * KSTEP < kend) {
    // Last, partial step of the reduction (in_dim not a multiple of KSTEP).
    const int kk = kbeg + nfull * KSTEP + g * VEC;
    const int valid = a.in_dim - kk;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const u32x4 xv = load_row_chunk<T, AL>(xrow[rb], kk, valid);
#pragma unroll
      for (int j = 0; j < NBT; ++j) acc[rb][j] = T::mma(acc[rb][j], load_row_chunk<T, AL>(arow[j], kk, valid), xv);
    }
  }

  const int ncols = a.part_cols;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int t = wrow0 + rb * 16 + r16;
    if (t >= end) continue;
    raw* mrow = static_cast<raw*>(a.mid) + static_cast<int64_t>(t) * a.mid_stride;
    float* prow = a.partials + (static_cast<int64_t>(kz) * a.rows + t) * ncols;
#pragma unroll
    for (int j = 0; j < NBT; ++j) {
      if (j >= nbt) continue;
      const int s = j / nb_act;
      const int n = (j - s * nb_act) * 16 + 4 * g;
      const int col = s * a.r_max + n;
      f32x4 v = acc[rb][j];
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] = (n + q < rank) ? v[q] : 0.f;
      if (a.ks == 1) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (n + q < a.r_max) mrow[col + q] = T::from_f32(v[q]);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (n + q < a.r_max) prow[col + q] = v[q];
      }
    }
  }
  if (kz == 0) zero_mid_cols<T>(a, row0, rows_here, nb_act * 16);
}

// Long segments, 16-bit types, 16-byte aligned rows: x and A tiles staged
// through LDS.  A stage is 64*RB rows x kLdsKt reduction elements; each row's
// 2*kLdsKt bytes are read by 16 consecutive lanes, so every row is streamed
// in 256-byte pieces rather than the 64-byte pieces that MFMA-layout loads
// give.  The next stage's loads are in flight in registers while the waves
// run the current stage's MFMAs from LDS.  Wave w owns rows
// [w*16*RB, (w+1)*16*RB) of the tile and every rank block.
constexpr int kLdsKt = 128;             // reduction elements per stage
constexpr int kLdsStride = kLdsKt + 8;  // LDS row stride (elements): 16-byte pad, conflict-free fragment reads

template <class T, int NBT, int RB>
__global__ __launch_bounds__(256) void shrink_lds_kernel(ShrinkArgs a) {
  using raw = typename T::raw_t;
  static_assert(sizeof(raw) == 2, "16-bit types only");
  constexpr int BM = 64 * RB;
  constexpr int NA = NBT * 16;
  constexpr int CPR = kLdsKt / 8;     // 16-byte chunks per row per stage
  constexpr int XC = BM * CPR / 256;  // x chunks per thread per stage
  constexpr int AC = NA * CPR / 256;  // A chunks per thread per stage
  static_assert(XC >= 1 && AC >= 1, "tile too small for 256 threads");
  __shared__ __attribute__((aligned(16))) raw xs[BM * kLdsStride];
  __shared__ __attribute__((aligned(16))) raw as[NA * kLdsStride];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int r16 = lane & 15;
  const int g = lane >> 4;

  const int bid = blockIdx.x;
  const int kz = bid % a.ks;
  TileRef tr;
  if (!dense_tile(a.meta, a.rows, bid / a.ks, BM, &tr)) return;
  const int end = tr.end;
  const int row0 = tr.start + tr.mt * BM;
  const int rows_here = min(BM, end - row0);
  const int slot = tr.slot;
  const int rank = slot_rank_of(a.meta, slot, a.r_max, a.rank_mult);
  if (rank == 0) {
    if (kz == 0) zero_mid_cols<T>(a, row0, rows_here, 0);
    return;
  }
  const int nb_act = (rank + 15) >> 4;
  const int nbt = a.n_slices * nb_act;

  // Source rows of this thread's chunks (clamped into the segment / rank).
  // Chunk i of this thread is row tid/CPR + i*(256/CPR) of the tile, at
  // column (tid % CPR) * 8 of the stage.
  const int col = (tid % CPR) * 8;
  const raw* xsrc[XC];
#pragma unroll
  for (int i = 0; i < XC; ++i)
    xsrc[i] = static_cast<const raw*>(a.x) +
              static_cast<int64_t>(min(row0 + (tid + i * 256) / CPR, end - 1)) * a.x_stride;
  const raw* asrc[AC];
#pragma unroll
  for (int i = 0; i < AC; ++i) {
    const int ar = (tid + i * 256) / CPR;
    const int j = min(ar >> 4, nbt - 1);
    const int s = j / nb_act;
    asrc[i] = slice_a<raw>(a.slices, s, slot, min((j - s * nb_act) * 16 + (ar & 15), rank - 1));
  }

  const int kbeg = kz * a.k_per_split;
  const int kend = min(a.in_dim, kbeg + a.k_per_split);
  const int nst = (kend - kbeg + kLdsKt - 1) / kLdsKt;

  u32x4 xr[XC], ar[AC];
  auto fetch = [&](int k0) {
#pragma unroll
    for (int i = 0; i < XC; ++i) xr[i] = load_row_chunk<T, true>(xsrc[i], k0 + col, kend - (k0 + col));
#pragma unroll
    for (int i = 0; i < AC; ++i) ar[i] = load_row_chunk<T, true>(asrc[i], k0 + col, kend - (k0 + col));
  };

  f32x4 acc[RB][NBT];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int j = 0; j < NBT; ++j) acc[rb][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  fetch(kbeg);
  for (int st = 0; st < nst; ++st) {
#pragma unroll
    for (int i = 0; i < XC; ++i) *reinterpret_cast<u32x4*>(xs + ((tid + i * 256) / CPR) * kLdsStride + col) = xr[i];
#pragma unroll
    for (int i = 0; i < AC; ++i) *reinterpret_cast<u32x4*>(as + ((tid + i * 256) / CPR) * kLdsStride + col) = ar[i];
    __syncthreads();
    if (st + 1 < nst) fetch(kbeg + (st + 1) * kLdsKt);
#pragma unroll
    for (int ks = 0; ks < kLdsKt / 32; ++ks) {
      const int kk = ks * 32 + g * 8;
      u32x4 xf[RB], af[NBT];
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
        xf[rb] = *reinterpret_cast<const u32x4*>(xs + (wave * RB * 16 + rb * 16 + r16) * kLdsStride + kk);
#pragma unroll
      for (int j = 0; j < NBT; ++j) af[j] = *reinterpret_cast<const u32x4*>(as + (j * 16 + r16) * kLdsStride + kk);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int j = 0; j < NBT; ++j) acc[rb][j] = T::mma(acc[rb][j], af[j], xf[rb]);
    }
    __syncthreads();
  }

  const int ncols = a.part_cols;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int t = row0 + wave * RB * 16 + rb * 16 + r16;
    if (t >= end) continue;
    raw* mrow = static_cast<raw*>(a.mid) + static_cast<int64_t>(t) * a.mid_stride;
    float* prow = a.partials + (static_cast<int64_t>(kz) * a.rows + t) * ncols;
#pragma unroll
    for (int j = 0; j < NBT; ++j) {
      if (j >= nbt) break;
      const int s = j / nb_act;
      const int n = (j - s * nb_act) * 16 + 4 * g;
      const int col = s * a.r_max + n;
      f32x4 v = acc[rb][j];
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] = (n + q < rank) ? v[q] : 0.f;
      if (a.ks == 1) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (n + q < a.r_max) mrow[col + q] = T::from_f32(v[q]);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (n + q < a.r_max) prow[col + q] = v[q];
      }
    }
  }
  if (kz == 0) zero_mid_cols<T>(a, row0, rows_here, nb_act * 16);
}

// Long segments, 16-bit types, aligned rows, K split in multiples of the
// stage width KT: x and A stages go from HBM straight to LDS
// (global_load_lds_dwordx4: lane l of a wave instruction fills LDS bytes
// [16 l, 16 l + 16) above the instruction's base), S stages in flight, so
// loads hold no VGPRs and occupancy is set by LDS alone.  A workgroup is BM
// token rows (BM / 16 waves of 16 rows each) against the NAL A rows of the
// slices' live rank blocks.  A stage is the BM x rows and the NAL A rows, KT
// elements each (2 KT bytes, KT / 8 chunks of 16 bytes); rows are not
// padded: the chunk c of LDS row r holds source chunk c ^ dma_swz(r), which
// makes the MFMA fragment reads (16 rows, one chunk each) hit 16 different
// bank groups.  A stage is (BM + NAL) / (64 / CPR) load instructions, dealt
// to the waves round-robin.  Per stage: wait for this wave's loads of the
// stage (vmcnt), one barrier (all waves' loads landed, the buffer of stage
// st - 1 is free), request stage st + S - 1 into that buffer, MFMAs from LDS.
// The planned instance is BM 64, KT 64, S 3: 128-row tiles (eight waves)
// and 4 to 9 stages of 32 or 64 elements measured no faster at prefill
// gate|up and down, and neither did the same loads without the MFMAs or
// the A fragment reads (the kernel is bound by its loads).  All row tiles of
// a split walk K in step, so the A rows in flight at any time are few and
// stay in the L2; a stream-K grid (equal runs of (tile, stage) units per
// workgroup) loses that and measured slower (gate|up 23.0 vs 18.2 us).
constexpr int kDmaKt = 64;  // reduction elements per stage
constexpr int kDmaStages = 3;

// Swizzle of LDS row r for rows of CPR 16-byte chunks: the 16 rows of one
// MFMA fragment read land on 16 different 16-byte bank groups.
template <int CPR>
__device__ __forceinline__ int dma_swz(int r) { return (r / (16 / CPR)) & (CPR - 1); }

typedef __attribute__((address_space(1))) void gvoid_t;
typedef __attribute__((address_space(3))) void lvoid_t;

// s_waitcnt vmcnt(n) for a wave-uniform n in [0, MAX] (larger n: MAX).
template <int MAX, int N = 0>
__device__ __forceinline__ void wait_vmcnt_upto(int n) {
  if constexpr (N >= MAX) {
    wait_vmcnt<MAX>();
  } else {
    if (n == N) {
      wait_vmcnt<N>();
      return;
    }
    wait_vmcnt_upto<MAX, N + 1>(n);
  }
}

// s_waitcnt vmcnt(A * live) for a wave-uniform live in [0, L].
template <int A, int L, int N = 0>
__device__ __forceinline__ void wait_vmcnt_times(int live) {
  if constexpr (N >= L) {
    wait_vmcnt<A * L>();
  } else {
    if (live == N) {
      wait_vmcnt<A * N>();
      return;
    }
    wait_vmcnt_times<A, L, N + 1>(live);
  }
}

template <class T, int NBT, int KT, int BM = 64, int S = kDmaStages>
__global__ __launch_bounds__(BM * 4) void shrink_dma_kernel(ShrinkArgs a) {
  using raw = typename T::raw_t;
  static_assert(sizeof(raw) == 2, "16-bit types only");
  constexpr int W = BM / 16;                      // waves
  constexpr int NAL = 16 * (NBT < 2 ? 2 : NBT);  // A rows loaded per stage
  constexpr int ROWS = BM + NAL;
  constexpr int ROW_BYTES = KT * 2;               // 128 or 64
  constexpr int CPR = KT / 8;                     // 16-byte chunks per row per stage
  constexpr int RPI = 64 / CPR;                   // rows per wave instruction
  constexpr int NX = BM / RPI;                    // x instructions per stage
  constexpr int NI = ROWS / RPI;                  // instructions per stage
  constexpr int L = (NI + W - 1) / W;             // most instructions of one wave per stage
  constexpr int STAGE_BYTES = ROWS * ROW_BYTES;
  static_assert(BM % RPI == 0 && NAL % RPI == 0, "whole instructions");
  static_assert(S >= 3 && (S - 2) * L < 64, "vmcnt range");
  __shared__ __attribute__((aligned(1024))) unsigned char lds[S * STAGE_BYTES];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15;
  const int g = lane >> 4;

  const int bid = blockIdx.x;
  const int kz = bid % a.ks;
  TileRef tr;
  if (!dense_tile(a.meta, a.rows, bid / a.ks, BM, &tr)) return;
  const int end = tr.end;
  const int row0 = tr.start + tr.mt * BM;
  const int rows_here = min(BM, end - row0);
  const int slot = tr.slot;
  const int rank = slot_rank_of(a.meta, slot, a.r_max, a.rank_mult);
  if (rank == 0) {
    if (kz == 0) zero_mid_cols<T>(a, row0, rows_here, 0);
    return;
  }
  const int nb_act = (rank + 15) >> 4;
  const int nbt = a.n_slices * nb_act;

  // Load instruction j of this wave is stage instruction i = wave + W j:
  // x rows [i RPI, i RPI + RPI) for i < NX, else A rows [(i - NX) RPI, ...).
  // Lane l fills LDS row (stage-local) i RPI + l / CPR, chunk l % CPR, from
  // source chunk (l % CPR) ^ swz(row).  Instructions whose rows are all past
  // the segment (x) or past the live rank blocks (A) are skipped: they would
  // only fetch a clamped row again, and the products of their LDS rows are
  // discarded.  The same instructions are live in every stage.  An A
  // instruction's rows lie in one 16-row block, so its slice is uniform and
  // the slice's pointers come by scalar loads.
  const int c8 = lane & (CPR - 1);
  const raw* src[L];
  uint32_t live_mask = 0;
  int live = 0;
#pragma unroll
  for (int j = 0; j < L; ++j) {
    const int i = wave + W * j;
    const int r = i * RPI + lane / CPR;  // stage-local LDS row
    if (i < NX) {
      src[j] = static_cast<const raw*>(a.x) + static_cast<int64_t>(min(row0 + r, end - 1)) * a.x_stride +
               ((c8 ^ dma_swz<CPR>(r)) << 3);
    } else {
      const int ra = min(r - BM, NAL - 1);
      const int jb = min(min((i - NX) * RPI, NAL - 1) >> 4, nbt - 1);  // the block of all the instruction's rows
      const int s = jb / nb_act;
      const raw* arow = slice_a<raw>(a.slices, s, slot, min((jb - s * nb_act) * 16 + (ra & 15), rank - 1));
      src[j] = arow + ((c8 ^ dma_swz<CPR>(r)) << 3);
    }
    const bool on = i < NI && (i < NX ? i * RPI < rows_here : (i - NX) * RPI < nbt * 16);
    if (on) {
      live_mask |= 1u << j;
      ++live;
    }
  }

  const int kbeg = kz * a.k_per_split;
  const int kend = min(a.in_dim, kbeg + a.k_per_split);
  const int nst = (kend - kbeg) / KT;  // the dispatch makes the split a multiple of KT

  // Instructions j < XJ of every wave are x loads (W XJ = NX).  x is read
  // once, so those loads carry the non-temporal hint (nt): the L2 keeps the
  // A rows, which every row tile of the segment reads again, in preference.
  constexpr int XJ = NX / W;
  static_assert(XJ * W == NX, "x instructions split evenly over the waves");
  auto issue = [&](int st) {
    unsigned char* base = lds + (st % S) * STAGE_BYTES;
    const int k0 = kbeg + st * KT;
#pragma unroll
    for (int j = 0; j < L; ++j)
      if (live_mask & (1u << j)) {
        gvoid_t* gp = (gvoid_t*)(src[j] + k0);
        lvoid_t* lp = (lvoid_t*)(base + (wave + W * j) * 1024);
        if (j < XJ)
          __builtin_amdgcn_global_load_lds(gp, lp, 16, 0, kCpolNt);
        else
          __builtin_amdgcn_global_load_lds(gp, lp, 16, 0, 0);
      }
  };

  f32x4 acc[NBT];
#pragma unroll
  for (int j = 0; j < NBT; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int st = 0; st < S - 1; ++st)
    if (st < nst) issue(st);
  for (int st = 0; st < nst; ++st) {
    // This wave's loads of stage st have landed once at most those of the
    // stages issued after it are still in flight.
    const int ahead = min(S - 2, nst - 1 - st);
    if (ahead == S - 2)
      wait_vmcnt_times<S - 2, L>(live);
    else
      wait_vmcnt_upto<(S - 2) * L>(ahead * live);
    // A bare barrier: a fenced one would also wait for the stages still in
    // flight.  The barrier makes the wait above true of every wave.
    __builtin_amdgcn_s_barrier();
    if (st + S - 1 < nst) issue(st + S - 1);
    const unsigned char* base = lds + (st % S) * STAGE_BYTES;
#pragma unroll
    for (int ks = 0; ks < KT / 32; ++ks) {
      const int c = ks * 4 + g;
      const int xr = wave * 16 + r16;
      const u32x4 xf = *reinterpret_cast<const u32x4*>(base + xr * ROW_BYTES + ((c ^ dma_swz<CPR>(xr)) << 4));
#pragma unroll
      for (int j = 0; j < NBT; ++j) {
        const int ar = BM + j * 16 + r16;
        const u32x4 af = *reinterpret_cast<const u32x4*>(base + ar * ROW_BYTES + ((c ^ dma_swz<CPR>(ar)) << 4));
        acc[j] = T::mma(acc[j], af, xf);
      }
    }
  }

  const int ncols = a.part_cols;
  const int t = row0 + wave * 16 + r16;
  if (t < end) {
    raw* mrow = static_cast<raw*>(a.mid) + static_cast<int64_t>(t) * a.mid_stride;
    float* prow = a.partials + (static_cast<int64_t>(kz) * a.rows + t) * ncols;
#pragma unroll
    for (int j = 0; j < NBT; ++j) {
      if (j >= nbt) break;
      const int s = j / nb_act;
      const int n = (j - s * nb_act) * 16 + 4 * g;
      const int col = s * a.r_max + n;
      f32x4 v = acc[j];
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] = (n + q < rank) ? v[q] : 0.f;
      if (a.ks == 1) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (n + q < a.r_max) mrow[col + q] = T::from_f32(v[q]);
      } else if ((a.r_max & 3) == 0 && (reinterpret_cast<uintptr_t>(a.partials) & 15) == 0) {
        // n is a multiple of 4 below r_max, so all four columns exist and the
        // store is 16-byte aligned (rows of n_slices * r_max floats).
        if (n < a.r_max) *reinterpret_cast<f32x4*>(prow + col) = v;
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (n + q < a.r_max) prow[col + q] = v[q];
      }
    }
  }
  if (kz == 0) zero_mid_cols<T>(a, row0, rows_here, nb_act * 16);
}

// Sums the K splits of every live (row, column) in split order and rounds
// once to the storage type.  Workgroup = (segment, 16-row tile), whatever
// the shrink's tile height, so the reduction is spread over many CUs.
constexpr int kReduceRows = 16;

template <class T>
__global__ __launch_bounds__(256) void shrink_reduce_kernel(ShrinkArgs a) {
  using raw = typename T::raw_t;
  TileRef tr;
  if (!dense_tile(a.meta, a.rows, blockIdx.x, kReduceRows, &tr)) return;
  const int end = tr.end;
  const int row0 = tr.start + tr.mt * kReduceRows;
  const int rows_here = min(kReduceRows, end - row0);
  const int rank = slot_rank_of(a.meta, tr.slot, a.r_max, a.rank_mult);
  if (rank == 0) return;
  const int live = min(((rank + 15) >> 4) * 16, a.r_max);
  const int ncols = a.part_cols;
  const int per_row = a.n_slices * live;
  const int64_t zs = static_cast<int64_t>(a.rows) * ncols;
  raw* mid = static_cast<raw*>(a.mid);
  if (a.r_max % 4 == 0) {
    // Four columns per thread (live and r_max are multiples of 4 here), so
    // every split load is 16 bytes.
    const int quads = per_row / 4;
    for (int i = threadIdx.x; i < rows_here * quads; i += blockDim.x) {
      const int r = i / quads;
      const int c = (i - r * quads) * 4;
      const int s = c / live;
      const int n = c - s * live;
      const int t = row0 + r;
      const int col = s * a.r_max + n;
      const f32x4* p = reinterpret_cast<const f32x4*>(a.partials + static_cast<int64_t>(t) * ncols + col);
      const int64_t zq = zs / 4;
      f32x4 v[16];
#pragma unroll
      for (int z = 0; z < 16; ++z) v[z] = (z < a.ks) ? p[z * zq] : f32x4{0.f, 0.f, 0.f, 0.f};
      f32x4 sum = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int z = 0; z < 16; ++z) sum += v[z];
      raw* m = mid + static_cast<int64_t>(t) * a.mid_stride + col;
#pragma unroll
      for (int q = 0; q < 4; ++q) m[q] = T::from_f32(n + q < rank ? sum[q] : 0.f);
    }
    return;
  }
  for (int i = threadIdx.x; i < rows_here * per_row; i += blockDim.x) {
    const int r = i / per_row;
    const int c = i - r * per_row;
    const int s = c / live;
    const int n = c - s * live;
    const int t = row0 + r;
    const int col = s * a.r_max + n;
    // Independent loads issued together; added in split order.
    const float* p = a.partials + static_cast<int64_t>(t) * ncols + col;
    float v[16];
#pragma unroll
    for (int z = 0; z < 16; ++z) v[z] = (z < a.ks) ? p[z * zs] : 0.f;
    float sum = 0.f;
#pragma unroll
    for (int z = 0; z < 16; ++z) sum += v[z];
    mid[static_cast<int64_t>(t) * a.mid_stride + col] = T::from_f32(n < rank ? sum : 0.f);
  }
}

// The same reduction for a mid that only the apply path's expand reads
// (16-bit, columns in quads): thread = (row, 4 columns) over every row and
// every column, so the split sums are requested at once, with no look-up of
// the segment table (two dependent round trips) before them.  Rows that no
// live segment covers, and columns past a slot's rank, get whatever the
// split sums held there; the expand never reads them (it skips rank-0
// segments, reads only its segments' rows, and masks y to the rank).  Live
// values are bit-identical to shrink_reduce_kernel's: the same 16-term sum
// in split order, rounded once.  Measured per call (graph-timed): the
// 32-layer step's q|k|v 27.66 -> 26.65 us, gate|up 49.26 -> 48.07; prefill
// gate|up 124.9 -> 123.7, down 50.17 -> 49.24.
template <class T>
__global__ __launch_bounds__(256) void shrink_reduce_rows_kernel(ShrinkArgs a) {
  using raw = typename T::raw_t;
  static_assert(sizeof(raw) == 2, "16-bit types only");
  const int ncols = a.part_cols;
  const int quads = ncols / 4;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= static_cast<int64_t>(a.rows) * quads) return;
  const int t = static_cast<int>(idx / quads);
  const int col = static_cast<int>(idx - static_cast<int64_t>(t) * quads) * 4;
  const f32x4* p = reinterpret_cast<const f32x4*>(a.partials + static_cast<int64_t>(t) * ncols + col);
  const int64_t zq = static_cast<int64_t>(a.rows) * ncols / 4;
  f32x4 v[16];
#pragma unroll
  for (int z = 0; z < 16; ++z) v[z] = (z < a.ks) ? p[z * zq] : f32x4{0.f, 0.f, 0.f, 0.f};
  f32x4 sum = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int z = 0; z < 16; ++z) sum += v[z];
  uint2 w;
  w.x = static_cast<uint32_t>(T::from_f32(sum[0])) | (static_cast<uint32_t>(T::from_f32(sum[1])) << 16);
  w.y = static_cast<uint32_t>(T::from_f32(sum[2])) | (static_cast<uint32_t>(T::from_f32(sum[3])) << 16);
  *reinterpret_cast<uint2*>(static_cast<raw*>(a.mid) + static_cast<int64_t>(t) * a.mid_stride + col) = w;
}

// The in-order reduction of the split sums into mid: over every row when
// the apply path owns mid, else over dense row tiles.
template <class T>
hipError_t launch_reduce(const ShrinkPlan& p, const ShrinkArgs& args, hipStream_t stream) {
  if constexpr (sizeof(typename T::raw_t) == 2) {
    if (args.row_reduce && args.part_cols % 4 == 0 && args.mid_stride % 4 == 0 &&
        reinterpret_cast<uintptr_t>(args.mid) % 8 == 0 && reinterpret_cast<uintptr_t>(args.partials) % 16 == 0) {
      const int64_t n = (static_cast<int64_t>(args.rows) * (args.part_cols / 4) + 255) / 256;
      if (n <= 0) return hipSuccess;
      if (!grid_fits(n)) return hipErrorInvalidConfiguration;
      hipLaunchKernelGGL((shrink_reduce_rows_kernel<T>), dim3(static_cast<unsigned>(n)), dim3(256), 0, stream, args);
      return hipGetLastError();
    }
  }
  const int64_t r_tiles = dense_tiles(args.meta.bs, p.m_tiles * (p.bm / kReduceRows), args.rows, kReduceRows);
  if (r_tiles <= 0) return hipSuccess;
  if (!grid_fits(r_tiles)) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL((shrink_reduce_kernel<T>), dim3(static_cast<unsigned>(r_tiles)), dim3(256), 0, stream, args);
  return hipGetLastError();
}

// The short kernel (bm 16) runs one workgroup per segment and split; the
// long kernels and the reduction run over dense row tiles.
template <class T>
hipError_t launch_with(void (*kern)(ShrinkArgs), const ShrinkPlan& p, const ShrinkArgs& args, hipStream_t stream,
                       int threads = 256) {
  const int64_t tiles = p.bm == 16 ? static_cast<int64_t>(args.meta.bs) * p.m_tiles
                                   : dense_tiles(args.meta.bs, p.m_tiles, args.rows, p.bm);
  if (tiles <= 0) return hipSuccess;
  if (!grid_fits(tiles * p.ks)) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(tiles * p.ks)), dim3(threads), 0, stream, args);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.ks == 1 || args.skip_reduce) return e;
  return launch_reduce<T>(p, args, stream);
}

// The streamed kernel's instance for the plan's (rows, stage width, stages).
template <class T, int NBT>
hipError_t launch_dma(const ShrinkPlan& p, const ShrinkArgs& args, hipStream_t stream) {
  if (p.bm == 64 && p.kt == 64 && p.stages == 3)
    return launch_with<T>(shrink_dma_kernel<T, NBT, 64, 64, 3>, p, args, stream, 256);
  if (p.bm == 128 && p.kt == 64 && p.stages == 3)
    return launch_with<T>(shrink_dma_kernel<T, NBT, 64, 128, 3>, p, args, stream, 512);
  return hipErrorInvalidValue;
}

template <class T, int NBT, bool AL>
hipError_t launch_nbt_al(const ShrinkPlan& p, const ShrinkArgs& args, hipStream_t stream) {
  constexpr int RB = kShrinkRb<NBT>;
  if (p.bm == 16) return launch_with<T>(shrink_kernel<T, 1, NBT, AL>, p, args, stream);
  if constexpr (AL && sizeof(typename T::raw_t) == 2 && NBT <= 8) {
    // Direct-to-LDS stages when every split is a whole number of them
    // (measured at prefill gate|up 25.3 vs 33.7 us, down 39.5 vs 43.5 us).
    // 64-element stages for every block count: with eight A blocks, 32-element
    // stages (36 KB of LDS, twice the occupancy) measured slower at prefill
    // gate|up, 30.8 vs 26 us.
    if (p.kt > 0 && args.in_dim % p.kt == 0 && p.k_per_split % p.kt == 0) return launch_dma<T, NBT>(p, args, stream);
  }
  if (p.bm != 64 * RB) return hipErrorInvalidValue;
  if constexpr (AL && sizeof(typename T::raw_t) == 2 && NBT <= 8)
    return launch_with<T>(shrink_lds_kernel<T, NBT, RB>, p, args, stream);
  return launch_with<T>(shrink_rows_kernel<T, NBT, RB, AL>, p, args, stream);
}

template <class T, bool AL>
hipError_t launch_al(const ShrinkPlan& p, const ShrinkArgs& args, hipStream_t stream) {
  switch (p.nbt) {
    case 1: return launch_nbt_al<T, 1, AL>(p, args, stream);
    case 2: return launch_nbt_al<T, 2, AL>(p, args, stream);
    case 4: return launch_nbt_al<T, 4, AL>(p, args, stream);
    case 8: return launch_nbt_al<T, 8, AL>(p, args, stream);
    default: return launch_nbt_al<T, 16, AL>(p, args, stream);
  }
}

template <class T>
hipError_t launch_dtype(const ShrinkPlan& p, const ShrinkArgs& args, bool aligned, hipStream_t stream) {
  if (p.spg >= args.n_slices)
    return aligned ? launch_al<T, true>(p, args, stream) : launch_al<T, false>(p, args, stream);
  // One launch per group of slices, each writing its own columns of mid and
  // of the split sums (same values as one launch over all slices), then one
  // reduction over every column.
  using raw = typename T::raw_t;
  for (int s0 = 0; s0 < args.n_slices; s0 += p.spg) {
    ShrinkArgs g = args;
    g.n_slices = min(p.spg, args.n_slices - s0);
    for (int i = 0; i < g.n_slices; ++i) g.slices[i] = args.slices[s0 + i];
    g.mid = static_cast<raw*>(args.mid) + static_cast<int64_t>(s0) * args.r_max;
    g.partials = args.partials ? args.partials + static_cast<int64_t>(s0) * args.r_max : nullptr;
    g.skip_reduce = 1;
    const hipError_t e = aligned ? launch_al<T, true>(p, g, stream) : launch_al<T, false>(p, g, stream);
    if (e != hipSuccess) return e;
  }
  if (p.ks == 1 || args.skip_reduce) return hipSuccess;
  return launch_reduce<T>(p, args, stream);
}

}  // namespace

bool plan_shrink(int in_dim, int r_max, int n_slices, int rows, int bs, int max_len, int dtype, int num_cus,
                 ShrinkPlan* plan) {
  if (in_dim <= 0 || r_max <= 0 || n_slices < 1 || n_slices > kMaxSlices || bs < 0 || max_len < 0 || rows < 0)
    return false;
  const int kstep = (dtype == MLORA_F32) ? F32::KSTEP : BF16::KSTEP;
  // Over 8 blocks of A the slices run in groups of at most 8 blocks, one
  // launch each (3 slices at r_max 64: q|k, then v), rather than one
  // 16-block instance at occupancy 1.
  const int per_slice = cdiv(r_max, 16);
  ShrinkPlan p{};
  p.spg = (n_slices * per_slice > 8 && per_slice <= 8) ? 8 / per_slice : n_slices;
  const int blocks = p.spg * per_slice;
  p.nbt = 1;
  while (p.nbt < blocks) p.nbt *= 2;
  if (p.nbt > 16) return false;
  const int rb = 1;  // kShrinkRb
  p.bm = (max_len <= 16) ? 16 : 64 * rb;
  p.m_tiles = cdiv(max_len > 0 ? max_len : 1, p.bm);
  const int ksteps = cdiv(in_dim, kstep);
  const int64_t base = (p.bm == 16) ? static_cast<int64_t>(bs) * p.m_tiles : dense_tiles(bs, p.m_tiles, rows, p.bm);
  int ks = 1;
  if (p.bm == 16) {
    // Decode-shaped rows: enough workgroups to cover the chip twice.
    while (ks < 16 && base * ks < 2LL * num_cus && cdiv(ksteps, ks * 2) >= 16) ks *= 2;
    const int steps_per_split = cdiv(ksteps, ks);
    p.k_per_split = steps_per_split * kstep;
  } else {
    // Long segments.  Each split is a whole number of `unit` elements (the
    // streamed kernel's 64-element stage when it will run, else one K-step).
    // The split count is sized by the batch's rows counted in full 64-row
    // tiles: about 1.7 workgroups of full tiles per CU, at most 12 splits.
    // Measured on prefill gate|up / down (4073 rows: 6 splits, 25.3 / 37.5 us
    // with the reduce, against 30 / 46 us at 8) and on the 32-layer step's
    // mixed batch (1088 rows: 8 splits at K 4096, 12 at K 14336); neither
    // full occupancy nor a wave count predicted these.  Splits keep at least
    // 512 reduction elements, and split sums (written and read back as fp32,
    // 8 bytes per column and split) cost at most the x bytes (at gate|up, six
    // splits move 0.75 of the x bytes in sums and still beat four).
    const bool streamed = dtype != MLORA_F32 && p.nbt <= 8 && in_dim % kDmaKt == 0;
    if (streamed) {
      p.kt = kDmaKt;
      p.stages = kDmaStages;
    }
    // Long reductions over long segments: 128-row tiles (eight waves), so a
    // stage carries twice the x rows for the same A rows.  Prefill down
    // (K 14336, 8 segments of 64..1024 rows): shrink + reduce 33.8 -> 31.0 us
    // at the same six splits (12 splits, what the tile count below would
    // give for 128-row tiles, 32.4 us; 256-row tiles 31.2 us at 12 splits, a
    // fourth stage 31.5 us).  At K 4096 (prefill gate|up) they do not pay
    // (22.5 vs 22.0 us), and batches of short segments keep 64 rows.  At
    // most four A blocks a launch: with eight, three 128-row stages need
    // 96 KB of LDS, one workgroup a CU.
    if (streamed && in_dim >= kLongKRows128 && rows >= 256LL * bs && p.nbt <= 4) {
      p.bm = 128;
      p.m_tiles = cdiv(max_len > 0 ? max_len : 1, p.bm);
    }
    const int unit = streamed ? kDmaKt : kstep;
    const int units = cdiv(in_dim, unit);
    const int ncols = n_slices * r_max;
    const int64_t x_row_bytes = static_cast<int64_t>(in_dim) * (dtype == MLORA_F32 ? 4 : 2);
    const double full_tiles = rows > 64 ? rows / 64.0 : 1.0;
    int want = static_cast<int>(1.7 * num_cus / full_tiles);
    want = want < 1 ? 1 : (want > 12 ? 12 : want);
    int per = cdiv(units, want);
    for (; want > 1; --want) {
      per = cdiv(units, want);
      const int n = cdiv(units, per);
      if (per * unit >= 512 && static_cast<int64_t>(n) * ncols * 8 <= x_row_bytes) break;
    }
    if (want == 1) per = units;
    const int best_units = per;
    p.k_per_split = best_units * unit;
  }
  p.ks = cdiv(in_dim, p.k_per_split);
  p.ws_bytes = (p.ks > 1) ? static_cast<size_t>(p.ks) * rows * n_slices * r_max * sizeof(float) : 0;
  *plan = p;
  return true;
}

hipError_t launch_shrink(const ShrinkPlan& plan, ShrinkArgs args, int dtype, bool aligned, hipStream_t stream) {
  ShrinkPlan p = plan;
  if (p.bm > 64 && !aligned) {
    // 128-row tiles are the streamed kernel's, which needs aligned rows; the
    // register-staged kernels take 64-row tiles, at most twice as many a
    // segment.
    p.bm = 64;
    p.m_tiles *= 2;
  }
  args.m_tiles = p.m_tiles;
  args.ks = p.ks;
  args.k_per_split = p.k_per_split;
  args.part_cols = args.n_slices * args.r_max;
  switch (dtype) {
    case MLORA_BF16: return launch_dtype<BF16>(p, args, aligned, stream);
    case MLORA_F16: return launch_dtype<F16>(p, args, aligned, stream);
    default: return launch_dtype<F32>(p, args, aligned, stream);
  }
}

}  // namespace mlora
