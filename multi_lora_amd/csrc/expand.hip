// Segment expand with residual accumulate on gfx950:
//   out[t, out_col_s + n] += round(scaling[slot] * sum_{k<rank} mid[t, s*r_max+k] * B_s[slot, n, k])
//
// Behaviour follows the reference's segment GEMM for LoRA B
// (multi_lora/kernels/sgemm_lora_b.py:10-90 tiled form, :93-153 decode form):
// fp32 accumulation over k < rank, multiply by the slot's scaling, round the
// delta to the storage type, add the existing output in fp32 and round again.
// Rank-0 segments return before touching `out`.  Unlike the reference's tiled
// form (whose output mask omits the column bound, sgemm_lora_b.py:88-90),
// every access here is bounded by out_dim, so any output width is safe.
//
// Work decomposition (256 threads = 4 wave64s per workgroup):
//   workgroup = (dense tile of BM tokens of one segment, tile of 256 output
//               columns of one slice); the n-tile index runs fastest
//   wave      = 64 output columns (4 MFMA n-blocks) x all BM tokens
//   MFMA tile = D[n][t] += B[n][k] * mid[t][k]   (16 columns x 16 tokens)
// expand_kernel (32-row tiles for mixed batches, 16 for decode-shaped ones,
// any dtype): the output tile is prefetched into registers before the MFMA
// loop so its HBM latency overlaps the B/mid reads; the rounded deltas go
// through LDS so the read-modify-write of `out` is done with row-contiguous
// 16-byte chunks.  expand_dma_kernel (64-row tiles when segments are long):
// the output tile is streamed into LDS instead and updated there.  All loads
// are unconditional (rows clamped, chunks masked), so they issue back to
// back.
#include "expand_dma.h"
#include "expand_tile.h"
#include "kernels.h"
#include "loads.h"

namespace mlora {

namespace {

// FUSED: y is added up from the shrink's split sums (a separate instance, so
// the common one keeps its registers and occupancy).
template <class T, int BM, bool AL, bool FUSED>
__global__ __launch_bounds__(256) void expand_kernel(ExpandArgs a) {
  __shared__ __attribute__((aligned(16))) ExpandTileLds<T, BM, FUSED> lds;
  const int bid = blockIdx.x;
  TileRef tr;
  if (!dense_tile(a.meta, a.rows, bid / a.n_tiles, BM, &tr)) return;
  expand_tile<T, BM, AL, FUSED>(a, tr, bid % a.n_tiles, lds);
}

// Streamed form for long segments (16-bit types, aligned rows, 64-row tiles,
// four workgroups a CU); the body is expand_dma_tile (NT: non-temporal
// output tile).
template <class T, int BM, bool NT>
__global__ __launch_bounds__(256, 4) void expand_dma_kernel(ExpandArgs a) {
  __shared__ __attribute__((aligned(1024))) unsigned char tile[expand_dma_lds_bytes<BM>()];
  const int bid = blockIdx.x;
  TileRef tr;
  if (!dense_tile(a.meta, a.rows, bid / a.n_tiles, BM, &tr)) return;
  expand_dma_tile<T, BM, NT>(a, tr, bid % a.n_tiles, tile);
}

template <class T, int BM, bool AL>
hipError_t launch_t(const ExpandArgs& args, hipStream_t stream) {
  const int64_t blocks = dense_tiles(args.meta.bs, args.m_tiles, args.rows, BM) * args.n_tiles;
  if (blocks <= 0) return hipSuccess;
  if (!grid_fits(blocks)) return hipErrorInvalidConfiguration;
  if constexpr (sizeof(typename T::raw_t) == 2) {
    if (args.ks > 1) {
      hipLaunchKernelGGL((expand_kernel<T, BM, AL, true>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                         args);
      return hipGetLastError();
    }
  }
  hipLaunchKernelGGL((expand_kernel<T, BM, AL, false>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, args);
  return hipGetLastError();
}

template <class T, int BM>
hipError_t launch_al(const ExpandArgs& args, bool aligned, hipStream_t stream) {
  return aligned ? launch_t<T, BM, true>(args, stream) : launch_t<T, BM, false>(args, stream);
}

}  // namespace

template <class T>
hipError_t launch_streamed(ExpandArgs args, hipStream_t stream) {
  constexpr int BM = kExpandStreamBM;
  // m_tiles counts 32-row tiles of the longest segment; half of them,
  // rounded up, bound its 64-row tiles.
  args.m_tiles = (args.m_tiles + 1) / 2;
  const int64_t blocks = dense_tiles(args.meta.bs, args.m_tiles, args.rows, BM) * args.n_tiles;
  if (blocks <= 0) return hipSuccess;
  if (!grid_fits(blocks)) return hipErrorInvalidConfiguration;
  // The output tile's loads and stores carry the non-temporal hint in
  // launches of at least kStreamNtTilesPerCu tiles a CU (1.5 rounds of four
  // workgroups): prefill gate|up (7728 tiles) expand 106.2 -> 97.8 us.  In a
  // launch of about one round the hint costs: prefill down (1104 tiles)
  // 17.3 -> 20.1 us.
  if (args.cus > 0 && blocks >= static_cast<int64_t>(kStreamNtTilesPerCu) * args.cus)
    hipLaunchKernelGGL((expand_dma_kernel<T, BM, true>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                       args);
  else
    hipLaunchKernelGGL((expand_dma_kernel<T, BM, false>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                       args);
  return hipGetLastError();
}

hipError_t launch_expand(int bm, ExpandArgs args, int dtype, bool aligned, hipStream_t stream) {
  // Long segments on average (at least kExpandStreamBM rows a segment),
  // 16-bit and aligned: 64-row tiles with the output streamed into LDS
  // (measured at prefill gate|up 113.9 vs 126.7 us, down 21.1 vs 21.7 us),
  // when the 64-row tiles give every CU four workgroups: fewer, and the
  // 32-row tiles' twice as many workgroups are faster (two 512-row prompts,
  // out 4096: 5.9 vs 8.8 us; q|k|v 4096->[4096,1024,1024]: 7.6 vs 10.1 us).
  // Mixed batches, whose tiles are mostly one-row decode segments, keep the
  // 32-row tiles.
  const int64_t streamed = dense_tiles(args.meta.bs, (args.m_tiles + 1) / 2, args.rows, kExpandStreamBM) * args.n_tiles;
  if (aligned && bm == kExpandLongBM && (dtype == MLORA_BF16 || dtype == MLORA_F16) && args.ks <= 1 &&
      static_cast<int64_t>(args.rows) >= static_cast<int64_t>(kExpandStreamBM) * args.meta.bs &&
      (args.cus <= 0 || streamed >= 4 * static_cast<int64_t>(args.cus)))
    return dtype == MLORA_BF16 ? launch_streamed<BF16>(args, stream) : launch_streamed<F16>(args, stream);
  switch (dtype) {
    case MLORA_BF16:
      return bm == 16 ? launch_al<BF16, 16>(args, aligned, stream) : launch_al<BF16, kExpandLongBM>(args, aligned, stream);
    case MLORA_F16:
      return bm == 16 ? launch_al<F16, 16>(args, aligned, stream) : launch_al<F16, kExpandLongBM>(args, aligned, stream);
    default: return launch_al<F32, 16>(args, aligned, stream);
  }
}

}  // namespace mlora
