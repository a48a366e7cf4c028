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

typedef __attribute__((address_space(1))) void gvoid_t;
typedef __attribute__((address_space(3))) void lvoid_t;

// Streamed form for long segments (16-bit types, aligned rows, 64-row tiles,
// four workgroups a CU):
// the output tile goes from HBM straight into LDS (global_load_lds_dwordx4;
// lane l of a wave instruction fills LDS bytes [16 l, 16 l + 16) above the
// instruction's base), so the prefetch holds no VGPRs and a 64-row tile
// fits.  Rows are 512 bytes, unpadded; chunk p of LDS row r holds output
// chunk p ^ (r & 15), which spreads both the MFMA-layout accesses (16 rows,
// one chunk each) and the row reads over the banks.  The rounded delta is
// added into the tile in place, then whole rows are stored.
template <class T, int BM>
__global__ __launch_bounds__(256, 4) void expand_dma_kernel(ExpandArgs a) {
  using raw = typename T::raw_t;
  static_assert(sizeof(raw) == 2, "16-bit types only");
  constexpr int VEC = T::VEC;
  constexpr int KSTEP = T::KSTEP;
  constexpr int BN = kExpandBN;
  constexpr int TB = BM / 16;
  constexpr int ROWB = BN * 2;           // bytes of a tile row
  constexpr int CPR = BN / VEC;          // 16-byte chunks per tile row (32)
  constexpr int IPW = BM * CPR / 256;    // DMA instructions per wave (64 chunks each)
  constexpr int RPI = 64 / CPR;          // tile rows per instruction (2)
  __shared__ __attribute__((aligned(1024))) unsigned char tile[BM * ROWB];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int r16 = lane & 15;
  const int g = lane >> 4;

  const int bid = blockIdx.x;
  const int nt_g = bid % a.n_tiles;
  TileRef tr;
  if (!dense_tile(a.meta, a.rows, bid / a.n_tiles, BM, &tr)) return;
  const int end = tr.end;
  const int row0 = tr.start + tr.mt * BM;
  const int slot = tr.slot;

  int s = 0;
  while (s + 1 < a.n_slices && nt_g >= a.tile_base[s + 1]) ++s;
  const int n0 = (nt_g - a.tile_base[s]) * BN;
  const int out_dim = a.slices[s].out_dim;
  raw* out = static_cast<raw*>(a.out) + a.slices[s].out_col;

  // Clamped to the pool: an out-of-pool slot has rank 0, and its loads are
  // discarded.
  const int pslot = min(max(slot, 0), a.meta.num_slots - 1);
  const raw* B = static_cast<const raw*>(a.slices[s].b) + static_cast<int64_t>(pslot) * a.slices[s].b_slot_stride;
  const int64_t brs = a.slices[s].b_row_stride;
  const raw* brow[4];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
    brow[nb] = B + static_cast<int64_t>(min(n0 + (wave * 4 + nb) * 16 + r16, out_dim - 1)) * brs;
  const raw* mrow[TB];
#pragma unroll
  for (int tb = 0; tb < TB; ++tb)
    mrow[tb] = static_cast<const raw*>(a.mid) + s * a.r_max +
               static_cast<int64_t>(min(row0 + tb * 16 + r16, end - 1)) * a.mid_stride;

  // The slot's rank and scaling word go out first, as vector loads (lane0 is
  // 0 in every lane, but not known to be uniform), and are waited for
  // together with the first fragments: as scalar loads they were waited for
  // before any request below went out (scalar loads return out of order, so
  // a wait for one waits for all), a round trip of about 1.3 us under load.
  const int lane0 = static_cast<int>(__builtin_amdgcn_mbcnt_lo(0u, 0u));
  const int rank_word = a.meta.ranks[pslot + lane0];
  const bool scal16 = a.meta.scal_dtype == MLORA_BF16 || a.meta.scal_dtype == MLORA_F16;
  const char* scal_byte = static_cast<const char*>(a.meta.scalings) + (scal16 ? 2 : 4) * static_cast<int64_t>(pslot);
  const int scal_hi = scal16 ? static_cast<int>(reinterpret_cast<uintptr_t>(scal_byte) & 3) : 0;
  const uint32_t scal_word = reinterpret_cast<const uint32_t*>(scal_byte - scal_hi)[lane0];

  // The first K-step's mid and B fragments go out before the output tile,
  // unmasked (masked at the MFMA): loads complete in issue order, so waiting
  // for them leaves the tile's loads in flight.
  u32x4 yv0[TB], bv0[4];
  {
    const int kk = g * VEC;
    const int off = kk < a.r_max ? kk : 0;
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) yv0[tb] = ld_chunk(mrow[tb] + off);
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) bv0[nb] = ld_chunk(brow[nb] + off);
  }

  // Output tile -> LDS, every instruction issued (a fixed count keeps the
  // wait below exact): a row past the segment reads the segment's last row
  // and chunks past out_dim read the tile's first chunk, both discarded at
  // the store.
#pragma unroll
  for (int i = 0; i < IPW; ++i) {
    const int ins = wave * IPW + i;
    const int r = ins * RPI + lane / CPR;
    const int q = (lane % CPR) ^ (r & 15);
    const int n = n0 + q * VEC < out_dim ? n0 + q * VEC : n0;
    const raw* src = out + static_cast<int64_t>(min(row0 + r, end - 1)) * a.out_stride + n;
    __builtin_amdgcn_global_load_lds((gvoid_t*)src, (lvoid_t*)(tile + ins * 64 * 16), 16, 0, 0);
  }
  // The rank, scaling and fragments have landed; the scheduling barrier
  // keeps their uses (and the wait) below the tile's loads.
  wait_vmcnt<IPW>();
  __builtin_amdgcn_sched_barrier(0);
  const int rank = (slot >= 0 && slot < a.meta.num_slots)
                       ? min(max(__builtin_amdgcn_readfirstlane(rank_word), 0), a.r_max) : 0;
  float scale;
  {
    const uint32_t w = __builtin_amdgcn_readfirstlane(scal_word);
    const uint16_t h = static_cast<uint16_t>(scal_hi ? (w >> 16) : (w & 0xffffu));
    scale = !scal16 ? __uint_as_float(w) : (a.meta.scal_dtype == MLORA_BF16 ? BF16::to_f32(h) : F16::to_f32(h));
  }
  // A rank-0 (or out-of-pool) slot leaves the output as it is; the tile's
  // loads into LDS must land before the waves leave.
  if (rank == 0) {
    wait_vmcnt<0>();
    return;
  }

  f32x4 acc[4][TB];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) acc[nb][tb] = f32x4{0.f, 0.f, 0.f, 0.f};
  {
    const u32x4 m = keep_mask<T>(rank - g * VEC);
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
      for (int tb = 0; tb < TB; ++tb) acc[nb][tb] = T::mma(acc[nb][tb], bv0[nb] & m, yv0[tb] & m);
  }
  for (int k0 = KSTEP; k0 < rank; k0 += KSTEP) {
    const int kk = k0 + g * VEC;
    const int valid = rank - kk;
    u32x4 yv[TB];
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) yv[tb] = load_row_chunk<T, true>(mrow[tb], kk, valid);
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      const u32x4 bv = load_row_chunk<T, true>(brow[nb], kk, valid);
#pragma unroll
      for (int tb = 0; tb < TB; ++tb) acc[nb][tb] = T::mma(acc[nb][tb], bv, yv[tb]);
    }
  }

  // Every wave's tile loads have landed (this wave's by vmcnt, the others'
  // by the barrier, which is bare: the waits it would add are done here).
  __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));  // vmcnt(0)
  __builtin_amdgcn_s_barrier();

  // out = round(out + round(scale * acc)), in place, 4 columns a lane.
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) {
    const int nl = (wave * 4 + nb) * 16 + 4 * g;  // tile column of v[0]
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
      const int t = tb * 16 + r16;
      const f32x4 v = acc[nb][tb];
      uint2* p = reinterpret_cast<uint2*>(tile + t * ROWB + (((nl / VEC) ^ (t & 15)) << 4) + (nl % VEC) * 2);
      const uint2 o = *p;
      // Two elements a conversion (the same rounding as one at a time).
      const uint32_t dlo = T::pack2(v[0] * scale, v[1] * scale), dhi = T::pack2(v[2] * scale, v[3] * scale);
      auto lo = [](uint32_t u) { return T::to_f32(static_cast<raw>(u & 0xffffu)); };
      auto hi = [](uint32_t u) { return T::to_f32(static_cast<raw>(u >> 16)); };
      uint2 w;
      w.x = T::pack2(lo(o.x) + lo(dlo), hi(o.x) + hi(dlo));
      w.y = T::pack2(lo(o.y) + lo(dhi), hi(o.y) + hi(dhi));
      *p = w;
    }
  }
  __syncthreads();

#pragma unroll
  for (int i = 0; i < IPW; ++i) {
    const int c = tid + i * 256;
    const int r = c / CPR;
    const int q = c % CPR;
    const int n = n0 + q * VEC;
    const int t = row0 + r;
    if (t < end && n < out_dim)
      st_chunk(out + static_cast<int64_t>(t) * a.out_stride + n,
               *reinterpret_cast<const u32x4*>(tile + r * ROWB + ((q ^ (r & 15)) << 4)));
  }
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
  hipLaunchKernelGGL((expand_dma_kernel<T, BM>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, args);
  return hipGetLastError();
}

hipError_t launch_expand(int bm, ExpandArgs args, int dtype, bool aligned, hipStream_t stream) {
  // Long segments on average (at least kExpandStreamBM rows a segment),
  // 16-bit and aligned: 64-row tiles with the output streamed into LDS
  // (measured at prefill gate|up 113.9 vs 126.7 us, down 21.1 vs 21.7 us).
  // Mixed batches, whose tiles are mostly one-row decode segments, keep the
  // 32-row tiles.
  if (aligned && bm == kExpandLongBM && (dtype == MLORA_BF16 || dtype == MLORA_F16) && args.ks <= 1 &&
      static_cast<int64_t>(args.rows) >= static_cast<int64_t>(kExpandStreamBM) * args.meta.bs)
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
