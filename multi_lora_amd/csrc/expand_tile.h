// Tiled segment expand body shared by expand_kernel (expand.hip) and the
// mixed-batch expand (grouped.hip): one workgroup's (row tile, 256-column
// tile) of
//   out[t, out_col_s + n] += round(scaling[slot] * sum_{k<rank} y[t, k] * B_s[slot, n, k])
// with y read from `mid`, or (FUSED) added up from the shrink's split sums.
//   wave      = 64 output columns (4 MFMA n-blocks) x all BM tokens
//   MFMA tile = D[n][t] += B[n][k] * y[t][k]   (16 columns x 16 tokens)
// The output tile is prefetched into registers before the MFMA loop so its
// HBM latency overlaps the B / y reads; the rounded deltas go through LDS
// so the read-modify-write of `out` is done with row-contiguous 16-byte
// chunks.  All loads are unconditional (rows clamped, chunks masked).
#pragma once

#include "kernels.h"
#include "loads.h"

namespace mlora {

// Per-workgroup LDS of expand_tile.
template <class T, int BM, bool FUSED>
struct ExpandTileLds {
  using raw = typename T::raw_t;
  static constexpr int LDS_STRIDE = kExpandBN + T::VEC;  // padded row, keeps 16-byte alignment
  static constexpr int YS = kFuseMaxRank + T::VEC;       // y tile row (split sums added here)
  raw delta[BM * LDS_STRIDE];
  raw ytile[FUSED ? BM * YS : 1];
};

// Tile `tr` (rows [tr.start + tr.mt * BM, ...) of one segment), column tile
// nt_g of the call's slices.  Every thread of the workgroup calls it.
template <class T, int BM, bool AL, bool FUSED>
__device__ __forceinline__ void expand_tile(const ExpandArgs& a, const TileRef& tr, int nt_g,
                                            ExpandTileLds<T, BM, FUSED>& lds) {
  using raw = typename T::raw_t;
  constexpr int VEC = T::VEC;
  constexpr int KSTEP = T::KSTEP;
  constexpr int BN = kExpandBN;
  constexpr int TB = BM / 16;
  constexpr int LDS_STRIDE = ExpandTileLds<T, BM, FUSED>::LDS_STRIDE;
  constexpr int CPR = BN / VEC;             // chunks per tile row
  constexpr int RPT = BM * CPR / 256;       // chunks per thread in the RMW
  constexpr int YS = ExpandTileLds<T, BM, FUSED>::YS;
  raw* delta = lds.delta;
  raw* ytile = lds.ytile;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int r16 = lane & 15;
  const int g = lane >> 4;

  // Aligned y from mid (kEarly): the first K-step's mid and B fragments are
  // requested before the output tile, and the slot's rank and scaling with
  // them (see below); otherwise the rank comes first.
  constexpr bool kEarly = AL && !FUSED;
  const int end = tr.end;
  const int row0 = tr.start + tr.mt * BM;
  const int slot = tr.slot;
  int rank = 0;
  float scale = 0.f;
  if constexpr (!kEarly) {
    rank = slot_rank_of(a.meta, slot, a.r_max, 1);
    if (rank == 0) return;
  }

  int s = 0;
  while (s + 1 < a.n_slices && nt_g >= a.tile_base[s + 1]) ++s;
  const int n0 = (nt_g - a.tile_base[s]) * BN;
  const int out_dim = a.slices[s].out_dim;
  if constexpr (!kEarly) scale = load_scaling_uniform(a.meta.scalings, slot, a.meta.scal_dtype);

  raw* out = static_cast<raw*>(a.out) + a.slices[s].out_col;

  // Clamped to the pool: an out-of-pool slot has rank 0 (its loads, made
  // before the rank is known, are discarded).
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

  // kEarly: the slot's rank and scaling word are vector loads (lane0 is 0
  // in every lane, but not known to be uniform), then the first K-step's mid
  // and B fragments, unmasked (masked at the MFMA), all before the output
  // tile.  Loads complete in issue order, so the first MFMAs wait for these
  // only, with the tile's loads still in flight.  (As scalar loads the rank
  // and scaling were waited for before any request went out: scalar loads
  // return out of order, so a wait for one waits for all.)
  u32x4 yv0[TB], bv0[4];
  int rank_word = 0, scal_hi = 0;
  uint32_t scal_word = 0;
  const bool scal16 = a.meta.scal_dtype == MLORA_BF16 || a.meta.scal_dtype == MLORA_F16;
  if constexpr (kEarly) {
    const int lane0 = static_cast<int>(__builtin_amdgcn_mbcnt_lo(0u, 0u));
    rank_word = a.meta.ranks[pslot + lane0];
    const char* scal_byte = static_cast<const char*>(a.meta.scalings) + (scal16 ? 2 : 4) * static_cast<int64_t>(pslot);
    scal_hi = scal16 ? static_cast<int>(reinterpret_cast<uintptr_t>(scal_byte) & 3) : 0;
    scal_word = reinterpret_cast<const uint32_t*>(scal_byte - scal_hi)[lane0];
    const int kk = g * VEC;
    const int off = kk < a.r_max ? kk : 0;
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) yv0[tb] = ld_chunk(mrow[tb] + off);
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) bv0[nb] = ld_chunk(brow[nb] + off);
  }

  // Prefetch this thread's share of the output tile (rows clamped to the
  // segment; chunks past out_dim read the row start and are masked).  The
  // tile is read and written once: aligned rows go with the non-temporal
  // hint (the 32-layer step's mixed batch, per layer: q|k|v 26.6 -> 24.7 us,
  // o 18.1 -> 16.3, down 24.3 -> 21.7).
  u32x4 ov[RPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int c = tid + i * 256;
    const int row = c / CPR;
    const int n = n0 + (c - row * CPR) * VEC;
    const int t = min(row0 + row, end - 1);
    if constexpr (AL)
      ov[i] = ld_chunk_nt(out + static_cast<int64_t>(t) * a.out_stride + (n < out_dim ? n : 0)) &
              keep_mask<T>(out_dim - n);
    else
      ov[i] = load_row_chunk<T, AL>(out + static_cast<int64_t>(t) * a.out_stride, n, out_dim - n);
  }

  f32x4 acc[4][TB];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) acc[nb][tb] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Split sums: the workgroup adds up the tile's y (four columns a thread,
  // sixteen split terms in split order with zeros past ks, as the split
  // reduce does) and rounds it into LDS; columns at and past the rank are 0.
  if constexpr (FUSED) {
    static_assert(sizeof(raw) == 2, "split sums are taken for 16-bit types");
    {
      const int ncols = a.n_slices * a.r_max;
      const int quads = a.r_max / 4;
      const int64_t zq = static_cast<int64_t>(a.rows) * ncols / 4;
      for (int q = tid; q < BM * quads; q += 256) {
        const int row = q / quads;
        const int c4 = (q - row * quads) * 4;
        const int t = min(row0 + row, end - 1);
        const f32x4* p = reinterpret_cast<const f32x4*>(a.partials + static_cast<int64_t>(t) * ncols + s * a.r_max + c4);
        f32x4 sum = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int z0 = 0; z0 < 16; z0 += 8) {
          f32x4 v[8];
#pragma unroll
          for (int z = 0; z < 8; ++z) v[z] = (z0 + z < a.ks) ? p[(z0 + z) * zq] : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int z = 0; z < 8; ++z) sum += v[z];
        }
        raw* y = ytile + row * YS + c4;
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = T::from_f32(c4 + e < rank ? sum[e] : 0.f);
      }
      __syncthreads();
    }
  }

  int k_first = 0;
  if constexpr (kEarly) {
    // The scheduling barrier keeps these MFMAs (and their waits) below the
    // output tile's loads.
    __builtin_amdgcn_sched_barrier(0);
    rank = (slot >= 0 && slot < a.meta.num_slots) ? min(max(__builtin_amdgcn_readfirstlane(rank_word), 0), a.r_max)
                                                   : 0;
    const uint32_t w = __builtin_amdgcn_readfirstlane(scal_word);
    const uint16_t h = static_cast<uint16_t>(scal_hi ? (w >> 16) : (w & 0xffffu));
    scale = !scal16 ? __uint_as_float(w) : (a.meta.scal_dtype == MLORA_BF16 ? BF16::to_f32(h) : F16::to_f32(h));
    // A rank-0 (or out-of-pool) slot leaves the output as it is.
    if (rank == 0) {
      wait_vmcnt<0>();
      return;
    }
    const u32x4 m = keep_mask<T>(rank - g * VEC);
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
      for (int tb = 0; tb < TB; ++tb) acc[nb][tb] = T::mma(acc[nb][tb], bv0[nb] & m, yv0[tb] & m);
    k_first = KSTEP;
  }
  for (int k0 = k_first; k0 < rank; k0 += KSTEP) {
    const int kk = k0 + g * VEC;
    const int valid = rank - kk;
    u32x4 yv[TB];
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
      if constexpr (FUSED)
        // Masked to the rank: when r_max is not a multiple of the chunk,
        // the chunk's tail past r_max lies in LDS the fill never wrote.
        yv[tb] = (kk < a.r_max) ? *reinterpret_cast<const u32x4*>(ytile + (tb * 16 + r16) * YS + kk) &
                                      keep_mask<T>(valid)
                                : zero_chunk();
      else
        yv[tb] = load_row_chunk<T, AL>(mrow[tb], kk, valid);
    }
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      const u32x4 bv = load_row_chunk<T, AL>(brow[nb], kk, valid);
#pragma unroll
      for (int tb = 0; tb < TB; ++tb) acc[nb][tb] = T::mma(acc[nb][tb], bv, yv[tb]);
    }
  }

  // Scaled, rounded deltas -> LDS as [token][column].
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) {
    const int nl = (wave * 4 + nb) * 16 + 4 * g;
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
      const int tl = tb * 16 + r16;
      const f32x4 v = acc[nb][tb];
      raw* p = delta + tl * LDS_STRIDE + nl;
      if constexpr (sizeof(raw) == 2) {
        uint2 w;
        w.x = T::pack2(v[0] * scale, v[1] * scale);
        w.y = T::pack2(v[2] * scale, v[3] * scale);
        *reinterpret_cast<uint2*>(p) = w;
      } else {
        *reinterpret_cast<f32x4*>(p) = v * scale;
      }
    }
  }
  __syncthreads();

#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int c = tid + i * 256;
    const int row = c / CPR;
    const int cc = c - row * CPR;
    const int n = n0 + cc * VEC;
    const int t = row0 + row;
    if (t < end && n < out_dim) {
      const u32x4 d = *reinterpret_cast<const u32x4*>(delta + row * LDS_STRIDE + cc * VEC);
      float f[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) f[e] = chunk_elem<T>(ov[i], e) + chunk_elem<T>(d, e);
      if (AL && out_dim - n >= VEC)
        st_chunk_nt(out + static_cast<int64_t>(t) * a.out_stride + n, pack_chunk<T>(f));
      else
        store_row_chunk<T, AL>(out + static_cast<int64_t>(t) * a.out_stride + n, pack_chunk<T>(f), out_dim - n);
    }
  }
}

}  // namespace mlora
