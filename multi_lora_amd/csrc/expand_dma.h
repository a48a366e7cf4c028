// Streamed segment expand body shared by expand_dma_kernel (expand.hip) and
// the mixed-batch expand (grouped.hip): one workgroup's (BM-row tile of a
// long segment, 256-column tile) of
//   out[t, out_col_s + n] += round(scaling[slot] * sum_{k<rank} mid[t, s*r_max+k] * B_s[slot, n, k])
// for 16-bit types and 16-byte aligned rows.
#pragma once

#include "kernels.h"
#include "loads.h"

namespace mlora {

typedef __attribute__((address_space(1))) void gvoid_t;
typedef __attribute__((address_space(3))) void lvoid_t;

// Bytes of LDS the tile needs (BM rows of 256 columns, 16-bit), to be
// aligned to 1024 bytes.
template <int BM>
constexpr int expand_dma_lds_bytes() { return BM * kExpandBN * 2; }

// Tile `tr` (rows [tr.start + tr.mt * BM, ...) of one segment), column tile
// nt_g of the call's slices; `tile` is expand_dma_lds_bytes<BM>() of LDS.
// Every thread of the workgroup calls it, with the LDS free (a barrier after
// any earlier use).  NT: the output tile's loads and stores carry the
// non-temporal hint (large launches; see launch_streamed).  The output tile
// goes from HBM straight into LDS
// (global_load_lds_dwordx4;
// lane l of a wave instruction fills LDS bytes [16 l, 16 l + 16) above the
// instruction's base), so the prefetch holds no VGPRs and a 64-row tile
// fits.  Rows are 512 bytes, unpadded; chunk p of LDS row r holds output
// chunk p ^ (r & 15), which spreads both the MFMA-layout accesses (16 rows,
// one chunk each) and the row reads over the banks.  The rounded delta is
// added into the tile in place, then whole rows are stored.
template <class T, int BM, bool NT = false>
__device__ __forceinline__ void expand_dma_tile(const ExpandArgs& a, const TileRef& tr, int nt_g,
                                                unsigned char* tile) {
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

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int r16 = lane & 15;
  const int g = lane >> 4;

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
    __builtin_amdgcn_global_load_lds((gvoid_t*)src, (lvoid_t*)(tile + ins * 64 * 16), 16, 0, NT ? kCpolNt : 0);
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
    if (t < end && n < out_dim) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(tile + r * ROWB + ((q ^ (r & 15)) << 4));
      if constexpr (NT)
        st_chunk_nt(out + static_cast<int64_t>(t) * a.out_stride + n, v);
      else
        st_chunk(out + static_cast<int64_t>(t) * a.out_stride + n, v);
    }
  }
}

}  // namespace mlora
