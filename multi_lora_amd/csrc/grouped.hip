// Slot-grouped expand items for batches that mix long and short segments
// (gfx950).
//
// In such a batch every short (decode-like) segment would otherwise take a
// row tile of its own and re-read its adapter's B tile for one row.  Here an
// item is (distinct slot of the short segments, 256 output columns): it
// finds the rows its slot owns with a workgroup-wide scan of the segment
// table (stable: the rows come out in ascending order), requests its B
// fragments and the output rows, takes y from `mid` (or adds the shrink's
// split sums in split order and rounds them to the storage type, the
// reference's `mid` rounding, sgemm_lora_a.py:109), multiplies with B on
// MFMA, scales and rounds (sgemm_lora_b.py:84-89), and adds into the output
// rows through an LDS transpose.  The long segments' row tiles follow in the
// same launch (expand_tile.h).
#include "expand_dma.h"
#include "expand_tile.h"
#include "kernels.h"
#include "loads.h"

namespace mlora {

namespace {

// Where an expand item takes y from.
constexpr int kSumF32 = 0;  // the shrink's fp32 split sums, added here
constexpr int kSumMid = 3;  // `mid` (already summed and rounded)
constexpr int kPollBatch = 16;  // split sums requested together

// One thread's view of one segment of the table: its slot and row range.
struct SegEntry {
  int slot, p0, p1;
};

__device__ __forceinline__ SegEntry load_seg(const SegView& m, int seg) {
  const int sc = min(seg, m.bs - 1);  // callers guarantee bs >= 1
  const int w = m.widx[sc];
  return SegEntry{seg < m.bs ? w : -1, m.indptr[sc], m.indptr[sc + 1]};
}

// One 256-segment block of the slot's row list: entry `e` of this thread;
// `total` rows of the slot precede the block.  short_only: segments of more
// than kShortSegRows rows are left out.
__device__ __forceinline__ void slot_rows_block(const SegEntry& e, int rows, int slot, int w0, int* list, int* tmp,
                                                int* total, bool short_only) {
  int st = 0, len = 0;
  if (e.slot == slot) {
    st = max(e.p0, 0);
    len = max(min(e.p1, rows) - st, 0);
    if (short_only && len > kShortSegRows) len = 0;
  }
  int sum;
  const int off = block_exclusive_scan<4>(len, tmp, &sum) + *total;
  const int lo = max(w0 - off, 0);
  const int hi = min(w0 + kGroupRows - off, len);
  for (int i = lo; i < hi; ++i) list[off + i - w0] = st + i;
  *total += sum;
}

// Rows owned by `slot` in ascending order.  Positions [w0, w0 + kGroupRows)
// of that list go to `list`; returns the full count.  `first` is this
// thread's entry of the first 256 segments, loaded at kernel start so the
// table read overlaps the other first loads.  All threads call it.  The
// first block is kept out of the loop over further blocks: a path that
// joins the loop's freshly loaded entries would make the compiler wait for
// every load in flight (the caller's A or B fragments included) before the
// scan, instead of for `first` alone.
__device__ int slot_rows(const SegView& m, const SegEntry& first, int rows, int slot, int w0, int* list, int* tmp,
                         bool short_only) {
  int total = 0;
  slot_rows_block(first, rows, slot, w0, list, tmp, &total, short_only);
  for (int base = 256; base < m.bs; base += 256)
    slot_rows_block(load_seg(m, base + threadIdx.x), rows, slot, w0, list, tmp, &total, short_only);
  lds_barrier();
  return total;
}

__device__ __forceinline__ int slot_rank(const GroupedArgs& a, int slot) {
  const int r = (slot < a.meta.num_slots) ? a.meta.ranks[slot] : 0;
  return max(min(r, a.r_max), 0);
}

// Sum over the splits, in split order, of the sums at word `idx`; split z's
// word sits at idx + z * zstride.
__device__ __forceinline__ float chunk_sum(const GroupedArgs& a, int64_t idx, int64_t zstride) {
  float sum = 0.f;
  for (int z0 = 0; z0 < a.kc; z0 += kPollBatch) {
    // Every word of the batch is requested before any is used: indices past
    // the last split read the last split again (in bounds) and count as 0.
    float v[kPollBatch];
    const float* p = a.partials + idx;
#pragma unroll
    for (int u = 0; u < kPollBatch; ++u) v[u] = p[min(z0 + u, a.kc - 1) * zstride];
#pragma unroll
    for (int u = 0; u < kPollBatch; ++u) sum += (z0 + u < a.kc) ? v[u] : 0.f;
  }
  return sum;
}

template <class T, int WN>
struct ExpandLds {
  using raw = typename T::raw_t;
  raw delta[16 * (kExpandBN * WN + T::VEC)];
  raw ytile[16 * (kGroupMaxRank + T::VEC)];
  int rows[kGroupRows];
  int tmp[4];
};

// WN: 256-column blocks per item (each wave 64 * WN columns); RS: MFMA
// K-steps of the expand (r_max <= 32 * RS).
template <class T, int FMT, int WN, int RS>
__device__ void expand_item(const GroupedArgs& a, int slot, int nt_g, ExpandLds<T, WN>& lds) {
  using raw = typename T::raw_t;
  constexpr int VEC = T::VEC;
  constexpr int KSTEP = T::KSTEP;
  constexpr int BN = kExpandBN * WN;
  constexpr int NBW = 4 * WN;  // 16-column blocks per wave
  constexpr int LDS_STRIDE = BN + VEC;
  constexpr int CPR = BN / VEC;
  constexpr int RPT = 16 * CPR / 256;
  constexpr int YS = kGroupMaxRank + VEC;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int r16 = lane & 15;
  const int g = lane >> 4;

  const SegEntry first = load_seg(a.meta, tid);
  const int rank = slot_rank(a, slot);
  // A scalar load, so the B and output-row loads go out at once.
  float scale = 0.f;
  if (slot < a.meta.num_slots) scale = load_scaling_uniform(a.meta.scalings, slot, a.meta.scal_dtype);
  if (rank == 0) return;
  int s = 0;
  while (s + 1 < a.n_slices && nt_g >= a.tile_base[s + 1]) ++s;
  const int n0 = (nt_g - a.tile_base[s]) * BN;
  const int out_dim = a.slices[s].out_dim;

  // B fragments: rows clamped to out_dim; loaded unmasked and masked to the
  // rank where the MFMA uses them, so no instruction between here and the
  // output-row loads needs their data.
  const raw* B = static_cast<const raw*>(a.slices[s].b) + static_cast<int64_t>(slot) * a.slices[s].b_slot_stride;
  u32x4 bf[RS][NBW];
#pragma unroll
  for (int nb = 0; nb < NBW; ++nb) {
    const raw* brow = B + static_cast<int64_t>(min(n0 + (wave * NBW + nb) * 16 + r16, out_dim - 1)) * a.slices[s].b_row_stride;
#pragma unroll
    for (int ks = 0; ks < RS; ++ks) {
      const int kk = ks * KSTEP + g * VEC;
      bf[ks][nb] = ld_chunk(brow + (kk < rank ? kk : 0));
    }
  }

  raw* out = static_cast<raw*>(a.out) + a.slices[s].out_col;
  const int ncols = a.n_slices * a.r_max;
  const int64_t zstride = static_cast<int64_t>(a.rows) * ncols;
  // Columns with sums: whole 16-column blocks up to the rank.
  const int live = min(((rank + 15) >> 4) * 16, a.r_max);
  int total = slot_rows(a.meta, first, a.rows, slot, 0, lds.rows, lds.tmp, a.short_only != 0);
  for (int w0 = 0; w0 < total; w0 += kGroupRows) {
    if (w0 > 0) total = slot_rows(a.meta, first, a.rows, slot, w0, lds.rows, lds.tmp, a.short_only != 0);
    const int cnt = min(kGroupRows, total - w0);
    for (int tt = 0; tt < cnt; tt += 16) {
      u32x4 ov[RPT];
#pragma unroll
      for (int i = 0; i < RPT; ++i) {
        const int cidx = tid + i * 256;
        const int row = cidx / CPR;
        const int n = n0 + (cidx - row * CPR) * VEC;
        const int t = lds.rows[min(tt + row, cnt - 1)];
        ov[i] = load_row_chunk<T, true>(out + static_cast<int64_t>(t) * a.out_stride, n, out_dim - n);
      }
      // The B fragments are masked only after this point: an empty asm that
      // rewrites them keeps the compiler from hoisting the mask, and with it
      // a wait for B, above the output-row loads.
      fence_regs(bf);
      const int rows_here = min(16, cnt - tt);
      // y = in-order sum of the K-chunk sums, rounded like the reference's
      // mid; zero at and past the rank.  One (row, column) per thread.
      for (int idx = tid; idx < 16 * a.r_max; idx += 256) {
        const int yr = idx / a.r_max;
        const int yc = idx - yr * a.r_max;
        float v = 0.f;
        if (yr < rows_here && yc < live) {
          if constexpr (FMT == kSumMid)
            v = T::to_f32(static_cast<const raw*>(a.mid)[static_cast<int64_t>(lds.rows[tt + yr]) * a.mid_stride +
                                                         s * a.r_max + yc]);
          else
            v = chunk_sum(a, static_cast<int64_t>(lds.rows[tt + yr]) * ncols + s * a.r_max + yc, zstride);
        }
        lds.ytile[yr * YS + yc] = T::from_f32(yc < rank ? v : 0.f);
      }
      lds_barrier();

      f32x4 acc[NBW];
#pragma unroll
      for (int nb = 0; nb < NBW; ++nb) acc[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < RS; ++ks) {
        if (ks * KSTEP >= rank) break;
        const int kk = ks * KSTEP + g * VEC;
        const u32x4 yv = (kk < a.r_max) ? *reinterpret_cast<const u32x4*>(lds.ytile + r16 * YS + kk) : zero_chunk();
#pragma unroll
        for (int nb = 0; nb < NBW; ++nb) acc[nb] = T::mma(acc[nb], bf[ks][nb] & keep_mask<T>(rank - kk), yv);
      }
#pragma unroll
      for (int nb = 0; nb < NBW; ++nb) {
        const f32x4 v = acc[nb];
        uint2 w;
        w.x = static_cast<uint32_t>(T::from_f32(v[0] * scale)) | (static_cast<uint32_t>(T::from_f32(v[1] * scale)) << 16);
        w.y = static_cast<uint32_t>(T::from_f32(v[2] * scale)) | (static_cast<uint32_t>(T::from_f32(v[3] * scale)) << 16);
        *reinterpret_cast<uint2*>(lds.delta + r16 * LDS_STRIDE + (wave * NBW + nb) * 16 + 4 * g) = w;
      }
      lds_barrier();
#pragma unroll
      for (int i = 0; i < RPT; ++i) {
        const int cidx = tid + i * 256;
        const int row = cidx / CPR;
        const int cc = cidx - row * CPR;
        const int n = n0 + cc * VEC;
        if (tt + row < cnt && n < out_dim) {
          const u32x4 d = *reinterpret_cast<const u32x4*>(lds.delta + row * LDS_STRIDE + cc * VEC);
          float f[VEC];
#pragma unroll
          for (int e = 0; e < VEC; ++e) f[e] = chunk_elem<T>(ov[i], e) + chunk_elem<T>(d, e);
          st_chunk(out + static_cast<int64_t>(lds.rows[tt + row]) * a.out_stride + n, pack_chunk<T>(f));
        }
      }
      // The output rows are used above only under a condition; this use on
      // every path lets the next tile start without a wait for their loads.
      fence_regs(ov);
      lds_barrier();
    }
  }
}

// ---------------------------------------------------------------- mixed batches
// Distinct slots of the short segments (1..kShortSegRows rows after clamping
// to the call's rows, slot in [0, num_slots)), as a bitmap over the pool in
// LDS, with each word's exclusive count of set bits in `offs`; returns how
// many there are.  Every thread calls it.
__device__ int short_slot_map(const GroupedArgs& a, unsigned* bits, int* offs, int* tmp) {
  const int nwords = (a.meta.num_slots + 31) >> 5;
  for (int i = threadIdx.x; i < nwords; i += 256) bits[i] = 0u;
  lds_barrier();
  for (int base = 0; base < a.meta.bs; base += 256) {
    const int seg = base + threadIdx.x;
    if (seg < a.meta.bs) {
      const int p0 = max(a.meta.indptr[seg], 0);
      const int len = min(a.meta.indptr[seg + 1], a.rows) - p0;
      const int w = a.meta.widx[seg];
      if (len >= 1 && len <= kShortSegRows && w >= 0 && w < a.meta.num_slots)
        atomicOr(&bits[w >> 5], 1u << (w & 31));
    }
  }
  lds_barrier();
  const int cnt = threadIdx.x < nwords ? __popc(bits[threadIdx.x]) : 0;
  int total;
  const int off = block_exclusive_scan<4>(cnt, tmp, &total);
  if (threadIdx.x < nwords) offs[threadIdx.x] = off;
  lds_barrier();
  return total;
}

// Slot number k (< the map's count) of the map, in increasing slot order.
// Every thread calls it; the result is uniform.
__device__ int short_slot(const unsigned* bits, const int* offs, int nwords, int k, int* out) {
  const int w = threadIdx.x;
  if (w < nwords) {
    unsigned b = bits[w];
    const int c = __popc(b);
    if (k >= offs[w] && k < offs[w] + c) {
      for (int i = offs[w]; i < k; ++i) b &= b - 1u;  // drop the lower set bits
      *out = w * 32 + __ffs(static_cast<int>(b)) - 1;
    }
  }
  lds_barrier();
  const int slot = *out;
  lds_barrier();
  return slot;
}

// One launch over a mixed batch: slot-grouped items for the short segments,
// then tiled units for the long ones (see launch_mixed).  FUSED: y from
// the shrink's split sums (ea.partials, ea.ks splits), else from mid.  LBM:
// rows of a long-segment tile, 32 (expand_kernel's register-prefetched
// tile) or 64 (expand_dma_kernel's tile streamed through LDS; y from mid
// only).  A workgroup runs units of one kind, so the kinds share one LDS
// area.  A long unit is ea.n_tiles workgroups (256-column tiles), a short
// unit ga.n_tiles (WS * 256-column tiles), the column fastest.
// Unit order: the short units first, or (interleave) a short and a long
// unit alternating while both last, then the rest.
template <class T, bool FUSED, int RS, int LBM, bool NT>
__global__ __launch_bounds__(256, RS == 1 ? 3 : 4) void expand_mixed_kernel(ExpandArgs ea, GroupedArgs ga, int long_units,
                                                              int short_units, int interleave) {
  constexpr bool STREAMED = LBM == kExpandStreamBM;
  constexpr int WS = RS == 1 ? kMixedShortWn : 1;  // wider short items fit the registers at one K-step
  static_assert(LBM == kExpandLongBM || (STREAMED && !FUSED), "32-row tiles, or 64-row streamed ones from mid");
  using TileLds = ExpandTileLds<T, kExpandLongBM, FUSED>;
  constexpr int kLongBytes = STREAMED ? expand_dma_lds_bytes<LBM>() : static_cast<int>(sizeof(TileLds));
  constexpr int kShortBytes = static_cast<int>(sizeof(ExpandLds<T, WS>));
  __shared__ __attribute__((aligned(1024))) unsigned char area[kLongBytes > kShortBytes ? kLongBytes : kShortBytes];
  __shared__ unsigned bits[kMixedMaxSlots / 32];
  __shared__ int offs[kMixedMaxSlots / 32];
  __shared__ int pick;
  const int nt = ea.n_tiles;
  const int ns = ga.n_tiles;
  const int b = blockIdx.x;
  const int m = interleave ? min(long_units, short_units) : 0;
  bool is_short;
  int idx, nt_g;
  if (b < m * (ns + nt)) {
    const int pair = b / (ns + nt);
    const int off = b - pair * (ns + nt);
    is_short = off < ns;
    idx = pair;
    nt_g = is_short ? off : off - ns;
  } else {
    int rb = b - m * (ns + nt);
    if (interleave)
      is_short = short_units > long_units;
    else if (rb < short_units * ns)
      is_short = true;
    else {
      is_short = false;
      rb -= short_units * ns;
    }
    const int w = is_short ? ns : nt;
    idx = m + rb / w;
    nt_g = rb - (rb / w) * w;
  }
  if (is_short) {
    auto& gl = *reinterpret_cast<ExpandLds<T, WS>*>(area);
    const int j = idx;
    const int n_short = short_slot_map(ga, bits, offs, gl.tmp);
    const int nwords = (ga.meta.num_slots + 31) >> 5;
    // More short slots than the launch has units for (by design when the
    // kinds are interleaved, or a summary from an earlier table, e.g. in a
    // replayed graph): this unit also takes slots j + short_units,
    // j + 2 short_units, ...
    for (int k = j; k < n_short; k += short_units) {
      const int slot = short_slot(bits, offs, nwords, k, &pick);
      expand_item<T, FUSED ? kSumF32 : kSumMid, WS, RS>(ga, slot, nt_g, gl);
      __syncthreads();
    }
    return;
  }
  const int u = idx;
  TileRef tr;
  bool found;
  const int total = long_tile(ea.meta, ea.rows, u, LBM, kShortSegRows, &tr, &found);
  if (found) {
    if constexpr (STREAMED)
      expand_dma_tile<T, LBM, NT>(ea, tr, nt_g, area);
    else
      expand_tile<T, LBM, true, FUSED>(ea, tr, nt_g, *reinterpret_cast<TileLds*>(area));
  }
  // More long tiles than the launch has units for: this unit also takes
  // tiles u + long_units, u + 2 long_units, ...  Streamed tiles go as two
  // halves of 32 rows here: the 64-row body inside a loop does not fit the
  // registers (values hoisted out of the loop stay live across it).
  for (int t = u + long_units; t < total; t += long_units) {
    __syncthreads();
    long_tile(ea.meta, ea.rows, t, LBM, kShortSegRows, &tr, &found);
    if (!found) continue;
    if constexpr (STREAMED) {
      constexpr int HBM = LBM / 2;
      TileRef h = tr;
      h.mt = 2 * tr.mt;
      expand_dma_tile<T, HBM, NT>(ea, h, nt_g, area);
      h.mt += 1;
      if (h.start + h.mt * HBM < h.end) {
        __syncthreads();
        expand_dma_tile<T, HBM, NT>(ea, h, nt_g, area);
      }
    } else {
      expand_tile<T, LBM, true, FUSED>(ea, tr, nt_g, *reinterpret_cast<TileLds*>(area));
    }
  }
}

// Long-segment tiles of LBM rows: at most (rows + (LBM - 1) segs) / LBM.
// At least one unit, which loops over every long tile should the summary
// have none.
template <int LBM>
int64_t mixed_long_units(int64_t long_rows, int long_segs) {
  return std::max<int64_t>(1, (long_rows + static_cast<int64_t>(LBM - 1) * long_segs) / LBM);
}

// The short items' column tiles: `wn` 256-column tiles of one slice each.
void set_short_tiles(const ExpandArgs& ea, int wn, GroupedArgs* ga) {
  ga->tile_base[0] = 0;
  for (int s = 0; s < kMaxSlices; ++s)
    ga->tile_base[s + 1] = ga->tile_base[s] + (s < ea.n_slices ? cdiv(ea.slices[s].out_dim, kExpandBN * wn) : 0);
  ga->n_tiles = ga->tile_base[ea.n_slices];
  ga->expand_wn = wn;
}

template <class T, bool FUSED, int LBM, bool NT = false>
hipError_t launch_mixed_t(const ExpandArgs& ea, GroupedArgs ga, int64_t long_rows, int long_segs,
                          int short_units, int cus, hipStream_t stream) {
  // Measurements below are on a mixed batch of 2 x 512 prompt rows and 64
  // one-row segments over 35 rank-16 adapters (gate|up: 4096 -> 2 x 14336;
  // q|k|v: 4096 -> [4096, 1024, 1024]).
  // One K-step (r_max <= 32): short items of kMixedShortWn tiles (gate|up
  // 38.3 vs 39.3 us for the expand); two: one tile, as the registers allow.
  set_short_tiles(ea, ga.r_max <= T::KSTEP ? kMixedShortWn : 1, &ga);
  const int64_t lu = mixed_long_units<LBM>(long_rows, long_segs);
  if (lu > INT32_MAX) return hipErrorInvalidConfiguration;
  const int long_units = static_cast<int>(lu);
  // Short items are latency-bound, long tiles bandwidth-bound.  Short items
  // that fit in one round of workgroup slots (four a CU) go first, and the
  // long tiles fill the other slots (q|k|v: 672 short items, 24.6 vs 25.0
  // us interleaved); more than that, and short-first would run rounds of
  // short items alone before the first long tile, so the kinds alternate
  // (gate|up: 3136 short items, 49.7 vs 51.3 us), and each short unit
  // takes two slots one after the other, which halves the workgroups that
  // wait on their table scans (48.2 vs 49.4 us; three slots a unit: 48.5).
  const int interleave = static_cast<int64_t>(short_units) * ga.n_tiles > 4 * static_cast<int64_t>(cus) ? 1 : 0;
  if (interleave) short_units = (short_units + 1) / 2;
  const int64_t blocks = static_cast<int64_t>(long_units) * ea.n_tiles + static_cast<int64_t>(short_units) * ga.n_tiles;
  if (blocks <= 0) return hipSuccess;
  if (!grid_fits(blocks)) return hipErrorInvalidConfiguration;
  if (ga.r_max <= T::KSTEP)
    hipLaunchKernelGGL((expand_mixed_kernel<T, FUSED, 1, LBM, NT>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       stream, ea, ga, long_units, short_units, interleave);
  else
    hipLaunchKernelGGL((expand_mixed_kernel<T, FUSED, 2, LBM, NT>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       stream, ea, ga, long_units, short_units, interleave);
  return hipGetLastError();
}

template <class T>
hipError_t launch_mixed_dt(const ExpandArgs& ea, const GroupedArgs& ga, bool fused, int64_t long_rows, int long_segs,
                           int short_units, int cus, hipStream_t stream) {
  if (fused) return launch_mixed_t<T, true, kExpandLongBM>(ea, ga, long_rows, long_segs, short_units, cus, stream);
  // Streamed 64-row tiles when they give every CU at least its four
  // workgroups (the mixed batch's gate|up: 1792 of them, 39.4 vs 40.7 us);
  // fewer, larger tiles leave CUs idle (its q|k|v: 384, 13.0 vs 12.1 us).
  // With at least kStreamNtTilesPerCu streamed tiles a CU, their output
  // tiles are read and written with the non-temporal hint (gate|up, 1792
  // tiles: expand 38.4 -> 33.1 us).
  const int64_t streamed = mixed_long_units<kExpandStreamBM>(long_rows, long_segs) * ea.n_tiles;
  if (cus > 0 && streamed >= static_cast<int64_t>(kStreamNtTilesPerCu) * cus)
    return launch_mixed_t<T, false, kExpandStreamBM, true>(ea, ga, long_rows, long_segs, short_units, cus, stream);
  if (streamed >= 4 * static_cast<int64_t>(cus))
    return launch_mixed_t<T, false, kExpandStreamBM>(ea, ga, long_rows, long_segs, short_units, cus, stream);
  return launch_mixed_t<T, false, kExpandLongBM>(ea, ga, long_rows, long_segs, short_units, cus, stream);
}

}  // namespace

hipError_t launch_mixed(const ExpandArgs& args, int dtype, int64_t long_rows, int long_segs, int short_units,
                        int cus, hipStream_t stream) {
  GroupedArgs ga{};
  ga.rows = args.rows;
  for (int s = 0; s < kMaxSlices; ++s) ga.slices[s] = args.slices[s];
  ga.n_slices = args.n_slices;
  ga.r_max = args.r_max;
  ga.out = args.out;
  ga.out_stride = args.out_stride;
  ga.meta = args.meta;
  ga.partials = const_cast<float*>(args.partials);
  ga.kc = args.ks > 1 ? args.ks : 1;
  ga.short_only = 1;
  ga.mid = args.mid;
  ga.mid_stride = args.mid_stride;
  const bool fused = args.ks > 1 && args.partials != nullptr;
  return dtype == MLORA_BF16 ? launch_mixed_dt<BF16>(args, ga, fused, long_rows, long_segs, short_units, cus, stream)
                             : launch_mixed_dt<F16>(args, ga, fused, long_rows, long_segs, short_units, cus, stream);
}

}  // namespace mlora
