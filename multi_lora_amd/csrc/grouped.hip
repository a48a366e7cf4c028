// Slot-grouped shrink+expand for decode-shaped batches (gfx950).
//
// The reference launches one program per segment and, in decode, streams
// the segment's whole A / B slice per token (multi_lora/kernels/sgemm_lora_a.py:118-183,
// sgemm_lora_b.py:93-153), so an adapter used by n tokens is read n times.
// Here workgroups are indexed by (slot, chunk) instead: each finds the rows
// its slot owns with a workgroup-wide scan of the segment table (stable: the
// rows come out in ascending order), and reads that slot's A / B chunk once
// for all of them.  No planning pass and no host-side state are involved, so
// the two launches are safe to capture in a HIP graph.
//
//   grouped_shrink  workgroup = (slot, 256-wide K chunk); the 4 waves take
//                   2 K-steps each, A fragments stay in registers while the
//                   slot's rows go by 16 at a time; the four wave sums are
//                   added in LDS and the chunk's fp32 sums are stored per row.
//   grouped_expand  workgroup = (slot, 256 output columns of one slice);
//                   B fragments are loaded first, then for each 16-row tile
//                   the K-chunk sums are added in chunk order, rounded to
//                   the storage type (the reference's `mid` rounding,
//                   sgemm_lora_a.py:109), multiplied with B on MFMA, scaled
//                   and rounded (sgemm_lora_b.py:84-89), and added into the
//                   output rows through an LDS transpose.
// Arithmetic per row is the same as the segment kernels' (fp32 sums, two
// roundings), only the split of the K reduction differs.
#include "kernels.h"
#include "loads.h"

namespace mlora {

namespace {

// One thread's view of one segment of the table: its slot and row range.
struct SegEntry {
  int slot, p0, p1;
};

__device__ __forceinline__ SegEntry load_seg(const SegView& m, int seg) {
  const int sc = min(seg, m.bs - 1);  // callers guarantee bs >= 1
  const int w = m.widx[sc];
  return SegEntry{seg < m.bs ? w : -1, m.indptr[sc], m.indptr[sc + 1]};
}

// Rows owned by `slot` in ascending order.  Positions [w0, w0 + kGroupRows)
// of that list go to `list`; returns the full count.  `first` is this
// thread's entry of the first 256 segments, loaded by the caller at kernel
// start so the table read overlaps the other first loads.  All threads call it.
__device__ int slot_rows(const SegView& m, const SegEntry& first, int rows, int slot, int w0, int* list, int* tmp) {
  int total = 0;
  for (int base = 0; base < m.bs; base += 256) {
    const SegEntry e = (base == 0) ? first : load_seg(m, base + threadIdx.x);
    int st = 0, len = 0;
    if (e.slot == slot) {
      st = max(e.p0, 0);
      len = max(min(e.p1, rows) - st, 0);
    }
    int sum;
    const int off = block_exclusive_scan(len, tmp, &sum) + total;
    const int lo = max(w0 - off, 0);
    const int hi = min(w0 + kGroupRows - off, len);
    for (int i = lo; i < hi; ++i) list[off + i - w0] = st + i;
    total += sum;
  }
  __syncthreads();
  return total;
}

__device__ __forceinline__ int slot_rank(const GroupedArgs& a, int slot) {
  int r = (slot < a.meta.num_slots) ? a.meta.ranks[slot] : 0;
  return max(min(r, a.r_max), 0);
}

template <class T, int NBT>
__global__ __launch_bounds__(256) void grouped_shrink_kernel(GroupedArgs a) {
  using raw = typename T::raw_t;
  constexpr int VEC = T::VEC;
  constexpr int KSTEP = T::KSTEP;
  __shared__ int s_rows[kGroupRows];
  __shared__ int s_tmp[4];
  __shared__ f32x4 red[3 * NBT][kWave];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int r16 = lane & 15;
  const int g = lane >> 4;
  const int slot = blockIdx.x / a.kc;
  const int c = blockIdx.x - slot * a.kc;

  // First loads, issued together: the slot's rank and this thread's entry of
  // the segment table.
  const SegEntry first = load_seg(a.meta, tid);
  const int rank = slot_rank(a, slot);
  if (rank == 0) return;
  const int nb_act = (rank + 15) >> 4;
  const int nbt = a.n_slices * nb_act;
  const int kbeg = c * a.k_chunk;

  // This wave's A fragments for the chunk, kept for every row tile.
  u32x4 af[kGroupSteps][NBT];
#pragma unroll
  for (int j = 0; j < NBT; ++j) {
    const int jj = j < nbt ? j : 0;
    const int s = jj / nb_act;
    const raw* arow = slice_a<raw>(a.slices, s, slot, min((jj - s * nb_act) * 16 + r16, rank - 1));
#pragma unroll
    for (int sp = 0; sp < kGroupSteps; ++sp) {
      const int kk = kbeg + (wave + 4 * sp) * KSTEP + g * VEC;
      af[sp][j] = load_row_chunk<T, true>(arow, kk, a.in_dim - kk);
    }
  }

  const int ncols = a.n_slices * a.r_max;
  int total = slot_rows(a.meta, first, a.rows, slot, 0, s_rows, s_tmp);
  for (int w0 = 0; w0 < total; w0 += kGroupRows) {
    if (w0 > 0) total = slot_rows(a.meta, first, a.rows, slot, w0, s_rows, s_tmp);
    const int cnt = min(kGroupRows, total - w0);
    for (int tt = 0; tt < cnt; tt += 16) {
      const raw* xrow = static_cast<const raw*>(a.x) + static_cast<int64_t>(s_rows[min(tt + r16, cnt - 1)]) * a.x_stride;
      f32x4 acc[NBT];
#pragma unroll
      for (int j = 0; j < NBT; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int sp = 0; sp < kGroupSteps; ++sp) {
        const int kk = kbeg + (wave + 4 * sp) * KSTEP + g * VEC;
        const u32x4 xv = load_row_chunk<T, true>(xrow, kk, a.in_dim - kk);
#pragma unroll
        for (int j = 0; j < NBT; ++j)
          if (j < nbt) acc[j] = T::mma(acc[j], af[sp][j], xv);
      }
      if (wave > 0) {
#pragma unroll
        for (int j = 0; j < NBT; ++j)
          if (j < nbt) red[(wave - 1) * NBT + j][lane] = acc[j];
      }
      __syncthreads();
      if (wave == 0) {
#pragma unroll
        for (int w2 = 0; w2 < 3; ++w2)
#pragma unroll
          for (int j = 0; j < NBT; ++j)
            if (j < nbt) acc[j] += red[w2 * NBT + j][lane];
        if (tt + r16 < cnt) {
          float* prow = a.partials + (static_cast<int64_t>(c) * a.rows + s_rows[tt + r16]) * ncols;
#pragma unroll
          for (int j = 0; j < NBT; ++j) {
            if (j >= nbt) break;
            const int s = j / nb_act;
            const int n = (j - s * nb_act) * 16 + 4 * g;
            if (n < a.r_max) *reinterpret_cast<f32x4*>(prow + s * a.r_max + n) = acc[j];
          }
        }
      }
      __syncthreads();
    }
  }
}

template <class T>
__global__ __launch_bounds__(256) void grouped_expand_kernel(GroupedArgs a) {
  using raw = typename T::raw_t;
  constexpr int VEC = T::VEC;
  constexpr int KSTEP = T::KSTEP;
  constexpr int BN = kExpandBN;
  constexpr int LDS_STRIDE = BN + VEC;
  constexpr int CPR = BN / VEC;
  constexpr int RPT = 16 * CPR / 256;
  constexpr int YS = kGroupMaxRank + VEC;
  constexpr int RS = kGroupMaxRank / KSTEP;
  __shared__ __attribute__((aligned(16))) raw delta[16 * LDS_STRIDE];
  __shared__ __attribute__((aligned(16))) raw ytile[16 * YS];
  __shared__ int s_rows[kGroupRows];
  __shared__ int s_tmp[4];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int r16 = lane & 15;
  const int g = lane >> 4;
  const int slot = blockIdx.x / a.n_tiles;
  const int nt_g = blockIdx.x - slot * a.n_tiles;

  const SegEntry first = load_seg(a.meta, tid);
  const int rank = slot_rank(a, slot);
  const float scale = (slot < a.meta.num_slots) ? load_scaling(a.meta.scalings, slot, a.meta.scal_dtype) : 0.f;
  if (rank == 0) return;
  int s = 0;
  while (s + 1 < a.n_slices && nt_g >= a.tile_base[s + 1]) ++s;
  const int n0 = (nt_g - a.tile_base[s]) * BN;
  const int out_dim = a.slices[s].out_dim;

  // B fragments: rows clamped to out_dim, K masked to the rank.
  const raw* B = static_cast<const raw*>(a.slices[s].b) + static_cast<int64_t>(slot) * a.slices[s].b_slot_stride;
  u32x4 bf[RS][4];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) {
    const raw* brow = B + static_cast<int64_t>(min(n0 + (wave * 4 + nb) * 16 + r16, out_dim - 1)) * a.slices[s].b_row_stride;
#pragma unroll
    for (int ks = 0; ks < RS; ++ks) {
      const int kk = ks * KSTEP + g * VEC;
      bf[ks][nb] = load_row_chunk<T, true>(brow, kk, rank - kk);
    }
  }

  raw* out = static_cast<raw*>(a.out) + a.slices[s].out_col;
  const int ncols = a.n_slices * a.r_max;
  const int yrow = tid >> 4;
  const int ycol = (tid & 15) * 4;
  int total = slot_rows(a.meta, first, a.rows, slot, 0, s_rows, s_tmp);
  for (int w0 = 0; w0 < total; w0 += kGroupRows) {
    if (w0 > 0) total = slot_rows(a.meta, first, a.rows, slot, w0, s_rows, s_tmp);
    const int cnt = min(kGroupRows, total - w0);
    for (int tt = 0; tt < cnt; tt += 16) {
      u32x4 ov[RPT];
#pragma unroll
      for (int i = 0; i < RPT; ++i) {
        const int cidx = tid + i * 256;
        const int row = cidx / CPR;
        const int n = n0 + (cidx - row * CPR) * VEC;
        const int t = s_rows[min(tt + row, cnt - 1)];
        ov[i] = load_row_chunk<T, true>(out + static_cast<int64_t>(t) * a.out_stride, n, out_dim - n);
      }
      // y = in-order sum of the K-chunk sums, rounded like the reference's mid.
      if (ycol < a.r_max) {
        const int t = s_rows[min(tt + yrow, cnt - 1)];
        const float* p = a.partials + static_cast<int64_t>(t) * ncols + s * a.r_max + ycol;
        const int64_t zstride = static_cast<int64_t>(a.rows) * ncols;
        // Issue the chunk loads in groups of 8 before adding, keeping the
        // addition order z = 0, 1, 2, ... (the loads are independent).
        f32x4 sum = f32x4{0.f, 0.f, 0.f, 0.f};
        int z = 0;
        for (; z + 8 <= a.kc; z += 8) {
          f32x4 v[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) v[u] = *reinterpret_cast<const f32x4*>(p + (z + u) * zstride);
#pragma unroll
          for (int u = 0; u < 8; ++u) sum += v[u];
        }
        for (; z < a.kc; ++z) sum += *reinterpret_cast<const f32x4*>(p + z * zstride);
        raw* yp = ytile + yrow * YS + ycol;
#pragma unroll
        for (int q = 0; q < 4; ++q) yp[q] = T::from_f32(ycol + q < rank ? sum[q] : 0.f);
      }
      __syncthreads();

      f32x4 acc[4];
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) acc[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < RS; ++ks) {
        if (ks * KSTEP >= rank) break;
        const int kk = ks * KSTEP + g * VEC;
        const u32x4 yv = (kk < a.r_max) ? *reinterpret_cast<const u32x4*>(ytile + r16 * YS + kk) : zero_chunk();
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) acc[nb] = T::mma(acc[nb], bf[ks][nb], yv);
      }
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) {
        const f32x4 v = acc[nb];
        uint2 w;
        w.x = static_cast<uint32_t>(T::from_f32(v[0] * scale)) | (static_cast<uint32_t>(T::from_f32(v[1] * scale)) << 16);
        w.y = static_cast<uint32_t>(T::from_f32(v[2] * scale)) | (static_cast<uint32_t>(T::from_f32(v[3] * scale)) << 16);
        *reinterpret_cast<uint2*>(delta + r16 * LDS_STRIDE + (wave * 4 + nb) * 16 + 4 * g) = w;
      }
      __syncthreads();
#pragma unroll
      for (int i = 0; i < RPT; ++i) {
        const int cidx = tid + i * 256;
        const int row = cidx / CPR;
        const int cc = cidx - row * CPR;
        const int n = n0 + cc * VEC;
        if (tt + row < cnt && n < out_dim) {
          const u32x4 d = *reinterpret_cast<const u32x4*>(delta + row * LDS_STRIDE + cc * VEC);
          float f[VEC];
#pragma unroll
          for (int e = 0; e < VEC; ++e) f[e] = chunk_elem<T>(ov[i], e) + chunk_elem<T>(d, e);
          st_chunk(out + static_cast<int64_t>(s_rows[tt + row]) * a.out_stride + n, pack_chunk<T>(f));
        }
      }
    }
  }
}

template <class T, int NBT>
hipError_t launch_t(const GroupedArgs& args, int phases, hipStream_t stream) {
  const int64_t g1 = static_cast<int64_t>(args.meta.num_slots) * args.kc;
  const int64_t g2 = static_cast<int64_t>(args.meta.num_slots) * args.n_tiles;
  if (g1 <= 0 || g2 <= 0) return hipSuccess;
  if (phases & 1) {
    hipLaunchKernelGGL((grouped_shrink_kernel<T, NBT>), dim3(static_cast<unsigned>(g1)), dim3(256), 0, stream, args);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (phases & 2) {
    hipLaunchKernelGGL((grouped_expand_kernel<T>), dim3(static_cast<unsigned>(g2)), dim3(256), 0, stream, args);
    return hipGetLastError();
  }
  return hipSuccess;
}

template <class T>
hipError_t launch_dtype(const GroupedArgs& args, int nbt, int phases, hipStream_t stream) {
  switch (nbt) {
    case 1: return launch_t<T, 1>(args, phases, stream);
    case 2: return launch_t<T, 2>(args, phases, stream);
    case 4: return launch_t<T, 4>(args, phases, stream);
    case 8: return launch_t<T, 8>(args, phases, stream);
    default: return launch_t<T, 16>(args, phases, stream);
  }
}

}  // namespace

bool plan_grouped(int in_dim, int r_max, int n_slices, int rows, int dtype, int* kc, int* k_chunk, int* nbt,
                  size_t* ws_bytes) {
  if (dtype != MLORA_BF16 && dtype != MLORA_F16) return false;
  if (in_dim <= 0 || rows <= 0 || n_slices < 1 || n_slices > kMaxSlices) return false;
  if (r_max <= 0 || r_max > kGroupMaxRank || r_max % 8 != 0 || in_dim % 8 != 0) return false;
  const int blocks = n_slices * cdiv(r_max, 16);
  int b = 1;
  while (b < blocks) b *= 2;
  if (b > 16) return false;
  *nbt = b;
  *k_chunk = 4 * kGroupSteps * BF16::KSTEP;
  *kc = cdiv(in_dim, *k_chunk);
  *ws_bytes = static_cast<size_t>(*kc) * rows * n_slices * r_max * sizeof(float);
  return true;
}

hipError_t launch_grouped(GroupedArgs args, int dtype, int nbt, int phases, hipStream_t stream) {
  if (dtype == MLORA_BF16) return launch_dtype<BF16>(args, nbt, phases, stream);
  return launch_dtype<F16>(args, nbt, phases, stream);
}

}  // namespace mlora
