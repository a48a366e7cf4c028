// Single-launch slot-grouped shrink+expand for decode-shaped batches (gfx950).
//
// Workgroup = (slot, 512 output columns of one slice).  Every workgroup of a
// slot computes that slot's y = x A^T for all of the slot's rows itself (the
// whole reduction over in_dim), then the expand of its own columns:
//   out[t, col] += round(scaling * round(y[t]) . B[slot, col, :rank])
// The roundings are those of the segment kernels (mid rounded to the storage
// type, multi_lora/kernels/sgemm_lora_a.py:109; scaled delta rounded before
// the residual add, multi_lora/kernels/sgemm_lora_b.py:84-89).
//
// No workgroup depends on another, so one launch suffices.  The price is that
// the workgroups of a slot each read the slot's A; the block -> (slot, chunk)
// map puts all workgroups of a slot on the same XCD (blocks are dealt to the
// 8 XCDs round-robin), so A comes from HBM once per slot and is shared
// through that XCD's L2.  The host uses this path when one slot's A is small
// (rank 16 at 4096 inputs is 128 KiB) and the two-launch grouped path
// otherwise.
//
// Load schedule: the slot's rank/scaling, this thread's segment-table entry
// and the B fragments are requested at kernel start; the row scan then
// issues the output-row prefetch; the K loop keeps 8 steps of A and x loads
// in flight per wave.
#include "kernels.h"
#include "loads.h"

namespace mlora {

namespace {

constexpr int kFusedBN = 512;          // output columns per workgroup (4 waves x 8 n-blocks)
constexpr int kFusedPipe = 8;          // K-steps in flight per wave

struct SegEntry2 {
  int slot, p0, p1;
};

__device__ __forceinline__ SegEntry2 load_entry(const SegView& m, int seg) {
  const int sc = min(seg, m.bs - 1);
  const int w = m.widx[sc];
  return SegEntry2{seg < m.bs ? w : -1, m.indptr[sc], m.indptr[sc + 1]};
}

// Rows of `slot`, ascending; window [w0, w0 + kGroupRows) into `list`.
__device__ int fused_slot_rows(const SegView& m, const SegEntry2& first, int rows, int slot, int w0, int* list,
                               int* tmp) {
  int total = 0;
  for (int base = 0; base < m.bs; base += 256) {
    const SegEntry2 e = (base == 0) ? first : load_entry(m, base + threadIdx.x);
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

template <class T, int NB>
__global__ __launch_bounds__(256) void fused_decode_kernel(GroupedArgs a, int chunks) {
  using raw = typename T::raw_t;
  constexpr int VEC = T::VEC;
  constexpr int KSTEP = T::KSTEP;
  constexpr int RS = (NB * 16 + KSTEP - 1) / KSTEP;   // K-steps of the expand
  constexpr int NBW = kFusedBN / 64;                  // n-blocks per wave in the expand (8)
  constexpr int LDS_STRIDE = kFusedBN + VEC;
  constexpr int CPR = kFusedBN / VEC;
  constexpr int RPT = 16 * CPR / 256;
  constexpr int YS = NB * 16 + VEC;
  __shared__ f32x4 red[3 * NB][kWave];
  __shared__ __attribute__((aligned(16))) raw ytile[16 * YS];
  __shared__ __attribute__((aligned(16))) raw delta[16 * LDS_STRIDE];
  __shared__ int s_rows[kGroupRows];
  __shared__ int s_tmp[4];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int r16 = lane & 15;
  const int g = lane >> 4;

  // block -> (slot, chunk): the chunks of one slot share blockIdx % 8.
  const int bid = blockIdx.x;
  const int slot = (bid / (8 * chunks)) * 8 + (bid & 7);
  const int c = (bid >> 3) % chunks;
  if (slot >= a.meta.num_slots) return;

  const SegEntry2 first = load_entry(a.meta, tid);
  const int rank = max(min(a.meta.ranks[slot], a.r_max), 0);
  const float scale = load_scaling(a.meta.scalings, slot, a.meta.scal_dtype);

  // Output chunk -> slice, first column.
  int s = 0;
  while (s + 1 < a.n_slices && c >= a.tile_base[s + 1]) ++s;
  const int n0 = (c - a.tile_base[s]) * kFusedBN;
  const int out_dim = a.slices[s].out_dim;

  if (rank == 0) return;

  // B fragments of this wave's 8 n-blocks (rows clamped, columns past the rank
  // masked: a reused slot may hold stale columns there).
  const raw* B = static_cast<const raw*>(a.slices[s].b) + static_cast<int64_t>(slot) * a.slices[s].b_slot_stride;
  u32x4 bf[RS][NBW];
#pragma unroll
  for (int nb = 0; nb < NBW; ++nb) {
    const raw* brow =
        B + static_cast<int64_t>(min(n0 + (wave * NBW + nb) * 16 + r16, out_dim - 1)) * a.slices[s].b_row_stride;
#pragma unroll
    for (int ks = 0; ks < RS; ++ks) {
      const int kk = ks * KSTEP + g * VEC;
      bf[ks][nb] = load_row_chunk<T, true>(brow, kk, rank - kk);
    }
  }

  // A row pointers: n-block j covers rows j*16 .. j*16+15 (clamped to r_max).
  const raw* arow[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) arow[j] = slice_a<raw>(a.slices, s, slot, min(j * 16 + r16, a.r_max - 1));

  raw* out = static_cast<raw*>(a.out) + a.slices[s].out_col;
  const int nsteps = a.in_dim / KSTEP;  // in_dim is a multiple of 8; the tail is handled below
  const int ytail = a.in_dim - nsteps * KSTEP;

  int total = fused_slot_rows(a.meta, first, a.rows, slot, 0, s_rows, s_tmp);
  for (int w0 = 0; w0 < total; w0 += kGroupRows) {
    if (w0 > 0) total = fused_slot_rows(a.meta, first, a.rows, slot, w0, s_rows, s_tmp);
    const int cnt = min(kGroupRows, total - w0);
    for (int tt = 0; tt < cnt; tt += 16) {
      // Output rows of this tile: requested before the reduction runs.
      u32x4 ov[RPT];
#pragma unroll
      for (int i = 0; i < RPT; ++i) {
        const int cidx = tid + i * 256;
        const int row = cidx / CPR;
        const int n = n0 + (cidx - row * CPR) * VEC;
        const int t = s_rows[min(tt + row, cnt - 1)];
        ov[i] = load_row_chunk<T, true>(out + static_cast<int64_t>(t) * a.out_stride, n, out_dim - n);
      }

      // y^T[n][t] over the whole reduction; wave w takes steps w, w+4, ...
      const raw* xrow = static_cast<const raw*>(a.x) + static_cast<int64_t>(s_rows[min(tt + r16, cnt - 1)]) * a.x_stride;
      f32x4 acc[NB];
#pragma unroll
      for (int j = 0; j < NB; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
      int i = wave;
      for (; i + 4 * (kFusedPipe - 1) < nsteps; i += 4 * kFusedPipe) {
        u32x4 xv[kFusedPipe], av[kFusedPipe][NB];
#pragma unroll
        for (int p = 0; p < kFusedPipe; ++p) {
          const int kk = (i + 4 * p) * KSTEP + g * VEC;
          xv[p] = ld_chunk(xrow + kk);
#pragma unroll
          for (int j = 0; j < NB; ++j) av[p][j] = ld_chunk(arow[j] + kk);
        }
#pragma unroll
        for (int p = 0; p < kFusedPipe; ++p)
#pragma unroll
          for (int j = 0; j < NB; ++j) acc[j] = T::mma(acc[j], av[p][j], xv[p]);
      }
      for (; i < nsteps; i += 4) {
        const int kk = i * KSTEP + g * VEC;
        const u32x4 xv = ld_chunk(xrow + kk);
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[j] = T::mma(acc[j], ld_chunk(arow[j] + kk), xv);
      }
      if (ytail > 0 && wave == (nsteps & 3)) {
        const int kk = nsteps * KSTEP + g * VEC;
        const int valid = a.in_dim - kk;
        const u32x4 xv = load_row_chunk<T, true>(xrow, kk, valid);
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[j] = T::mma(acc[j], load_row_chunk<T, true>(arow[j], kk, valid), xv);
      }

      // Sum the four waves in wave order; round y like `mid`; zero past the rank.
      if (wave > 0) {
#pragma unroll
        for (int j = 0; j < NB; ++j) red[(wave - 1) * NB + j][lane] = acc[j];
      }
      __syncthreads();
      if (wave == 0) {
#pragma unroll
        for (int w2 = 0; w2 < 3; ++w2)
#pragma unroll
          for (int j = 0; j < NB; ++j) acc[j] += red[w2 * NB + j][lane];
#pragma unroll
        for (int j = 0; j < NB; ++j) {
          const int n = j * 16 + 4 * g;
          raw* yp = ytile + r16 * YS + n;
#pragma unroll
          for (int q = 0; q < 4; ++q) yp[q] = T::from_f32(n + q < rank ? acc[j][q] : 0.f);
        }
      }
      __syncthreads();

      // Expand this workgroup's columns: D[col][t] = B[col][k] . y[t][k].
      f32x4 e[NBW];
#pragma unroll
      for (int nb = 0; nb < NBW; ++nb) e[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < RS; ++ks) {
        const int kk = ks * KSTEP + g * VEC;
        const u32x4 yv = (kk < NB * 16) ? *reinterpret_cast<const u32x4*>(ytile + r16 * YS + kk) : zero_chunk();
#pragma unroll
        for (int nb = 0; nb < NBW; ++nb) e[nb] = T::mma(e[nb], bf[ks][nb], yv);
      }
#pragma unroll
      for (int nb = 0; nb < NBW; ++nb) {
        const f32x4 v = e[nb];
        uint2 w;
        w.x = static_cast<uint32_t>(T::from_f32(v[0] * scale)) | (static_cast<uint32_t>(T::from_f32(v[1] * scale)) << 16);
        w.y = static_cast<uint32_t>(T::from_f32(v[2] * scale)) | (static_cast<uint32_t>(T::from_f32(v[3] * scale)) << 16);
        *reinterpret_cast<uint2*>(delta + r16 * LDS_STRIDE + (wave * NBW + nb) * 16 + 4 * g) = w;
      }
      __syncthreads();
#pragma unroll
      for (int ii = 0; ii < RPT; ++ii) {
        const int cidx = tid + ii * 256;
        const int row = cidx / CPR;
        const int cc = cidx - row * CPR;
        const int n = n0 + cc * VEC;
        if (tt + row < cnt && n < out_dim) {
          const u32x4 d = *reinterpret_cast<const u32x4*>(delta + row * LDS_STRIDE + cc * VEC);
          float f[VEC];
#pragma unroll
          for (int ee = 0; ee < VEC; ++ee) f[ee] = chunk_elem<T>(ov[ii], ee) + chunk_elem<T>(d, ee);
          st_chunk(out + static_cast<int64_t>(s_rows[tt + row]) * a.out_stride + n, pack_chunk<T>(f));
        }
      }
      __syncthreads();
    }
  }
}

template <class T, int NB>
hipError_t launch_nb(const GroupedArgs& args, hipStream_t stream) {
  const int chunks = args.n_tiles;
  const int64_t blocks = static_cast<int64_t>(cdiv(args.meta.num_slots, 8)) * 8 * chunks;
  if (blocks <= 0) return hipSuccess;
  hipLaunchKernelGGL((fused_decode_kernel<T, NB>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, args,
                     chunks);
  return hipGetLastError();
}

template <class T>
hipError_t launch_dtype(const GroupedArgs& args, hipStream_t stream) {
  const int nb = cdiv(args.r_max, 16);
  if (nb <= 1) return launch_nb<T, 1>(args, stream);
  if (nb <= 2) return launch_nb<T, 2>(args, stream);
  return launch_nb<T, 4>(args, stream);
}

}  // namespace

int fused_chunks(const int* out_dims, int n_slices, int* tile_base) {
  int tiles = 0;
  for (int s = 0; s < n_slices; ++s) {
    tile_base[s] = tiles;
    tiles += cdiv(out_dims[s], kFusedBN);
  }
  tile_base[n_slices] = tiles;
  return tiles;
}

hipError_t launch_fused_decode(GroupedArgs args, int dtype, hipStream_t stream) {
  if (dtype == MLORA_BF16) return launch_dtype<BF16>(args, stream);
  return launch_dtype<F16>(args, stream);
}

}  // namespace mlora
