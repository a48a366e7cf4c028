// Segment shrink on gfx950: mid[t, s*r_max + n] = sum_k x[t,k] * A_s[slot,n,k].
//
// Behaviour follows the reference's segment GEMM for LoRA A
// (multi_lora/kernels/sgemm_lora_a.py:10-115 tiled form, :118-183 decode
// form): segment -> slot -> rank lookup from device metadata, fp32
// accumulation, one rounding to the storage type, columns at or past the rank
// stay zero.  Unlike the reference, rank-0 segments write zeros (the
// per-segment PyTorch path returns a zero-initialised tensor,
// multi_lora/backend/torch_backend.py:30-48), so `mid` is fully defined.
//
// Work decomposition (one 256-thread workgroup = 4 wave64s):
//   workgroup  = (segment, row tile of BM tokens, K split kz)
//   wave       = 16 token rows (WM waves along M) x 1/WK of the K-steps
//   MFMA tile  = 16 rank rows x 16 tokens, D[n][t] += A[n][k] * x[t][k]
// The K reduction runs inside the MFMA accumulators; waves that split K
// inside a workgroup are summed through LDS in wave order, and K splits
// across workgroups are summed by the last-arriving workgroup of the tile in
// split order.  Both orders are fixed, so results are deterministic.
#include "kernels.h"
#include "loads.h"

namespace mlora {

namespace {

template <class T, int WM, int MAXS, int NBS>
__device__ __forceinline__ void write_mid_tile(const ShrinkArgs& a, const f32x4 (&acc)[MAXS * NBS],
                                               int row0, int end, int wm, int nb_act) {
  using raw = typename T::raw_t;
  raw* mid = static_cast<raw*>(a.mid);
  const int lane = threadIdx.x & 63;
  const int t = row0 + wm * 16 + (lane & 15);
  if (t >= end) return;
  const int g = lane >> 4;
  const bool vec = (a.align & kAlMid) != 0;
  raw* mrow = mid + static_cast<int64_t>(t) * a.mid_stride;
#pragma unroll
  for (int s = 0; s < MAXS; ++s) {
    if (s >= a.n_slices) break;
#pragma unroll
    for (int nb = 0; nb < NBS; ++nb) {
      if (nb >= nb_act) break;
      const int n = nb * 16 + 4 * g;
      const f32x4 v = acc[s * NBS + nb];
      raw* p = mrow + s * a.r_max + n;
      if (vec && n + 3 < a.r_max) {
        if constexpr (sizeof(raw) == 2) {
          uint2 w;
          w.x = static_cast<uint32_t>(T::from_f32(v[0])) | (static_cast<uint32_t>(T::from_f32(v[1])) << 16);
          w.y = static_cast<uint32_t>(T::from_f32(v[2])) | (static_cast<uint32_t>(T::from_f32(v[3])) << 16);
          *reinterpret_cast<uint2*>(p) = w;
        } else {
          *reinterpret_cast<f32x4*>(p) = v;
        }
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (n + q < a.r_max) p[q] = T::from_f32(v[q]);
      }
    }
  }
}

// Columns [nb_act*16, r_max) of every slice are never produced by an MFMA
// tile; they are zero by definition.
template <class T>
__device__ __forceinline__ void zero_mid_tail(const ShrinkArgs& a, int row0, int rows_here, int col_from) {
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

template <class T, int WM, int MAXS, int NBS>
__global__ __launch_bounds__(256) void shrink_kernel(ShrinkArgs a) {
  using raw = typename T::raw_t;
  constexpr int WK = 4 / WM;
  constexpr int BM = 16 * WM;
  constexpr int NACC = MAXS * NBS;
  constexpr int VEC = T::VEC;
  constexpr int KSTEP = T::KSTEP;
  __shared__ f32x4 red[WK > 1 ? (WK - 1) * NACC : 1][kWave];
  __shared__ int s_last;

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
    if (kz == 0) zero_mid_tail<T>(a, row0, rows_here, 0);
    return;
  }
  const int nb_act = (rank + 15) >> 4;

  const raw* x = static_cast<const raw*>(a.x);
  const int trow = row0 + wm * 16 + r16;
  const bool xrow_ok = trow < end;
  const raw* xrow = x + static_cast<int64_t>(xrow_ok ? trow : row0) * a.x_stride;
  const bool alx = (a.align & kAlX) != 0;
  const bool ala = (a.align & kAlA) != 0;

  f32x4 acc[NACC];
#pragma unroll
  for (int j = 0; j < NACC; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int kbeg = kz * a.k_per_split;
  const int kend = min(a.in_dim, kbeg + a.k_per_split);
  for (int k0 = kbeg + wk * KSTEP; k0 < kend; k0 += WK * KSTEP) {
    const int kk = k0 + g * VEC;
    const int valid = a.in_dim - kk;
    const u32x4 xv = xrow_ok ? load_chunk<T>(xrow + kk, valid, alx) : zero_chunk();
#pragma unroll
    for (int s = 0; s < MAXS; ++s) {
      if (s >= a.n_slices) break;
      const raw* A = static_cast<const raw*>(a.slices[s].a) +
                     static_cast<int64_t>(slot) * a.slices[s].a_slot_stride;
#pragma unroll
      for (int nb = 0; nb < NBS; ++nb) {
        if (nb >= nb_act) break;
        const int n = nb * 16 + r16;
        const u32x4 av = (n < rank)
            ? load_chunk<T>(A + static_cast<int64_t>(n) * a.slices[s].a_row_stride + kk, valid, ala)
            : zero_chunk();
        acc[s * NBS + nb] = T::mma(acc[s * NBS + nb], av, xv);
      }
    }
  }

  if constexpr (WK > 1) {
    if (wk > 0) {
#pragma unroll
      for (int j = 0; j < NACC; ++j) red[(wk - 1) * NACC + j][lane] = acc[j];
    }
    __syncthreads();
    if (wk == 0) {
#pragma unroll
      for (int w2 = 1; w2 < WK; ++w2)
#pragma unroll
        for (int j = 0; j < NACC; ++j) acc[j] += red[(w2 - 1) * NACC + j][lane];
    }
  }

  if (a.ks == 1) {
    if (wk == 0) write_mid_tile<T, WM, MAXS, NBS>(a, acc, row0, end, wm, nb_act);
    zero_mid_tail<T>(a, row0, rows_here, nb_act * 16);
    return;
  }

  // Split-K: publish this split's partial tile, then the last workgroup of
  // the tile to arrive sums the splits in order and writes `mid`.
  const int nbst = a.n_slices * a.nb_slice;
  f32x4* parts = reinterpret_cast<f32x4*>(a.partials);
  if (wk == 0) {
    f32x4* dst = parts + ((static_cast<int64_t>(tile) * a.ks + kz) * WM + wm) * nbst * kWave + lane;
#pragma unroll
    for (int s = 0; s < MAXS; ++s) {
      if (s >= a.n_slices) break;
#pragma unroll
      for (int nb = 0; nb < NBS; ++nb) {
        if (nb >= nb_act) break;
        dst[(s * a.nb_slice + nb) * kWave] = acc[s * NBS + nb];
      }
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  __syncthreads();
  if (tid == 0) {
    const int prev = __hip_atomic_fetch_add(a.counters + tile, 1, __ATOMIC_ACQ_REL,
                                            __HIP_MEMORY_SCOPE_AGENT);
    s_last = (prev == a.ks - 1) ? 1 : 0;
  }
  __syncthreads();
  if (!s_last) return;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");

  if (wk == 0) {
#pragma unroll
    for (int s = 0; s < MAXS; ++s) {
      if (s >= a.n_slices) break;
#pragma unroll
      for (int nb = 0; nb < NBS; ++nb) {
        if (nb >= nb_act) break;
        f32x4 sum = f32x4{0.f, 0.f, 0.f, 0.f};
        for (int z = 0; z < a.ks; ++z) {
          const f32x4* src = parts + ((static_cast<int64_t>(tile) * a.ks + z) * WM + wm) * nbst * kWave;
          sum += src[(s * a.nb_slice + nb) * kWave + lane];
        }
        acc[s * NBS + nb] = sum;
      }
    }
    write_mid_tile<T, WM, MAXS, NBS>(a, acc, row0, end, wm, nb_act);
  }
  zero_mid_tail<T>(a, row0, rows_here, nb_act * 16);
  if (tid == 0) __hip_atomic_store(a.counters + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <class T, int WM, int MAXS, int NBS>
hipError_t launch_t(const ShrinkPlan& p, const ShrinkArgs& args, hipStream_t stream) {
  const int64_t blocks = static_cast<int64_t>(args.meta.bs) * p.m_tiles * p.ks;
  if (blocks <= 0) return hipSuccess;
  hipLaunchKernelGGL((shrink_kernel<T, WM, MAXS, NBS>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     stream, args);
  return hipGetLastError();
}

template <class T, int WM>
hipError_t launch_wm(const ShrinkPlan& p, const ShrinkArgs& args, hipStream_t stream) {
  if (p.maxs == 1) {
    if (p.nbs == 1) return launch_t<T, WM, 1, 1>(p, args, stream);
    if (p.nbs == 4) return launch_t<T, WM, 1, 4>(p, args, stream);
    return launch_t<T, WM, 1, 8>(p, args, stream);
  }
  if (p.nbs == 1) return launch_t<T, WM, 4, 1>(p, args, stream);
  return launch_t<T, WM, 4, 4>(p, args, stream);
}

template <class T>
hipError_t launch_dtype(const ShrinkPlan& p, const ShrinkArgs& args, hipStream_t stream) {
  if (p.bm == 16) return launch_wm<T, 1>(p, args, stream);
  return launch_wm<T, 4>(p, args, stream);
}

}  // namespace

bool plan_shrink(int in_dim, int r_max, int n_slices, int bs, int max_len, int dtype, int num_cus,
                 ShrinkPlan* plan) {
  if (in_dim <= 0 || r_max <= 0 || n_slices < 1 || n_slices > kMaxSlices || bs < 0 || max_len < 0)
    return false;
  const int kstep = (dtype == MLORA_F32) ? F32::KSTEP : BF16::KSTEP;
  const int nb_slice = cdiv(r_max, 16);
  ShrinkPlan p{};
  p.maxs = (n_slices == 1) ? 1 : 4;
  if (nb_slice <= 1) p.nbs = 1;
  else if (nb_slice <= 4) p.nbs = 4;
  else if (nb_slice <= 8 && p.maxs == 1) p.nbs = 8;
  else return false;
  p.bm = (max_len <= 16) ? 16 : 64;
  p.m_tiles = cdiv(max_len > 0 ? max_len : 1, p.bm);
  const int ksteps = cdiv(in_dim, kstep);
  const int64_t base = static_cast<int64_t>(bs) * p.m_tiles;
  const int min_steps = (p.bm == 16) ? 4 : 2;
  int ks = 1;
  while (ks < 8 && base * ks < 2LL * num_cus && cdiv(ksteps, ks * 2) >= min_steps) ks *= 2;
  const int steps_per_split = cdiv(ksteps, ks);
  p.k_per_split = steps_per_split * kstep;
  p.ks = cdiv(ksteps, steps_per_split);
  p.ws_bytes = 0;
  if (p.ks > 1) {
    const int wm = p.bm / 16;
    const size_t counters = (static_cast<size_t>(base) * 4 + 255) / 256 * 256;
    p.ws_bytes = counters + static_cast<size_t>(base) * p.ks * wm * n_slices * nb_slice * kWave * sizeof(f32x4);
  }
  *plan = p;
  return true;
}

hipError_t launch_shrink(const ShrinkPlan& plan, ShrinkArgs args, int dtype, hipStream_t stream) {
  args.m_tiles = plan.m_tiles;
  args.ks = plan.ks;
  args.k_per_split = plan.k_per_split;
  args.nb_slice = cdiv(args.r_max, 16);
  switch (dtype) {
    case MLORA_BF16: return launch_dtype<BF16>(plan, args, stream);
    case MLORA_F16: return launch_dtype<F16>(plan, args, stream);
    default: return launch_dtype<F32>(plan, args, stream);
  }
}

}  // namespace mlora
