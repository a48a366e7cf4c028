// Pool upload scatter on gfx950: copies staged adapter banks into their slots.
//
// Behaviour follows the reference's upload kernel
// (multi_lora/kernels/scatter_bank.py:17-68, driven by pool.py:157-316): a
// staged row i holds one adapter's bank, every key's A block [rank, in] and
// then every key's B block [out, rank] at offsets fixed per rank; A goes to
// rows [0, rank) of A[key][slot] (contiguous in the slot), B to columns
// [0, rank) of every row of B[key][slot] (row stride max_rank).  Rows past
// the rank, other slots and other keys are not touched.
//
// Work decomposition: workgroup = (block of kScatterElems elements, key,
// adapter); one block covers the same element range of the key's A block and
// of its B block.  A is a straight copy in 16-byte chunks; B is copied one
// rank-wide row piece at a time, in 16-byte chunks when the rank and the row
// stride allow.  Pure data movement: the bound is HBM bandwidth (each element
// read once from the stage and written once to the pool), so the 16-byte
// copies carry the non-temporal hint (the Llama-3-8B bank of 4 adapters:
// 137.4 -> 135.4 us), and blocks are small: a workgroup moves one 16-byte
// chunk of A and one of B a thread, so many blocks are in flight.
#include "kernels.h"
#include "loads.h"

namespace mlora {

namespace {

template <class R>
__device__ __forceinline__ void copy_run(const R* src, R* dst, int64_t n0, int64_t n1, bool vec) {
  // Elements [n0, n1) of src to the same positions of dst.
  constexpr int V = 16 / sizeof(R);
  if (vec) {
    for (int64_t e = n0 + static_cast<int64_t>(threadIdx.x) * V; e < n1; e += static_cast<int64_t>(blockDim.x) * V)
      st_chunk_nt(dst + e, ld_chunk_nt(src + e));
  } else {
    for (int64_t e = n0 + threadIdx.x; e < n1; e += blockDim.x) dst[e] = src[e];
  }
}

template <class R>
__global__ __launch_bounds__(256) void scatter_kernel(ScatterArgs a) {
  constexpr int V = 16 / sizeof(R);
  const int blk = blockIdx.x;
  const int key = blockIdx.y % a.n_keys;
  const int i = blockIdx.y / a.n_keys;
  const int slot = a.slots[i];
  if (slot < 0 || slot >= a.num_slots) return;
  const mlora_pool_key k = a.keys[key];
  const R* row = static_cast<const R*>(a.stage) + static_cast<int64_t>(i) * a.stage_stride;
  const int64_t e0 = static_cast<int64_t>(blk) * kScatterElems;

  // A: [rank, in] block -> rows [0, rank) of the slot, one contiguous run.
  const int64_t a_numel = static_cast<int64_t>(a.rank) * k.in_dim;
  if (e0 < a_numel) {
    const R* src = row + k.a_off;
    R* dst = static_cast<R*>(k.a) + static_cast<int64_t>(slot) * k.a_slot_stride;
    const bool vec = a.vec && (reinterpret_cast<uintptr_t>(k.a) & 15) == 0 && (k.a_off % V) == 0 &&
                     (k.a_slot_stride % V) == 0 && (a_numel % V) == 0;
    copy_run<R>(src, dst, e0, min(e0 + kScatterElems, a_numel), vec);
  }

  // B: [out, rank] block -> columns [0, rank) of rows [0, out) of the slot.
  const int64_t b_numel = static_cast<int64_t>(k.out_dim) * a.rank;
  if (e0 < b_numel) {
    const R* src = row + k.b_off;
    R* dst = static_cast<R*>(k.b) + static_cast<int64_t>(slot) * k.b_slot_stride;
    const int64_t e1 = min(e0 + kScatterElems, b_numel);
    const bool vec = a.vec && (reinterpret_cast<uintptr_t>(k.b) & 15) == 0 && (k.b_off % V) == 0 &&
                     (a.rank % V) == 0 && (k.b_row_stride % V) == 0 && (k.b_slot_stride % V) == 0;
    if (vec) {
      const int per_row = a.rank / V;  // 16-byte pieces per rank-wide row
      for (int64_t q = e0 / V + threadIdx.x; q < e1 / V; q += blockDim.x) {
        const int64_t o = q / per_row;
        const int64_t c = (q - o * per_row) * V;
        st_chunk_nt(dst + o * k.b_row_stride + c, ld_chunk_nt(src + q * V));
      }
    } else {
      for (int64_t e = e0 + threadIdx.x; e < e1; e += blockDim.x) {
        const int64_t o = e / a.rank;
        dst[o * k.b_row_stride + (e - o * a.rank)] = src[e];
      }
    }
  }
}

}  // namespace

hipError_t launch_scatter(const ScatterArgs& args, int64_t max_numel, int elem_bytes, hipStream_t stream) {
  const int64_t nblk = (max_numel + kScatterElems - 1) / kScatterElems;
  const int64_t ny = static_cast<int64_t>(args.n_keys) * args.h;
  if (nblk <= 0 || ny <= 0) return hipSuccess;
  if (!grid_fits(nblk) || ny > 0xffffffffLL) return hipErrorInvalidConfiguration;
  const dim3 grid(static_cast<unsigned>(nblk), static_cast<unsigned>(ny));
  if (elem_bytes == 2)
    hipLaunchKernelGGL((scatter_kernel<uint16_t>), grid, dim3(256), 0, stream, args);
  else
    hipLaunchKernelGGL((scatter_kernel<float>), grid, dim3(256), 0, stream, args);
  return hipGetLastError();
}

}  // namespace mlora
