// Slot-grouped shrink+expand for decode-shaped batches (gfx950).
//
// The reference launches one program per segment and, in decode, streams
// the segment's whole A / B slice per token (multi_lora/kernels/sgemm_lora_a.py:118-183,
// sgemm_lora_b.py:93-153), so an adapter used by n tokens is read n times.
// Here work items are indexed by (slot, chunk) instead: each finds the rows
// its slot owns with a workgroup-wide scan of the segment table (stable: the
// rows come out in ascending order) and reads that slot's A / B chunk once
// for all of them.  No planning pass and no host-side state are involved.
//
//   shrink item  (slot, K chunk: 256 wide in the single launch, 512 with two
//                launches): the 4 waves take 2 or 4 K-steps each,
//                A fragments stay in registers while the slot's rows go by
//                16 at a time; the four wave sums are added in LDS and the
//                chunk's fp32 sums are published per (chunk, row, column).
//   expand item  (slot, 256 output columns of one slice): B fragments and
//                the output rows are requested first; the K-chunk sums are
//                added in chunk order and rounded to the storage type (the
//                reference's `mid` rounding, sgemm_lora_a.py:109), multiplied
//                with B on MFMA, scaled and rounded (sgemm_lora_b.py:84-89),
//                and added into the output rows through an LDS transpose.
//
// Two schedules share these bodies:
//   two launches  shrink items, then expand items; the kernel boundary
//                 orders them and the sums travel as plain fp32.
//   linked        one launch holding the shrink items followed by the expand
//                 items.  Each sum is published as one 64-bit word
//                 {tag, fp32 bits} with an atomic store; the tag is an odd
//                 32-bit function of this launch's dispatch id (the packet
//                 index on its hardware queue, fresh for every launch and
//                 every graph replay) and of the queue.  An expand item first
//                 waits, one lane per K chunk, for one sentinel word of each
//                 chunk, then reads every word it needs and checks every tag,
//                 waiting on any word still missing.  Words left by earlier
//                 launches carry other tags, so the workspace is never
//                 cleared and no counter is kept.  Two launches on one queue
//                 get equal tags only 2^31 packets apart: a word would have
//                 to stay unwritten that long and then be read by exactly
//                 such a launch.  Each wait is bounded: on timeout the item
//                 raises the workspace's error word and goes on, so no wave
//                 can hang.  Shrink items never wait and workgroups are
//                 dispatched in index order, so every shrink item is placed
//                 before any expand item that waits on it.  Every
//                 cross-workgroup access is a relaxed agent-scope atomic on a
//                 single word: device-coherent on gfx950 without any cache
//                 flush, and a word's tag and value always arrive together.
//                 Segments that overlap (one row in two segments, outside the
//                 reference's contract too) can make a wait time out; the
//                 error word reports it.
// Arithmetic per row is the same as the segment kernels' (fp32 sums, two
// roundings); only the split of the K reduction differs.
#include "expand_tile.h"
#include "kernels.h"
#include "loads.h"

namespace mlora {

// The launch's dispatch id (its AQL packet index on the hardware queue),
// through the LLVM intrinsic; declared outside the anonymous namespace so the
// bodiless declaration has external linkage.
__device__ uint64_t hw_dispatch_id() __asm("llvm.amdgcn.dispatch.id");

namespace {

// How shrink items pass their K-chunk sums to expand items.
constexpr int kSumF32 = 0;     // two launches: fp32 words
constexpr int kSumLinked = 2;  // one launch: 64-bit words tagged with the launch, polled
constexpr int kSumMid = 3;     // mixed-batch expand: y read from `mid` (already summed and rounded)
constexpr int kSpinLimit = 1 << 20;   // polls before an expand item gives up
constexpr int kPollBatch = 16;        // K-chunk words requested together

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

// This launch's tag: odd (a zero-filled workspace never matches), equal for
// every workgroup of the launch, different for launches on one queue fewer
// than 2^31 packets apart; the queue address salts it.
__device__ __forceinline__ uint32_t launch_tag() {
  const uint64_t q = reinterpret_cast<uint64_t>(__builtin_amdgcn_queue_ptr());
  const uint32_t salt = static_cast<uint32_t>(q ^ (q >> 32)) * 0x9E3779B1u;
  return ((static_cast<uint32_t>(hw_dispatch_id()) + salt) << 1) | 1u;
}

__device__ __forceinline__ uint64_t tagged(uint32_t tag, float v) {
  return (static_cast<uint64_t>(tag) << 32) | __float_as_uint(v);
}

// Linked-schedule workspace: [error word | pad to 256 B][tagged sums
// [kc][rows][n_slices * r_max]].
struct LinkedView {
  int* error;
  uint64_t* sums;
};

__device__ __forceinline__ LinkedView linked_view(const GroupedArgs& a) {
  char* base = reinterpret_cast<char*>(a.partials);
  return LinkedView{reinterpret_cast<int*>(base), reinterpret_cast<uint64_t*>(base + kLinkedHeader)};
}

// Shrink item (slot, slice group sg, K chunk c).  With a.s_groups == 1 the
// item covers every slice; otherwise slice sg only.  SP: K-steps per wave
// (a.k_chunk = 4 * SP * KSTEP).
template <class T, int NBT, int FMT, int SP>
__device__ void shrink_item(const GroupedArgs& a, int slot, int sg, int c, int* s_rows, int* s_tmp,
                            f32x4 (*red)[kWave]) {
  using raw = typename T::raw_t;
  constexpr int VEC = T::VEC;
  constexpr int KSTEP = T::KSTEP;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int r16 = lane & 15;
  const int g = lane >> 4;

  // First loads, issued together: the slot's rank and this thread's entry of
  // the segment table.
  const SegEntry first = load_seg(a.meta, tid);
  const int rank = slot_rank(a, slot);
  if (rank == 0) return;
  const int nb_act = (rank + 15) >> 4;
  const int s_first = (a.s_groups == 1) ? 0 : sg;
  const int nbt = ((a.s_groups == 1) ? a.n_slices : 1) * nb_act;
  const int kbeg = c * a.k_chunk;

  // This wave's A fragments for the chunk, kept for every row tile.  They
  // are loaded unmasked and masked to in_dim where the MFMA uses them, so no
  // instruction between here and the x loads needs their data.
  u32x4 af[SP][NBT];
#pragma unroll
  for (int j = 0; j < NBT; ++j) {
    const int jj = j < nbt ? j : 0;
    const int sl = jj / nb_act;  // slice within the item
    const raw* arow = slice_a<raw>(a.slices, s_first + sl, slot, min((jj - sl * nb_act) * 16 + r16, rank - 1));
#pragma unroll
    for (int sp = 0; sp < SP; ++sp) {
      const int kk = kbeg + (wave + 4 * sp) * KSTEP + g * VEC;
      af[sp][j] = ld_chunk(arow + (kk < a.in_dim ? kk : 0));
    }
  }

  const int ncols = a.n_slices * a.r_max;
  int total = slot_rows(a.meta, first, a.rows, slot, 0, s_rows, s_tmp, false);
  for (int w0 = 0; w0 < total; w0 += kGroupRows) {
    if (w0 > 0) total = slot_rows(a.meta, first, a.rows, slot, w0, s_rows, s_tmp, false);
    const int cnt = min(kGroupRows, total - w0);
    for (int tt = 0; tt < cnt; tt += 16) {
      const raw* xrow = static_cast<const raw*>(a.x) + static_cast<int64_t>(s_rows[min(tt + r16, cnt - 1)]) * a.x_stride;
      f32x4 acc[NBT];
#pragma unroll
      for (int j = 0; j < NBT; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
      // Both x chunks are requested before the first MFMA waits for data.
      u32x4 xv[SP];
#pragma unroll
      for (int sp = 0; sp < SP; ++sp) {
        const int kk = kbeg + (wave + 4 * sp) * KSTEP + g * VEC;
        xv[sp] = load_row_chunk<T, true>(xrow, kk, a.in_dim - kk);
      }
      // The A fragments are masked only after this point (their mask needs
      // their data); an empty asm that rewrites them keeps the compiler from
      // hoisting the mask, and with it a wait for A, above the x loads.
      fence_regs(af);
#pragma unroll
      for (int sp = 0; sp < SP; ++sp) {
        const int kk = kbeg + (wave + 4 * sp) * KSTEP + g * VEC;
#pragma unroll
        for (int j = 0; j < NBT; ++j)
          if (j < nbt) acc[j] = T::mma(acc[j], af[sp][j] & keep_mask<T>(a.in_dim - kk), xv[sp]);
      }
      if (wave > 0) {
#pragma unroll
        for (int j = 0; j < NBT; ++j)
          if (j < nbt) red[(wave - 1) * NBT + j][lane] = acc[j];
      }
      lds_barrier();
      if (wave == 0) {
        // One wave's sums at a time keeps the register peak at two sets.
#pragma unroll 1
        for (int w2 = 0; w2 < 3; ++w2)
#pragma unroll
          for (int j = 0; j < NBT; ++j)
            if (j < nbt) acc[j] += red[w2 * NBT + j][lane];
        if (tt + r16 < cnt) {
          const int64_t rowoff = (static_cast<int64_t>(c) * a.rows + s_rows[tt + r16]) * ncols;
#pragma unroll
          for (int j = 0; j < NBT; ++j) {
            if (j >= nbt) break;
            const int sl = j / nb_act;  // slice within the item
            const int s = s_first + sl;
            const int n = (j - sl * nb_act) * 16 + 4 * g;
            if (n >= a.r_max) continue;
            if constexpr (FMT == kSumLinked) {
              uint64_t* p = linked_view(a).sums + rowoff + s * a.r_max + n;
              const uint32_t tag = launch_tag();
#pragma unroll
              for (int q = 0; q < 4; ++q)
                __hip_atomic_store(p + q, tagged(tag, acc[j][q]), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            } else {
              *reinterpret_cast<f32x4*>(a.partials + rowoff + s * a.r_max + n) = acc[j];
            }
          }
        }
      }
      lds_barrier();
    }
  }
}

// Bounded wait for one linked word to carry the tag; returns the word (its
// value is unreliable if the wait timed out, which raises the error word).
__device__ uint64_t wait_word(const LinkedView& lv, const uint64_t* p, uint32_t tag) {
  for (int spin = 0;; ++spin) {
    const uint64_t w = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (static_cast<uint32_t>(w >> 32) == tag) return w;
    if (spin >= kSpinLimit) {
      __hip_atomic_store(lv.error, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return w;
    }
    // Once any wait has timed out, every other wait of the launch ends
    // within 1024 polls instead of running to its own limit.
    if ((spin & 1023) == 1023 && __hip_atomic_load(lv.error, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) return w;
    __builtin_amdgcn_s_sleep(2);
  }
}

// Sum over the K chunks, in chunk order, of the sums published for one
// (row, column) at word `idx`; chunk z's word sits at idx + z * zstride.  In
// the linked schedule every word's tag is checked, and a word that has not
// arrived yet is waited for.
template <int FMT>
__device__ __forceinline__ float chunk_sum(const GroupedArgs& a, int64_t idx, int64_t zstride) {
  float sum = 0.f;
  for (int z0 = 0; z0 < a.kc; z0 += kPollBatch) {
    // Every word of the batch is requested before any is used: indices past
    // the last chunk read the last chunk again (in bounds) and count as 0.
    float v[kPollBatch];
    if constexpr (FMT == kSumLinked) {
      const LinkedView lv = linked_view(a);
      const uint32_t tag = launch_tag();
      const uint64_t* p = lv.sums + idx;
      uint64_t w[kPollBatch];
#pragma unroll
      for (int u = 0; u < kPollBatch; ++u)
        w[u] = __hip_atomic_load(p + min(z0 + u, a.kc - 1) * zstride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
      for (int u = 0; u < kPollBatch; ++u)
        if (z0 + u < a.kc && static_cast<uint32_t>(w[u] >> 32) != tag) w[u] = wait_word(lv, p + (z0 + u) * zstride, tag);
#pragma unroll
      for (int u = 0; u < kPollBatch; ++u) v[u] = (z0 + u < a.kc) ? __uint_as_float(static_cast<uint32_t>(w[u])) : 0.f;
    } else {
      const float* p = a.partials + idx;
#pragma unroll
      for (int u = 0; u < kPollBatch; ++u) v[u] = p[min(z0 + u, a.kc - 1) * zstride];
#pragma unroll
      for (int u = 0; u < kPollBatch; ++u) v[u] = (z0 + u < a.kc) ? v[u] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < kPollBatch; ++u) sum += v[u];
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
  // The scalar load lets the B and output-row loads go out at once.  In the
  // single launch the vector load is kept: its wait holds those loads back
  // about 1 us, while the shrink items of the launch are still reading A and
  // x (decode q_proj 8.43 vs 8.65 us with the scalar load).
  float scale = 0.f;
  if (slot < a.meta.num_slots)
    scale = (FMT == kSumLinked) ? load_scaling(a.meta.scalings, slot, a.meta.scal_dtype)
                                : load_scaling_uniform(a.meta.scalings, slot, a.meta.scal_dtype);
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
  // Columns the shrink items publish: whole 16-column blocks up to the rank.
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
      // The B fragments are masked only after this point (see the A
      // fragments in shrink_item).
      fence_regs(bf);
      const int rows_here = min(16, cnt - tt);
      if constexpr (FMT == kSumLinked) {
        // Light polling first: one lane per K chunk waits for the word its
        // shrink item stores last for this tile and slice (last row, last
        // live column); the full read below then rarely finds a word
        // missing.  Polling every word would flood the memory system the
        // shrink items are reading from.
        if (wave == 0) {
          const int64_t sidx = static_cast<int64_t>(lds.rows[tt + rows_here - 1]) * ncols + s * a.r_max + live - 1;
          const LinkedView lv = linked_view(a);
          const uint32_t tag = launch_tag();
          for (int z = lane; z < a.kc; z += kWave) wait_word(lv, lv.sums + z * zstride + sidx, tag);
        }
        lds_barrier();
      }
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
            v = chunk_sum<FMT>(a, static_cast<int64_t>(lds.rows[tt + yr]) * ncols + s * a.r_max + yc, zstride);
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

template <class T, int NBT, int FMT, int SP>
__global__ __launch_bounds__(256) void grouped_shrink_kernel(GroupedArgs a) {
  __shared__ int s_rows[kGroupRows];
  __shared__ int s_tmp[4];
  __shared__ f32x4 red[3 * NBT][kWave];
  const int per_slot = a.s_groups * a.kc;
  const int slot = blockIdx.x / per_slot;
  const int rem = blockIdx.x - slot * per_slot;
  shrink_item<T, NBT, FMT, SP>(a, slot, rem / a.kc, rem % a.kc, s_rows, s_tmp, red);
}

// Four workgroups a CU except for 512-column items at r_max > 32 (169
// VGPRs).  512-column items at r_max <= 32 fit in 126 VGPRs without spills:
// q|k|v at 128 rank-32 adapters 39.5 vs 40.0 us for the pair at three a CU.
template <class T, int FMT, int WN, int RS>
__global__ __launch_bounds__(256, WN == 1 || RS == 1 ? 4 : 2) void grouped_expand_kernel(GroupedArgs a) {
  __shared__ __attribute__((aligned(16))) ExpandLds<T, WN> lds;
  const int slot = blockIdx.x / a.n_tiles;
  expand_item<T, FMT, WN, RS>(a, slot, blockIdx.x - slot * a.n_tiles, lds);
}

// Shrink items are workgroups [0, num_slots * kc); expand items follow.
// Four waves per SIMD (at most 128 VGPRs) keep four workgroups resident per
// CU, so expand items are placed, and run their prologue, while the shrink
// items still run; with 8 or more A blocks the A fragments alone need more.
template <class T, int NBT, int WN, int RS>
__global__ __launch_bounds__(256, (NBT >= 8 || WN > 1) ? 2 : 4) void grouped_linked_kernel(GroupedArgs a) {
  __shared__ __attribute__((aligned(16))) ExpandLds<T, WN> lds;
  __shared__ f32x4 red[3 * NBT][kWave];
  const int per_slot = a.s_groups * a.kc;
  const int ns = a.meta.num_slots * per_slot;
  const int b = blockIdx.x;
  if (b < ns) {
    const int slot = b / per_slot;
    const int rem = b - slot * per_slot;
    shrink_item<T, NBT, kSumLinked, kGroupStepsLinked>(a, slot, rem / a.kc, rem % a.kc, lds.rows, lds.tmp, red);
  } else {
    const int e = b - ns;
    const int slot = e / a.n_tiles;
    expand_item<T, kSumLinked, WN, RS>(a, slot, e - slot * a.n_tiles, lds);
  }
}

template <class T, int NBT, int WN, int RS>
hipError_t launch_t(const GroupedArgs& args, int mode, int phases, hipStream_t stream) {
  const int64_t g1 = static_cast<int64_t>(args.meta.num_slots) * args.s_groups * args.kc;
  const int64_t g2 = static_cast<int64_t>(args.meta.num_slots) * args.n_tiles;
  if (g1 <= 0 || g2 <= 0) return hipSuccess;
  if (!grid_fits(g1 + g2)) return hipErrorInvalidConfiguration;
  if (mode == kGroupLinked) {
    hipLaunchKernelGGL((grouped_linked_kernel<T, NBT, WN, RS>), dim3(static_cast<unsigned>(g1 + g2)), dim3(256), 0, stream,
                       args);
    return hipGetLastError();
  }
  if (phases & 1) {
    hipLaunchKernelGGL((grouped_shrink_kernel<T, NBT, kSumF32, kGroupStepsTwo>), dim3(static_cast<unsigned>(g1)), dim3(256), 0,
                       stream, args);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (phases & 2) {
    hipLaunchKernelGGL((grouped_expand_kernel<T, kSumF32, WN, RS>), dim3(static_cast<unsigned>(g2)), dim3(256), 0, stream,
                       args);
    return hipGetLastError();
  }
  return hipSuccess;
}

template <class T, int WN, int RS>
hipError_t launch_nbt(const GroupedArgs& args, int nbt, int mode, int phases, hipStream_t stream) {
  switch (nbt) {
    case 1: return launch_t<T, 1, WN, RS>(args, mode, phases, stream);
    case 2: return launch_t<T, 2, WN, RS>(args, mode, phases, stream);
    default: return launch_t<T, 4, WN, RS>(args, mode, phases, stream);
  }
}

template <class T>
hipError_t launch_dtype(const GroupedArgs& args, int nbt, int mode, int phases, hipStream_t stream) {
  const bool rs1 = args.r_max <= T::KSTEP;
  if (args.expand_wn == 2)
    return rs1 ? launch_nbt<T, 2, 1>(args, nbt, mode, phases, stream) : launch_nbt<T, 2, 2>(args, nbt, mode, phases, stream);
  return rs1 ? launch_nbt<T, 1, 1>(args, nbt, mode, phases, stream) : launch_nbt<T, 1, 2>(args, nbt, mode, phases, stream);
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
// the shrink's split sums (ea.partials, ea.ks splits), else from mid.
template <class T, bool FUSED, int RS>
__global__ __launch_bounds__(256, 4) void expand_mixed_kernel(ExpandArgs ea, GroupedArgs ga, int long_units,
                                                              int short_units) {
  __shared__ __attribute__((aligned(16))) ExpandTileLds<T, kExpandLongBM, FUSED> tl;
  __shared__ __attribute__((aligned(16))) ExpandLds<T, 1> gl;
  __shared__ unsigned bits[kMixedMaxSlots / 32];
  __shared__ int offs[kMixedMaxSlots / 32];
  __shared__ int pick;
  const int nt = ea.n_tiles;
  const int b = blockIdx.x;
  if (b < short_units * nt) {
    const int j = b / nt;
    const int nt_g = b - j * nt;
    const int n_short = short_slot_map(ga, bits, offs, gl.tmp);
    const int nwords = (ga.meta.num_slots + 31) >> 5;
    // More short slots than the launch has units for (a summary from an
    // earlier table, e.g. in a replayed graph): this unit also takes slots
    // j + short_units, j + 2 short_units, ...  These units come first in the
    // grid, so such extra work overlaps the long tiles'.
    for (int k = j; k < n_short; k += short_units) {
      const int slot = short_slot(bits, offs, nwords, k, &pick);
      expand_item<T, FUSED ? kSumF32 : kSumMid, 1, RS>(ga, slot, nt_g, gl);
      __syncthreads();
    }
    return;
  }
  const int u = (b - short_units * nt) / nt;
  const int nt_g = (b - short_units * nt) - u * nt;
  TileRef tr;
  bool found;
  const int total = long_tile(ea.meta, ea.rows, u, kExpandLongBM, kShortSegRows, &tr, &found);
  if (found) expand_tile<T, kExpandLongBM, true, FUSED>(ea, tr, nt_g, tl);
  // More long tiles than the launch has units for: this unit also takes
  // tiles u + long_units, u + 2 long_units, ...
  for (int t = u + long_units; t < total; t += long_units) {
    __syncthreads();
    long_tile(ea.meta, ea.rows, t, kExpandLongBM, kShortSegRows, &tr, &found);
    if (found) expand_tile<T, kExpandLongBM, true, FUSED>(ea, tr, nt_g, tl);
  }
}

template <class T, bool FUSED>
hipError_t launch_mixed_t(const ExpandArgs& ea, const GroupedArgs& ga, int long_units, int short_units,
                          hipStream_t stream) {
  const int64_t blocks = (static_cast<int64_t>(long_units) + short_units) * ea.n_tiles;
  if (blocks <= 0) return hipSuccess;
  if (!grid_fits(blocks)) return hipErrorInvalidConfiguration;
  if (ga.r_max <= T::KSTEP)
    hipLaunchKernelGGL((expand_mixed_kernel<T, FUSED, 1>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                       ea, ga, long_units, short_units);
  else
    hipLaunchKernelGGL((expand_mixed_kernel<T, FUSED, 2>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                       ea, ga, long_units, short_units);
  return hipGetLastError();
}

}  // namespace

bool plan_grouped(int in_dim, int r_max, int n_slices, int rows, int dtype, int* kc, int* k_chunk, int* nbt,
                  int* s_groups, size_t* linked_bytes, size_t* plain_bytes) {
  if (dtype != MLORA_BF16 && dtype != MLORA_F16) return false;
  if (in_dim <= 0 || rows <= 0 || n_slices < 1 || n_slices > kMaxSlices) return false;
  if (r_max <= 0 || r_max > kGroupMaxRank || r_max % 8 != 0 || in_dim % 8 != 0) return false;
  // More than four 16-row A blocks in all: one shrink item per slice, so an
  // item never holds more than four blocks of A fragments.
  const int blocks = n_slices * cdiv(r_max, 16);
  *s_groups = (blocks > 4) ? n_slices : 1;
  const int item_blocks = blocks / *s_groups;
  int b = 1;
  while (b < item_blocks) b *= 2;
  *nbt = b;
  *k_chunk = 4 * kGroupStepsLinked * BF16::KSTEP;
  *kc = cdiv(in_dim, *k_chunk);
  const size_t words = static_cast<size_t>(*kc) * rows * n_slices * r_max;
  *linked_bytes = kLinkedHeader + words * sizeof(uint64_t);
  *plain_bytes = words * sizeof(float);
  return true;
}

hipError_t launch_grouped(GroupedArgs args, int dtype, int nbt, int mode, int phases, hipStream_t stream) {
  if (dtype == MLORA_BF16) return launch_dtype<BF16>(args, nbt, mode, phases, stream);
  return launch_dtype<F16>(args, nbt, mode, phases, stream);
}

hipError_t launch_mixed(const ExpandArgs& args, int dtype, int long_units, int short_units, hipStream_t stream) {
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
  ga.n_tiles = args.n_tiles;
  for (int s = 0; s <= kMaxSlices; ++s) ga.tile_base[s] = args.tile_base[s];
  ga.expand_wn = 1;
  ga.short_only = 1;
  ga.mid = args.mid;
  ga.mid_stride = args.mid_stride;
  const bool fused = args.ks > 1 && args.partials != nullptr;
  if (dtype == MLORA_BF16)
    return fused ? launch_mixed_t<BF16, true>(args, ga, long_units, short_units, stream)
                 : launch_mixed_t<BF16, false>(args, ga, long_units, short_units, stream);
  return fused ? launch_mixed_t<F16, true>(args, ga, long_units, short_units, stream)
               : launch_mixed_t<F16, false>(args, ga, long_units, short_units, stream);
}

}  // namespace mlora
