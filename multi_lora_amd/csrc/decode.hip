// Slot-planned shrink+expand for decode-shaped batches (gfx950).
//
// The reference runs one GEMV program per token in decode, so every token
// streams its adapter's whole A and B (multi_lora/kernels/sgemm_lora_a.py:118-183,
// sgemm_lora_b.py:93-153).  Here the work follows a per-step *plan* of the
// segment table: one entry per (referenced slot, up to 16 of its rows), with
// the slot, its rank and scaling, the rows, and their position in the
// workspace (layout in include/mlora_hip.h).  Slots no row uses, and rank-0
// slots, have no entry, so their A and B are never read.
//
//   shrink item  (entry, slice group, K chunk of 4 waves x SP x 32): the
//                entry (with its rows) comes in one scalar load, then the
//                chunk's A fragments and the entry's x rows together; they
//                are multiplied on MFMA (16 rank rows x 16 token rows a
//                tile), the four waves' sums added in LDS, and the chunk's
//                fp32 sums stored to the workspace.
//   expand item  (entry, 256 output columns of one slice): B fragments and
//                the output rows are requested first; once the sums of every
//                K chunk are there they are added (four chunk groups, each in
//                chunk order, then the groups in order) and rounded to the
//                storage type (the
//                reference's `mid` rounding, sgemm_lora_a.py:109), multiplied
//                with B on MFMA, scaled and rounded (sgemm_lora_b.py:84-89),
//                and added into the output rows through an LDS transpose.
//
// Single launch (linked).  Workgroup b is item b / E of entry slot b % E,
// with E a multiple of 8.  Workgroups are placed on the XCDs round-robin
// (b mod 8), so every item of an entry runs on one XCD and shares its L2.
// A shrink item stores its fp32 sums with plain stores, which stay in that
// L2, waits for their acknowledgement (vmcnt(0)), then stores the chunk's
// 64-bit flag {launch tag, XCC id}.  Expand items poll the flags and read
// the sums with device-scope (sc1) loads, which skip the CU's L1 and are
// served by the L2 (a workgroup-scope load may be served by the L1, which
// keeps the first value it fetched while another CU updates the line;
// device-scope stores would write through past the L2, so the reads after
// them go to memory).  The tag is an odd function of the launch's dispatch
// id on its hardware queue (fresh for every launch and graph replay), so
// the workspace is never cleared.  An expand item takes a chunk once its
// flag carries this launch's tag and its own XCC id; a chunk it does not
// get that way before a deadline (a late producer, or one on another XCD,
// whose L2 it cannot see) it computes itself from x and A, bit for bit as
// the shrink item would, and publishes it; the workspace header counts such
// chunks.  So results never depend on placement or timing, only speed
// does.  Shrink items come first in the grid and never wait, so every wait
// also ends on its own.  (Sums carried as 64-bit words {tag, value}, which
// need no flag and no acknowledgement, were measured slower: twice the
// bytes to store under load.)
//
// Two launches: shrink items, then expand items, with the same bodies and
// the same sums (bit-identical results); the kernel boundary orders them.
//
// Fused RMSNorm (two launches): the shrink launch also holds the RMSNorm of
// the call's rows (the RMSNorm kernel's row body, so the same y, and each
// row's rsqrt(mean(x^2) + eps) stored), and its shrink items multiply
// round(x * w) instead of y; the expand items scale a row's summed chunks by
// that rstd before the mid rounding.
#include "kernels.h"
#include "loads.h"
#include "rmsnorm_row.h"

namespace mlora {

// Per-phase timestamps of the planned kernel, in builds made with
// MLORA_TIMELINE (the calibration library; the product library has none):
// lane 0 of each wave keeps the low 32 bits of s_memrealtime (100 MHz) at
// the phases below in LDS, and the workgroup writes them out once, at its
// end, to tl_stamps[workgroup][wave][phase] (workgroup = its linear id,
// y * gridDim.x + x).  Phases of a shrink item: 0
// start, 1 plan entry in, 2 this wave's A and x in, 3 the four waves' sums
// in LDS, 4 flag stored (wave 0, after the sums' acknowledgement), 5 item
// done.  Of an expand item: 0 start, 1 entry in, 2 B and output requested,
// 3 every chunk flag seen (or given up), 4 sums gathered, 5 y in LDS, 6
// output stored and acknowledged.  A wait for vmcnt(0) precedes the
// data-arrival stamps.
#ifdef MLORA_TIMELINE
constexpr int kTlBlocks = 8192;
constexpr int kTlPhases = 8;
__device__ uint32_t tl_stamps[kTlBlocks][4][kTlPhases];
__shared__ uint32_t tl_lds[4][kTlPhases];
#define MLORA_STAMP(k)                                                                                  \
  do {                                                                                                  \
    const uint32_t t_ = static_cast<uint32_t>(__builtin_amdgcn_s_memrealtime());                        \
    if ((threadIdx.x & 63) == 0) tl_lds[threadIdx.x >> 6][k] = t_;                                      \
  } while (0)
#define MLORA_STAMP_AFTER_LOADS(k) \
  do {                             \
    wait_vmcnt<0>();               \
    MLORA_STAMP(k);                \
  } while (0)
#define MLORA_STAMP_BEGIN()                                                    \
  do {                                                                         \
    if (threadIdx.x < 4 * kTlPhases) (&tl_lds[0][0])[threadIdx.x] = 0u;        \
    lds_barrier();                                                             \
    MLORA_STAMP(0);                                                            \
  } while (0)
#define MLORA_STAMP_FLUSH()                                                                               \
  do {                                                                                                    \
    lds_barrier();                                                                                        \
    const unsigned b_ = blockIdx.y * gridDim.x + blockIdx.x;                                              \
    if (threadIdx.x < 4 * kTlPhases && b_ < kTlBlocks)                                                    \
      (&tl_stamps[b_][0][0])[threadIdx.x] = (&tl_lds[0][0])[threadIdx.x];                                 \
  } while (0)
#else
#define MLORA_STAMP(k) \
  do {                 \
  } while (0)
#define MLORA_STAMP_AFTER_LOADS(k) \
  do {                             \
  } while (0)
#define MLORA_STAMP_BEGIN() \
  do {                      \
  } while (0)
#define MLORA_STAMP_FLUSH() \
  do {                      \
  } while (0)
#endif

// The launch's dispatch id (its AQL packet index on the hardware queue).
__device__ uint64_t planned_dispatch_id() __asm("llvm.amdgcn.dispatch.id");

namespace {

constexpr int kDefaultWaitTicks = 20000;  // 200 us of s_memrealtime (100 MHz)
constexpr int kGroups = 4;                // chunk groups summed separately, then in order

struct Entry {
  int slot;
  int rank;   // clamped to [0, r_max]; 0 for a slot outside the call's pool
  int nr;     // rows, [0, 16]
  int pos;    // first workspace row
  float scale;
};

// Entry e of the plan; e is wave-uniform, so these are scalar loads.
__device__ __forceinline__ Entry load_entry(const int32_t* plan, int e, int r_max, int num_slots) {
  const int32_t* p = plan + kPlanHeaderWords + static_cast<int64_t>(e) * kPlanEntryWords;
  Entry en;
  en.slot = p[kPlanSlot];
  const int r = p[kPlanRank];
  en.scale = __int_as_float(p[kPlanScale]);
  en.nr = min(max(p[kPlanRowCount], 0), kPlanRows);
  en.pos = p[kPlanPos];
  en.rank = (en.slot >= 0 && en.slot < num_slots) ? min(max(r, 0), r_max) : 0;
  return en;
}

// Row i (< 16) of entry e (a vector load: its address needs no other load,
// so it goes out together with the entry's scalar loads), clamped to
// [0, rows).  The plan pads an entry's unused row words with its first row.
__device__ __forceinline__ int load_entry_row(const int32_t* plan, int e, int i) {
  return plan[kPlanHeaderWords + static_cast<int64_t>(e) * kPlanEntryWords + kPlanRowWord + i];
}

__device__ __forceinline__ int clamp_row(int r, int rows) { return min(max(r, 0), rows - 1); }

// This launch's tag: odd (a zero-filled workspace never matches), equal for
// every workgroup of the launch, different for launches on one queue fewer
// than 2^31 packets apart; the queue address salts it.
__device__ __forceinline__ uint32_t launch_tag() {
  const uint64_t q = reinterpret_cast<uint64_t>(__builtin_amdgcn_queue_ptr());
  const uint32_t salt = static_cast<uint32_t>(q ^ (q >> 32)) * 0x9E3779B1u;
  return ((static_cast<uint32_t>(planned_dispatch_id()) + salt) << 1) | 1u;
}

__device__ __forceinline__ uint32_t xcc_id() {
  uint32_t v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
  return v & 0xfu;
}

__device__ __forceinline__ uint64_t flag_word() { return (static_cast<uint64_t>(launch_tag()) << 32) | xcc_id(); }

__device__ __forceinline__ uint64_t* flag_ptr(const DecodeArgs& a, int e, int sg, int c) {
  return a.flags + (static_cast<int64_t>(e) * a.s_groups + sg) * a.kc + c;
}

// Workspace row `pos`, chunk c, column col: fp32 sum of one K chunk.
__device__ __forceinline__ int64_t sum_index(const DecodeArgs& a, int pos, int c, int col) {
  return (static_cast<int64_t>(pos) * a.kc + c) * (a.n_slices * a.r_max) + col;
}

// One K chunk of one entry's shrink, for the slices of group sg:
// sums[i][n] = sum over the chunk of x[row_i, k] * A_s[slot, n, k], stored to
// the workspace by wave 0 for the entry's rows, then (flag != 0) the chunk's
// flag once the sums are acknowledged.  xrow: this lane's x row (row
// lane & 15 of the entry).  All threads call it; it ends with an LDS barrier.
// LEAN: one A block's fragments in flight at a time instead of all NBT (the
// same products in the same order, so the same sums), for the expand items'
// rare recompute when it has four A blocks and one expand K-step, so that
// the single launch keeps four workgroups a CU without spilling (q|k|v at
// rank 16: 12.6 vs 14.0 us at 64 tokens, 19.2 vs 20.9 at 256).
// NORM (the fused RMSNorm launch): the MFMA takes round(x * w) with the
// RMSNorm weight nw.
template <class T, int NBT, int SP, bool LEAN = false, bool NORM = false>
__device__ void shrink_chunk(const DecodeArgs& a, int e, const Entry& en, int xrow, int sg, int c,
                             f32x4 (*red)[kWave], uint64_t flag, const typename T::raw_t* nw = nullptr) {
  static_assert(!(NORM && LEAN), "the fused RMSNorm shrink has no recompute path");
  using raw = typename T::raw_t;
  constexpr int VEC = T::VEC;
  constexpr int KSTEP = T::KSTEP;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int r16 = lane & 15;
  const int g = lane >> 4;
  const int rank = en.rank;
  const int nb_act = (rank + 15) >> 4;
  const int s_first = (a.s_groups == 1) ? 0 : sg;
  const int nbt = ((a.s_groups == 1) ? a.n_slices : 1) * nb_act;
  const int kbeg = c * a.k_chunk;

  // A fragments, loaded unmasked (clamped in bounds) and dropped past in_dim
  // where the MFMA uses them, so nothing between here and the x loads waits
  // for them.  in_dim is a multiple of the chunk: a chunk is wholly inside
  // or wholly outside.
  auto a_row = [&](int j) {
    const int jj = j < nbt ? j : 0;
    const int sl = jj / nb_act;  // slice within the group
    return slice_a<raw>(a.slices, s_first + sl, en.slot, min((jj - sl * nb_act) * 16 + r16, rank - 1));
  };
  auto x_frags = [&](u32x4 (&xv)[SP]) {
    const raw* xr = static_cast<const raw*>(a.x) + static_cast<int64_t>(xrow) * a.x_stride;
#pragma unroll
    for (int sp = 0; sp < SP; ++sp) {
      const int kk = kbeg + (wave + 4 * sp) * KSTEP + g * VEC;
      const u32x4 v = ld_chunk(xr + (kk < a.in_dim ? kk : 0));
      xv[sp] = kk < a.in_dim ? v : zero_chunk();
    }
  };
  f32x4 acc[NBT];
#pragma unroll
  for (int j = 0; j < NBT; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  if constexpr (!LEAN) {
    u32x4 af[SP][NBT];
#pragma unroll
    for (int j = 0; j < NBT; ++j) {
      const int jj = j < nbt ? j : 0;
      const int sl = jj / nb_act;  // slice within the group
      const raw* arow = slice_a<raw>(a.slices, s_first + sl, en.slot, min((jj - sl * nb_act) * 16 + r16, rank - 1));
#pragma unroll
      for (int sp = 0; sp < SP; ++sp) {
        const int kk = kbeg + (wave + 4 * sp) * KSTEP + g * VEC;
        af[sp][j] = ld_chunk(arow + (kk < a.in_dim ? kk : 0));
      }
    }
    const raw* xr = static_cast<const raw*>(a.x) + static_cast<int64_t>(xrow) * a.x_stride;
    u32x4 xv[SP];
#pragma unroll
    for (int sp = 0; sp < SP; ++sp) {
      const int kk = kbeg + (wave + 4 * sp) * KSTEP + g * VEC;
      const u32x4 v = ld_chunk(xr + (kk < a.in_dim ? kk : 0));
      xv[sp] = kk < a.in_dim ? v : zero_chunk();
    }
    u32x4 wv[SP];
    if constexpr (NORM) {
#pragma unroll
      for (int sp = 0; sp < SP; ++sp) {
        const int kk = kbeg + (wave + 4 * sp) * KSTEP + g * VEC;
        const u32x4 v = ld_chunk(nw + (kk < a.in_dim ? kk : 0));
        wv[sp] = kk < a.in_dim ? v : zero_chunk();
      }
    }
    fence_regs(af);
    if constexpr (NORM) {
#pragma unroll
      for (int sp = 0; sp < SP; ++sp) {
        float f[VEC];
#pragma unroll
        for (int q = 0; q < VEC; ++q) f[q] = chunk_elem<T>(xv[sp], q) * chunk_elem<T>(wv[sp], q);
        xv[sp] = pack_chunk<T>(f);
      }
    }
#pragma unroll
    for (int sp = 0; sp < SP; ++sp) {
      const int kk = kbeg + (wave + 4 * sp) * KSTEP + g * VEC;
#pragma unroll
      for (int j = 0; j < NBT; ++j)
        if (j < nbt) acc[j] = T::mma(acc[j], kk < a.in_dim ? af[sp][j] : zero_chunk(), xv[sp]);
    }
  } else {
    u32x4 xv[SP];
    x_frags(xv);
#pragma unroll
    for (int j = 0; j < NBT; ++j) {
      if (j >= nbt) break;
      const raw* arow = a_row(j);
      u32x4 af[SP];
#pragma unroll
      for (int sp = 0; sp < SP; ++sp) {
        const int kk = kbeg + (wave + 4 * sp) * KSTEP + g * VEC;
        af[sp] = ld_chunk(arow + (kk < a.in_dim ? kk : 0));
      }
#pragma unroll
      for (int sp = 0; sp < SP; ++sp) {
        const int kk = kbeg + (wave + 4 * sp) * KSTEP + g * VEC;
        acc[j] = T::mma(acc[j], kk < a.in_dim ? af[sp] : zero_chunk(), xv[sp]);
      }
    }
  }
  MLORA_STAMP_AFTER_LOADS(2);
  if (wave > 0) {
#pragma unroll
    for (int j = 0; j < NBT; ++j)
      if (j < nbt) red[(wave - 1) * NBT + j][lane] = acc[j];
  }
  lds_barrier();
  MLORA_STAMP(3);
  if (wave == 0) {
#pragma unroll 1
    for (int w2 = 0; w2 < 3; ++w2)
#pragma unroll
      for (int j = 0; j < NBT; ++j)
        if (j < nbt) acc[j] += red[w2 * NBT + j][lane];
    // Lane l holds token row l & 15 and rank columns 4 (l >> 4) .. + 3 of
    // each 16-column block.
    if (r16 < en.nr) {
#pragma unroll
      for (int j = 0; j < NBT; ++j) {
        if (j >= nbt) break;
        const int sl = j / nb_act;
        const int n = (j - sl * nb_act) * 16 + 4 * g;
        if (n >= a.r_max) continue;
        *reinterpret_cast<f32x4*>(a.partials + sum_index(a, en.pos + r16, c, (s_first + sl) * a.r_max + n)) = acc[j];
      }
    }
    if (flag != 0) {
      // The flag goes out only once every sum of the chunk has reached the L2.
      asm volatile("" ::: "memory");
      wait_vmcnt<0>();
      asm volatile("" ::: "memory");
      if (lane == 0) __hip_atomic_store(flag_ptr(a, e, sg, c), flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      MLORA_STAMP(4);
    }
  }
  lds_barrier();
  MLORA_STAMP(5);
}

template <class T, int WN>
struct DecodeLds {
  using raw = typename T::raw_t;
  raw delta[16 * (kExpandBN * WN + T::VEC)];
  raw ytile[16 * (kGroupMaxRank + T::VEC)];
  f32x4 part[kGroups][16][kGroupMaxRank / 4];  // per chunk group: sums of each (row, 4 columns)
  uint64_t missing;                             // chunks not received
};

// 16 bytes of the workspace at byte offset `off`, read past the L1 (sc1):
// the L2 holds what other workgroups of this XCD stored.
__device__ __forceinline__ u32x4 load16_l2(__amdgpu_buffer_rsrc_t rsrc, int64_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, static_cast<int>(off), 0, /*sc1*/ 16));
}

// The y sums of rows < nr and columns < rank of slice s into lds.part: wave
// g adds the chunks of group g in chunk order, lane l the (row l / 16, quad
// l % 16) unit (and l + 64, ... for more rows), up to four chunks' sums
// requested together.  The mapping uses shifts only: the item's set-up is
// on the decode path's critical chain, and every instruction a wave issues
// there costs about 4 cycles at four waves a SIMD.
template <class T, int WN>
__device__ void gather_sums(const DecodeArgs& a, const Entry& en, int s, DecodeLds<T, WN>& lds) {
  static_assert(kGroups == 4 && kGroupMaxRank / 4 <= 16, "one chunk group per wave, at most 16 quads a row");
  const int quads = (en.rank + 3) >> 2;
  const int per = (a.kc + kGroups - 1) / kGroups;  // chunks per group
  const int ncols = a.n_slices * a.r_max;
  const int64_t bytes = static_cast<int64_t>(a.ws_rows) * a.kc * ncols * 4;
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
      a.partials, 0, static_cast<int>(bytes < 0x7fffffff ? bytes : 0x7fffffff), kBufferRsrcWord3);
  const int grp = threadIdx.x >> 6;
  const int c0 = grp * per;
  const int c1 = min(c0 + per, a.kc);
  for (int u = threadIdx.x & 63; u < en.nr * 16; u += 64) {
    const int row = u >> 4;
    const int q = u & 15;
    if (q >= quads) continue;
    const int64_t base = sum_index(a, en.pos + row, 0, s * a.r_max + 4 * q);
    f32x4 sum = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int cb = c0; cb < c1; cb += 4) {
      u32x4 w[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) w[k] = load16_l2(rsrc, (base + static_cast<int64_t>(min(cb + k, c1 - 1)) * ncols) * 4);
#pragma unroll
      for (int k = 0; k < 4; ++k)
        if (cb + k < c1) sum += __builtin_bit_cast(f32x4, w[k]);
    }
    lds.part[grp][row][q] = sum;
  }
  lds_barrier();
}

// Output chunks per thread of an expand item, and the entry row of chunk i
// of thread tid.
template <class T, int WN>
struct ExpandRows {
  static constexpr int CPR = kExpandBN * WN / T::VEC;  // chunks per output row
  static constexpr int RPT = 16 * CPR / 256;
  __device__ static __forceinline__ int row_of(int tid, int i) { return (tid + i * 256) / CPR; }
};

// Expand item (entry e, column tile nt_g).  LINKED: the sums come as tagged
// words from this launch's shrink items (or are computed here), else as
// fp32 from the previous launch.
// NORM (expand half of the fused RMSNorm launch): y = round(rstd * sum),
// with the rstd of the thread's row t / 16 (table row yrow_raw) requested
// with B and the output rows.
template <class T, int NBT, int SP, int WN, int RS, bool LINKED, bool NORM = false>
__device__ void expand_entry(const DecodeArgs& a, const int32_t* plan, int e, const Entry& en, int nt_g,
                             const int (&orow_raw)[ExpandRows<T, WN>::RPT], DecodeLds<T, WN>& lds,
                             f32x4 (*red)[kWave], const float* rstd = nullptr, int yrow_raw = 0) {
  static_assert(!(NORM && LINKED), "the fused RMSNorm path runs as two launches");
  using raw = typename T::raw_t;
  constexpr int VEC = T::VEC;
  constexpr int KSTEP = T::KSTEP;
  constexpr int BN = kExpandBN * WN;
  constexpr int NBW = 4 * WN;  // 16-column blocks per wave
  constexpr int LDS_STRIDE = BN + VEC;
  constexpr int CPR = BN / VEC;  // chunks per output row
  constexpr int RPT = 16 * CPR / 256;
  constexpr int YS = kGroupMaxRank + VEC;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int r16 = lane & 15;
  const int g = lane >> 4;
  const int rank = en.rank;

  int s = 0;
  while (s + 1 < a.n_slices && nt_g >= a.tile_base[s + 1]) ++s;
  const int n0 = (nt_g - a.tile_base[s]) * BN;
  const int out_dim = a.slices[s].out_dim;
  const int sg = (a.s_groups == 1) ? 0 : s;

  // The workspace's wait limit (written by other launches, so a vector load).
  const int over = LINKED ? a.header[kWsWaitOverride] : 0;
  raw* out = static_cast<raw*>(a.out) + a.slices[s].out_col;
  int orow[RPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i) orow[i] = clamp_row(orow_raw[i], a.rows);
  // B fragments: rows clamped to out_dim, loaded unmasked and masked to the
  // rank where the MFMA uses them.
  const raw* B = static_cast<const raw*>(a.slices[s].b) + static_cast<int64_t>(en.slot) * a.slices[s].b_slot_stride;
  u32x4 bf[RS][NBW];
  u32x4 ov[RPT];
  auto load_b = [&]() {
#pragma unroll
    for (int nb = 0; nb < NBW; ++nb) {
      const raw* brow =
          B + static_cast<int64_t>(min(n0 + (wave * NBW + nb) * 16 + r16, out_dim - 1)) * a.slices[s].b_row_stride;
#pragma unroll
      for (int ks = 0; ks < RS; ++ks) {
        const int kk = ks * KSTEP + g * VEC;
        bf[ks][nb] = ld_chunk(brow + (kk < rank ? kk : 0));
      }
    }
  };
  // The output rows are read and written once, with the non-temporal hint
  // (decode_q 6.88 -> 6.80 us, decode_q_resident 6.88 -> 6.73, decode_qkv
  // 37.09 -> 36.83; the same hint on the A, x and B loads measured slower,
  // 7.30 -> 7.46 us at decode_q over 20-call regions).
  auto load_out = [&]() {
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const int cidx = tid + i * 256;
      const int row = cidx / CPR;
      const int n = n0 + (cidx - row * CPR) * VEC;
      ov[i] = ld_chunk_nt(out + static_cast<int64_t>(orow[i]) * a.out_stride + (n < out_dim ? n : 0)) &
              keep_mask<T>(out_dim - n);
    }
  };
  // B and the output rows are requested at once: requested later (after a
  // delay, or once the flags are in), their arrival moves the end of the
  // item by as much (measured: +0.5 us per 0.5 us of delay).
  load_b();
  load_out();
  // The rstd of the row whose y this thread forms below: one load, issued
  // before the sums, so the gather's wait covers it.
  float rs = 1.f;
  if constexpr (NORM) rs = rstd[clamp_row(yrow_raw, a.rows)];
  MLORA_STAMP(2);

  if constexpr (LINKED) {
    // Wave 0 polls the flags of the chunks this slice needs (at most 64),
    // one lane per chunk, until each carries this launch's tag and this XCD,
    // or the deadline passes; the rest are computed here.
    const uint64_t want = flag_word();
    if (wave == 0) {
      // 0 waiting, 1 arrived, 2 this launch's tag from another XCD (its sums
      // sit in that XCD's L2, out of reach of these loads).
      int st = lane >= a.kc ? 1 : 0;
      const uint64_t* fp = flag_ptr(a, e, sg, min(lane, a.kc - 1));
      const uint64_t limit = over > 0 ? static_cast<uint64_t>(over) : kDefaultWaitTicks;
      const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
      // A negative limit skips the wait: every chunk is computed here.  The
      // clock (a scalar memory round trip) is read every eighth poll only.
      uint32_t polls = 0;
      while (over >= 0) {
        if (st == 0) {
          const uint64_t w = __hip_atomic_load(fp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          if (w == want)
            st = 1;
          else if ((w >> 32) == (want >> 32))
            st = 2;
        }
        if (__all(st != 0)) break;
        if ((++polls & 7) == 0 && __builtin_amdgcn_s_memrealtime() - t0 >= limit) break;
      }
      const uint64_t miss = __ballot(st != 1);
      if (lane == 0) lds.missing = miss;
    }
    lds_barrier();
    MLORA_STAMP(3);
    uint64_t miss = lds.missing;
    if (miss != 0) {
      // Compute the missing chunks here, bit for bit as their shrink items
      // would, and publish them for the entry's other expand items.
      const int xrow = clamp_row(load_entry_row(plan, e, r16), a.rows);
      if (tid == 0) atomicAdd(a.header + kWsFallbacks, __popcll(miss));
      while (miss != 0) {
        const int z = __builtin_ctzll(miss);
        miss &= miss - 1;
        shrink_chunk<T, NBT, SP, (NBT >= 4 && RS == 1)>(a, e, en, xrow, sg, z, red, want);
      }
      // The prefetched B fragments and output rows are requested again, so
      // they hold no registers across the computation above (a rare path).
      load_b();
      load_out();
    }
  }
  gather_sums<T, WN>(a, en, s, lds);
  MLORA_STAMP(4);
  fence_regs(bf);

  // y = the chunk groups' sums added in group order, rounded like the
  // reference's mid; zero at and past the rank and for rows past the entry's.
  {
    // Thread t: row t / 16, columns 4 (t % 16) .. + 3 (16 rows x 64 columns).
    const int row = tid >> 4;
    const int c4 = (tid & 15) * 4;
    if (c4 < a.r_max) {
      f32x4 sum = f32x4{0.f, 0.f, 0.f, 0.f};
      if (row < en.nr && c4 < rank) {
#pragma unroll
        for (int grp = 0; grp < kGroups; ++grp) sum += lds.part[grp][row][c4 / 4];
        if constexpr (NORM) {
#pragma unroll
          for (int q2 = 0; q2 < 4; ++q2) sum[q2] *= rs;
        }
      }
      raw* y = lds.ytile + row * YS + c4;
#pragma unroll
      for (int q2 = 0; q2 < 4; ++q2) y[q2] = T::from_f32(c4 + q2 < rank ? sum[q2] : 0.f);
    }
  }
  lds_barrier();
  MLORA_STAMP(5);

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
  const float scale = en.scale;
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
    // A plan row outside the call's rows (a plan made for a longer table)
    // is not stored: its clamped reads served only memory safety.  The
    // first column tile counts each such row as a plan error.
    const bool in_rows = orow_raw[i] == orow[i];
    if (row < en.nr && n < out_dim && in_rows) {
      const u32x4 d = *reinterpret_cast<const u32x4*>(lds.delta + row * LDS_STRIDE + cc * VEC);
      float f[VEC];
#pragma unroll
      for (int q = 0; q < VEC; ++q) f[q] = chunk_elem<T>(ov[i], q) + chunk_elem<T>(d, q);
      st_chunk_nt(out + static_cast<int64_t>(orow[i]) * a.out_stride + n, pack_chunk<T>(f));
    } else if (row < en.nr && !in_rows && cc == 0 && nt_g == 0) {
      atomicAdd(a.header + kWsPlanErrors, 1);
    }
  }
  MLORA_STAMP_AFTER_LOADS(6);
  lds_barrier();
}

// Shrink items of entries j, j + e_grid, ... (item: K chunk, and slice group
// when the slices' A blocks are split over items).  en / xrow_raw: entry j
// and this thread's row word, already requested.
template <class T, int NBT, int SCHED, bool NORM = false>
__device__ void shrink_items(const int32_t* plan, const DecodeArgs& a, int j, int item, int n_ent, Entry en,
                             int xrow_raw, f32x4 (*red)[kWave], const typename T::raw_t* nw = nullptr) {
  constexpr int SP = kGroupStepsLinked;
  int sg = 0, c = item;
  if (a.s_groups != 1) {
    sg = item / a.kc;
    c = item - sg * a.kc;
  }
  const uint64_t flag = SCHED == kGroupLinked ? flag_word() : 0;
  // The first entry is taken apart from the loop over the others (rare: a
  // grid smaller than the plan), so nothing the loop hoists runs before it.
  MLORA_STAMP(1);
  if (en.rank > 0 && en.nr > 0 && en.pos >= 0 && en.pos + en.nr <= a.ws_rows)
    shrink_chunk<T, NBT, SP, false, NORM>(a, j, en, clamp_row(xrow_raw, a.rows), sg, c, red, flag, nw);
  else if (en.rank > 0 && en.nr > 0 && threadIdx.x == 0 && item == 0)
    atomicAdd(a.header + kWsPlanErrors, 1);
  for (int e = j + a.e_grid; e < n_ent; e += a.e_grid) {
    xrow_raw = load_entry_row(plan, e, threadIdx.x & 15);
    en = load_entry(plan, e, a.r_max, a.num_slots);
    if (en.rank > 0 && en.nr > 0 && en.pos >= 0 && en.pos + en.nr <= a.ws_rows)
      shrink_chunk<T, NBT, SP, false, NORM>(a, e, en, clamp_row(xrow_raw, a.rows), sg, c, red, flag, nw);
    else if (en.rank > 0 && en.nr > 0 && threadIdx.x == 0 && item == 0)
      atomicAdd(a.header + kWsPlanErrors, 1);
  }
}

// Expand items (column tile `tile`) of entries j, j + e_grid, ...;
// count_errors: this launch has no shrink items, so tile 0 reports entries
// it cannot take.
// NORM: rstd holds each table row's rstd; yrow_raw is the row word of entry
// j's row threadIdx.x / 16.
template <class T, int NBT, int WN, int RS, int SCHED, bool NORM = false>
__device__ void expand_items(const int32_t* plan, const DecodeArgs& a, int j, int tile, int n_ent, Entry en,
                             int (&rows_raw)[ExpandRows<T, WN>::RPT], DecodeLds<T, WN>& lds, f32x4 (*red)[kWave],
                             bool count_errors, const float* rstd = nullptr, int yrow_raw = 0) {
  constexpr int SP = kGroupStepsLinked;
  constexpr int RPT = ExpandRows<T, WN>::RPT;
  for (int e = j;;) {
    MLORA_STAMP(1);
    if (en.rank > 0 && en.nr > 0 && en.pos >= 0 && en.pos + en.nr <= a.ws_rows)
      expand_entry<T, NBT, SP, WN, RS, SCHED == kGroupLinked, NORM>(a, plan, e, en, tile, rows_raw, lds, red, rstd,
                                                                      yrow_raw);
    else if (count_errors && en.rank > 0 && en.nr > 0 && threadIdx.x == 0 && tile == 0)
      atomicAdd(a.header + kWsPlanErrors, 1);
    e += a.e_grid;
    if (e >= n_ent) break;
#pragma unroll
    for (int i = 0; i < RPT; ++i) rows_raw[i] = load_entry_row(plan, e, ExpandRows<T, WN>::row_of(threadIdx.x, i));
    if constexpr (NORM) yrow_raw = load_entry_row(plan, e, threadIdx.x >> 4);
    en = load_entry(plan, e, a.r_max, a.num_slots);
  }
}

// Three workgroups a CU for the single launch over four A blocks (r_max 48
// and 64): at four, the loop invariants of its expand items (their row
// words and pointers) spilled 12-20 bytes a lane to scratch; at three it
// holds them in 135-138 VGPRs (rank 64: 14.07 vs 13.88 us, rank 48: 11.58
// vs 11.62 us).
//
// Workgroup (j, item) of the grid (e_grid x items) is item `item` of entry
// j, then of entries j + e_grid, ... while the plan has them; items [0,
// n_shrink) are shrink items, the next n_tiles expand items.  Workgroups go
// to the XCDs round-robin in x-fastest order and e_grid is a multiple of 8,
// so every item of entry j runs on XCD j mod 8.  plan_cap and n_shrink come
// as leading arguments (preloaded in SGPRs), so the first entry, the row
// words and the plan's entry count are requested at once, together with
// every cache line of the other arguments.
template <class T, int NBT, int WN, int RS, int SCHED>
__global__ __launch_bounds__(256, NBT >= 8 ? 2 : (NBT >= 4 && SCHED == kGroupLinked && RS == 2) ? 3 : 4) void planned_kernel(const int32_t* __restrict__ plan,
                                                                       int plan_cap, int n_shrink, DecodeArgs a) {
  __shared__ __attribute__((aligned(16))) DecodeLds<T, WN> lds;
  __shared__ f32x4 red[3 * NBT][kWave];
  MLORA_STAMP_BEGIN();
  constexpr int RPT = ExpandRows<T, WN>::RPT;
  const int j = blockIdx.x;
  const int item = blockIdx.y;
  const bool shrink = item < n_shrink;
  const int ef = min(j, plan_cap - 1);
  int rows_raw[RPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i)
    rows_raw[i] = load_entry_row(plan, ef, shrink ? (threadIdx.x & 15) : ExpandRows<T, WN>::row_of(threadIdx.x, i));
  const Entry en = load_entry(plan, ef, a.r_max, a.num_slots);
  const int p0 = plan[0];
  {
    // Touch every cache line of the kernel arguments in the round trip that
    // brings the entry, so the argument loads the compiler places over the
    // item's set-up hit the scalar cache (which every launch starts cold).
    const char* ks = (const char*)__builtin_amdgcn_kernarg_segment_ptr();
    constexpr int kLines = static_cast<int>((sizeof(DecodeArgs) + 16 + 63) / 64);
    int acc = 0;
#pragma unroll
    for (int i = 0; i < kLines; ++i) acc |= *reinterpret_cast<const int*>(ks + i * 64);
    asm volatile("" ::"s"(acc), "s"(p0), "s"(en.slot), "s"(en.rank), "s"(en.nr), "s"(en.pos));
  }
  const int n_ent = min(p0, min(plan_cap, a.e_cap));
  if (j == 0 && item == 0 && threadIdx.x == 0 && p0 > min(plan_cap, a.e_cap)) atomicAdd(a.header + kWsPlanErrors, 1);
  if (j < n_ent) {
    if (shrink) {
      if constexpr (SCHED != kGroupExpandOnly) shrink_items<T, NBT, SCHED>(plan, a, j, item, n_ent, en, rows_raw[0], red);
    } else if constexpr (SCHED != kGroupShrinkOnly) {
      expand_items<T, NBT, WN, RS, SCHED>(plan, a, j, item - n_shrink, n_ent, en, rows_raw, lds, red, n_shrink == 0);
    }
  }
  MLORA_STAMP_FLUSH();
}

template <class T, int NBT, int WN, int RS>
hipError_t launch_sched(const int32_t* plan, const DecodeArgs& a, int sched, int n_items, hipStream_t stream) {
  if (n_items <= 0 || a.e_grid <= 0) return hipSuccess;
  if (n_items > 65535 || !grid_fits(static_cast<int64_t>(n_items) * a.e_grid)) return hipErrorInvalidConfiguration;
  const dim3 grid(static_cast<unsigned>(a.e_grid), static_cast<unsigned>(n_items));
  const int n_shrink = sched == kGroupExpandOnly ? 0 : a.s_groups * a.kc;
  switch (sched) {
    case kGroupLinked:
      hipLaunchKernelGGL((planned_kernel<T, NBT, WN, RS, kGroupLinked>), grid, dim3(256), 0, stream, plan, a.plan_cap,
                         n_shrink, a);
      break;
    case kGroupShrinkOnly:
      hipLaunchKernelGGL((planned_kernel<T, NBT, WN, RS, kGroupShrinkOnly>), grid, dim3(256), 0, stream, plan,
                         a.plan_cap, n_shrink, a);
      break;
    default:
      hipLaunchKernelGGL((planned_kernel<T, NBT, WN, RS, kGroupExpandOnly>), grid, dim3(256), 0, stream, plan,
                         a.plan_cap, n_shrink, a);
      break;
  }
  return hipGetLastError();
}

template <class T, int NBT, int WN, int RS>
hipError_t launch_t(const int32_t* plan, const DecodeArgs& a, int mode, int phases, hipStream_t stream) {
  const int n_shrink = a.s_groups * a.kc;
  if (mode == kGroupLinked) return launch_sched<T, NBT, WN, RS>(plan, a, kGroupLinked, n_shrink + a.n_tiles, stream);
  // Two launches: the shrink grid holds the shrink items, the expand grid
  // the expand items (item i of entry j is workgroup i * e_grid + j there).
  if (phases & 1) {
    const hipError_t e = launch_sched<T, NBT, WN, RS>(plan, a, kGroupShrinkOnly, n_shrink, stream);
    if (e != hipSuccess) return e;
  }
  if (phases & 2) return launch_sched<T, NBT, WN, RS>(plan, a, kGroupExpandOnly, a.n_tiles, stream);
  return hipSuccess;
}

template <class T, int WN, int RS>
hipError_t launch_nbt(const int32_t* plan, const DecodeArgs& a, int nbt, int mode, int phases, hipStream_t stream) {
  switch (nbt) {
    case 1: return launch_t<T, 1, WN, RS>(plan, a, mode, phases, stream);
    case 2: return launch_t<T, 2, WN, RS>(plan, a, mode, phases, stream);
    default: return launch_t<T, 4, WN, RS>(plan, a, mode, phases, stream);
  }
}

template <class T>
hipError_t launch_dtype(const int32_t* plan, const DecodeArgs& a, int nbt, int mode, int phases, hipStream_t stream) {
  if (a.r_max <= T::KSTEP) return launch_nbt<T, 1, 1>(plan, a, nbt, mode, phases, stream);
  return launch_nbt<T, 1, 2>(plan, a, nbt, mode, phases, stream);
}

// ------------------------------------------- fused RMSNorm + decode shrink
// Shrink launch: grid (e_grid, norm rows + n_shrink).  Workgroup (j, i)
// for i < n_norm is RMSNorm row block i * e_grid + j (256 / tpr rows),
// written as the RMSNorm kernel writes it, with each row's rstd stored; the
// items after them are the shrink items of the two-launch schedule, with
// round(x * w) on the MFMA.  The norm rows come first in the grid, so they
// run beside the first shrink items instead of after the last.  Nothing in
// the launch waits on another workgroup.
template <class T, int NBT>
__global__ __launch_bounds__(256, NBT >= 8 ? 2 : 4) void planned_norm_shrink_kernel(const int32_t* __restrict__ plan,
                                                                                     int plan_cap, int n_norm,
                                                                                     DecodeArgs a, NormShrinkArgs na) {
  __shared__ f32x4 red[3 * NBT][kWave];
  __shared__ float nred[4];
  const int j = blockIdx.x;
  const int item = static_cast<int>(blockIdx.y) - n_norm;
  if (item < 0) {
    const int64_t blk = static_cast<int64_t>(blockIdx.y) * gridDim.x + j;
    // At most two chunks a thread held (the rest streamed twice): the same
    // chunks in the same order as the RMSNorm kernel's, so the same bits.
    if (blk * (256 / na.rms.tpr) < na.rms.rows)
      rmsnorm_block<T, 2, true, true, false, true>(na.rms, blk, nred, min(na.rms.nc, 2), na.rstd);
    return;
  }
  const int ef = min(j, plan_cap - 1);
  const int row_raw = load_entry_row(plan, ef, threadIdx.x & 15);
  const Entry en = load_entry(plan, ef, a.r_max, a.num_slots);
  const int p0 = plan[0];
  {
    // As in planned_kernel: every line of the kernel arguments is touched in
    // the round trip that brings the entry.
    const char* ks = (const char*)__builtin_amdgcn_kernarg_segment_ptr();
    constexpr int kLines = static_cast<int>((sizeof(DecodeArgs) + sizeof(NormShrinkArgs) + 16 + 63) / 64);
    int acc = 0;
#pragma unroll
    for (int i = 0; i < kLines; ++i) acc |= *reinterpret_cast<const int*>(ks + i * 64);
    asm volatile("" ::"s"(acc), "s"(p0), "s"(en.slot), "s"(en.rank), "s"(en.nr), "s"(en.pos));
  }
  const int n_ent = min(p0, min(plan_cap, a.e_cap));
  if (j == 0 && item == 0 && threadIdx.x == 0 && p0 > min(plan_cap, a.e_cap)) atomicAdd(a.header + kWsPlanErrors, 1);
  if (j < n_ent)
    shrink_items<T, NBT, kGroupShrinkOnly, true>(plan, a, j, item, n_ent, en, row_raw, red,
                                                 static_cast<const typename T::raw_t*>(na.rms.w));
}

// Expand launch: the expand items of the two-launch schedule, y scaled by
// each row's rstd before its rounding.
template <class T, int WN, int RS>
__global__ __launch_bounds__(256, 4) void planned_norm_expand_kernel(const int32_t* __restrict__ plan, int plan_cap,
                                                                     DecodeArgs a, const float* __restrict__ rstd) {
  __shared__ __attribute__((aligned(16))) DecodeLds<T, WN> lds;
  constexpr int RPT = ExpandRows<T, WN>::RPT;
  const int j = blockIdx.x;
  const int ef = min(j, plan_cap - 1);
  int rows_raw[RPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i) rows_raw[i] = load_entry_row(plan, ef, ExpandRows<T, WN>::row_of(threadIdx.x, i));
  const int yrow_raw = load_entry_row(plan, ef, threadIdx.x >> 4);
  const Entry en = load_entry(plan, ef, a.r_max, a.num_slots);
  const int p0 = plan[0];
  {
    // As in planned_kernel: every line of the kernel arguments is touched in
    // the round trip that brings the entry.
    const char* ks = (const char*)__builtin_amdgcn_kernarg_segment_ptr();
    constexpr int kLines = static_cast<int>((sizeof(DecodeArgs) + 32 + 63) / 64);
    int acc = 0;
#pragma unroll
    for (int i = 0; i < kLines; ++i) acc |= *reinterpret_cast<const int*>(ks + i * 64);
    asm volatile("" ::"s"(acc), "s"(p0), "s"(en.slot), "s"(en.rank), "s"(en.nr), "s"(en.pos));
  }
  const int n_ent = min(p0, min(plan_cap, a.e_cap));
  if (j == 0 && blockIdx.y == 0 && threadIdx.x == 0 && p0 > min(plan_cap, a.e_cap))
    atomicAdd(a.header + kWsPlanErrors, 1);
  if (j < n_ent)
    expand_items<T, 1, WN, RS, kGroupExpandOnly, true>(plan, a, j, blockIdx.y, n_ent, en, rows_raw, lds, nullptr,
                                                       true, rstd, yrow_raw);
}

template <class T, int NBT>
hipError_t launch_norm_shrink(const int32_t* plan, const DecodeArgs& a, const NormShrinkArgs& na, hipStream_t stream) {
  const int n_shrink = a.s_groups * a.kc;
  if (a.e_grid <= 0 || na.rms.rows <= 0) return hipSuccess;
  const int64_t blocks = (na.rms.rows + (256 / na.rms.tpr) - 1) / (256 / na.rms.tpr);
  const int64_t n_norm = (blocks + a.e_grid - 1) / a.e_grid;
  const int64_t items = n_norm + n_shrink;
  if (items > 65535 || !grid_fits(items * a.e_grid)) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL((planned_norm_shrink_kernel<T, NBT>), dim3(static_cast<unsigned>(a.e_grid), static_cast<unsigned>(items)),
                     dim3(256), 0, stream, plan, a.plan_cap, static_cast<int>(n_norm), a, na);
  return hipGetLastError();
}

template <class T>
hipError_t launch_norm_t(const int32_t* plan, const DecodeArgs& a, const NormShrinkArgs& na, int nbt, int phases,
                         hipStream_t stream) {
  if (phases & 1) {
    hipError_t e;
    switch (nbt) {
      case 1: e = launch_norm_shrink<T, 1>(plan, a, na, stream); break;
      case 2: e = launch_norm_shrink<T, 2>(plan, a, na, stream); break;
      default: e = launch_norm_shrink<T, 4>(plan, a, na, stream); break;
    }
    if (e != hipSuccess) return e;
  }
  if ((phases & 2) && a.e_grid > 0 && a.n_tiles > 0) {
    if (a.n_tiles > 65535 || !grid_fits(static_cast<int64_t>(a.n_tiles) * a.e_grid)) return hipErrorInvalidConfiguration;
    const dim3 grid(static_cast<unsigned>(a.e_grid), static_cast<unsigned>(a.n_tiles));
    if (a.r_max <= T::KSTEP)
      hipLaunchKernelGGL((planned_norm_expand_kernel<T, 1, 1>), grid, dim3(256), 0, stream, plan, a.plan_cap, a,
                         na.rstd);
    else
      hipLaunchKernelGGL((planned_norm_expand_kernel<T, 1, 2>), grid, dim3(256), 0, stream, plan, a.plan_cap, a,
                         na.rstd);
    return hipGetLastError();
  }
  return hipSuccess;
}

// Plan of a segment table, built on the device by one workgroup of NT
// threads (for callers that pass no plan): the same plan, word for word, as
// the host's (multi_lora_amd/batch_info.py: build_plan).  Entries follow the
// slots in ascending order; a slot's rows, in row order, fill entries of 16.
// Segment bounds are clamped to [0, rows); slots outside [0, num_slots) and
// rank-0 slots get no entry.  Entries past `cap` are not written (the header
// still counts them, and the apply kernels report a plan error).
//
// The table is read once: every slot's rank and scaling and a pass of up to
// NT segments (one a thread) are requested together and kept in LDS, so a
// pass costs one round trip to memory; the rest is LDS work and stores.
// NT is 1024, or 256 (128) for tables of at most 256 (128) segments over
// pools of at most 512 (256) slots, so fewer waves meet at each barrier.
template <int NT>
__global__ __launch_bounds__(NT) void build_plan_kernel(SegView m, int rows, int32_t* plan, int cap) {
  constexpr int kBuildThreads = NT;
  constexpr int kBuildSegs = NT;  // segments staged in LDS per pass
  __shared__ int cnt[kPlanBuildMaxSlots];   // rows of each slot
  __shared__ int fill[kPlanBuildMaxSlots];  // rows of each slot placed by earlier passes
  __shared__ int eoff[kPlanBuildMaxSlots];  // first entry of each slot
  __shared__ int poff[kPlanBuildMaxSlots];  // first row position of each slot
  __shared__ int rank_of[kPlanBuildMaxSlots];
  __shared__ float scal_of[kPlanBuildMaxSlots];
  __shared__ __attribute__((aligned(16))) int seg_w[kBuildSegs];  // live slot of the pass's segments (-1: none)
  __shared__ int seg_a[kBuildSegs];
  __shared__ __attribute__((aligned(16))) int seg_n[kBuildSegs];
  __shared__ int tmp[kBuildThreads / kWave];
  __shared__ int run[2];
  const int tid = threadIdx.x;
  const int ns = m.num_slots;
  const int passes = (m.bs + kBuildSegs - 1) / kBuildSegs;
  // Ranks and scalings of every slot and the first pass of segments,
  // requested at once.
  for (int s = tid; s < ns; s += kBuildThreads) {
    rank_of[s] = m.ranks[s];
    scal_of[s] = load_scaling(m.scalings, s, m.scal_dtype);
    cnt[s] = 0;
    fill[s] = 0;
  }
  auto stage = [&](int b0) {
    // Segment b0 + tid (one per thread: kBuildSegs == kBuildThreads).
    const int i = b0 + tid;
    int a0 = 0, a1 = 0, w = -1;
    if (i < m.bs) {
      a0 = min(max(m.indptr[i], 0), rows);
      a1 = min(max(m.indptr[i + 1], 0), rows);
      w = m.widx[i];
    }
    return int3{a0, a1, w};
  };
  int3 sg = stage(0);
  __syncthreads();
  auto publish = [&](int3 v) {
    const bool live = v.z >= 0 && v.z < ns && v.y > v.x && rank_of[v.z] > 0;
    seg_w[tid] = live ? v.z : -1;
    seg_a[tid] = v.x;
    seg_n[tid] = live ? v.y - v.x : 0;
  };
  // Pass 1 counts every slot's rows.
  for (int pass = 0; pass < passes; ++pass) {
    if (pass > 0) sg = stage(pass * kBuildSegs);
    publish(sg);
    if (seg_w[tid] >= 0) atomicAdd(&cnt[seg_w[tid]], seg_n[tid]);
    __syncthreads();
  }
  // Exclusive scans over the slots (in chunks of kBuildThreads): entries and rows.
  if (tid == 0) run[0] = run[1] = 0;
  __syncthreads();
  for (int s0 = 0; s0 < ns; s0 += kBuildThreads) {
    const int s = s0 + tid;
    const int c = s < ns ? cnt[s] : 0;
    int tot_e, tot_r;
    const int ex_e = block_exclusive_scan<kBuildThreads / kWave>((c + kPlanRows - 1) / kPlanRows, tmp, &tot_e);
    const int ex_r = block_exclusive_scan<kBuildThreads / kWave>(c, tmp, &tot_r);
    if (s < ns) {
      eoff[s] = run[0] + ex_e;
      poff[s] = run[1] + ex_r;
    }
    __syncthreads();
    if (tid == 0) {
      run[0] += tot_e;
      run[1] += tot_r;
    }
    __syncthreads();
  }
  const int n_entries = run[0];
  if (tid < kPlanHeaderWords) plan[tid] = tid == 0 ? n_entries : tid == 1 ? run[1] : tid == 2 ? cap : 0;
  // Entry words other than the rows: one thread per (slot, entry).
  for (int s = tid; s < ns; s += kBuildThreads) {
    const int c = cnt[s];
    if (c == 0) continue;
    const float sc = scal_of[s];
    for (int k = 0; k * kPlanRows < c; ++k) {
      const int e = eoff[s] + k;
      if (e >= cap) break;
      int32_t* p = plan + kPlanHeaderWords + static_cast<int64_t>(e) * kPlanEntryWords;
      const int nr = min(kPlanRows, c - k * kPlanRows);
      *reinterpret_cast<int4*>(p) = int4{s, rank_of[s], __float_as_int(sc), nr};
      *reinterpret_cast<int4*>(p + 4) = int4{poff[s] + k * kPlanRows, 0, 0, 0};
      *reinterpret_cast<int4*>(p + 24) = int4{0, 0, 0, 0};
      *reinterpret_cast<int4*>(p + 28) = int4{0, 0, 0, 0};
    }
  }
  // Pass 2 places the rows: segment i's rows follow the rows of the same
  // slot in earlier segments (earlier passes: fill; this pass: a scan of the
  // staged segments before it).  The thread that places an entry's first
  // row also fills the entry's unused row words with it.
  for (int pass = 0; pass < passes; ++pass) {
    if (passes > 1) {
      __syncthreads();
      sg = stage(pass * kBuildSegs);
      publish(sg);
      __syncthreads();
    }
    const int w = seg_w[tid];
    // Rows of slot w in this pass's segments before this one: a wave-uniform
    // loop (eight segments a step, read as 16-byte words) up to the wave's
    // last segment of the pass, counting those before this thread's.
    int before = 0;
    const int in_pass = min(m.bs - pass * kBuildSegs, kBuildSegs);
    const int wave0 = tid & ~(kWave - 1);
    const int lim = wave0 < in_pass ? min(wave0 + kWave, (in_pass + 7) & ~7) : 0;
    for (int j0 = 0; j0 < lim; j0 += 8) {
      const int4 wa = *reinterpret_cast<const int4*>(seg_w + j0);
      const int4 wb = *reinterpret_cast<const int4*>(seg_w + j0 + 4);
      const int4 na = *reinterpret_cast<const int4*>(seg_n + j0);
      const int4 nb = *reinterpret_cast<const int4*>(seg_n + j0 + 4);
      before += (j0 + 0 < tid && wa.x == w) ? na.x : 0;
      before += (j0 + 1 < tid && wa.y == w) ? na.y : 0;
      before += (j0 + 2 < tid && wa.z == w) ? na.z : 0;
      before += (j0 + 3 < tid && wa.w == w) ? na.w : 0;
      before += (j0 + 4 < tid && wb.x == w) ? nb.x : 0;
      before += (j0 + 5 < tid && wb.y == w) ? nb.y : 0;
      before += (j0 + 6 < tid && wb.z == w) ? nb.z : 0;
      before += (j0 + 7 < tid && wb.w == w) ? nb.w : 0;
    }
    if (w >= 0) {
      int q = fill[w] + before;
      const int a0 = seg_a[tid];
      const int n = seg_n[tid];
      const int c = cnt[w];
      for (int r = 0; r < n; ++r, ++q) {
        const int e = eoff[w] + q / kPlanRows;
        if (e >= cap) continue;
        int32_t* rw = plan + kPlanHeaderWords + static_cast<int64_t>(e) * kPlanEntryWords + kPlanRowWord;
        rw[q % kPlanRows] = a0 + r;
        if (q % kPlanRows == 0)
          for (int i = min(kPlanRows, c - q); i < kPlanRows; ++i) rw[i] = a0 + r;
      }
    }
    __syncthreads();
    if (w >= 0) atomicAdd(&fill[w], seg_n[tid]);
  }
}

}  // namespace

namespace {
size_t round256(size_t b) { return (b + 255) / 256 * 256; }
}  // namespace

bool plan_decode(int in_dim, int r_max, int n_slices, int rows, int dtype, DecodeShape* sh) {
  if (dtype != MLORA_BF16 && dtype != MLORA_F16) return false;
  if (in_dim <= 0 || rows <= 0 || n_slices < 1 || n_slices > kMaxSlices) return false;
  if (r_max <= 0 || r_max > kGroupMaxRank || r_max % 8 != 0 || in_dim % 8 != 0) return false;
  // More than four 16-row A blocks in all: one shrink item per slice, so an
  // item never holds more than four blocks of A fragments.
  const int blocks = n_slices * cdiv(r_max, 16);
  sh->s_groups = (blocks > 4) ? n_slices : 1;
  const int item_blocks = blocks / sh->s_groups;
  int b = 1;
  while (b < item_blocks) b *= 2;
  sh->nbt = b;
  sh->k_chunk = 4 * kGroupStepsLinked * BF16::KSTEP;
  sh->kc = cdiv(in_dim, sh->k_chunk);
  if (sh->kc > kWave) return false;  // one polling lane per chunk: in_dim <= 16384
  // Every entry holds at least one row: at most `rows` entries.
  sh->e_cap = rows;
  const size_t n_sums = static_cast<size_t>(rows) * sh->kc * n_slices * r_max;
  if (n_sums * sizeof(float) >= 0x7fffffffu) return false;  // read through a 32-bit buffer range
  sh->flags_off = kWsHeaderBytes;
  sh->partials_off = sh->flags_off + round256(static_cast<size_t>(sh->e_cap) * sh->s_groups * sh->kc * sizeof(uint64_t));
  sh->plan_off = sh->partials_off + round256(n_sums * sizeof(float));
  sh->rstd_off =
      sh->plan_off + round256(sizeof(int32_t) * (kPlanHeaderWords + static_cast<size_t>(sh->e_cap) * kPlanEntryWords));
  sh->bytes = sh->rstd_off + sizeof(float) * static_cast<size_t>(rows);
  return true;
}

hipError_t launch_build_plan(const SegView& m, int rows, int32_t* plan, int cap, hipStream_t stream) {
  // Decode q_proj table (128 segments, 64 slots): 7.4 us at 128 threads,
  // 7.8 at 256, 8.5 at 1024 (rocprof).
  if (m.bs <= 128 && m.num_slots <= 256)
    hipLaunchKernelGGL((build_plan_kernel<128>), dim3(1), dim3(128), 0, stream, m, rows, plan, cap);
  else if (m.bs <= 256 && m.num_slots <= 512)
    hipLaunchKernelGGL((build_plan_kernel<256>), dim3(1), dim3(256), 0, stream, m, rows, plan, cap);
  else
    hipLaunchKernelGGL((build_plan_kernel<1024>), dim3(1), dim3(1024), 0, stream, m, rows, plan, cap);
  return hipGetLastError();
}

hipError_t launch_planned(const int32_t* plan, const DecodeArgs& args, int dtype, int nbt, int mode, int phases,
                          hipStream_t stream) {
  if (dtype == MLORA_BF16) return launch_dtype<BF16>(plan, args, nbt, mode, phases, stream);
  return launch_dtype<F16>(plan, args, nbt, mode, phases, stream);
}

hipError_t launch_planned_norm(const int32_t* plan, const DecodeArgs& args, const NormShrinkArgs& na, int dtype,
                               int nbt, int phases, hipStream_t stream) {
  if (dtype == MLORA_BF16) return launch_norm_t<BF16>(plan, args, na, nbt, phases, stream);
  return launch_norm_t<F16>(plan, args, na, nbt, phases, stream);
}

}  // namespace mlora

#ifdef MLORA_TIMELINE
// Calibration builds: clear and read the planned kernel's timestamps
// ([kTlBlocks][4 waves][kTlPhases] uint32, the low word of a 100 MHz
// counter: differences modulo 2^32 are ticks of 10 ns).
extern "C" int mlora_tl_words(void) { return mlora::kTlBlocks * 4 * mlora::kTlPhases; }

// Zero the first `words` stamp words (a phase left at 0 was not reached).
extern "C" int mlora_tl_clear(int words, void* stream) {
  if (words < 0 || words > mlora_tl_words()) return -1;
  void* p = nullptr;
  hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(mlora::tl_stamps));
  if (e == hipSuccess) e = hipMemsetAsync(p, 0, sizeof(uint32_t) * words, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? 0 : static_cast<int>(e);
}

extern "C" int mlora_tl_read(uint32_t* host, int words) {
  if (host == nullptr || words < 0 || words > mlora_tl_words()) return -1;
  const hipError_t e = hipMemcpyFromSymbol(host, HIP_SYMBOL(mlora::tl_stamps), sizeof(uint32_t) * words);
  return e == hipSuccess ? 0 : static_cast<int>(e);
}
#endif
