// Launch-side contracts between the C ABI layer (api.hip) and the kernel
// translation units.  Every *Args struct is passed to a kernel by value.
#pragma once

#include "common.h"

namespace mlora {

inline int cdiv(int a, int b) { return (a + b - 1) / b; }

// A launch's work-items per grid dimension must fit in 32 bits: at most this
// many 256-thread workgroups.  Launchers return hipErrorInvalidConfiguration
// beyond it instead of launching a truncated grid.
constexpr int64_t kMaxBlocks = ((int64_t{1} << 32) - 1) / 256;
inline bool grid_fits(int64_t blocks) { return blocks <= kMaxBlocks; }

// Workgroups that cover every dense row tile of bm rows (dense_tile): each
// segment has ceil(len / bm) tiles and the segments' lengths add up to at
// most `rows`, so there are at most (rows + bs * (bm - 1)) / bm tiles, and at
// most bs * m_tiles (m_tiles = ceil(max_len / bm)).
inline int64_t dense_tiles(int bs, int m_tiles, int rows, int bm) {
  const int64_t seg_major = static_cast<int64_t>(bs) * m_tiles;
  const int64_t bound = (static_cast<int64_t>(rows) + static_cast<int64_t>(bs) * (bm - 1)) / bm;
  return seg_major < bound ? seg_major : bound;
}

// -------------------------------------------------------------- shrink
struct ShrinkArgs {
  const void* x;
  int64_t x_stride;
  int rows;         // rows of x / mid; segment bounds are clamped to it
  int in_dim;
  SliceView slices[kMaxSlices];
  int n_slices;
  int r_max;
  int rank_mult;
  void* mid;
  int64_t mid_stride;
  SegView meta;
  int m_tiles;      // row tiles per segment (ceil(max_len / bm)); bounds the grid
  int ks;           // K splits per row tile
  int k_per_split;  // reduction elements per split (multiple of KSTEP)
  float* partials;  // ks > 1: [ks][rows][part_cols] fp32 split sums (this launch's columns first)
  int part_cols;    // row width of the split sums: n_slices * r_max of the whole call
  int skip_reduce;  // ks > 1: leave the split sums for the expand (no reduce launch)
  int row_reduce;   // ks > 1, mid private to the apply path: reduce every row and column, no table lookup
};

struct ShrinkPlan {
  int bm;         // token rows per tile: 16, 64, or 128 (streamed kernel only)
  int m_tiles;
  int ks;
  int k_per_split;
  int nbt;        // compiled bound on 16-row blocks of A over the slices of one launch
  int spg;        // slices per launch: calls over 8 A blocks run one launch per group of slices
  int kt;         // streamed kernel: reduction elements per stage (0: not planned)
  int stages;     // streamed kernel: stages in flight
  size_t ws_bytes;
};

bool plan_shrink(int in_dim, int r_max, int n_slices, int rows, int bs, int max_len, int dtype, int num_cus,
                 ShrinkPlan* plan);
// Launches the shrink and, when K is split, the in-order split reduction.
hipError_t launch_shrink(const ShrinkPlan& plan, ShrinkArgs args, int dtype, bool aligned, hipStream_t stream);

// -------------------------------------------------------------- expand
constexpr int kExpandBN = 256;  // output columns per tile
// Token rows per tile for long segments: 32 keeps the accumulators at 32
// registers a lane, so four workgroups fit on a CU and their output tiles
// are in flight together.
constexpr int kExpandLongBM = 32;
// Token rows per tile of the streamed expand (output tile staged in LDS by
// direct-to-LDS loads, no prefetch registers), used when segments average
// at least this many rows.
constexpr int kExpandStreamBM = 64;

struct ExpandArgs {
  const void* mid;
  int64_t mid_stride;
  int rows;         // rows of mid / out; segment bounds are clamped to it
  SliceView slices[kMaxSlices];
  int n_slices;
  int r_max;
  void* out;
  int64_t out_stride;
  SegView meta;
  int m_tiles;
  int n_tiles;                     // n-tiles over all slices
  int tile_base[kMaxSlices + 1];   // first n-tile of each slice
  // ks > 1: y is not read from `mid` but added up here from the shrink's
  // fp32 split sums [ks][rows][n_slices * r_max], in split order, and
  // rounded once (the values the split reduce would have written to mid).
  const float* partials;
  int ks;
  int cus;  // compute units of the device (sizes the streamed expand's choice of cache hint)
};
// Streamed expand launches of at least this many tiles a CU read and write
// their output tiles with the non-temporal hint (the tile is read and written
// once; the hint keeps B and mid, which other tiles read again, in the L2).
constexpr int kStreamNtTilesPerCu = 6;
// Reductions of at least this many elements over long segments take the
// streamed shrink's 128-row tiles.
constexpr int kLongKRows128 = 8192;
// Largest r_max, and widest output in 256-column tiles, for which the
// expand takes split sums.
constexpr int kFuseMaxRank = 64;
constexpr int kFuseMaxTiles = 16;

hipError_t launch_expand(int bm, ExpandArgs args, int dtype, bool aligned, hipStream_t stream);

// -------------------------------------------------------------- slot-grouped items
// Shared by the mixed-batch expand (grouped.hip): work items indexed by
// (slot, column tile) that find their slot's rows by scanning the segment
// table and read each slot's B tile once for all of them.
constexpr int kGroupRows = 256;  // rows gathered per pass
// K-steps per wave per K chunk of the planned decode shrink (chunk = 4 waves
// x steps x 32 = 256 elements).
constexpr int kGroupStepsLinked = 2;
constexpr int kGroupAuto = 0;    // mode: the library's choice (the single launch)
constexpr int kGroupLinked = 1;  // mode: one launch, sums handed over through the L2
constexpr int kGroupTwo = 2;     // mode: two launches
constexpr int kGroupShrinkOnly = 3;  // launch schedules of the two-launch mode
constexpr int kGroupExpandOnly = 4;
// kGroupAuto takes the single launch while the grid holds at most this many
// work items per CU, else two launches.
constexpr int kLinkedItemsPerCu = 16;

struct GroupedArgs {
  const void* x;
  int64_t x_stride;
  int rows;
  int in_dim;
  SliceView slices[kMaxSlices];
  int n_slices;
  int r_max;
  void* out;
  int64_t out_stride;
  SegView meta;
  float* partials;   // split sums [kc][rows][n_slices * r_max]
  int kc;            // K splits
  int k_chunk;
  int s_groups;
  int n_tiles;       // expand items per slot (column tiles over all slices)
  int tile_base[kMaxSlices + 1];
  int expand_wn;     // 256-column blocks per expand item
  // Expand items take the rows of the slot's short segments only (at most
  // kShortSegRows rows), and y from `mid` (or, with split sums, from
  // `partials` with kc = the split count).
  int short_only;
  const void* mid;
  int64_t mid_stride;
};

// Largest r_max (per slice) the grouped and planned paths handle.
constexpr int kGroupMaxRank = 64;

// -------------------------------------------------------------- planned decode
// Plan of a segment table (int32 words; the layout callers see in
// include/mlora_hip.h).  Header: [0] entries, [1] rows planned, [2] entry
// capacity.  Entry: slot, rank, scaling (fp32 bits), row count (1..16),
// workspace position of its first row, then 16 row numbers (unused ones
// repeat the first).
constexpr int kPlanHeaderWords = MLORA_PLAN_HEADER_WORDS;
constexpr int kPlanEntryWords = MLORA_PLAN_ENTRY_WORDS;
constexpr int kPlanRows = MLORA_PLAN_ROWS;
constexpr int kPlanSlot = 0;
constexpr int kPlanRank = 1;
constexpr int kPlanScale = 2;
constexpr int kPlanRowCount = 3;
constexpr int kPlanPos = 4;
constexpr int kPlanRowWord = MLORA_PLAN_ROW_WORD;
// Pools of up to this many slots get their plan built on the device when
// the caller passes none (LDS tables of the builder).
constexpr int kPlanBuildMaxSlots = 2048;

// Workspace of the planned decode: a header of int32 words, the chunk
// flags (64-bit) and the fp32 K-chunk sums, each region 256-byte aligned,
// then a plan region used when the caller passes no plan.
constexpr size_t kWsHeaderBytes = 256;
constexpr int kWsFallbacks = MLORA_WS_FALLBACKS;       // chunks an expand item computed itself
constexpr int kWsWaitOverride = MLORA_WS_WAIT_TICKS;   // wait limit in 10 ns ticks: 0 default, < 0 none
constexpr int kWsPlanErrors = MLORA_WS_PLAN_ERRORS;    // entries the call could not take
// Buffer resource word 3 for raw buffer loads on gfx9 (data format 32 bit).
constexpr int kBufferRsrcWord3 = 0x00020000;

struct DecodeArgs {
  const void* x;
  int64_t x_stride;
  int rows;
  int in_dim;
  SliceView slices[kMaxSlices];
  int n_slices;
  int r_max;
  void* out;
  int64_t out_stride;
  int num_slots;     // slots of the call's stacks (entries of other slots are skipped)
  int kc;            // K chunks
  int k_chunk;       // reduction elements per chunk
  int s_groups;      // shrink items per (entry, chunk): 1 (all slices) or n_slices (one each)
  int n_tiles;       // expand items per entry (256-column tiles over all slices)
  int tile_base[kMaxSlices + 1];
  int e_grid;        // entries per row of the grid (multiple of 8)
  int e_cap;         // entries the workspace flags hold
  int plan_cap;      // entries the plan holds
  int ws_rows;       // rows the workspace sums hold
  int* header;
  uint64_t* flags;   // [plan_cap][s_groups][kc] {launch tag, XCC id}
  float* partials;   // [ws_rows][kc][n_slices * r_max]
};

// Shape check and plan of the work: K chunks, A blocks per shrink item,
// shrink items per chunk, and the workspace regions.
struct DecodeShape {
  int kc, k_chunk, nbt, s_groups;
  size_t flags_off, partials_off, plan_off, rstd_off, bytes;
  int e_cap;
};
bool plan_decode(int in_dim, int r_max, int n_slices, int rows, int dtype, DecodeShape* sh);
hipError_t launch_planned(const int32_t* plan, const DecodeArgs& args, int dtype, int nbt, int mode, int phases,
                          hipStream_t stream);
hipError_t launch_build_plan(const SegView& m, int rows, int32_t* plan, int cap, hipStream_t stream);

// ------------------------------------------------------ mixed-batch expand
// Segments of at most this many rows are "short" (decode-like) in a mixed
// batch; the host summary in mlora_seg_meta uses the same bound.
constexpr int kShortSegRows = 16;
// Pools of up to this many slots (a bitmap of 32-bit words in LDS).
constexpr int kMixedMaxSlots = 2048;
// 256-column tiles a short item of the mixed expand covers.
constexpr int kMixedShortWn = 2;
// One launch for a batch mixing long and short segments: units
// [0, short_units * n_tiles) are slot-grouped items (distinct slot of the
// short segments, in slot order; 256-column tile), which read each adapter's
// B tile once for all of that slot's short rows; the next units are (row
// tile of a long segment, 256-column tile): 64 rows streamed through LDS as
// expand_dma_kernel's when y comes from mid and such tiles give each of the
// `cus` CUs four workgroups, else 32 rows as expand_kernel's.  The long
// units are counted from the summary's long_rows and long_segs.  The kernel
// recounts both kinds from the table: a count given too small is covered by
// looping, one too large leaves units that exit.
hipError_t launch_mixed(const ExpandArgs& args, int dtype, int64_t long_rows, int long_segs, int short_units,
                        int cus, hipStream_t stream);


// -------------------------------------------------------------- rmsnorm
struct RmsArgs {
  const void* x;
  int64_t x_stride_outer;
  int64_t x_stride_inner;
  int64_t inner;
  const void* w;
  int w_dtype;
  void* y;
  int64_t y_stride;
  int64_t rows;
  int hidden;
  float eps;
  int tpr;      // threads per row (power of two, 16..256)
  int nc;       // 16-byte chunks per thread held in registers (1, 2, 4 or 8)
  int aligned;  // x rows and y rows readable as 16-byte chunks
  int w_vec;    // weight has x's dtype and is readable as 16-byte chunks
  void* residual;            // non-null: h = x + residual is stored here and normalised
  int64_t residual_stride;
};

hipError_t launch_rmsnorm(RmsArgs args, int dtype, hipStream_t stream);

// Threads per row and registered chunks per thread of the RMSNorm kernel for
// rows of `hidden` elements (the fused RMSNorm + decode shrink takes the same,
// so both write the same bits).
void rmsnorm_shape(int hidden, int dtype, int* tpr, int* nc);

// ------------------------------------------- fused RMSNorm + decode shrink
// The two-launch planned decode with the RMSNorm of its input rows folded
// into the shrink launch.  That launch holds norm workgroups that write
// y = RMSNorm(x) for every row (the RMSNorm kernel's rows, same bits) and
// each row's rstd = rsqrt(mean(x^2) + eps), and the shrink items, which read
// the raw x rows and the weight and multiply round(x * w) with A on MFMA
// instead of y.  The expand items scale a row's summed chunks by its rstd
// before rounding them to the storage type as y . A^T.
struct NormShrinkArgs {
  RmsArgs rms;  // the call's rows: x, weight (data dtype, 16-byte aligned), y, eps
  float* rstd;  // [rows]: each row's rstd, as the norm rows computed it
};
hipError_t launch_planned_norm(const int32_t* plan, const DecodeArgs& args, const NormShrinkArgs& na, int dtype,
                               int nbt, int phases, hipStream_t stream);

// -------------------------------------------------------------- pool upload
// Elements per workgroup and block of the pool upload: one 16-byte chunk of
// A and one of B a thread (Llama-3-8B bank of 4 adapters, 671 MB: 108.8 us
// against 122.1 at 4096, 131.4 at 8192, 139.1 at 1024).
constexpr int64_t kScatterElems = 2048;

struct ScatterArgs {
  const void* stage;          // [h, stage_stride] staged banks
  int64_t stage_stride;
  int h;                      // adapters staged
  const int32_t* slots;       // [h] destination slot of each staged bank (device)
  const mlora_pool_key* keys; // [n_keys] per-key layout (device)
  int n_keys;
  int rank;
  int num_slots;
  int vec;                    // stage and pool 16-byte aligned
};

hipError_t launch_scatter(const ScatterArgs& args, int64_t max_numel, int elem_bytes, hipStream_t stream);

// Base pointer of slice `s`'s A (or B) for one slot, selected with
// compile-time indexing so the kernel-argument array is never indexed
// dynamically.
template <class R>
__device__ __forceinline__ const R* slice_a(const SliceView (&sl)[kMaxSlices], int s, int slot, int n) {
  const SliceView* p = &sl[0];
#pragma unroll
  for (int i = 1; i < kMaxSlices; ++i)
    if (s == i) p = &sl[i];
  return static_cast<const R*>(p->a) + static_cast<int64_t>(slot) * p->a_slot_stride +
         static_cast<int64_t>(n) * p->a_row_stride;
}

}  // namespace mlora
