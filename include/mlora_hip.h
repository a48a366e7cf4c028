/*
 * mlora_hip.h — C ABI of libmlora_hip.so, the MI355X (gfx950) segment-LoRA
 * hot path: segment shrink, segment expand with residual accumulate (single
 * and multi-slice), the slot-grouped decode apply, and fused RMSNorm.
 *
 * Conventions shared by every entry point
 *   - All tensor arguments are raw device pointers; strides are in ELEMENTS
 *     and the innermost stride is always 1.  The library never allocates or
 *     frees device memory: outputs and workspaces are owned by the caller.
 *   - Every call is launch-only on `stream` (a hipStream_t passed as void*):
 *     no host synchronisation, no allocation, so it can be captured into a
 *     HIP graph.  Per-step values (segment bounds, slots, ranks, scalings) are
 *     read from device memory; only `bs` and `max_len` size the grid.  A
 *     replayed call keeps the host values it was captured with, so a table
 *     rewritten in place between replays must have at most `bs` segments of
 *     at most `max_len` rows (the table summary and plan counts only size
 *     grids whose kernels recount from the device and loop).
 *   - Return value: 0 = ok, < 0 = invalid argument (nothing launched),
 *     > 0 = a hipError_t from the launch.  mlora_last_error() returns a
 *     thread-local message for the last non-zero return on this thread.
 *   - No C++ exception crosses this boundary.
 */
#ifndef MLORA_HIP_H_
#define MLORA_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types.  Data tensors (x, A, B, mid, out) share one dtype per call;
 * scalings and RMSNorm weights carry their own. */
enum mlora_dtype { MLORA_F32 = 0, MLORA_F16 = 1, MLORA_BF16 = 2 };

/* Per-step segment table (device pointers, int32).  Mirrors
 * KernelInputMetaData (multi_lora/batch_info.py:25-42):
 *   seg_indptr[bs+1]      segment s owns rows [seg_indptr[s], seg_indptr[s+1])
 *   weight_indices[bs]    pool slot of segment s
 *   lora_ranks[num_slots] rank of each slot (0 = base model, no LoRA)
 *   scalings[num_slots]   per-slot scaling, dtype `scal_dtype`
 * A slot outside [0, num_slots) is treated as rank 0 (the segment is skipped),
 * a rank above the tensor's r_max is clamped to r_max, and segment bounds are
 * clamped to [0, num_rows) of the call, so an inconsistent table can produce
 * wrong rows but never an access outside the caller's tensors.  Segments are
 * expected not to overlap: the segment kernels launch as many row tiles as
 * non-overlapping segments of num_rows rows in all can have, and tiles
 * beyond that (possible only when segments overlap) are not computed.
 * max_len bounds the segment lengths the same way.
 *
 * Optional host-side summary of the table (no counterpart in the reference's
 * KernelInputMetaData; -1 in all three when not known):
 *   long_segs    segments of more than 16 rows (after clamping to the call's
 *                rows), and long_rows the rows they hold;
 *   short_slots  distinct slots in [0, num_slots) among the segments of 1 to
 *                16 rows.
 * With it, a batch mixing long and short segments gets its expand as one
 * launch sized to the work: tiles over the long segments, and slot-grouped
 * items that read each adapter's B once for all of its short rows (pools of
 * up to 2048 slots, 16-bit data, r_max <= 64).  The kernels recount both
 * from the table, so a wrong summary costs time, never results. */
typedef struct mlora_seg_meta {
  const int32_t* seg_indptr;
  const int32_t* weight_indices;
  const int32_t* lora_ranks;
  const void* scalings;
  int32_t bs;
  int32_t max_len;
  int32_t num_slots;
  int32_t scal_dtype;
  int32_t long_segs;
  int32_t long_rows;
  int32_t short_slots;
  /* Optional plan of the table for mlora_apply_grouped (device pointer,
   * layout below), NULL when none; plan_cap: entries it holds;
   * plan_entries: its entry count if the host knows it, else -1 (it only
   * sizes the grid). */
  const int32_t* plan;
  int32_t plan_cap;
  int32_t plan_entries;
} mlora_seg_meta;

/* Plan of a segment table (no counterpart in the reference: it is the
 * slot-grouped gather list of the table, made once per table and used by
 * every mlora_apply_grouped call on it).  int32 words:
 *   header [MLORA_PLAN_HEADER_WORDS]: [0] entries, [1] rows planned,
 *     [2] entry capacity, rest 0;
 *   entry e at MLORA_PLAN_HEADER_WORDS + e * MLORA_PLAN_ENTRY_WORDS:
 *     [0] slot, [1] its rank (lora_ranks[slot]), [2] its scaling as fp32
 *     bits, [3] rows n (1..MLORA_PLAN_ROWS), [4] position of the entry's
 *     first row among all planned rows, [5..7] 0,
 *     [MLORA_PLAN_ROW_WORD + i] row i of the entry (i < n; words i >= n
 *     repeat row 0), remaining words 0.
 * Entries take the slots in ascending order, slots outside [0, num_slots)
 * and rank-0 slots excluded; a slot's rows (segment bounds clamped to the
 * call's rows), in row order, fill consecutive entries of MLORA_PLAN_ROWS,
 * and positions count the rows of all earlier entries. */
#define MLORA_PLAN_HEADER_WORDS 16
#define MLORA_PLAN_ENTRY_WORDS 32
#define MLORA_PLAN_ROWS 16
#define MLORA_PLAN_ROW_WORD 8

/* Header words (int32) at the start of an mlora_apply_grouped workspace. */
#define MLORA_WS_FALLBACKS 0   /* K chunks a waiting work item computed itself (counter) */
#define MLORA_WS_WAIT_TICKS 1  /* wait limit in 10 ns ticks: 0 = library default; < 0 = no wait at all:
                                  every waiting work item computes each K chunk itself (a test mode) */
#define MLORA_WS_PLAN_ERRORS 2 /* plan entries the call could not take (counter; should stay 0) */

/* One LoRA slice of a (possibly fused) projection.
 *   a: A stack [num_slots, r_max, in_dim]   (a_slot_stride, a_row_stride)
 *   b: B stack [num_slots, out_dim, r_max]  (b_slot_stride, b_row_stride)
 *   out_col: first column of this slice in the output rows;
 *            out_col + out_dim must not exceed the output row stride.
 * The pool layout of multi_lora/pool.py:146-155 is exactly this. */
typedef struct mlora_slice {
  const void* a;
  int64_t a_slot_stride;
  int64_t a_row_stride;
  const void* b;
  int64_t b_slot_stride;
  int64_t b_row_stride;
  int32_t out_dim;
  int32_t out_col;
} mlora_slice;

#define MLORA_MAX_SLICES 4

/* ABI version of this header; bumped on any signature change. */
int mlora_abi_version(void);

/* Thread-local text of the last error returned on this thread ("" if none). */
const char* mlora_last_error(void);

/* Bytes of caller-owned workspace mlora_shrink needs for this launch shape
 * (0 when none is needed, or when the shape is invalid — mlora_shrink then
 * reports why).  When the reduction is split over workgroups the workspace
 * holds their fp32 sums, which a second launch adds in a fixed order; its
 * contents need no initialisation.  Calls that overlap in time (on different
 * streams) need separate workspaces. */
size_t mlora_shrink_workspace_bytes(int32_t in_dim, int32_t r_max, int32_t n_slices, int32_t num_rows,
                                    int32_t bs, int32_t max_len, int32_t dtype);

/* Segment shrink: mid[t, s*r_max + n] = sum_k x[t,k] * A_s[slot, n, k] for
 * n < rank(slot) (fp32 accumulate, rounded once to `dtype`), zeros for
 * rank <= n < r_max and for rank-0 segments.  Rows outside every segment
 * are not written.
 * Replaces sgemm_lora_a_fwd (multi_lora/kernels/sgemm_lora_a.py:186-274) and
 * TritonLoRABackend.run_lora_a_sgemm (multi_lora/backend/triton_backend.py:34-45);
 * n_slices > 1 is the fused-QKV / gate-up form (x read once).
 * rank_mult implements the reference's stack_num (rank*stack_num rows of A
 * are live, sgemm_lora_a.py:51); pass 1 otherwise. */
int mlora_shrink(const void* x, int64_t x_row_stride, int32_t num_rows, int32_t in_dim,
                 const mlora_slice* slices, int32_t n_slices, int32_t r_max,
                 int32_t rank_mult, void* mid, int64_t mid_row_stride,
                 const mlora_seg_meta* meta, int32_t dtype, void* workspace,
                 size_t workspace_bytes, void* stream);

/* Segment expand with residual accumulate, for every slice s:
 *   out[t, out_col_s + n] = round(out[t, out_col_s + n]
 *                                 + round(scaling[slot] * sum_{k<rank} mid[t, s*r_max + k] * B_s[slot, n, k]))
 * fp32 accumulate; the scaled delta is rounded to `dtype` before the add,
 * as the reference kernel does (multi_lora/kernels/sgemm_lora_b.py:84-89).
 * Rank-0 segments leave `out` bit-identical.  `out` may be a strided view.
 * Replaces sgemm_lora_b_fwd (multi_lora/kernels/sgemm_lora_b.py:156-237) and
 * TritonLoRABackend.run_lora_b_sgemm (multi_lora/backend/triton_backend.py:47-61). */
int mlora_expand(const void* mid, int64_t mid_row_stride, int32_t num_rows, const mlora_slice* slices,
                 int32_t n_slices, int32_t r_max, void* out, int64_t out_row_stride,
                 const mlora_seg_meta* meta, int32_t dtype, void* stream);

/* Bytes of workspace mlora_apply_segments needs: a mid region
 * [num_rows, n_slices * r_max] of `dtype` (256-byte aligned), then the split
 * sums of mlora_shrink_workspace_bytes.  0 for an invalid shape. */
size_t mlora_apply_segments_workspace_bytes(int32_t in_dim, int32_t r_max, int32_t n_slices, int32_t num_rows,
                                            int32_t bs, int32_t max_len, int32_t dtype);

/* Segment shrink then expand in one call, with the same results as
 * mlora_shrink followed by mlora_expand element for element; the rank-r
 * intermediate lives in the workspace instead of a caller `mid`.  When the
 * shrink's K reduction is split over workgroups (16-bit data, r_max <= 64,
 * segments not all long) the expand adds the split sums up itself, in split
 * order with the same rounding, and no reduce launch or mid round trip
 * happens.  Replaces LoRABackend.apply_lora (multi_lora/backend/base.py:60-89)
 * for batches the grouped path does not take (prefill and mixed batches).
 * The workspace is scratch for this call only (no initialisation needed);
 * calls that overlap in time need separate workspaces. */
int mlora_apply_segments(const void* x, int64_t x_row_stride, int32_t num_rows, int32_t in_dim,
                         const mlora_slice* slices, int32_t n_slices, int32_t r_max, void* out,
                         int64_t out_row_stride, const mlora_seg_meta* meta, int32_t dtype, void* workspace,
                         size_t workspace_bytes, void* stream);

/* Bytes of workspace mlora_apply_grouped needs for this shape (any mode; 0
 * when the shape is not eligible or mode is not 0..2): a 256-byte header
 * (MLORA_WS_* words), per-entry chunk flags, the fp32 sums of each 256-wide
 * K chunk for every row and slice, and room for a plan of num_rows entries
 * (used when the caller passes none).  `num_slots` is accepted for layouts
 * that depend on it; none does now. */
size_t mlora_grouped_workspace_bytes(int32_t in_dim, int32_t r_max, int32_t n_slices, int32_t num_rows,
                                     int32_t num_slots, int32_t dtype, int32_t mode);

/* Slot-grouped shrink + expand for decode-shaped batches:
 *   out[t, out_col_s + n] += round(scaling * round(x[t] . A_s[slot,:rank]) . B_s[slot, n, :rank])
 * with the same roundings as mlora_shrink followed by mlora_expand; no `mid`
 * is materialised.  Work follows the table's plan (meta->plan, or one built
 * on the device into the workspace first when it is NULL; pools of up to
 * 2048 slots then): each entry's A and B are read once per call for all of
 * its rows, and slots no row uses are never read.
 * `mode`: 0 = the library's choice (the single launch while the work items
 * fit on the chip about at once, at most 16 a CU, else two launches); 1 = single launch
 * (work items of one entry run on one XCD and hand the K-chunk sums over
 * through its L2; a work item that does not receive a chunk in time, or
 * from its own XCD, computes it itself, so results never depend on timing
 * or placement); 2 = two launches (shrink items, then expand items).  All
 * modes give bit-identical results.
 * The workspace must be zero-filled before its first use and is never
 * cleared afterwards (sums are tagged with the launch's dispatch id on its
 * hardware queue); calls that overlap in time need separate workspaces, and
 * one workspace serves one stream.  Its MLORA_WS_* header words count chunks
 * computed after a wait gave up and plan errors, and may set the wait
 * limit.
 * `phases` (two-launch mode only; must be 3 otherwise): 1 = shrink half
 * (leaves its sums in the workspace), 2 = expand half (consumes them), 3 = both.
 * Requirements (else -2 and nothing launched): bf16 or fp16; r_max <= 64 and
 * a multiple of 8; 16-byte aligned rows of x, A, B and out (pointers, strides,
 * in_dim and every out_dim multiples of 8 elements).
 * Replaces LoRABackend.apply_lora (multi_lora/backend/base.py:60-89) with the
 * reference's decode kernels (sgemm_lora_a.py:118-183, sgemm_lora_b.py:93-153). */
int mlora_apply_grouped(const void* x, int64_t x_row_stride, int32_t num_rows, int32_t in_dim,
                        const mlora_slice* slices, int32_t n_slices, int32_t r_max, void* out,
                        int64_t out_row_stride, const mlora_seg_meta* meta, int32_t dtype, void* workspace,
                        size_t workspace_bytes, int32_t mode, int32_t phases, void* stream);

/* mlora_apply_grouped without a caller workspace, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid it); no counterpart in the reference.  The library
 * keeps its own workspace, MLORA_STATIC_SCRATCH_BYTES of device memory per
 * GPU held for the life of the process; a shape that needs more (see
 * mlora_grouped_workspace_bytes) returns -3 with nothing launched.  The
 * call allocates nothing.  Every call on one GPU shares that workspace:
 * calls that overlap in time on one GPU (on different streams) race, and
 * must not be made.  Arguments and results are those of mlora_apply_grouped. */
#define MLORA_STATIC_SCRATCH_BYTES (16 << 20)
int mlora_apply_grouped_static(const void* x, int64_t x_row_stride, int32_t num_rows, int32_t in_dim,
                               const mlora_slice* slices, int32_t n_slices, int32_t r_max, void* out,
                               int64_t out_row_stride, const mlora_seg_meta* meta, int32_t dtype, int32_t mode,
                               int32_t phases, void* stream);

/* RMSNorm fused into the slot-grouped apply (two launches), for a decoder
 * layer's input norm feeding LoRA-wrapped projections:
 *   y[t] = round(x[t] * rsqrt(mean(x[t]^2) + eps) * w)     (every row t)
 *   out[t, out_col_s + n] += round(scaling * round(rstd_t * (round(x[t] * w) . A_s[slot,:rank]))
 *                                  . B_s[slot, n, :rank])
 * The first launch (phases & 1) writes y, the same bits mlora_rmsnorm writes,
 * with each row's rstd_t = rsqrt(mean(x[t]^2) + eps) kept in the workspace,
 * and the shrink's K-chunk sums: the shrink reads x and multiplies
 * round(x * w) with A on MFMA, so it needs no y and no pass before it.  The
 * second launch (phases & 2) adds a row's chunk sums, scales them by rstd_t
 * before the reference's `mid` rounding, and runs the expand as
 * mlora_apply_grouped does.  In a layer the base GEMM on y runs between the two
 * halves (phases 1, GEMM, phases 2), since the expand adds into its output.
 * Against the unfused path (mlora_rmsnorm, then mlora_apply_grouped on y)
 * only the rounding of the MFMA inputs differs (round(x * w) scaled after
 * the sum instead of round(x * rstd * w)), within the tolerance of an fp32
 * reference.  The weight has the data dtype; y must not overlap x.  In
 * fp16, every x * w must be finite in fp16 (the unfused path rounds
 * x * rstd * w instead, which is smaller where mean(x^2) > 1).
 * Workspace: mlora_grouped_workspace_bytes (any mode), the same conditions
 * as mlora_apply_grouped (zero-filled before its first use, one stream);
 * a table without LoRA work still writes y.
 * Requirements (else -2): bf16 or fp16, the grouped path's shape and
 * alignment conditions, and 16-byte aligned rows of y and of the weight.
 * No counterpart is called in the reference: it fuses rmsnorm_fwd
 * (multi_lora/kernels/rmsnorm.py:48-92) into the decode shrink it feeds
 * (sgemm_lora_a.py:118-183); the expand half replaces sgemm_lora_b.py:93-153. */
int mlora_rmsnorm_apply_grouped(const void* x, int64_t x_row_stride, int32_t num_rows, int32_t in_dim,
                                const void* norm_w, float eps, void* y, int64_t y_row_stride,
                                const mlora_slice* slices, int32_t n_slices, int32_t r_max, void* out,
                                int64_t out_row_stride, const mlora_seg_meta* meta, int32_t dtype, void* workspace,
                                size_t workspace_bytes, int32_t phases, void* stream);

/* Bytes of a plan with room for `entries_cap` entries. */
size_t mlora_plan_bytes(int32_t entries_cap);

/* Build the plan of meta's table for calls of num_rows rows into `plan`
 * (device memory of mlora_plan_bytes(plan_cap) bytes), on the device: the
 * same words the layout above defines.  Entries past plan_cap are not
 * written (the header still counts them).  Pools of up to 2048 slots.
 * No counterpart in the reference; the slot-grouped gather indices of its
 * batch metadata (multi_lora/batch_info.py:128-179) made on the device. */
int mlora_build_plan(const mlora_seg_meta* meta, int32_t num_rows, int32_t* plan, int32_t plan_cap, void* stream);

/* Fused RMSNorm: y[row] = round(x[row] * rsqrt(mean(x[row]^2) + eps) * w) in
 * fp32, one rounding.  Row `row` of x starts at
 *   (row / inner) * x_stride_outer + (row % inner) * x_stride_inner,
 * the two-level addressing of rmsnorm_fwd (multi_lora/kernels/rmsnorm.py:48-92);
 * y is [rows, hidden] with row stride y_row_stride.  w has dtype w_dtype. */
int mlora_rmsnorm(const void* x, int64_t x_stride_outer, int64_t x_stride_inner,
                  int64_t inner, const void* w, int32_t w_dtype, void* y,
                  int64_t y_row_stride, int64_t rows, int32_t hidden, float eps,
                  int32_t dtype, void* stream);

/* Residual add fused with the next RMSNorm of a decoder layer:
 *   h = round(x + residual); residual <- h; y = round(h * rsqrt(mean(h^2) + eps) * w)
 * (fp32 math, h rounded to `dtype` as an unfused tensor add stores it).  x, residual
 * and y are [rows, hidden] with their own row strides; y may be x (in place),
 * residual must not overlap x or y.  No counterpart is called in the
 * reference: it is the fusion the reference plans as fused_add_rms_norm
 * (OPTIMIZATION_TODO.md T22) around multi_lora/kernels/rmsnorm.py:17-48. */
int mlora_add_rmsnorm(const void* x, int64_t x_row_stride, void* residual, int64_t residual_row_stride,
                      const void* w, int32_t w_dtype, void* y, int64_t y_row_stride, int64_t rows,
                      int32_t hidden, float eps, int32_t dtype, void* stream);

/* Layout of one module key in the slot pool and in a staged bank, for
 * mlora_pool_scatter.  A[key] is [num_slots, max_rank, in_dim] and B[key] is
 * [num_slots, out_dim, max_rank] (multi_lora/pool.py:146-155); a bank holds
 * the key's A block [rank, in_dim] at a_off and its B block [out_dim, rank]
 * at b_off (elements), as multi_lora/pool.py:23-58 packs them. */
typedef struct mlora_pool_key {
  void* a;
  int64_t a_slot_stride;   /* elements between slots of A[key] (max_rank * in_dim) */
  int64_t a_off;
  void* b;
  int64_t b_slot_stride;   /* elements between slots of B[key] (out_dim * max_rank) */
  int64_t b_row_stride;    /* elements between rows of one B slot (max_rank) */
  int64_t b_off;
  int32_t in_dim;
  int32_t out_dim;
} mlora_pool_key;

/* Pool upload: for each staged adapter i < h and each key, copy the bank's A
 * block into rows [0, rank) of A[key][slots[i]] and its B block into columns
 * [0, rank) of B[key][slots[i]]; nothing else in the pool changes.  `stage`
 * is [h, stage_row_stride] on the device; `slots` (int32[h]) and `keys`
 * (mlora_pool_key[n_keys]) are device arrays, so a captured graph follows
 * their rewrites.  Slots outside [0, num_slots) are skipped.  `max_numel` is
 * the largest rank*in_dim or out_dim*rank over the keys (it sizes the grid);
 * n_keys * h must not exceed 65535.  Data dtype F16, BF16 or F32 (a bit
 * copy: only the element size matters).
 * Replaces scatter_stage / _scatter_stage_kernel
 * (multi_lora/kernels/scatter_bank.py:17-93), called from the pool's upload
 * (multi_lora/pool.py:199-243). */
int mlora_pool_scatter(const void* stage, int64_t stage_row_stride, int32_t h, const int32_t* slots,
                       const mlora_pool_key* keys, int32_t n_keys, int32_t rank, int32_t num_slots,
                       int64_t max_numel, int32_t dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MLORA_HIP_H_ */
