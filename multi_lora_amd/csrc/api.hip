// extern "C" entry points of libmlora_hip.so (declared in include/mlora_hip.h).
// Each entry point validates its arguments on the host, picks a launch
// shape, and launches on the caller's stream.  Nothing here allocates,
// frees or synchronises.
#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "kernels.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  std::snprintf(g_err, sizeof(g_err), "%s: %s", what, hipGetErrorString(e));
  return static_cast<int>(e);
}

constexpr int kBadArg = -1;
constexpr int kUnsupported = -2;
constexpr int kWorkspace = -3;

int elem_bytes(int dtype) { return dtype == MLORA_F32 ? 4 : 2; }
int vec_elems(int dtype) { return dtype == MLORA_F32 ? 4 : 8; }
bool valid_dtype(int d) { return d == MLORA_F32 || d == MLORA_F16 || d == MLORA_BF16; }
bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int num_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

int check_meta(const mlora_seg_meta* m) {
  if (m == nullptr) return fail(kBadArg, "segment metadata is null");
  if (m->bs < 0 || m->max_len < 0 || m->num_slots < 0)
    return fail(kBadArg, "negative bs/max_len/num_slots (%d/%d/%d)", m->bs, m->max_len, m->num_slots);
  if (!valid_dtype(m->scal_dtype)) return fail(kBadArg, "bad scalings dtype %d", m->scal_dtype);
  if (m->long_segs < -1 || m->long_rows < -1 || m->short_slots < -1)
    return fail(kBadArg, "table summary below -1 (%d/%d/%d)", m->long_segs, m->long_rows, m->short_slots);
  if (m->bs > 0 && (m->seg_indptr == nullptr || m->weight_indices == nullptr || m->lora_ranks == nullptr))
    return fail(kBadArg, "null segment table pointer");
  if (m->bs > 0 && m->num_slots > 0 && m->scalings == nullptr) return fail(kBadArg, "null scalings pointer");
  if (m->plan != nullptr && m->plan_cap < 1) return fail(kBadArg, "plan given with capacity %d", m->plan_cap);
  return 0;
}

mlora::SegView seg_view(const mlora_seg_meta* m) {
  mlora::SegView v;
  v.indptr = m->seg_indptr;
  v.widx = m->weight_indices;
  v.ranks = m->lora_ranks;
  v.scalings = m->scalings;
  v.bs = m->bs;
  v.num_slots = m->num_slots;
  v.scal_dtype = m->scal_dtype;
  return v;
}

mlora::SliceView slice_view(const mlora_slice& s) {
  mlora::SliceView v;
  v.a = s.a;
  v.a_slot_stride = s.a_slot_stride;
  v.a_row_stride = s.a_row_stride;
  v.b = s.b;
  v.b_slot_stride = s.b_slot_stride;
  v.b_row_stride = s.b_row_stride;
  v.out_dim = s.out_dim;
  v.out_col = s.out_col;
  return v;
}

// Bytes of the mid region at the start of a segment workspace (256-byte
// aligned, so the split sums after it are too).
size_t mid_region_bytes(int32_t rows, int32_t n_slices, int32_t r_max, int32_t dtype) {
  const size_t b = static_cast<size_t>(rows) * n_slices * r_max * elem_bytes(dtype);
  return (b + 255) / 256 * 256;
}

// Shrink; with skip_reduce the split sums stay in the workspace for the
// expand (no reduce launch).  private_mid: only the apply path's expand
// reads mid, so the split reduce may fill every row and column of it
// (values the expand never reads included) without looking up the table.
int shrink_impl(const void* x, int64_t x_row_stride, int32_t num_rows, int32_t in_dim, const mlora_slice* slices,
                int32_t n_slices, int32_t r_max, int32_t rank_mult, void* mid, int64_t mid_row_stride,
                const mlora_seg_meta* meta, int32_t dtype, void* workspace, size_t workspace_bytes, bool skip_reduce,
                bool private_mid, void* stream) {
  if (!valid_dtype(dtype)) return fail(kBadArg, "bad dtype %d", dtype);
  if (int rc = check_meta(meta)) return rc;
  if (n_slices < 1 || n_slices > MLORA_MAX_SLICES) return fail(kBadArg, "n_slices %d not in [1, %d]", n_slices, MLORA_MAX_SLICES);
  if (slices == nullptr) return fail(kBadArg, "slices is null");
  if (in_dim <= 0 || r_max <= 0 || rank_mult < 1 || num_rows < 0)
    return fail(kBadArg, "in_dim %d, r_max %d, rank_mult %d, num_rows %d", in_dim, r_max, rank_mult, num_rows);
  if (x_row_stride < in_dim) return fail(kBadArg, "x row stride %lld < in_dim %d", (long long)x_row_stride, in_dim);
  if (mid_row_stride < static_cast<int64_t>(n_slices) * r_max)
    return fail(kBadArg, "mid row stride %lld < n_slices*r_max %d", (long long)mid_row_stride, n_slices * r_max);
  if (meta->bs == 0 || num_rows == 0) return 0;
  if (x == nullptr || mid == nullptr) return fail(kBadArg, "x or mid is null");
  for (int s = 0; s < n_slices; ++s) {
    if (slices[s].a == nullptr) return fail(kBadArg, "slice %d: A is null", s);
    if (slices[s].a_row_stride < in_dim || slices[s].a_slot_stride < static_cast<int64_t>(r_max) * slices[s].a_row_stride)
      return fail(kBadArg, "slice %d: A strides (%lld, %lld) do not hold [r_max=%d, in=%d] rows", s,
                  (long long)slices[s].a_slot_stride, (long long)slices[s].a_row_stride, r_max, in_dim);
  }

  mlora::ShrinkPlan plan;
  if (!mlora::plan_shrink(in_dim, r_max, n_slices, num_rows, meta->bs, meta->max_len, dtype, num_cus(), &plan))
    return fail(kUnsupported, "shrink shape unsupported: %d slices x r_max %d exceeds 16 blocks of 16 rows",
                n_slices, r_max);
  if (plan.ws_bytes > 0 && (workspace == nullptr || workspace_bytes < plan.ws_bytes))
    return fail(kWorkspace, "shrink workspace too small: need %zu bytes, got %zu", plan.ws_bytes, workspace_bytes);

  const int vec = vec_elems(dtype);
  bool aligned = al16(x) && x_row_stride % vec == 0 && in_dim % vec == 0;
  for (int s = 0; s < n_slices; ++s)
    aligned = aligned && al16(slices[s].a) && slices[s].a_slot_stride % vec == 0 && slices[s].a_row_stride % vec == 0;

  mlora::ShrinkArgs args{};
  args.x = x;
  args.x_stride = x_row_stride;
  args.rows = num_rows;
  args.in_dim = in_dim;
  for (int s = 0; s < n_slices; ++s) args.slices[s] = slice_view(slices[s]);
  args.n_slices = n_slices;
  args.r_max = r_max;
  args.rank_mult = rank_mult;
  args.mid = mid;
  args.mid_stride = mid_row_stride;
  args.meta = seg_view(meta);
  args.partials = static_cast<float*>(workspace);
  args.skip_reduce = skip_reduce ? 1 : 0;
  args.row_reduce = private_mid ? 1 : 0;
  hipError_t e = mlora::launch_shrink(plan, args, dtype, aligned, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "shrink launch");
  return 0;
}

// Expand; with partials (ks > 1) y is added up from the shrink's split sums
// instead of read from mid.
int expand_impl(const void* mid, int64_t mid_row_stride, int32_t num_rows, const mlora_slice* slices, int32_t n_slices,
                int32_t r_max, void* out, int64_t out_row_stride, const mlora_seg_meta* meta, int32_t dtype,
                const float* partials, int ks, void* stream) {
  if (!valid_dtype(dtype)) return fail(kBadArg, "bad dtype %d", dtype);
  if (int rc = check_meta(meta)) return rc;
  if (n_slices < 1 || n_slices > MLORA_MAX_SLICES) return fail(kBadArg, "n_slices %d not in [1, %d]", n_slices, MLORA_MAX_SLICES);
  if (slices == nullptr) return fail(kBadArg, "slices is null");
  if (r_max <= 0 || num_rows < 0) return fail(kBadArg, "r_max %d, num_rows %d", r_max, num_rows);
  if (mid_row_stride < static_cast<int64_t>(n_slices) * r_max)
    return fail(kBadArg, "mid row stride %lld < n_slices*r_max %d", (long long)mid_row_stride, n_slices * r_max);
  // No slot in the pool: every segment has rank 0 and the output is untouched.
  if (meta->bs == 0 || num_rows == 0 || meta->num_slots == 0) return 0;
  if (mid == nullptr || out == nullptr) return fail(kBadArg, "mid or out is null");

  const int vec = vec_elems(dtype);
  const int eb = elem_bytes(dtype);
  mlora::ExpandArgs args{};
  int tiles = 0;
  bool aligned = r_max % vec == 0 && out_row_stride % vec == 0 && al16(mid) && mid_row_stride % vec == 0;
  for (int s = 0; s < n_slices; ++s) {
    const mlora_slice& sl = slices[s];
    if (sl.b == nullptr) return fail(kBadArg, "slice %d: B is null", s);
    if (sl.out_dim <= 0 || sl.out_col < 0) return fail(kBadArg, "slice %d: out_dim %d, out_col %d", s, sl.out_dim, sl.out_col);
    if (static_cast<int64_t>(sl.out_col) + sl.out_dim > out_row_stride)
      return fail(kBadArg, "slice %d: columns [%d, %lld) exceed the output row stride %lld", s, sl.out_col,
                  static_cast<long long>(sl.out_col) + sl.out_dim, (long long)out_row_stride);
    if (sl.b_row_stride < r_max || sl.b_slot_stride < static_cast<int64_t>(sl.out_dim) * sl.b_row_stride)
      return fail(kBadArg, "slice %d: B strides (%lld, %lld) do not hold [out=%d, r_max=%d] rows", s,
                  (long long)sl.b_slot_stride, (long long)sl.b_row_stride, sl.out_dim, r_max);
    args.slices[s] = slice_view(sl);
    args.tile_base[s] = tiles;
    tiles += mlora::cdiv(sl.out_dim, mlora::kExpandBN);
    aligned = aligned && al16(sl.b) && sl.b_slot_stride % vec == 0 && sl.b_row_stride % vec == 0 &&
              al16(static_cast<const char*>(out) + static_cast<int64_t>(sl.out_col) * eb) && sl.out_dim % vec == 0;
  }
  args.tile_base[n_slices] = tiles;

  const int bm = (dtype == MLORA_F32 || meta->max_len <= 16) ? 16 : mlora::kExpandLongBM;
  // A batch mixing long and short segments, with the host's summary of the
  // table: one launch of tiles over the long segments and slot-grouped items
  // over the short ones.  Batches long on average keep the streamed tiles.
  const bool mixed = bm == mlora::kExpandLongBM && aligned && (dtype == MLORA_BF16 || dtype == MLORA_F16) &&
                     meta->long_segs >= 0 && meta->long_rows >= 0 && meta->short_slots > 0 &&
                     meta->num_slots <= mlora::kMixedMaxSlots && r_max <= mlora::kGroupMaxRank && r_max % 8 == 0 &&
                     static_cast<int64_t>(num_rows) < static_cast<int64_t>(mlora::kExpandStreamBM) * meta->bs;
  args.mid = mid;
  args.mid_stride = mid_row_stride;
  args.rows = num_rows;
  args.n_slices = n_slices;
  args.r_max = r_max;
  args.out = out;
  args.out_stride = out_row_stride;
  args.meta = seg_view(meta);
  args.m_tiles = mlora::cdiv(meta->max_len > 0 ? meta->max_len : 1, bm);
  args.cus = num_cus();
  args.n_tiles = tiles;
  args.partials = partials;
  args.ks = ks;
  hipError_t e;
  if (mixed) {
    e = mlora::launch_mixed(args, dtype, meta->long_rows, meta->long_segs, meta->short_slots, num_cus(),
                            static_cast<hipStream_t>(stream));
  } else {
    e = mlora::launch_expand(bm, args, dtype, aligned, static_cast<hipStream_t>(stream));
  }
  if (e != hipSuccess) return hip_fail(e, "expand launch");
  return 0;
}

}  // namespace

extern "C" {

int mlora_abi_version(void) { return 6; }

const char* mlora_last_error(void) { return g_err; }

size_t mlora_shrink_workspace_bytes(int32_t in_dim, int32_t r_max, int32_t n_slices, int32_t num_rows, int32_t bs,
                                    int32_t max_len, int32_t dtype) {
  if (!valid_dtype(dtype)) return 0;
  mlora::ShrinkPlan p;
  if (!mlora::plan_shrink(in_dim, r_max, n_slices, num_rows, bs, max_len, dtype, num_cus(), &p)) return 0;
  return p.ws_bytes;
}

int mlora_shrink(const void* x, int64_t x_row_stride, int32_t num_rows, int32_t in_dim, const mlora_slice* slices,
                 int32_t n_slices, int32_t r_max, int32_t rank_mult, void* mid, int64_t mid_row_stride,
                 const mlora_seg_meta* meta, int32_t dtype, void* workspace, size_t workspace_bytes,
                 void* stream) {
  g_err[0] = '\0';
  return shrink_impl(x, x_row_stride, num_rows, in_dim, slices, n_slices, r_max, rank_mult, mid, mid_row_stride, meta,
                     dtype, workspace, workspace_bytes, false, false, stream);
}

int mlora_expand(const void* mid, int64_t mid_row_stride, int32_t num_rows, const mlora_slice* slices, int32_t n_slices,
                 int32_t r_max, void* out, int64_t out_row_stride, const mlora_seg_meta* meta, int32_t dtype,
                 void* stream) {
  g_err[0] = '\0';
  return expand_impl(mid, mid_row_stride, num_rows, slices, n_slices, r_max, out, out_row_stride, meta, dtype, nullptr,
                     0, stream);
}

size_t mlora_apply_segments_workspace_bytes(int32_t in_dim, int32_t r_max, int32_t n_slices, int32_t num_rows,
                                            int32_t bs, int32_t max_len, int32_t dtype) {
  if (!valid_dtype(dtype) || num_rows < 0 || r_max <= 0 || n_slices < 1) return 0;
  mlora::ShrinkPlan p;
  if (!mlora::plan_shrink(in_dim, r_max, n_slices, num_rows, bs, max_len, dtype, num_cus(), &p)) return 0;
  return mid_region_bytes(num_rows, n_slices, r_max, dtype) + p.ws_bytes;
}

int mlora_apply_segments(const void* x, int64_t x_row_stride, int32_t num_rows, int32_t in_dim,
                         const mlora_slice* slices, int32_t n_slices, int32_t r_max, void* out,
                         int64_t out_row_stride, const mlora_seg_meta* meta, int32_t dtype, void* workspace,
                         size_t workspace_bytes, void* stream) {
  g_err[0] = '\0';
  if (!valid_dtype(dtype)) return fail(kBadArg, "bad dtype %d", dtype);
  if (int rc = check_meta(meta)) return rc;
  if (n_slices < 1 || n_slices > MLORA_MAX_SLICES) return fail(kBadArg, "n_slices %d not in [1, %d]", n_slices, MLORA_MAX_SLICES);
  if (in_dim <= 0 || r_max <= 0 || num_rows < 0) return fail(kBadArg, "in_dim %d, r_max %d, num_rows %d", in_dim, r_max, num_rows);
  if (meta->bs == 0 || num_rows == 0) return 0;
  mlora::ShrinkPlan plan;
  if (!mlora::plan_shrink(in_dim, r_max, n_slices, num_rows, meta->bs, meta->max_len, dtype, num_cus(), &plan))
    return fail(kUnsupported, "shrink shape unsupported: %d slices x r_max %d exceeds 16 blocks of 16 rows",
                n_slices, r_max);
  const size_t mid_bytes = mid_region_bytes(num_rows, n_slices, r_max, dtype);
  if (workspace == nullptr || workspace_bytes < mid_bytes + plan.ws_bytes)
    return fail(kWorkspace, "segment workspace too small: need %zu bytes, got %zu", mid_bytes + plan.ws_bytes,
                workspace_bytes);
  // The expand adds up the split sums itself (no reduce launch, no mid)
  // when K is split, the data is 16-bit, the rank fits its y tile, the batch
  // is not one of long segments (those take the streamed expand, which reads
  // mid), and the output is at most kFuseMaxTiles column tiles wide: every
  // column tile of a row tile adds the same sums again, which costs more
  // than the reduce launch it saves on wide outputs (measured per layer at
  // the 32-layer step: o 20.5 vs 21.8 us, down 32.2 vs 32.9, but gate|up
  // 82.1 vs 64.7; q|k|v, 24 tiles, 25.6 vs 24.3 us with the mixed-batch
  // expand's non-temporal tiles).
  int col_tiles = 0;
  for (int s = 0; s < n_slices && slices != nullptr; ++s) col_tiles += mlora::cdiv(slices[s].out_dim, mlora::kExpandBN);
  const bool long_segments =
      meta->max_len > 16 && static_cast<int64_t>(num_rows) >= static_cast<int64_t>(mlora::kExpandStreamBM) * meta->bs;
  const bool fused = plan.ks > 1 && dtype != MLORA_F32 && r_max <= mlora::kFuseMaxRank && r_max % 4 == 0 &&
                     !long_segments && col_tiles <= mlora::kFuseMaxTiles;
  char* ws = static_cast<char*>(workspace);
  const int64_t mid_stride = static_cast<int64_t>(n_slices) * r_max;
  int rc = shrink_impl(x, x_row_stride, num_rows, in_dim, slices, n_slices, r_max, 1, ws, mid_stride, meta, dtype,
                       ws + mid_bytes, plan.ws_bytes, fused, true, stream);
  if (rc != 0) return rc;
  return expand_impl(ws, mid_stride, num_rows, slices, n_slices, r_max, out, out_row_stride, meta, dtype,
                     fused ? reinterpret_cast<const float*>(ws + mid_bytes) : nullptr, fused ? plan.ks : 0, stream);
}

size_t mlora_grouped_workspace_bytes(int32_t in_dim, int32_t r_max, int32_t n_slices, int32_t num_rows,
                                     int32_t num_slots, int32_t dtype, int32_t mode) {
  (void)num_slots;
  mlora::DecodeShape sh;
  if (mode < 0 || mode > 2) return 0;
  if (!mlora::plan_decode(in_dim, r_max, n_slices, num_rows, dtype, &sh)) return 0;
  return sh.bytes;
}

size_t mlora_plan_bytes(int32_t entries_cap) {
  if (entries_cap < 0) return 0;
  return sizeof(int32_t) * (MLORA_PLAN_HEADER_WORDS + static_cast<size_t>(entries_cap) * MLORA_PLAN_ENTRY_WORDS);
}

int mlora_build_plan(const mlora_seg_meta* meta, int32_t num_rows, int32_t* plan, int32_t plan_cap, void* stream) {
  g_err[0] = '\0';
  if (int rc = check_meta(meta)) return rc;
  if (plan == nullptr || plan_cap < 1 || num_rows < 0)
    return fail(kBadArg, "plan %p, plan_cap %d, num_rows %d", static_cast<void*>(plan), plan_cap, num_rows);
  if (meta->num_slots > mlora::kPlanBuildMaxSlots)
    return fail(kUnsupported, "device plan build takes pools of up to %d slots, got %d", mlora::kPlanBuildMaxSlots,
                meta->num_slots);
  const hipError_t e = mlora::launch_build_plan(seg_view(meta), num_rows, plan, plan_cap, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "plan build launch");
  return 0;
}

// The RMSNorm folded into a grouped call (mlora_rmsnorm_apply_grouped):
// weight of the data dtype, output rows y.
struct NormCall {
  const void* w;
  float eps;
  void* y;
  int64_t y_stride;
};

// RMSNorm arguments of a fused call over the call's rows of x.
static mlora::RmsArgs norm_rms_args(const NormCall& nc, const void* x, int64_t x_row_stride, int32_t num_rows,
                                    int32_t in_dim, int32_t dtype) {
  mlora::RmsArgs a{};
  a.x = x;
  a.x_stride_outer = x_row_stride;
  a.x_stride_inner = x_row_stride;
  a.inner = 1;
  a.w = nc.w;
  a.w_dtype = dtype;
  a.y = nc.y;
  a.y_stride = nc.y_stride;
  a.rows = num_rows;
  a.hidden = in_dim;
  a.eps = nc.eps;
  mlora::rmsnorm_shape(in_dim, dtype, &a.tpr, &a.nc);
  a.aligned = 1;
  a.w_vec = 1;
  return a;
}

// mlora_apply_grouped on a given workspace (the caller's, or the static
// scratch of mlora_apply_grouped_static); with `norm`, the fused RMSNorm
// form (two launches).
static int apply_grouped_impl(const void* x, int64_t x_row_stride, int32_t num_rows, int32_t in_dim,
                              const mlora_slice* slices, int32_t n_slices, int32_t r_max, void* out,
                              int64_t out_row_stride, const mlora_seg_meta* meta, int32_t dtype, void* workspace,
                              size_t workspace_bytes, int32_t mode, int32_t phases, void* stream,
                              const NormCall* norm = nullptr) {
  if (!valid_dtype(dtype)) return fail(kBadArg, "bad dtype %d", dtype);
  if (int rc = check_meta(meta)) return rc;
  if (n_slices < 1 || n_slices > MLORA_MAX_SLICES) return fail(kBadArg, "n_slices %d not in [1, %d]", n_slices, MLORA_MAX_SLICES);
  if (slices == nullptr) return fail(kBadArg, "slices is null");
  if (in_dim <= 0 || r_max <= 0 || num_rows < 0) return fail(kBadArg, "in_dim %d, r_max %d, num_rows %d", in_dim, r_max, num_rows);
  if (x_row_stride < in_dim) return fail(kBadArg, "x row stride %lld < in_dim %d", (long long)x_row_stride, in_dim);
  if (phases < 1 || phases > 3) return fail(kBadArg, "phases %d not in 1..3", phases);
  if (mode < 0 || mode > 2) return fail(kBadArg, "mode %d not in 0..2", mode);
  if (meta->bs == 0 || num_rows == 0 || meta->num_slots == 0) {
    // No LoRA work: the fused call still owes the RMSNorm rows.
    if (norm == nullptr || num_rows == 0 || !(phases & 1)) return 0;
    if (x == nullptr) return fail(kBadArg, "x is null");
    const hipError_t e = mlora::launch_rmsnorm(norm_rms_args(*norm, x, x_row_stride, num_rows, in_dim, dtype), dtype,
                                               static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "rmsnorm launch");
    return 0;
  }
  if (x == nullptr || out == nullptr) return fail(kBadArg, "x or out is null");
  if (mode != mlora::kGroupTwo && phases != 3)
    return fail(kBadArg, "phases %d: only the two-launch mode runs one half (use phases=3)", phases);
  mlora::DecodeShape sh;
  if (!mlora::plan_decode(in_dim, r_max, n_slices, num_rows, dtype, &sh))
    return fail(kUnsupported, "grouped path needs bf16/fp16, r_max <= %d and a multiple of 8, in_dim a multiple of 8",
                mlora::kGroupMaxRank);
  if (workspace == nullptr || workspace_bytes < sh.bytes)
    return fail(kWorkspace, "grouped workspace too small: need %zu bytes, got %zu", sh.bytes, workspace_bytes);
  if (meta->plan == nullptr && meta->num_slots > mlora::kPlanBuildMaxSlots)
    return fail(kUnsupported, "no plan given and the pool has %d slots (the device builder takes up to %d)",
                meta->num_slots, mlora::kPlanBuildMaxSlots);
  const int vec = vec_elems(dtype);
  const int eb = elem_bytes(dtype);
  bool aligned = al16(x) && x_row_stride % vec == 0 && out_row_stride % vec == 0 && al16(workspace);
  mlora::DecodeArgs args{};
  int tiles = 0;
  for (int s = 0; s < n_slices; ++s) {
    const mlora_slice& sl = slices[s];
    if (sl.a == nullptr || sl.b == nullptr) return fail(kBadArg, "slice %d: A or B is null", s);
    if (sl.out_dim <= 0 || sl.out_col < 0) return fail(kBadArg, "slice %d: out_dim %d, out_col %d", s, sl.out_dim, sl.out_col);
    if (static_cast<int64_t>(sl.out_col) + sl.out_dim > out_row_stride)
      return fail(kBadArg, "slice %d: columns [%d, %lld) exceed the output row stride %lld", s, sl.out_col,
                  static_cast<long long>(sl.out_col) + sl.out_dim, (long long)out_row_stride);
    if (sl.a_row_stride < in_dim || sl.a_slot_stride < static_cast<int64_t>(r_max) * sl.a_row_stride ||
        sl.b_row_stride < r_max || sl.b_slot_stride < static_cast<int64_t>(sl.out_dim) * sl.b_row_stride)
      return fail(kBadArg, "slice %d: A/B strides do not hold their [r_max, in] / [out, r_max] rows", s);
    aligned = aligned && al16(sl.a) && sl.a_slot_stride % vec == 0 && sl.a_row_stride % vec == 0 && al16(sl.b) &&
              sl.b_slot_stride % vec == 0 && sl.b_row_stride % vec == 0 && sl.out_dim % vec == 0 &&
              al16(static_cast<const char*>(out) + static_cast<int64_t>(sl.out_col) * eb);
    args.slices[s] = slice_view(sl);
    args.tile_base[s] = tiles;
    tiles += mlora::cdiv(sl.out_dim, mlora::kExpandBN);
  }
  args.tile_base[n_slices] = tiles;
  if (!aligned)
    return fail(kUnsupported, "grouped path needs 16-byte aligned rows (pointers, strides and widths)");
  char* ws = static_cast<char*>(workspace);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int32_t* plan = meta->plan;
  int plan_cap = meta->plan_cap;
  int known = meta->plan_entries;
  if (plan == nullptr) {
    int32_t* built = reinterpret_cast<int32_t*>(ws + sh.plan_off);
    plan_cap = sh.e_cap;
    const hipError_t e = mlora::launch_build_plan(seg_view(meta), num_rows, built, plan_cap, st);
    if (e != hipSuccess) return hip_fail(e, "plan build launch");
    plan = built;
    known = -1;
  }
  // Grid rows: the host's entry count when known, else a bound on it (each
  // slot's rows fill ceil(n / 16) entries).
  if (known < 0) {
    const int64_t bound = mlora::cdiv(num_rows, mlora::kPlanRows) + std::min(meta->bs, meta->num_slots);
    known = static_cast<int>(std::min<int64_t>(num_rows, bound));
  }
  known = std::max(1, std::min(known, std::min(plan_cap, sh.e_cap)));
  args.x = x;
  args.x_stride = x_row_stride;
  args.rows = num_rows;
  args.in_dim = in_dim;
  args.n_slices = n_slices;
  args.r_max = r_max;
  args.out = out;
  args.out_stride = out_row_stride;
  args.num_slots = meta->num_slots;
  args.kc = sh.kc;
  args.k_chunk = sh.k_chunk;
  args.s_groups = sh.s_groups;
  args.n_tiles = tiles;
  args.e_grid = (known + 7) / 8 * 8;
  args.e_cap = sh.e_cap;
  args.plan_cap = plan_cap;
  args.ws_rows = num_rows;
  args.header = reinterpret_cast<int*>(ws);
  args.flags = reinterpret_cast<uint64_t*>(ws + sh.flags_off);
  args.partials = reinterpret_cast<float*>(ws + sh.partials_off);
  // Mode 0: the single launch while its work items fit on the chip about at
  // once; beyond that expand items wait behind shrink items and two launches
  // are faster (q|k|v over 110 entries, 8064 items: 28.5 vs 34.6 us; the
  // 128-token q_proj batch, 1024 items: 7.4 vs 9.1 us).
  if (norm != nullptr) {
    mlora::NormShrinkArgs na{};
    na.rms = norm_rms_args(*norm, x, x_row_stride, num_rows, in_dim, dtype);
    na.rstd = reinterpret_cast<float*>(ws + sh.rstd_off);
    const hipError_t e = mlora::launch_planned_norm(plan, args, na, dtype, sh.nbt, phases, st);
    if (e != hipSuccess) return hip_fail(e, "fused RMSNorm grouped launch");
    return 0;
  }
  int m = mode;
  if (m == mlora::kGroupAuto) {
    const int64_t items = static_cast<int64_t>(args.e_grid) * (sh.s_groups * sh.kc + tiles);
    m = items <= static_cast<int64_t>(mlora::kLinkedItemsPerCu) * num_cus() ? mlora::kGroupLinked : mlora::kGroupTwo;
  }
  const hipError_t e = mlora::launch_planned(plan, args, dtype, sh.nbt, m, phases, st);
  if (e != hipSuccess) return hip_fail(e, "grouped launch");
  return 0;
}

int mlora_apply_grouped(const void* x, int64_t x_row_stride, int32_t num_rows, int32_t in_dim,
                        const mlora_slice* slices, int32_t n_slices, int32_t r_max, void* out,
                        int64_t out_row_stride, const mlora_seg_meta* meta, int32_t dtype, void* workspace,
                        size_t workspace_bytes, int32_t mode, int32_t phases, void* stream) {
  g_err[0] = '\0';
  return apply_grouped_impl(x, x_row_stride, num_rows, in_dim, slices, n_slices, r_max, out, out_row_stride, meta,
                            dtype, workspace, workspace_bytes, mode, phases, stream);
}

int mlora_rmsnorm_apply_grouped(const void* x, int64_t x_row_stride, int32_t num_rows, int32_t in_dim,
                                const void* norm_w, float eps, void* y, int64_t y_row_stride,
                                const mlora_slice* slices, int32_t n_slices, int32_t r_max, void* out,
                                int64_t out_row_stride, const mlora_seg_meta* meta, int32_t dtype, void* workspace,
                                size_t workspace_bytes, int32_t phases, void* stream) {
  g_err[0] = '\0';
  if (dtype != MLORA_BF16 && dtype != MLORA_F16) return fail(kUnsupported, "fused RMSNorm path needs bf16 or fp16, got dtype %d", dtype);
  if (in_dim <= 0 || num_rows < 0) return fail(kBadArg, "in_dim %d, num_rows %d", in_dim, num_rows);
  if (num_rows == 0) return 0;
  if (x == nullptr || norm_w == nullptr || y == nullptr) return fail(kBadArg, "null x, weight or y");
  if (x_row_stride < in_dim || y_row_stride < in_dim)
    return fail(kBadArg, "x / y row strides %lld / %lld below in_dim %d", (long long)x_row_stride,
                (long long)y_row_stride, in_dim);
  const int vec = vec_elems(dtype);
  if (!al16(x) || !al16(y) || !al16(norm_w) || in_dim % vec != 0 || x_row_stride % vec != 0 || y_row_stride % vec != 0)
    return fail(kUnsupported, "fused RMSNorm path needs 16-byte aligned rows of x, y and the weight");
  // The launch that writes y also reads x: the two must not share a byte.
  const int eb = elem_bytes(dtype);
  const uintptr_t x0 = reinterpret_cast<uintptr_t>(x);
  const uintptr_t y0 = reinterpret_cast<uintptr_t>(y);
  const uintptr_t x1 = x0 + static_cast<uintptr_t>((static_cast<int64_t>(num_rows - 1) * x_row_stride + in_dim) * eb);
  const uintptr_t y1 = y0 + static_cast<uintptr_t>((static_cast<int64_t>(num_rows - 1) * y_row_stride + in_dim) * eb);
  if (x0 < y1 && y0 < x1) return fail(kBadArg, "y overlaps x (the fused call reads x while it writes y)");
  const NormCall nc{norm_w, eps, y, y_row_stride};
  return apply_grouped_impl(x, x_row_stride, num_rows, in_dim, slices, n_slices, r_max, out, out_row_stride, meta,
                            dtype, workspace, workspace_bytes, mlora::kGroupTwo, phases, stream, &nc);
}

}  // extern "C"

// ------------------------------------------------------------ static scratch
// Workspace of mlora_apply_grouped_static: device memory the library holds
// for the life of the process, one copy per GPU (zero at load, which is
// what the launch-tagged flags need; never cleared afterwards).
static __device__ __align__(256) unsigned char scratch[MLORA_STATIC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {nullptr};

// The device address of `scratch` on the current device, looked up once per
// device (the host-side name is only a stand-in).  nullptr on failure, with
// the error text set.
void* scratch_ptr() {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    hip_fail(e, "hipGetDevice");
    return nullptr;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    fail(kUnsupported, "device %d beyond the %d the static scratch serves", dev, kMaxDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    // The first call on a device may come while the caller's stream is
    // being captured into a graph, and the lookup may load the code object
    // first.  The thread's capture mode is relaxed around it, so a lookup
    // made under capture is allowed, then restored.
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    const hipError_t ex = hipThreadExchangeStreamCaptureMode(&mode);
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (ex == hipSuccess) (void)hipThreadExchangeStreamCaptureMode(&mode);
    if (e != hipSuccess || p == nullptr) {
      hip_fail(e != hipSuccess ? e : hipErrorInvalidSymbol, "hipGetSymbolAddress(scratch)");
      return nullptr;
    }
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}

}  // namespace

extern "C" {

int mlora_apply_grouped_static(const void* x, int64_t x_row_stride, int32_t num_rows, int32_t in_dim,
                               const mlora_slice* slices, int32_t n_slices, int32_t r_max, void* out,
                               int64_t out_row_stride, const mlora_seg_meta* meta, int32_t dtype, int32_t mode,
                               int32_t phases, void* stream) {
  g_err[0] = '\0';
  const size_t need = mlora_grouped_workspace_bytes(in_dim, r_max, n_slices, num_rows, meta ? meta->num_slots : 0,
                                                    dtype, mode);
  if (need > MLORA_STATIC_SCRATCH_BYTES)
    return fail(kWorkspace, "shape needs %zu bytes of workspace, more than the %d of the static scratch", need,
                MLORA_STATIC_SCRATCH_BYTES);
  void* ws = scratch_ptr();
  if (ws == nullptr) return kUnsupported;
  return apply_grouped_impl(x, x_row_stride, num_rows, in_dim, slices, n_slices, r_max, out, out_row_stride, meta,
                            dtype, ws, MLORA_STATIC_SCRATCH_BYTES, mode, phases, stream);
}

}  // extern "C"

namespace {

int rmsnorm_call(const void* x, int64_t x_stride_outer, int64_t x_stride_inner, int64_t inner, void* residual,
                 int64_t residual_row_stride, const void* w, int32_t w_dtype, void* y, int64_t y_row_stride,
                 int64_t rows, int32_t hidden, float eps, int32_t dtype, void* stream) {
  g_err[0] = '\0';
  if (!valid_dtype(dtype) || !valid_dtype(w_dtype)) return fail(kBadArg, "bad dtype %d / weight dtype %d", dtype, w_dtype);
  if (hidden <= 0 || rows < 0 || inner < 1) return fail(kBadArg, "hidden %d, rows %lld, inner %lld", hidden, (long long)rows, (long long)inner);
  if (y_row_stride < hidden) return fail(kBadArg, "y row stride %lld < hidden %d", (long long)y_row_stride, hidden);
  if (residual != nullptr && residual_row_stride < hidden)
    return fail(kBadArg, "residual row stride %lld < hidden %d", (long long)residual_row_stride, hidden);
  if (rows == 0) return 0;
  if (x == nullptr || w == nullptr || y == nullptr) return fail(kBadArg, "null x, w or y");
  const int vec = vec_elems(dtype);
  mlora::RmsArgs a{};
  a.x = x;
  a.x_stride_outer = x_stride_outer;
  a.x_stride_inner = x_stride_inner;
  a.inner = inner;
  a.w = w;
  a.w_dtype = w_dtype;
  a.y = y;
  a.y_stride = y_row_stride;
  a.rows = rows;
  a.hidden = hidden;
  a.eps = eps;
  mlora::rmsnorm_shape(hidden, dtype, &a.tpr, &a.nc);
  a.aligned = al16(x) && al16(y) && hidden % vec == 0 && x_stride_outer % vec == 0 &&
              x_stride_inner % vec == 0 && y_row_stride % vec == 0 &&
              (residual == nullptr || (al16(residual) && residual_row_stride % vec == 0));
  a.w_vec = (w_dtype == dtype) && al16(w) && hidden % vec == 0;
  a.residual = residual;
  a.residual_stride = residual_row_stride;
  hipError_t e = mlora::launch_rmsnorm(a, dtype, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "rmsnorm launch");
  return 0;
}

}  // namespace

extern "C" {

int mlora_rmsnorm(const void* x, int64_t x_stride_outer, int64_t x_stride_inner, int64_t inner, const void* w,
                  int32_t w_dtype, void* y, int64_t y_row_stride, int64_t rows, int32_t hidden, float eps,
                  int32_t dtype, void* stream) {
  return rmsnorm_call(x, x_stride_outer, x_stride_inner, inner, nullptr, 0, w, w_dtype, y, y_row_stride, rows,
                      hidden, eps, dtype, stream);
}

int mlora_add_rmsnorm(const void* x, int64_t x_row_stride, void* residual, int64_t residual_row_stride,
                      const void* w, int32_t w_dtype, void* y, int64_t y_row_stride, int64_t rows, int32_t hidden,
                      float eps, int32_t dtype, void* stream) {
  if (residual == nullptr && rows > 0) {
    g_err[0] = '\0';
    return fail(kBadArg, "null residual");
  }
  return rmsnorm_call(x, x_row_stride, x_row_stride, 1, residual, residual_row_stride, w, w_dtype, y, y_row_stride,
                      rows, hidden, eps, dtype, stream);
}

int mlora_pool_scatter(const void* stage, int64_t stage_row_stride, int32_t h, const int32_t* slots,
                       const mlora_pool_key* keys, int32_t n_keys, int32_t rank, int32_t num_slots,
                       int64_t max_numel, int32_t dtype, void* stream) {
  g_err[0] = '\0';
  if (!valid_dtype(dtype)) return fail(kBadArg, "bad dtype %d", dtype);
  if (h < 0 || n_keys < 0 || rank < 1 || num_slots < 0 || max_numel < 0)
    return fail(kBadArg, "h %d, n_keys %d, rank %d, num_slots %d, max_numel %lld", h, n_keys, rank, num_slots,
                (long long)max_numel);
  if (h == 0 || n_keys == 0 || max_numel == 0) return 0;
  if (stage == nullptr || slots == nullptr || keys == nullptr) return fail(kBadArg, "null stage, slots or keys");
  if (static_cast<int64_t>(n_keys) * h > 65535)
    return fail(kBadArg, "n_keys * h = %lld above 65535", static_cast<long long>(n_keys) * h);
  const int eb = elem_bytes(dtype);
  mlora::ScatterArgs a{};
  a.stage = stage;
  a.stage_stride = stage_row_stride;
  a.h = h;
  a.slots = slots;
  a.keys = keys;
  a.n_keys = n_keys;
  a.rank = rank;
  a.num_slots = num_slots;
  a.vec = al16(stage) && (stage_row_stride * eb) % 16 == 0;
  const hipError_t e = mlora::launch_scatter(a, max_numel, eb, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "pool scatter launch");
  return 0;
}

}  // extern "C"
