// Fused RMSNorm on gfx950: y = round(x * rsqrt(mean(x^2) + eps) * w), fp32
// math and a single rounding, as the reference kernel computes it
// (multi_lora/kernels/rmsnorm.py:17-45).  Rows may be addressed with the
// reference's two-level stride (rmsnorm.py:56-75): row r starts at
// (r / inner) * stride_outer + (r % inner) * stride_inner.
//
// `tpr` threads cooperate on one row (a power of two from 16 to 256), each
// holding up to 8 16-byte chunks of the row in registers so x is read from
// HBM once.  The sum of squares is reduced with xor shuffles inside the wave
// and, for rows wider than one wave, through LDS.
#include "kernels.h"
#include "loads.h"

namespace mlora {

namespace {

constexpr int kMaxCached = 8;

__device__ __forceinline__ float load_w(const void* w, int dtype, int idx) {
  return load_scaling(w, idx, dtype);
}

template <class T, bool AL>
__global__ __launch_bounds__(256) void rmsnorm_kernel(RmsArgs a) {
  using raw = typename T::raw_t;
  constexpr int VEC = T::VEC;
  __shared__ float red[4];

  const int tid = threadIdx.x;
  const int tpr = a.tpr;
  const int rpb = 256 / tpr;
  const int lr = tid / tpr;
  const int li = tid - lr * tpr;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * rpb + lr;
  const bool row_ok = row < a.rows;
  const int hidden = a.hidden;
  const int nch = (hidden + VEC - 1) / VEC;

  const raw* x = static_cast<const raw*>(a.x);
  const int64_t r = row_ok ? row : 0;
  const raw* xrow = x + (r / a.inner) * a.x_stride_outer + (r % a.inner) * a.x_stride_inner;

  u32x4 cache[kMaxCached];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < kMaxCached; ++j) {
    const int c = li + j * tpr;
    cache[j] = load_row_chunk<T, AL>(xrow, c * VEC, (row_ok && c < nch) ? hidden - c * VEC : 0);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float v = chunk_elem<T>(cache[j], e);
      ss += v * v;
    }
  }
  for (int c = li + kMaxCached * tpr; row_ok && c < nch; c += tpr) {
    const u32x4 v = load_row_chunk<T, AL>(xrow, c * VEC, hidden - c * VEC);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float f = chunk_elem<T>(v, e);
      ss += f * f;
    }
  }

  const int width = tpr < kWave ? tpr : kWave;
  for (int off = 1; off < width; off <<= 1) ss += __shfl_xor(ss, off, kWave);
  if (tpr > kWave) {
    const int wave = tid >> 6;
    if ((tid & 63) == 0) red[wave] = ss;
    __syncthreads();
    const int wpr = tpr / kWave;
    const int w0 = (wave / wpr) * wpr;
    ss = 0.f;
    for (int w = 0; w < wpr; ++w) ss += red[w0 + w];
  }
  if (!row_ok) return;

  const float rstd = rsqrtf(ss / static_cast<float>(hidden) + a.eps);
  raw* yrow = static_cast<raw*>(a.y) + row * a.y_stride;
  auto emit = [&](int c, const u32x4& v) {
    float f[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const int col = c * VEC + e;
      const float wv = (col < hidden) ? load_w(a.w, a.w_dtype, col) : 0.f;
      f[e] = chunk_elem<T>(v, e) * rstd * wv;
    }
    store_row_chunk<T, AL>(yrow + c * VEC, pack_chunk<T>(f), hidden - c * VEC);
  };
#pragma unroll
  for (int j = 0; j < kMaxCached; ++j) {
    const int c = li + j * tpr;
    if (c < nch) emit(c, cache[j]);
  }
  for (int c = li + kMaxCached * tpr; c < nch; c += tpr)
    emit(c, load_row_chunk<T, AL>(xrow, c * VEC, hidden - c * VEC));
}

template <class T>
hipError_t launch_t(const RmsArgs& args, hipStream_t stream) {
  const int rpb = 256 / args.tpr;
  const int64_t blocks = (args.rows + rpb - 1) / rpb;
  if (blocks <= 0) return hipSuccess;
  if (args.aligned)
    hipLaunchKernelGGL((rmsnorm_kernel<T, true>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, args);
  else
    hipLaunchKernelGGL((rmsnorm_kernel<T, false>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, args);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_rmsnorm(RmsArgs args, int dtype, hipStream_t stream) {
  switch (dtype) {
    case MLORA_BF16: return launch_t<BF16>(args, stream);
    case MLORA_F16: return launch_t<F16>(args, stream);
    default: return launch_t<F32>(args, stream);
  }
}

}  // namespace mlora
