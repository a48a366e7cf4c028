// The RMSNorm rows of one workgroup, shared by the RMSNorm kernel and the
// norm workgroups of the fused RMSNorm + decode shrink launch, so both write
// the same bits: y = round(x * rsqrt(mean(x^2) + eps) * w), fp32 math and a
// single rounding, as the reference kernel computes it
// (multi_lora/kernels/rmsnorm.py:17-45).  With a residual row (ADD) the rows
// first form h = round(x + residual), store h back to the residual and
// normalise h: the residual add and the next RMSNorm of a decoder layer in
// one pass, the fusion the reference plans (OPTIMIZATION_TODO.md T22).  Rows
// may be addressed with the reference's two-level stride (rmsnorm.py:56-75):
// row r starts at (r / inner) * stride_outer + (r % inner) * stride_inner.
//
// `tpr` threads cooperate on one row (a power of two from 16 to 256), each
// holding `nc` (at most NC: 1, 2, 4 or 8) 16-byte chunks of the row and of
// the weight in registers, requested together, so x is read from HBM once.
// The sum of squares is reduced with xor shuffles inside the wave and, for
// rows wider than one wave, through LDS.
#pragma once

#include "kernels.h"
#include "loads.h"

namespace mlora {

// Weight chunk `c` as floats: one 16-byte load when the weight has the data
// type of x and is 16-byte aligned (WV), else element by element.
template <class T, bool WV>
__device__ __forceinline__ void weight_chunk(const RmsArgs& a, int c, float (&wf)[T::VEC]) {
  constexpr int VEC = T::VEC;
  if constexpr (WV) {
    const u32x4 v = load_row_chunk<T, true>(static_cast<const typename T::raw_t*>(a.w), c * VEC, a.hidden - c * VEC);
#pragma unroll
    for (int e = 0; e < VEC; ++e) wf[e] = chunk_elem<T>(v, e);
  } else {
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const int col = c * VEC + e;
      wf[e] = (col < a.hidden) ? load_scaling(a.w, col, a.w_dtype) : 0.f;
    }
  }
}

// x + residual rounded to the storage type (what an unfused bf16/fp16 add
// stores), written back to the residual row when ADD.
template <class T>
__device__ __forceinline__ u32x4 add_chunk(const u32x4& x, const u32x4& r) {
  float f[T::VEC];
#pragma unroll
  for (int e = 0; e < T::VEC; ++e) f[e] = chunk_elem<T>(x, e) + chunk_elem<T>(r, e);
  return pack_chunk<T>(f);
}

// The 256 / tpr rows of row block `block` (256 threads; every thread calls
// it).  `red`: 4 floats of LDS.  nc <= NC chunks a thread are held in
// registers (the RMSNorm kernel passes NC itself); rows wider than tpr * nc
// chunks stream the rest a second time.  RSTD: each row's
// rsqrt(mean(x^2) + eps) also goes to rstd_out[row].
template <class T, int NC, bool AL, bool WV, bool ADD, bool RSTD = false>
__device__ __forceinline__ void rmsnorm_block(const RmsArgs& a, int64_t block, float* red, int nc = NC,
                                              float* rstd_out = nullptr) {
  using raw = typename T::raw_t;
  constexpr int VEC = T::VEC;
  const int tid = threadIdx.x;
  const int tpr = a.tpr;
  const int rpb = 256 / tpr;
  const int lr = tid / tpr;
  const int li = tid - lr * tpr;
  const int64_t row = block * rpb + lr;
  const bool row_ok = row < a.rows;
  const int hidden = a.hidden;
  const int nch = (hidden + VEC - 1) / VEC;
  const raw* x = static_cast<const raw*>(a.x);
  const int64_t r = row_ok ? row : 0;
  const raw* xrow = x + (r / a.inner) * a.x_stride_outer + (r % a.inner) * a.x_stride_inner;
  raw* rrow = ADD ? static_cast<raw*>(a.residual) + r * a.residual_stride : nullptr;

  // The row's chunks and the matching weight chunks, all requested at once
  // (a weight of x's dtype stays in its 16-byte chunks until it is used).
  u32x4 cache[NC];
  u32x4 wraw[WV ? NC : 1];
  float wf[WV ? 1 : NC][VEC];
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    if (j >= nc) break;
    const int c = li + j * tpr;
    cache[j] = load_row_chunk<T, AL>(xrow, c * VEC, (row_ok && c < nch) ? hidden - c * VEC : 0);
  }
  // The weight chunks go out with the row's, before the add waits for them
  // (fused add + RMSNorm at 1088 x 4096: 9.9 vs 10.2 us).
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    if (j >= nc) break;
    const int c = li + j * tpr;
    if constexpr (WV)
      wraw[j] = load_row_chunk<T, true>(static_cast<const raw*>(a.w), c * VEC, hidden - c * VEC);
    else
      weight_chunk<T, WV>(a, c, wf[j]);
  }
  if constexpr (ADD) {
    u32x4 res[NC];
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      if (j >= nc) break;
      const int c = li + j * tpr;
      res[j] = load_row_chunk<T, AL>(rrow, c * VEC, (row_ok && c < nch) ? hidden - c * VEC : 0);
    }
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      if (j >= nc) break;
      const int c = li + j * tpr;
      cache[j] = add_chunk<T>(cache[j], res[j]);
      if (row_ok && c < nch) store_row_chunk<T, AL>(rrow + c * VEC, cache[j], hidden - c * VEC);
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    if (j >= nc) break;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float v = chunk_elem<T>(cache[j], e);
      ss += v * v;
    }
  }
  for (int c = li + nc * tpr; row_ok && c < nch; c += tpr) {
    u32x4 v = load_row_chunk<T, AL>(xrow, c * VEC, hidden - c * VEC);
    if constexpr (ADD) {
      v = add_chunk<T>(v, load_row_chunk<T, AL>(rrow, c * VEC, hidden - c * VEC));
      store_row_chunk<T, AL>(rrow + c * VEC, v, hidden - c * VEC);
    }
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
  if constexpr (RSTD) {
    if (li == 0) rstd_out[row] = rstd;
  }
  raw* yrow = static_cast<raw*>(a.y) + row * a.y_stride;
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    if (j >= nc) break;
    const int c = li + j * tpr;
    if (c >= nch) break;
    float f[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      float we;
      if constexpr (WV)
        we = chunk_elem<T>(wraw[j], e);
      else
        we = wf[j][e];
      f[e] = chunk_elem<T>(cache[j], e) * rstd * we;
    }
    store_row_chunk<T, AL>(yrow + c * VEC, pack_chunk<T>(f), hidden - c * VEC);
  }
  for (int c = li + nc * tpr; c < nch; c += tpr) {
    // Chunks past the cached ones: the sum was stored to the residual row
    // by this same thread in the first pass.
    const u32x4 v = ADD ? load_row_chunk<T, AL>(rrow, c * VEC, hidden - c * VEC)
                        : load_row_chunk<T, AL>(xrow, c * VEC, hidden - c * VEC);
    float w1[VEC];
    weight_chunk<T, WV>(a, c, w1);
    float f[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) f[e] = chunk_elem<T>(v, e) * rstd * w1[e];
    store_row_chunk<T, AL>(yrow + c * VEC, pack_chunk<T>(f), hidden - c * VEC);
  }
}

}  // namespace mlora
