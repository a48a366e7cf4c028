// Fused RMSNorm on gfx950: y = round(x * rsqrt(mean(x^2) + eps) * w), fp32
// math and a single rounding, optionally after the residual add of a decoder
// layer; the row body (rmsnorm_block) is in rmsnorm_row.h, shared with the
// norm workgroups of the fused RMSNorm + decode shrink launch.
#include "rmsnorm_row.h"

namespace mlora {

namespace {

template <class T, int NC, bool AL, bool WV, bool ADD>
__global__ __launch_bounds__(256) void rmsnorm_kernel(RmsArgs a) {
  __shared__ float red[4];
  rmsnorm_block<T, NC, AL, WV, ADD>(a, blockIdx.x, red);
}

template <class T, int NC, bool AL, bool ADD>
hipError_t launch_w(const RmsArgs& args, dim3 grid, hipStream_t stream) {
  if (args.w_vec)
    hipLaunchKernelGGL((rmsnorm_kernel<T, NC, AL, true, ADD>), grid, dim3(256), 0, stream, args);
  else
    hipLaunchKernelGGL((rmsnorm_kernel<T, NC, AL, false, ADD>), grid, dim3(256), 0, stream, args);
  return hipGetLastError();
}

template <class T, int NC, bool AL>
hipError_t launch_add(const RmsArgs& args, dim3 grid, hipStream_t stream) {
  return args.residual ? launch_w<T, NC, AL, true>(args, grid, stream) : launch_w<T, NC, AL, false>(args, grid, stream);
}

template <class T, int NC>
hipError_t launch_nc(const RmsArgs& args, dim3 grid, hipStream_t stream) {
  return args.aligned ? launch_add<T, NC, true>(args, grid, stream) : launch_add<T, NC, false>(args, grid, stream);
}

template <class T>
hipError_t launch_t(const RmsArgs& args, hipStream_t stream) {
  const int rpb = 256 / args.tpr;
  const int64_t blocks = (args.rows + rpb - 1) / rpb;
  if (blocks <= 0) return hipSuccess;
  if (!grid_fits(blocks)) return hipErrorInvalidConfiguration;
  const dim3 grid(static_cast<unsigned>(blocks));
  switch (args.nc) {
    case 1: return launch_nc<T, 1>(args, grid, stream);
    case 2: return launch_nc<T, 2>(args, grid, stream);
    case 4: return launch_nc<T, 4>(args, grid, stream);
    default: return launch_nc<T, 8>(args, grid, stream);
  }
}

}  // namespace

void rmsnorm_shape(int hidden, int dtype, int* tpr, int* nc) {
  const int nch = cdiv(hidden, dtype == MLORA_F32 ? F32::VEC : BF16::VEC);
  int t = 16;
  while (t < 256 && t * 2 <= nch) t *= 2;
  int n = 1;
  while (n < 8 && n * t < nch) n *= 2;
  *tpr = t;
  *nc = n;
}

hipError_t launch_rmsnorm(RmsArgs args, int dtype, hipStream_t stream) {
  switch (dtype) {
    case MLORA_BF16: return launch_t<BF16>(args, stream);
    case MLORA_F16: return launch_t<F16>(args, stream);
    default: return launch_t<F32>(args, stream);
  }
}

}  // namespace mlora
