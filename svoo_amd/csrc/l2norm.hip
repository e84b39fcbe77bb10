// Row L2 normalisation to fp32: y = x / sqrt(sum(x^2) + eps), one wave per row.
#include "svoo_common.h"

namespace svoo {

template <bool kBf16>
__global__ void __launch_bounds__(256) l2norm_rows_kernel(const void* __restrict__ x, float* __restrict__ y,
                                                          long long rows, int cols, float eps) {
  const long long row = (long long)blockIdx.x * 4 + threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  if (row >= rows) return;
  float s = 0.0f;
  for (int c = lane; c < cols; c += kWave) {
    const float v = kBf16 ? bf16_to_f32(((const uint16_t*)x)[row * cols + c]) : ((const float*)x)[row * cols + c];
    s = fmaf(v, v, s);
  }
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
  const float nrm = sqrtf(s + eps);
  for (int c = lane; c < cols; c += kWave) {
    const float v = kBf16 ? bf16_to_f32(((const uint16_t*)x)[row * cols + c]) : ((const float*)x)[row * cols + c];
    y[row * cols + c] = v / nrm;
  }
}

}  // namespace svoo

using namespace svoo;

extern "C" int svoo_l2norm_rows(const void* x, int x_is_bf16, float* y, long long rows, int cols, float eps,
                                void* stream) {
  SVOO_REQUIRE(x && y, SVOO_ERR_INVALID_ARG, "svoo_l2norm_rows: null pointer");
  SVOO_REQUIRE(rows >= 0 && cols > 0, SVOO_ERR_INVALID_ARG, "svoo_l2norm_rows: bad dims");
  if (rows == 0) return SVOO_OK;
  SVOO_REQUIRE((rows + 3) / 4 <= 2147483647ll, SVOO_ERR_UNSUPPORTED, "svoo_l2norm_rows: too many rows");
  dim3 grid((unsigned)((rows + 3) / 4));
  if (x_is_bf16)
    hipLaunchKernelGGL(l2norm_rows_kernel<true>, grid, dim3(256), 0, (hipStream_t)stream, x, y, rows, cols, eps);
  else
    hipLaunchKernelGGL(l2norm_rows_kernel<false>, grid, dim3(256), 0, (hipStream_t)stream, x, y, rows, cols, eps);
  return check_launch("svoo_l2norm_rows");
}
