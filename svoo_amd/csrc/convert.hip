// Element-type conversion at the operator boundary.  The hot path computes in bf16 (the MFMA operand type of
// every kernel here) on rows of 128 elements; fp16 and fp32 inputs are rounded to bf16 (to nearest even, through
// fp32, which holds both exactly), rows of a smaller head dim are padded with zeros, and results go back to the
// caller's type and row width.  One element per lane, grid-stride: the loads and stores of a wave are contiguous.
#include "svoo_common.h"

namespace svoo {

enum ElemType { kElemBf16 = 0, kElemF16 = 1, kElemF32 = 2 };

template <int S>
__device__ __forceinline__ float load_elem(const void* __restrict__ p, long long i) {
  if (S == kElemBf16) return bf16_to_f32(((const uint16_t*)p)[i]);
  if (S == kElemF16) return (float)__builtin_bit_cast(_Float16, ((const uint16_t*)p)[i]);
  return ((const float*)p)[i];
}

template <int D>
__device__ __forceinline__ void store_elem(void* __restrict__ p, long long i, float v) {
  if (D == kElemBf16) ((uint16_t*)p)[i] = f32_to_bf16(v);
  else if (D == kElemF16) ((uint16_t*)p)[i] = __builtin_bit_cast(uint16_t, (_Float16)v);
  else ((float*)p)[i] = v;
}

template <int S, int D>
__global__ void __launch_bounds__(256) convert_kernel(const void* __restrict__ src, void* __restrict__ dst,
                                                      long long n) {
  const long long stride = (long long)gridDim.x * blockDim.x;
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    store_elem<D>(dst, i, load_elem<S>(src, i));
}

// Rows of src_cols elements to rows of dst_cols: the first min(src_cols, dst_cols) converted, the rest zero.
template <int S, int D>
__global__ void __launch_bounds__(256) convert_rows_kernel(const void* __restrict__ src, int src_cols,
                                                           void* __restrict__ dst, int dst_cols, long long n) {
  const long long stride = (long long)gridDim.x * blockDim.x;
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const long long r = i / dst_cols;
    const int c = (int)(i - r * dst_cols);
    store_elem<D>(dst, i, c < src_cols ? load_elem<S>(src, r * src_cols + c) : 0.0f);
  }
}

template <int S>
static void launch_rows_from(const void* src, int src_cols, int dst_type, void* dst, int dst_cols, long long n,
                             unsigned blocks, hipStream_t s) {
  if (dst_type == kElemBf16)
    hipLaunchKernelGGL((convert_rows_kernel<S, kElemBf16>), dim3(blocks), dim3(256), 0, s, src, src_cols, dst, dst_cols, n);
  else if (dst_type == kElemF16)
    hipLaunchKernelGGL((convert_rows_kernel<S, kElemF16>), dim3(blocks), dim3(256), 0, s, src, src_cols, dst, dst_cols, n);
  else
    hipLaunchKernelGGL((convert_rows_kernel<S, kElemF32>), dim3(blocks), dim3(256), 0, s, src, src_cols, dst, dst_cols, n);
}

template <int S>
static void launch_from(const void* src, int dst_type, void* dst, long long n, unsigned blocks, hipStream_t s) {
  if (dst_type == kElemBf16) hipLaunchKernelGGL((convert_kernel<S, kElemBf16>), dim3(blocks), dim3(256), 0, s, src, dst, n);
  else if (dst_type == kElemF16) hipLaunchKernelGGL((convert_kernel<S, kElemF16>), dim3(blocks), dim3(256), 0, s, src, dst, n);
  else hipLaunchKernelGGL((convert_kernel<S, kElemF32>), dim3(blocks), dim3(256), 0, s, src, dst, n);
}

}  // namespace svoo

using namespace svoo;

extern "C" int svoo_convert(const void* src, int src_type, void* dst, int dst_type, long long n, void* stream) {
  SVOO_REQUIRE(src_type >= kElemBf16 && src_type <= kElemF32 && dst_type >= kElemBf16 && dst_type <= kElemF32,
               SVOO_ERR_INVALID_ARG, "svoo_convert: element types %d -> %d (0 bf16, 1 fp16, 2 fp32)", src_type,
               dst_type);
  SVOO_REQUIRE(n >= 0, SVOO_ERR_INVALID_ARG, "svoo_convert: n=%lld", n);
  if (n == 0) return SVOO_OK;
  SVOO_REQUIRE(src && dst, SVOO_ERR_INVALID_ARG, "svoo_convert: null pointer");
  const long long want = (n + 255) / 256;
  const unsigned blocks = (unsigned)(want < 65536 ? want : 65536);
  hipStream_t s = (hipStream_t)stream;
  if (src_type == kElemBf16) launch_from<kElemBf16>(src, dst_type, dst, n, blocks, s);
  else if (src_type == kElemF16) launch_from<kElemF16>(src, dst_type, dst, n, blocks, s);
  else launch_from<kElemF32>(src, dst_type, dst, n, blocks, s);
  return check_launch("svoo_convert");
}

extern "C" int svoo_convert_rows(const void* src, int src_type, int src_cols, void* dst, int dst_type, int dst_cols,
                                 long long rows, void* stream) {
  SVOO_REQUIRE(src_type >= kElemBf16 && src_type <= kElemF32 && dst_type >= kElemBf16 && dst_type <= kElemF32,
               SVOO_ERR_INVALID_ARG, "svoo_convert_rows: element types %d -> %d (0 bf16, 1 fp16, 2 fp32)", src_type,
               dst_type);
  SVOO_REQUIRE(rows >= 0 && src_cols > 0 && dst_cols > 0, SVOO_ERR_INVALID_ARG,
               "svoo_convert_rows: rows=%lld src_cols=%d dst_cols=%d", rows, src_cols, dst_cols);
  const long long n = rows * dst_cols;
  if (n == 0) return SVOO_OK;
  SVOO_REQUIRE(src && dst, SVOO_ERR_INVALID_ARG, "svoo_convert_rows: null pointer");
  const long long want = (n + 255) / 256;
  const unsigned blocks = (unsigned)(want < 65536 ? want : 65536);
  hipStream_t s = (hipStream_t)stream;
  if (src_type == kElemBf16) launch_rows_from<kElemBf16>(src, src_cols, dst_type, dst, dst_cols, n, blocks, s);
  else if (src_type == kElemF16) launch_rows_from<kElemF16>(src, src_cols, dst_type, dst, dst_cols, n, blocks, s);
  else launch_rows_from<kElemF32>(src, src_cols, dst_type, dst, dst_cols, n, blocks, s);
  return check_launch("svoo_convert_rows");
}
