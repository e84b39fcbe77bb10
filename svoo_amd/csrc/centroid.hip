// Centroid update over cluster-sorted tokens.
//
// accumulate: each wave owns 256 consecutive sorted positions.  Labels are non-decreasing along
//   sorted positions, so the wave walks its rows in order, keeping two fp64 partial sums per lane
//   (lane l owns dims 2l, 2l+1 of a 128-dim row) and flushing them with one fp64 atomicAdd per
//   lane whenever the label changes.  Sums of bf16 values are exact in fp64, so the result does
//   not depend on the order of the atomics.  Rows are fetched 8 at a time for memory parallelism.
// finalize: centroid = bf16(f32(sum) / f32(size)), size 0 keeps the old centroid; the sum buffer
//   is cleared on the way out so the next update starts from zero.
#include "svoo_common.h"

namespace svoo {

constexpr int kCentPosPerWave = 128;
constexpr int kCentUnroll = 8;

__global__ void __launch_bounds__(256) centroid_accumulate_kernel(const uint32_t* __restrict__ x,
                                                                  const int32_t* __restrict__ sorted_idx,
                                                                  const int32_t* __restrict__ sorted_labels,
                                                                  double* __restrict__ sums, int n, int k) {
  // D = 128 fixed: a row is 64 uint32 words (bf16 pairs), one per lane.
  const int b = blockIdx.y;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int p0 = (blockIdx.x * (blockDim.x / kWave) + wave) * kCentPosPerWave;
  if (p0 >= n) return;
  const int p1 = min(n, p0 + kCentPosPerWave);
  const int32_t* si = sorted_idx + (size_t)b * n;
  const int32_t* sl = sorted_labels + (size_t)b * n;
  const uint32_t* xb = x + (size_t)b * n * 64;
  double* sb = sums + (size_t)b * k * 128;
  int cur = sl[p0];
  double a0 = 0.0, a1 = 0.0;
  for (int p = p0; p < p1; p += kCentUnroll) {
    uint32_t w[kCentUnroll];
    int lab[kCentUnroll];
#pragma unroll
    for (int u = 0; u < kCentUnroll; ++u) {
      const int q = min(p + u, p1 - 1);
      lab[u] = sl[q];
      const int src = si[q];
      w[u] = ((unsigned)src < (unsigned)n) ? xb[(size_t)src * 64 + lane] : 0u;
    }
#pragma unroll
    for (int u = 0; u < kCentUnroll; ++u) {
      if (p + u >= p1) break;
      if (lab[u] != cur) {
        if ((unsigned)cur < (unsigned)k) {
          atomicAdd(&sb[(size_t)cur * 128 + 2 * lane], a0);
          atomicAdd(&sb[(size_t)cur * 128 + 2 * lane + 1], a1);
        }
        a0 = 0.0;
        a1 = 0.0;
        cur = lab[u];
      }
      a0 += (double)bf16_to_f32((uint16_t)(w[u] & 0xffffu));
      a1 += (double)bf16_to_f32((uint16_t)(w[u] >> 16));
    }
  }
  if ((unsigned)cur < (unsigned)k) {
    atomicAdd(&sb[(size_t)cur * 128 + 2 * lane], a0);
    atomicAdd(&sb[(size_t)cur * 128 + 2 * lane + 1], a1);
  }
}

__global__ void __launch_bounds__(256) centroid_finalize_kernel(double* __restrict__ sums,
                                                                const int32_t* __restrict__ sizes,
                                                                const uint16_t* old_c, uint16_t* new_c,
                                                                long long total, int d) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const long long row = i / d;
  const int cnt = sizes[row];
  const double s = sums[i];
  sums[i] = 0.0;
  if (cnt > 0) {
    const float mean = (float)s / (float)cnt;
    new_c[i] = f32_to_bf16(mean);
  } else {
    new_c[i] = old_c[i];
  }
}

__global__ void zero_f64_kernel(double* __restrict__ p, long long n) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.0;
}

}  // namespace svoo

using namespace svoo;

int svoo_zero_f64(double* p, long long n, hipStream_t stream) {
  if (n <= 0) return SVOO_OK;
  hipLaunchKernelGGL(zero_f64_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, p, n);
  return check_launch("zero_f64");
}

// sums must be zero on entry; it is zero again on return.
int svoo_centroid_update_impl(const uint16_t* x, const int32_t* sorted_idx, const int32_t* sorted_labels,
                              const int32_t* sizes, const uint16_t* old_c, uint16_t* new_c, int bh, int n, int k,
                              double* sums, hipStream_t stream) {
  const int waves_per_block = 4;
  const int pos_per_block = waves_per_block * kCentPosPerWave;
  dim3 grid((n + pos_per_block - 1) / pos_per_block, bh);
  hipLaunchKernelGGL(centroid_accumulate_kernel, grid, dim3(256), 0, stream, (const uint32_t*)x, sorted_idx,
                     sorted_labels, sums, n, k);
  const long long total = (long long)bh * k * 128;
  hipLaunchKernelGGL(centroid_finalize_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, sums,
                     sizes, old_c, new_c, total, 128);
  return check_launch("svoo_centroid_update");
}

extern "C" size_t svoo_centroid_update_workspace_size(int bh, int k, int d) {
  if (bh <= 0 || k <= 0 || d <= 0) return 256;
  return (size_t)bh * k * d * sizeof(double) + 256;
}

extern "C" int svoo_centroid_update(const uint16_t* x, const int32_t* sorted_idx, const int32_t* sorted_labels,
                                    const int32_t* sizes, const uint16_t* old_c, uint16_t* new_c, int bh, int n,
                                    int k, int d, void* workspace, size_t ws_bytes, void* stream) {
  SVOO_REQUIRE(x && sorted_idx && sorted_labels && sizes && old_c && new_c, SVOO_ERR_INVALID_ARG,
               "svoo_centroid_update: null pointer");
  SVOO_REQUIRE(bh > 0 && n > 0 && k > 0, SVOO_ERR_INVALID_ARG, "svoo_centroid_update: bad dims");
  SVOO_REQUIRE(d == 128, SVOO_ERR_UNSUPPORTED, "svoo_centroid_update: D=%d (only 128 supported)", d);
  SVOO_REQUIRE(bh <= 65535, SVOO_ERR_UNSUPPORTED, "svoo_centroid_update: bh too large");
  const size_t need = svoo_centroid_update_workspace_size(bh, k, d);
  SVOO_REQUIRE(workspace && ws_bytes >= need, SVOO_ERR_WORKSPACE, "svoo_centroid_update: workspace %zu < %zu",
               ws_bytes, need);
  hipStream_t s = (hipStream_t)stream;
  double* sums = (double*)workspace;
  if (int rc = svoo_zero_f64(sums, (long long)bh * k * d, s)) return rc;
  return svoo_centroid_update_impl(x, sorted_idx, sorted_labels, sizes, old_c, new_c, bh, n, k, sums, s);
}
