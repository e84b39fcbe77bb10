// Block-mask builder: one 256-thread block per (b, h, q-cluster) row.
//
//   s_j  = bf16(f32(Qc_i . Kc_j))            exact fp64 dot, rounded as a bf16 matmul output
//   t_j  = bf16(f32(s_j) * f32(1/sqrt(D)))   the reference's "/ D**0.5" on a bf16 tensor
//   p_j  = bf16(f32(w_j e^(t_j - max) / max(sum, 1e-12)))   weighted softmax, evaluated in fp64
//   sort (p desc, j asc) with a bitonic network on packed 32-bit keys in LDS
//   prefix_t = sum_{u<=t} floor(p_u * 2^60)  (exact int64 scan) -> bf16 -> compared with bf16(top_p)
//   kept length L = max(1 + #{t <= Kc-2 : prefix_t <= p}, preserve_h), capped by cap_h
// and the first L sorted clusters are written back as 1 in the bool map.
#include "svoo_common.h"

namespace svoo {

constexpr int kMaskThreads = 256;

template <int KP>
__global__ void __launch_bounds__(kMaskThreads) block_mask_kernel(const uint16_t* __restrict__ qc,
                                                                  const uint16_t* __restrict__ kc,
                                                                  const int32_t* __restrict__ ksz,
                                                                  const int32_t* __restrict__ preserve,
                                                                  const int32_t* __restrict__ cap, int h, int qn,
                                                                  int kn, float inv_sqrt_d, float p_st, int full,
                                                                  uint8_t* __restrict__ map,
                                                                  int32_t* __restrict__ lengths) {
  constexpr int E = KP / kMaskThreads;  // entries per thread
  __shared__ double qrow[128];
  __shared__ float tv[KP];
  __shared__ uint32_t keys[KP];
  __shared__ double red_d[kMaskThreads / kWave];
  __shared__ float red_f[kMaskThreads / kWave];
  __shared__ long long red_l[kMaskThreads / kWave];
  __shared__ int red_i[kMaskThreads / kWave];

  const int bh = blockIdx.y, i = blockIdx.x, tid = threadIdx.x;
  const int head = bh % h;
  uint8_t* mrow = map + ((size_t)bh * qn + i) * kn;
  if (full) {
    for (int j = tid; j < kn; j += kMaskThreads) mrow[j] = 1;
    if (tid == 0 && lengths) lengths[(size_t)bh * qn + i] = kn;
    return;
  }
  if (tid < 128) qrow[tid] = (double)bf16_to_f32(qc[((size_t)bh * qn + i) * 128 + tid]);
  __syncthreads();

  // Scores and row max.
  float lmax = -INFINITY;
  const uint16_t* kb = kc + (size_t)bh * kn * 128;
#pragma unroll
  for (int u = 0; u < E; ++u) {
    const int j = tid + u * kMaskThreads;
    float t = -INFINITY;
    if (j < kn) {
      const u32x4_t* row = (const u32x4_t*)(kb + (size_t)j * 128);
      double acc = 0.0;
      for (int c = 0; c < 16; ++c) {
        const u32x4_t w = row[c];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc = fma(qrow[c * 8 + 2 * e], (double)bf16_to_f32((uint16_t)(w[e] & 0xffffu)), acc);
          acc = fma(qrow[c * 8 + 2 * e + 1], (double)bf16_to_f32((uint16_t)(w[e] >> 16)), acc);
        }
      }
      const float sb = bf16_round_f32((float)acc);
      t = bf16_round_f32(sb * inv_sqrt_d);
      lmax = fmaxf(lmax, t);
    }
    tv[j] = t;
  }
  const float m = block_max_f32<kMaskThreads>(lmax, red_f);

  // Weighted softmax in fp64.
  const int32_t* wrow = ksz + (size_t)bh * kn;
  double we[E];
  double lsum = 0.0;
#pragma unroll
  for (int u = 0; u < E; ++u) {
    const int j = tid + u * kMaskThreads;
    we[u] = 0.0;
    if (j < kn) {
      we[u] = (double)wrow[j] * exp((double)tv[j] - (double)m);
      lsum += we[u];
    }
  }
  const double den = fmax(block_sum_f64<kMaskThreads>(lsum, red_d), 1e-12);
#pragma unroll
  for (int u = 0; u < E; ++u) {
    const int j = tid + u * kMaskThreads;
    uint32_t key = 0;
    if (j < kn) {
      const uint16_t pb = f32_to_bf16((float)(we[u] / den));
      key = ((uint32_t)pb << 16) | (uint32_t)(0xffff - j);
    }
    keys[j] = key;
  }
  __syncthreads();

  // Bitonic sort, descending.
  for (int size = 2; size <= KP; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
#pragma unroll
      for (int u = 0; u < E / 2 + (E == 1 ? 1 : 0); ++u) {
        const int idx = tid + u * kMaskThreads;
        if (idx < KP / 2) {
          const int pos = 2 * idx - (idx & (stride - 1));
          const int par = pos + stride;
          const bool desc = (pos & size) == 0;
          const uint32_t a = keys[pos], b = keys[par];
          if ((a < b) == desc) {
            keys[pos] = b;
            keys[par] = a;
          }
        }
      }
      __syncthreads();
    }
  }

  // Exact fixed-point prefix of the sorted probabilities (thread owns E consecutive positions).
  long long fx[E];
  long long run = 0;
#pragma unroll
  for (int u = 0; u < E; ++u) {
    const int t = tid * E + u;
    const float pbv = bf16_to_f32((uint16_t)(keys[t] >> 16));
    const long long v = (t < kn && pbv > 0.0f) ? (long long)ldexp((double)pbv, 60) : 0ll;
    run += v;
    fx[u] = run;
  }
  long long total;
  const long long excl = block_exclusive_scan_i64<kMaskThreads>(run, red_l, &total);
  int cnt = 0;
#pragma unroll
  for (int u = 0; u < E; ++u) {
    const int t = tid * E + u;
    if (t <= kn - 2) {
      const long long pre = excl + fx[u];
      const float cb = bf16_round_f32((float)((double)pre * 0x1p-60));
      if (cb <= p_st) ++cnt;
    }
  }
  const int le = block_sum_i32<kMaskThreads>(cnt, red_i);
  int len = 1 + le;
  len = max(len, (int)preserve[head]);
  if (cap[head] > 0) len = min(len, (int)cap[head]);
  len = min(len, kn);
#pragma unroll
  for (int u = 0; u < E; ++u) {
    const int t = tid * E + u;
    if (t < kn) {
      const int j = 0xffff - (int)(keys[t] & 0xffffu);
      mrow[j] = (t < len) ? 1 : 0;
    }
  }
  if (tid == 0 && lengths) lengths[(size_t)bh * qn + i] = len;
}

// Standalone weighted softmax (one block per row).
template <int KP>
__global__ void __launch_bounds__(kMaskThreads) weighted_softmax_kernel(const uint16_t* __restrict__ scores,
                                                                        const float* __restrict__ weights,
                                                                        long long wstride, uint16_t* __restrict__ out,
                                                                        int cols) {
  constexpr int E = KP / kMaskThreads;
  __shared__ double red_d[kMaskThreads / kWave];
  __shared__ float red_f[kMaskThreads / kWave];
  const long long r = blockIdx.x;
  const uint16_t* srow = scores + r * cols;
  const float* wrow = weights + r * wstride;
  float lmax = -INFINITY;
  float sv[E];
#pragma unroll
  for (int u = 0; u < E; ++u) {
    const int j = threadIdx.x + u * kMaskThreads;
    sv[u] = j < cols ? bf16_to_f32(srow[j]) : -INFINITY;
    lmax = fmaxf(lmax, sv[u]);
  }
  const float m = block_max_f32<kMaskThreads>(lmax, red_f);
  double we[E];
  double lsum = 0.0;
#pragma unroll
  for (int u = 0; u < E; ++u) {
    const int j = threadIdx.x + u * kMaskThreads;
    we[u] = j < cols ? (double)wrow[j] * exp((double)sv[u] - (double)m) : 0.0;
    lsum += we[u];
  }
  const double den = fmax(block_sum_f64<kMaskThreads>(lsum, red_d), 1e-12);
#pragma unroll
  for (int u = 0; u < E; ++u) {
    const int j = threadIdx.x + u * kMaskThreads;
    if (j < cols) out[r * cols + j] = f32_to_bf16((float)(we[u] / den));
  }
}

}  // namespace svoo

using namespace svoo;

extern "C" int svoo_block_mask(const uint16_t* qc, const uint16_t* kc, const int32_t* k_sizes,
                               const int32_t* preserve, const int32_t* cap, int b, int h, int qn, int kn, int d,
                               float p_storage, int full, uint8_t* map, int32_t* lengths, void* stream) {
  SVOO_REQUIRE(map && (full || (qc && kc && k_sizes && preserve && cap)), SVOO_ERR_INVALID_ARG,
               "svoo_block_mask: null pointer");
  SVOO_REQUIRE(b > 0 && h > 0 && qn > 0 && kn > 0, SVOO_ERR_INVALID_ARG, "svoo_block_mask: bad dims");
  SVOO_REQUIRE(d == 128, SVOO_ERR_UNSUPPORTED, "svoo_block_mask: D=%d (only 128 supported)", d);
  SVOO_REQUIRE(kn <= 4096, SVOO_ERR_UNSUPPORTED, "svoo_block_mask: Kc=%d exceeds 4096", kn);
  SVOO_REQUIRE(qn <= 65535 && (long long)b * h <= 65535, SVOO_ERR_UNSUPPORTED, "svoo_block_mask: grid too large");
  const float inv = 1.0f / (float)sqrt((double)d);
  dim3 grid(qn, b * h);
  hipStream_t s = (hipStream_t)stream;
#define SVOO_MASK_LAUNCH(KP)                                                                                    \
  hipLaunchKernelGGL(block_mask_kernel<KP>, grid, dim3(kMaskThreads), 0, s, qc, kc, k_sizes, preserve, cap, h, qn, \
                     kn, inv, p_storage, full, map, lengths)
  if (kn <= 256)
    SVOO_MASK_LAUNCH(256);
  else if (kn <= 512)
    SVOO_MASK_LAUNCH(512);
  else if (kn <= 1024)
    SVOO_MASK_LAUNCH(1024);
  else if (kn <= 2048)
    SVOO_MASK_LAUNCH(2048);
  else
    SVOO_MASK_LAUNCH(4096);
#undef SVOO_MASK_LAUNCH
  return check_launch("svoo_block_mask");
}

extern "C" int svoo_weighted_softmax(const uint16_t* scores, const float* weights, long long weight_row_stride,
                                     uint16_t* out, long long rows, int cols, void* stream) {
  SVOO_REQUIRE(scores && weights && out, SVOO_ERR_INVALID_ARG, "svoo_weighted_softmax: null pointer");
  SVOO_REQUIRE(rows > 0 && cols > 0 && rows <= 2147483647ll, SVOO_ERR_INVALID_ARG, "svoo_weighted_softmax: bad dims");
  SVOO_REQUIRE(cols <= 4096, SVOO_ERR_UNSUPPORTED, "svoo_weighted_softmax: cols=%d exceeds 4096", cols);
  hipStream_t s = (hipStream_t)stream;
  dim3 grid((unsigned)rows);
#define SVOO_WS_LAUNCH(KP) \
  hipLaunchKernelGGL(weighted_softmax_kernel<KP>, grid, dim3(kMaskThreads), 0, s, scores, weights, weight_row_stride, out, cols)
  if (cols <= 256)
    SVOO_WS_LAUNCH(256);
  else if (cols <= 1024)
    SVOO_WS_LAUNCH(1024);
  else
    SVOO_WS_LAUNCH(4096);
#undef SVOO_WS_LAUNCH
  return check_launch("svoo_weighted_softmax");
}
