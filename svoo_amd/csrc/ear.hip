// EAR: error-aware routing of key-cluster blocks (budget from centroid attention, greedy by an
// estimated pruning error) for the compensated variable-block-sparse attention.
//
// Kernels, in call order (all inputs cluster-contiguous, i.e. already permuted):
//   ear_value_kernel       one block per (bh, key cluster): value centroid vc_j (exact member sum),
//                          |vc_j|^2 and per token u_t = v_t - vc_j as {|u_t|^2, u_t . vc_j}
//   (centroid logits)      c_ij = bf16(bf16(qc_i . kc_j) * D^-0.5): svoo_centroid_scores (mask.hip)
//   ear_efficiency_kernel  MFMA over (32 query centroids x 32 tokens) tiles; per (i, j) the error
//                          err = sum_t || e_t v_t - pc vc_j ||^2,  e_t = e^{a_t - m},  pc = e^{c_ij - m},
//                          a_t = qc_i . k_t / sqrt(D), m = max(c_ij, max_t a_t) (online), then
//                          eff = max(log(err) + 2m, log eps) - gamma log(max(|Q_i||K_j|, eps)).
//                          The reference expands err as sum e^2|v|^2 - 2 pc sum e (vc.v) + pc^2|vc|^2|K|,
//                          which cancels catastrophically in fp32 where the centroid reproduces the
//                          block (a one-token cluster with a_t ~ c_ij); here, with d_t = e_t - pc,
//                            || e_t v_t - pc vc ||^2 = e_t^2 |u_t|^2 + 2 e_t d_t (u_t . vc) + d_t^2 |vc|^2,
//                          d_t = pc expm1(a_t - c_ij) near c_ij: equal in exact arithmetic, accurate in fp32.
//   ear_select_kernel      one block per (bh, query cluster): budget from the bf16 softmax of
//                          c + bf16(log(|K| + 1e-8)) (stable sort, exact fixed-point top-p prefix),
//                          guaranteed top clusters, greedy fill by efficiency (stable sort, exact
//                          int64 areas) -> uint8 map row.
// The compensated attention itself is the EAR variant of the VBSA kernel.
#include "svoo_common.h"

namespace svoo {

constexpr int kEarThreads = 256;

// ------------------------------------------------------------------------------------------ value side
__global__ void __launch_bounds__(kEarThreads) ear_value_kernel(const uint16_t* __restrict__ vp,
                                                                const int32_t* __restrict__ koff,
                                                                const int32_t* __restrict__ ks, int n, int kn,
                                                                int compute_vc, uint16_t* __restrict__ vc,
                                                                float* __restrict__ vc_sq,
                                                                float2* __restrict__ tok_stats) {
  __shared__ double part[16][128];
  __shared__ float vcs[128];
  const int j = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int lane = tid % kWave, wave = tid / kWave;
  const size_t cj = (size_t)b * kn + j;
  const int start = koff[cj], cnt = ks[cj];
  const uint16_t* vb = vp + ((size_t)b * n + start) * 128;
  if (compute_vc) {
    // 16 row groups x 16 chunks of 8 values: 16-byte loads, fp64 sums (exact for bf16 inputs)
    const int rg = tid / 16, c8 = tid % 16;
    double acc[8] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
    for (int t = rg; t < cnt; t += 16) {
      const u32x4_t w = ((const u32x4_t*)(vb + (size_t)t * 128))[c8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc[2 * e] += (double)bf16_to_f32((uint16_t)(w[e] & 0xffffu));
        acc[2 * e + 1] += (double)bf16_to_f32((uint16_t)(w[e] >> 16));
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) part[rg][8 * c8 + e] = acc[e];
    __syncthreads();
    if (tid < 128) {
      double sum = 0.0;
#pragma unroll
      for (int g = 0; g < 16; ++g) sum += part[g][tid];
      const int d = tid;
      // bf16 sum (rounded once), divided by the bf16-rounded count, rounded to bf16
      const float s_st = bf16_round_f32((float)sum);
      const float den = bf16_round_f32((float)max(cnt, 1));
      const uint16_t r = f32_to_bf16(s_st / den);
      vc[cj * 128 + d] = r;
      vcs[d] = bf16_to_f32(r);
    }
  } else if (tid < 128) {
    vcs[tid] = bf16_to_f32(vc[cj * 128 + tid]);
  }
  __syncthreads();
  if (wave == 0) {
    float q = vcs[2 * lane] * vcs[2 * lane] + vcs[2 * lane + 1] * vcs[2 * lane + 1];
    for (int o = 32; o > 0; o >>= 1) q += __shfl_xor(q, o);
    if (lane == 0) vc_sq[cj] = q;
  }
  // per token: 16 lanes x 8 elements, 4 tokens per wave and pass
  const int tg = lane / 16, ch = lane % 16;
  float cv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) cv[e] = vcs[8 * ch + e];
  for (int t0 = wave * 4; t0 < cnt; t0 += 16) {
    const int t = t0 + tg;
    float vn = 0.0f, cd = 0.0f;  // |u|^2, u . vc with u = v - vc (bf16 differences are exact in fp32)
    if (t < cnt) {
      const u32x4_t w = ((const u32x4_t*)(vb + (size_t)t * 128))[ch];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float u0 = bf16_to_f32((uint16_t)(w[e] & 0xffffu)) - cv[2 * e];
        const float u1 = bf16_to_f32((uint16_t)(w[e] >> 16)) - cv[2 * e + 1];
        vn = fmaf(u0, u0, vn);
        vn = fmaf(u1, u1, vn);
        cd = fmaf(cv[2 * e], u0, cd);
        cd = fmaf(cv[2 * e + 1], u1, cd);
      }
    }
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) {
      vn += __shfl_xor(vn, o);
      cd += __shfl_xor(cd, o);
    }
    if (t < cnt && ch == 0) tok_stats[(size_t)b * n + start + t] = make_float2(vn, cd);
  }
}

// ------------------------------------------------------------------------------------------ efficiency
// Block = 4 waves over kEffClusters consecutive key clusters of one head; wave w takes the query
// tiles w, w+4, ... (32 query centroids each).  S^T = K Q^T with v_mfma_f32_32x32x16_bf16: tokens
// on M, query centroids on N, so lane (n, h) holds 16 tokens of query centroid n and the sums over
// tokens stay in the lane until one exchange with lane n+32 per (i, j).  The contraction index is
// permuted (lane half h covers d in [64h, 64h+64), k-step s the 8 values at 64h + 8s) identically
// in both operands, so every lane loads 128 contiguous bytes of its row.
constexpr int kEffClusters = 8;
constexpr float kLog2e = 1.4426950408889634f, kLn2 = 0.6931471805599453f;

// expm1(x) for |x| <= 0.1 by its Taylor series to x^4 (truncation below 1e-6 relative); beyond
// 0.1 the difference e^a - e^c itself loses at most 6e-8 / 0.1 relative in fp32.
constexpr float kExpm1Lim = 0.1f;
__device__ __forceinline__ float expm1_small(float x) {
  float p = fmaf(x, 1.0f / 24.0f, 1.0f / 6.0f);
  p = fmaf(p, x, 0.5f);
  p = fmaf(p, x, 1.0f);
  return p * x;
}

__global__ void __launch_bounds__(kEarThreads) ear_efficiency_kernel(
    const uint16_t* __restrict__ qc, const uint16_t* __restrict__ kp, const uint16_t* __restrict__ clog,
    const float2* __restrict__ tok_stats, const float* __restrict__ vc_sq, const int32_t* __restrict__ qs,
    const int32_t* __restrict__ ks, const int32_t* __restrict__ koff, int n, int qn, int kn, float scale2,
    double inv_sqrt_d, float gamma, float log_eps, float eps, float* __restrict__ eff) {
  const int b = blockIdx.y, j0 = blockIdx.x * kEffClusters;
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave, h = lane / 32, l32 = lane % 32;
  const int j1 = min(kn, j0 + kEffClusters);
  const int qtiles = (qn + 31) / 32;
  const uint16_t* kb = kp + (size_t)b * n * 128;
  const float2* st = tok_stats + (size_t)b * n;
  for (int qt = wave; qt < qtiles; qt += 4) {
    const int i = qt * 32 + l32, ic = min(i, qn - 1);
    u32x4_t qop[8];
    {
      const u32x4_t* src = (const u32x4_t*)(qc + ((size_t)b * qn + ic) * 128) + 8 * h;
#pragma unroll
      for (int s = 0; s < 8; ++s) qop[s] = src[s];
    }
    const float qsz = (float)qs[(size_t)b * qn + ic];
    const uint16_t* crow = clog + ((size_t)b * qn + ic) * kn;
    for (int j = j0; j < j1; ++j) {
      const size_t cj = (size_t)b * kn + j;
      const int start = koff[cj], cnt = ks[cj];
      const float c = bf16_to_f32(crow[j]);
      const float c2 = c * kLog2e;
      // sums of e^2 |u|^2, e d (u . vc) and d^2, relative to the running max m2 (log2 units)
      float m2 = c2, sd = 0.0f, sg = 0.0f, sc = 0.0f;
      // A one-member cluster's key centroid is its member (a mean of one value is exact) and u = 0, so its error
      // d^2 |vc|^2 is set by x = a - c alone, which is the bf16 rounding of the logit: an fp32 dot (~1e-6
      // absolute) would leave x wrong by percents.  Every lane then loads the member's row and also forms
      // qc_i . k exactly in fp64 (bf16 products are exact there).
      const bool single = cnt == 1;
      float x_single = 0.0f;
      for (int tt = 0; tt < cnt; tt += 32) {
        const int row = single ? start : min(start + tt + l32, n - 1);
        const u32x4_t* kr = (const u32x4_t*)(kb + (size_t)row * 128) + 8 * h;
        u32x4_t ka[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) ka[s] = kr[s];
        if (single) {
          // operands re-read from memory (L1/L2 hits) in a rolled loop: fp64 copies of the register-resident
          // operands would be hoisted out of the cluster loop and cost 128 VGPRs
          const u32x4_t* qsrc = (const u32x4_t*)(qc + ((size_t)b * qn + ic) * 128) + 8 * h;
          double dot = 0.0;
#pragma unroll 1
          for (int s = 0; s < 8; ++s) {
            const u32x4_t qw = qsrc[s], kw = kr[s];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const double q0 = bf16_to_f32((uint16_t)(qw[e] & 0xffffu)), q1 = bf16_to_f32((uint16_t)(qw[e] >> 16));
              const double k0 = bf16_to_f32((uint16_t)(kw[e] & 0xffffu)), k1 = bf16_to_f32((uint16_t)(kw[e] >> 16));
              dot = fma(q1, k1, fma(q0, k0, dot));
            }
          }
          dot += __shfl_xor(dot, 32);
          x_single = (float)(dot * inv_sqrt_d - (double)c);
        }
        // token statistics of this lane's 16 tokens, loaded with the K rows (clamped rows are masked below)
        float2 sv[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) sv[r] = st[min(start + tt + (r / 4) * 8 + h * 4 + (r % 4), n - 1)];
        f32x16_t sacc = f32x16_t{};
#pragma unroll
        for (int s = 0; s < 8; ++s) sacc = mfma32x32x16(as_bf16x8(ka[s]), as_bf16x8(qop[s]), sacc);
        const bool full = tt + 32 <= cnt;  // wave-uniform: no masking inside the cluster
        float av[16];  // a_t in log2 units
        float tmax = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int tok = tt + (r / 4) * 8 + h * 4 + (r % 4);
          av[r] = (full || tok < cnt) ? sacc[r] * scale2 : -INFINITY;
          tmax = fmaxf(tmax, av[r]);
        }
        tmax = xhalf_max(tmax);
        if (tmax > m2) {
          const float f = __builtin_amdgcn_exp2f(m2 - tmax), f2 = f * f;
          sd *= f2;
          sg *= f2;
          sc *= f2;
          m2 = tmax;
        }
        const float pc = __builtin_amdgcn_exp2f(c2 - m2);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int tok = tt + (r / 4) * 8 + h * 4 + (r % 4);
          const float e = __builtin_amdgcn_exp2f(av[r] - m2);  // 0 for masked tokens
          const float x = single ? x_single : (av[r] - c2) * kLn2;  // a_t - c_ij
          float d = fabsf(x) <= kExpm1Lim ? pc * expm1_small(x) : e - pc;
          if (!full && tok >= cnt) d = 0.0f;
          sd = fmaf(e * e, sv[r].x, sd);
          sg = fmaf(e * d, sv[r].y, sg);
          sc = fmaf(d, d, sc);
        }
      }
      sd = xhalf_sum(sd);
      sg = xhalf_sum(sg);
      sc = xhalf_sum(sc);
      const float err = sd + 2.0f * sg + vc_sq[cj] * sc;
      // log(err) + 2m with m = m2 ln2, via the hardware log2
      const float lerr = fmaxf(err > 0.0f ? (__builtin_amdgcn_logf(err) + 2.0f * m2) * kLn2 : -INFINITY, log_eps);
      const float area = fmaxf(qsz * (float)cnt, eps);
      if (h == 0 && i < qn) eff[((size_t)b * qn + i) * kn + j] = lerr - gamma * logf(area);
    }
  }
}

// ------------------------------------------------------------------------------------------ selection
__device__ __forceinline__ uint32_t ord_f32(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

template <typename T, int KP>
__device__ __forceinline__ void bitonic_desc(T* keys) {
  constexpr int E = KP / kEarThreads;
  for (int size = 2; size <= KP; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
#pragma unroll
      for (int u = 0; u < (E / 2 > 0 ? E / 2 : 1); ++u) {
        const int idx = threadIdx.x + u * kEarThreads;
        if (idx < KP / 2) {
          const int pos = 2 * idx - (idx & (stride - 1));
          const int par = pos + stride;
          const bool desc = (pos & size) == 0;
          const T a = keys[pos], bb = keys[par];
          if ((a < bb) == desc) {
            keys[pos] = bb;
            keys[par] = a;
          }
        }
      }
      __syncthreads();
    }
  }
}

template <int KP>
__global__ void __launch_bounds__(kEarThreads) ear_select_kernel(const uint16_t* __restrict__ clog,
                                                                 const float* __restrict__ eff,
                                                                 const int32_t* __restrict__ qs,
                                                                 const int32_t* __restrict__ ks,
                                                                 const int32_t* __restrict__ preserve,
                                                                 const int32_t* __restrict__ budget_preserve, int h,
                                                                 int qn, int kn, float p_st,
                                                                 uint8_t* __restrict__ map) {
  constexpr int E = KP / kEarThreads;
  __shared__ uint32_t keys[KP];
  __shared__ unsigned long long keys2[KP];
  __shared__ uint8_t gflag[KP];
  __shared__ double red_d[kEarThreads / kWave];
  __shared__ float red_f[kEarThreads / kWave];
  __shared__ long long red_l[kEarThreads / kWave];
  __shared__ int red_i[kEarThreads / kWave];
  const int i = blockIdx.x, b = blockIdx.y, tid = threadIdx.x, head = b % h;
  const size_t row = (size_t)b * qn + i;
  const uint16_t* crow = clog + row * kn;
  const int32_t* ksb = ks + (size_t)b * kn;
  const long long qsz = qs[row];

  // 1. budget logits bf16(c + bf16(log(bf16(bf16(|K|) + 1e-8)))) and their softmax in fp64
  float lg[E];
  float lmax = -INFINITY;
#pragma unroll
  for (int u = 0; u < E; ++u) {
    const int j = tid + u * kEarThreads;
    lg[u] = -INFINITY;
    if (j < kn) {
      const float se = bf16_round_f32(bf16_round_f32((float)ksb[j]) + 1e-8f);
      const float lks = bf16_round_f32((float)log((double)se));
      lg[u] = bf16_round_f32(bf16_to_f32(crow[j]) + lks);
      lmax = fmaxf(lmax, lg[u]);
    }
  }
  const float m = block_max_f32<kEarThreads>(lmax, red_f);
  double ex[E];
  double lsum = 0.0;
#pragma unroll
  for (int u = 0; u < E; ++u) {
    const int j = tid + u * kEarThreads;
    ex[u] = j < kn ? exp((double)lg[u] - (double)m) : 0.0;
    lsum += ex[u];
  }
  const double den = block_sum_f64<kEarThreads>(lsum, red_d);
#pragma unroll
  for (int u = 0; u < E; ++u) {
    const int j = tid + u * kEarThreads;
    uint32_t key = 0;
    if (j < kn) key = ((uint32_t)f32_to_bf16((float)(ex[u] / den)) << 16) | (uint32_t)(0xffff - j);
    keys[j] = key;
    gflag[j] = 0;
  }
  __syncthreads();
  bitonic_desc<uint32_t, KP>(keys);

  // 2. budget length: 1 + #{t <= Kc-2 : bf16(prefix_t) <= p}, at least budget_preserve
  long long fx[E];
  long long run = 0;
#pragma unroll
  for (int u = 0; u < E; ++u) {
    const int t = tid * E + u;
    const float pbv = bf16_to_f32((uint16_t)(keys[t] >> 16));
    run += (t < kn && pbv > 0.0f) ? (long long)ldexp((double)pbv, 60) : 0ll;
    fx[u] = run;
  }
  long long total;
  const long long excl = block_exclusive_scan_i64<kEarThreads>(run, red_l, &total);
  int cnt = 0;
#pragma unroll
  for (int u = 0; u < E; ++u) {
    const int t = tid * E + u;
    if (t <= kn - 2 && bf16_round_f32((float)((double)(excl + fx[u]) * 0x1p-60)) <= p_st) ++cnt;
  }
  const int le = block_sum_i32<kEarThreads>(cnt, red_i);
  const int len = min(kn, max(1 + le, (int)budget_preserve[head]));
  const int pre = min(kn, (int)preserve[head]);

  // 3. budget and guaranteed cost (exact int64 areas)
  long long bsum = 0, gsum = 0;
#pragma unroll
  for (int u = 0; u < E; ++u) {
    const int t = tid * E + u;
    if (t < kn) {
      const int j = 0xffff - (int)(keys[t] & 0xffffu);
      const long long area = qsz * (long long)ksb[j];
      if (t < len) bsum += area;
      if (t < pre) {
        gsum += area;
        gflag[j] = 1;
      }
    }
  }
  long long bt, gt;
  block_exclusive_scan_i64<kEarThreads>(bsum, red_l, &bt);
  block_exclusive_scan_i64<kEarThreads>(gsum, red_l, &gt);
  const long long remaining = max(bt - gt, 0ll);
  __syncthreads();

  // 4. greedy fill in descending efficiency (guaranteed clusters last, ties by index)
#pragma unroll
  for (int u = 0; u < E; ++u) {
    const int j = tid + u * kEarThreads;
    unsigned long long key = 0ull;
    if (j < kn) {
      float e = gflag[j] ? -1e10f : eff[row * kn + j];
      if (e == 0.0f) e = 0.0f;  // -0 and +0 are one value (a tie), as in a comparison sort
      key = ((unsigned long long)ord_f32(e) << 16) | (unsigned long long)(0xffff - j);
    }
    keys2[j] = key;
  }
  __syncthreads();
  bitonic_desc<unsigned long long, KP>(keys2);
  long long ar[E];
  long long arun = 0;
#pragma unroll
  for (int u = 0; u < E; ++u) {
    const int t = tid * E + u;
    ar[u] = 0;
    if (t < kn) ar[u] = qsz * (long long)ksb[0xffff - (int)(keys2[t] & 0xffffu)];
    arun += ar[u];
  }
  long long atot;
  long long before = block_exclusive_scan_i64<kEarThreads>(arun, red_l, &atot);
  uint8_t* mrow = map + row * kn;
#pragma unroll
  for (int u = 0; u < E; ++u) {
    const int t = tid * E + u;
    if (t < kn) {
      const int j = 0xffff - (int)(keys2[t] & 0xffffu);
      mrow[j] = (before < remaining || gflag[j]) ? 1 : 0;
    }
    before += ar[u];
  }
}

}  // namespace svoo

using namespace svoo;

extern "C" int svoo_ear_value_stats(const uint16_t* v_perm, const int32_t* k_offsets, const int32_t* k_sizes, int bh,
                                    int n, int kn, int d, int compute_vc, uint16_t* v_cent, float* vc_sq,
                                    float* tok_stats, void* stream) {
  SVOO_REQUIRE(v_perm && k_offsets && k_sizes && v_cent && vc_sq && tok_stats, SVOO_ERR_INVALID_ARG,
               "svoo_ear_value_stats: null pointer");
  SVOO_REQUIRE_HEAD_DIM(d, "svoo_ear_value_stats");
  SVOO_REQUIRE(bh > 0 && n > 0 && kn > 0 && bh <= 65535, SVOO_ERR_INVALID_ARG, "svoo_ear_value_stats: bad dims");
  hipLaunchKernelGGL(ear_value_kernel, dim3(kn, bh), dim3(kEarThreads), 0, (hipStream_t)stream, v_perm, k_offsets,
                     k_sizes, n, kn, compute_vc, v_cent, vc_sq, (float2*)tok_stats);
  return check_launch("svoo_ear_value_stats");
}

extern "C" int svoo_ear_centroid_logits(const uint16_t* qc, const uint16_t* kc, int bh, int qn, int kn, int d,
                                        uint16_t* c_logits, void* stream) {
  SVOO_REQUIRE(qc && kc && c_logits, SVOO_ERR_INVALID_ARG, "svoo_ear_centroid_logits: null pointer");
  SVOO_REQUIRE_HEAD_DIM(d, "svoo_ear_centroid_logits");
  SVOO_REQUIRE(bh > 0 && qn > 0 && kn > 0 && bh <= 65535 && qn <= 65535, SVOO_ERR_INVALID_ARG,
               "svoo_ear_centroid_logits: bad dims");
  // c_ij = bf16(bf16(qc_i . kc_j) * f32(D^-1/2)): the centroid scores of the block mask
  return svoo_centroid_scores(qc, kc, bh, qn, kn, d, c_logits, stream);
}

extern "C" int svoo_ear_efficiency(const uint16_t* qc, const uint16_t* k_perm, const uint16_t* c_logits,
                                   const float* tok_stats, const float* vc_sq, const int32_t* q_sizes,
                                   const int32_t* k_sizes, const int32_t* k_offsets, int bh, int n, int qn, int kn,
                                   int d, float gamma, float eps, float* eff, void* stream) {
  SVOO_REQUIRE(qc && k_perm && c_logits && tok_stats && vc_sq && q_sizes && k_sizes && k_offsets && eff,
               SVOO_ERR_INVALID_ARG, "svoo_ear_efficiency: null pointer");
  SVOO_REQUIRE_HEAD_DIM(d, "svoo_ear_efficiency");
  SVOO_REQUIRE(bh > 0 && n > 0 && qn > 0 && kn > 0 && bh <= 65535 && eps > 0.0f, SVOO_ERR_INVALID_ARG,
               "svoo_ear_efficiency: bad dims");
  const float scale2 = (float)(1.4426950408889634 / sqrt((double)d));  // log2(e) / sqrt(D)
  dim3 grid((kn + kEffClusters - 1) / kEffClusters, bh);
  hipLaunchKernelGGL(ear_efficiency_kernel, grid, dim3(kEarThreads), 0, (hipStream_t)stream, qc, k_perm, c_logits,
                     (const float2*)tok_stats, vc_sq, q_sizes, k_sizes, k_offsets, n, qn, kn, scale2,
                     1.0 / sqrt((double)d), gamma, logf(eps), eps, eff);
  return check_launch("svoo_ear_efficiency");
}

extern "C" int svoo_ear_select(const uint16_t* c_logits, const float* eff, const int32_t* q_sizes,
                               const int32_t* k_sizes, const int32_t* preserve, const int32_t* budget_preserve, int b,
                               int h, int qn, int kn, float p_storage, uint8_t* map, void* stream) {
  SVOO_REQUIRE(c_logits && eff && q_sizes && k_sizes && preserve && budget_preserve && map, SVOO_ERR_INVALID_ARG,
               "svoo_ear_select: null pointer");
  SVOO_REQUIRE(b > 0 && h > 0 && qn > 0 && kn > 0, SVOO_ERR_INVALID_ARG, "svoo_ear_select: bad dims");
  SVOO_REQUIRE(kn <= 4096, SVOO_ERR_UNSUPPORTED, "svoo_ear_select: Kc=%d exceeds 4096", kn);
  SVOO_REQUIRE(qn <= 65535 && (long long)b * h <= 65535, SVOO_ERR_UNSUPPORTED, "svoo_ear_select: grid too large");
  dim3 grid(qn, b * h);
  hipStream_t s = (hipStream_t)stream;
#define SVOO_EAR_SEL(KP)                                                                                           \
  hipLaunchKernelGGL(ear_select_kernel<KP>, grid, dim3(kEarThreads), 0, s, c_logits, eff, q_sizes, k_sizes, preserve, \
                     budget_preserve, h, qn, kn, p_storage, map)
  if (kn <= 256)
    SVOO_EAR_SEL(256);
  else if (kn <= 512)
    SVOO_EAR_SEL(512);
  else if (kn <= 1024)
    SVOO_EAR_SEL(1024);
  else if (kn <= 2048)
    SVOO_EAR_SEL(2048);
  else
    SVOO_EAR_SEL(4096);
#undef SVOO_EAR_SEL
  return check_launch("svoo_ear_select");
}
