// Exact attention sparsity of one query row (the offline profile producer).
//
// For a row of scaled scores s_j (bf16 scores times scale, as the reference's fp32 softmax input)
// the count is the smallest c such that the c largest softmax weights hold at least `threshold` of
// the row's mass.  Softmax weights are exp(s_j - m) / Z with m the row max, so the count is the same
// for the unnormalised weights e_j = exp(s_j - m), computed here as float(exp(double(s_j - m))).
//
// Scores are bf16, so a row holds at most 65536 distinct values and the order of the weights is
// the order of the bf16 patterns.  One block per row, three passes over the row:
//   1. the largest score (as an order-preserving 16-bit key);
//   2. a 256-bin histogram over the key's high byte: counts and fp64 mass sums; the block finds the
//      bin where the mass counted from the top first reaches threshold * total;
//   3. a 256-bin count histogram over the low byte of the keys in that bin: every sub-bin is one
//      exact value, so the crossing element and its multiplicity are exact.
// All masses are fp64 sums of fp32 weights, so the count does not depend on summation order beyond
// 2^-53 of the mass.
#include "svoo_common.h"

namespace svoo {

constexpr int kSpThreads = 256;

// bf16 bit pattern <-> key whose unsigned order is the numeric order
__device__ __forceinline__ uint32_t sp_key(uint16_t b) { return (b & 0x8000u) ? (~b & 0xffffu) : (b | 0x8000u); }
__device__ __forceinline__ uint16_t sp_unkey(uint32_t k) {
  return (uint16_t)((k & 0x8000u) ? (k & 0x7fffu) : (~k & 0xffffu));
}

__device__ __forceinline__ float sp_weight(uint16_t b, float scale, float m) {
  const float s = bf16_to_f32(b) * scale;
  return (float)exp((double)(s - m));
}

// Lanes of a wave with the same bin combine their (count, weight) before one LDS atomic per
// distinct bin: scores concentrate in a few binades, and plain per-lane atomics would serialise.
__device__ __forceinline__ double wave_sum_f64(double v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
__device__ __forceinline__ void hist_add(int32_t* cnt, double* mass, int bin, double w, bool valid) {
  const int lane = threadIdx.x & (kWave - 1);
  unsigned long long todo = __ballot(valid);
  while (todo) {
    const int leader = __ffsll((long long)todo) - 1;
    const int lb = __shfl(bin, leader);
    const bool mine = valid && bin == lb;
    const unsigned long long mm = __ballot(mine);
    const double sum = wave_sum_f64(mine ? w : 0.0);
    if (lane == leader) {
      atomicAdd(&cnt[lb], (int)__popcll(mm));
      atomicAdd(&mass[lb], sum);
    }
    todo &= ~mm;
  }
}
__device__ __forceinline__ void count_add(int32_t* cnt, int bin, bool valid) {
  const int lane = threadIdx.x & (kWave - 1);
  unsigned long long todo = __ballot(valid);
  while (todo) {
    const int leader = __ffsll((long long)todo) - 1;
    const int lb = __shfl(bin, leader);
    const unsigned long long mm = __ballot(valid && bin == lb);
    if (lane == leader) atomicAdd(&cnt[lb], (int)__popcll(mm));
    todo &= ~mm;
  }
}

// Inclusive prefix, from the top bin down, of the 256 bins' masses and counts (thread t holds bin
// 255 - t); a fixed summation order.
__device__ void sp_scan(const int32_t* cnt, const double* mass, double* dsc, long long* isc) {
  const int tid = threadIdx.x;
  dsc[tid] = mass[255 - tid];
  isc[tid] = cnt[255 - tid];
  __syncthreads();
  for (int off = 1; off < kSpThreads; off <<= 1) {
    const double dv = tid >= off ? dsc[tid - off] : 0.0;
    const long long iv = tid >= off ? isc[tid - off] : 0;
    __syncthreads();
    dsc[tid] += dv;
    isc[tid] += iv;
    __syncthreads();
  }
}

// The bin (scanned from the top) at which the scanned mass first reaches `target`, with the mass
// and count strictly above it; the lowest non-empty bin when rounding leaves the total below the
// target.  Call after sp_scan.
struct SpCross {
  int bin;
  double mass_above;
  long long cnt_above;
};
__device__ SpCross sp_find(const int32_t* cnt, double target, const double* dsc, const long long* isc, int* found) {
  const int tid = threadIdx.x;
  if (tid == 0) *found = -1;
  __syncthreads();
  const double above = tid > 0 ? dsc[tid - 1] : 0.0;
  if (cnt[255 - tid] > 0 && above < target && dsc[tid] >= target) *found = tid;
  __syncthreads();
  if (*found < 0) {
    __syncthreads();
    if (tid == 0) {
      int last = 0;
      for (int i = 0; i < kSpThreads; ++i)
        if (cnt[255 - i] > 0) last = i;
      *found = last;
    }
    __syncthreads();
  }
  const int t = *found;
  SpCross r;
  r.bin = 255 - t;
  r.mass_above = t > 0 ? dsc[t - 1] : 0.0;
  r.cnt_above = t > 0 ? isc[t - 1] : 0;
  __syncthreads();
  return r;
}

__global__ void __launch_bounds__(kSpThreads) exact_count_kernel(const uint16_t* __restrict__ scores, int n,
                                                                   float scale, float threshold,
                                                                   int32_t* __restrict__ counts) {
  __shared__ int32_t cnt[256];
  __shared__ double mass[256];
  __shared__ double dsc[kSpThreads];
  __shared__ long long isc[kSpThreads];
  __shared__ int found;
  __shared__ uint32_t kmax_s;
  const size_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const uint16_t* sr = scores + row * (size_t)n;

  // 1. row max as a key
  uint32_t kmax = 0;
  for (int j = tid; j < n; j += kSpThreads) kmax = max(kmax, sp_key(sr[j]));
  for (int o = 32; o > 0; o >>= 1) kmax = max(kmax, (uint32_t)__shfl_xor((int)kmax, o));
  if (tid == 0) kmax_s = 0;
  cnt[tid] = 0;
  mass[tid] = 0.0;
  __syncthreads();
  if ((tid & (kWave - 1)) == 0) atomicMax(&kmax_s, kmax);
  __syncthreads();
  const float m = bf16_to_f32(sp_unkey(kmax_s)) * scale;

  // 2. high-byte histogram of counts and weights (whole-wave iterations: every lane takes part)
  for (int j0 = 0; j0 < n; j0 += kSpThreads) {
    const int j = j0 + tid;
    const bool valid = j < n;
    const uint16_t b = valid ? sr[j] : (uint16_t)0;
    const uint32_t k = sp_key(b);
    hist_add(cnt, mass, (int)(k >> 8), valid ? (double)sp_weight(b, scale, m) : 0.0, valid);
  }
  __syncthreads();
  sp_scan(cnt, mass, dsc, isc);
  const double total = dsc[kSpThreads - 1];
  const double target = (double)threshold * total;
  const SpCross c1 = sp_find(cnt, target, dsc, isc, &found);

  // 3. low-byte counts inside the crossing bin; each sub-bin is one exact value
  cnt[tid] = 0;
  __syncthreads();
  for (int j0 = 0; j0 < n; j0 += kSpThreads) {
    const int j = j0 + tid;
    const uint32_t k = j < n ? sp_key(sr[j]) : 0u;
    count_add(cnt, (int)(k & 255), j < n && (int)(k >> 8) == c1.bin);
  }
  __syncthreads();
  {
    const int sb = 255 - tid;
    mass[sb] = (double)cnt[sb] * (double)sp_weight(sp_unkey(((uint32_t)c1.bin << 8) | (uint32_t)sb), scale, m);
  }
  __syncthreads();
  sp_scan(cnt, mass, dsc, isc);
  const double rem = target - c1.mass_above;
  const SpCross c2 = sp_find(cnt, rem, dsc, isc, &found);
  if (tid == 0) {
    const double v = (double)sp_weight(sp_unkey(((uint32_t)c1.bin << 8) | (uint32_t)c2.bin), scale, m);
    const int mult = cnt[c2.bin];
    const double need = rem - c2.mass_above;
    long long k = 1;
    if (v > 0.0 && need > 0.0) {
      k = (long long)ceil(need / v);
      // the smallest k with k * v >= need (the division may round either way)
      while (k > 1 && (double)(k - 1) * v >= need) --k;
      while (k < mult && (double)k * v < need) ++k;
    }
    k = k < 1 ? 1 : (k > mult ? mult : k);
    counts[row] = (int32_t)(c1.cnt_above + c2.cnt_above + k);
  }
}

}  // namespace svoo

using namespace svoo;

extern "C" int svoo_exact_sparsity_counts(const uint16_t* scores, long long rows, int n, float scale, float threshold,
                                          int32_t* counts, void* stream) {
  SVOO_REQUIRE(scores && counts, SVOO_ERR_INVALID_ARG, "svoo_exact_sparsity_counts: null pointer");
  SVOO_REQUIRE(rows > 0 && rows < (1ll << 31) && n > 0, SVOO_ERR_INVALID_ARG,
               "svoo_exact_sparsity_counts: bad dims rows=%lld n=%d", rows, n);
  SVOO_REQUIRE(threshold > 0.0f && threshold <= 1.0f, SVOO_ERR_INVALID_ARG,
               "svoo_exact_sparsity_counts: threshold %g outside (0, 1]", (double)threshold);
  hipLaunchKernelGGL(exact_count_kernel, dim3((unsigned)rows), dim3(kSpThreads), 0, (hipStream_t)stream, scores, n,
                     scale, threshold, counts);
  return check_launch("svoo_exact_sparsity_counts");
}
