// Centroid scores and the block-mask builder.
//
// centroid_scores_kernel (one 4-wave block per 32 key centroids of a head):
//   t_ij = bf16(f32(bf16(Qc_i . Kc_j)) * f32(1/sqrt(D)))   the reference's bf16 matmul, then "/ D**0.5"
//   The dot runs on the bf16 MFMA, one k-step (16 exact products) per accumulator, and the eight partial
//   sums are added in fp64; a second MFMA over |Qc| and |Kc| gives a = sum |q_d k_d|.  Each partial is
//   the fp32 rounding of at most 16 additions, so |r - s| <= 16 * 2^-24 * a; with e = 2^-19 a (twice that,
//   which also covers the fp32 error of a itself and the rounding of the fp64 sum to fp32) every value in
//   [r - e, r + e] rounds (via fp32) to the same bf16 as the exact dot s when its two ends do.  The entries
//   that fail this test (2-3% of them on centroid data), or whose rows hold bf16 subnormals (which the MFMA
//   may flush), are computed exactly in fp64: by their lane, or (for the mask) by the mask kernel.
//
// block_mask_kernel (one 256-thread block per (b, h, q-cluster) row):
//   p_j  = bf16(f32(w_j e^(t_j - max) / max(sum, 1e-12)))   weighted softmax, evaluated in fp64
//   order (p desc, j asc), found by two-level histograms of the bf16 bits of p (no sort)
//   prefix_t = sum_{u<=t} floor(p_u * 2^60)  (exact int64) -> bf16 -> compared with bf16(top_p)
//   kept length L = max(1 + #{t <= Kc-2 : prefix_t <= p}, preserve_h), capped by cap_h
// and the first L clusters of that order are written back as 1 in the bool map.
#include "svoo_common.h"

namespace svoo {

constexpr int kMaskThreads = 256;

constexpr int kScoreThreads = 256;

// Dot of two bf16 rows of 128 in fp64 by 16 lanes (aligned groups of 16; lane c of the group takes the
// 16-byte chunk c of both rows): the products are exact in fp64, and so is their sum while the products'
// exponents span less than 2^30 (beyond that the sum is rounded in a fixed order).  Every lane of the group
// returns the dot.  `valid` may differ between groups; all 64 lanes must call it together.
__device__ __forceinline__ double group16_dot128(const uint16_t* __restrict__ x, const uint16_t* __restrict__ y,
                                                 bool valid) {
  const int c = threadIdx.x % 16;
  double acc = 0.0;
  if (valid) {
    const u32x4_t a = ((const u32x4_t*)x)[c], b = ((const u32x4_t*)y)[c];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      acc = fma((double)bf16_to_f32((uint16_t)(a[e] & 0xffffu)), (double)bf16_to_f32((uint16_t)(b[e] & 0xffffu)), acc);
      acc = fma((double)bf16_to_f32((uint16_t)(a[e] >> 16)), (double)bf16_to_f32((uint16_t)(b[e] >> 16)), acc);
    }
  }
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
  return acc;
}

// 1 when any of the 8 bf16 values of w is subnormal (exponent 0, mantissa not 0).
__device__ __forceinline__ uint32_t has_subnormal(u32x4_t w) {
  uint32_t any = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t lo = w[e] & 0xffffu, hi = w[e] >> 16;
    any |= ((lo & 0x7f80u) == 0 && (lo & 0x7fu) != 0) | ((hi & 0x7f80u) == 0 && (hi & 0x7fu) != 0);
  }
  return any;
}

// Marks an entry whose certificate failed when the exact dot is left to the mask kernel (not a value
// f32_to_bf16 produces: its NaNs are 0x7fc0).
constexpr uint16_t kDeferredScore = 0xffffu;
// k-steps (16 products each) summed in fp32 per partial; the partials are added in fp64.  The certificate's
// half-width is 2^-24 * 32 * kStepsPerPartial * a: twice the worst-case fp32 rounding of a partial of
// 16 * kStepsPerPartial products, which also covers the fp32 error of a itself and the final rounding.
constexpr int kStepsPerPartial = 1;

// Lane layout (v_mfma_f32_32x32x16_bf16, keys on M, query centroids on N): lane (l32, h) supplies key
// row kt*32 + l32 and query row qt*32 + l32, the 8 values at d = 64h + 8s in k-step s (the same
// permutation of the contraction index in both operands), and receives entry r at key (r/4)*8 + 4h + r%4,
// query l32.  defer != 0 writes kDeferredScore for the entries that fail the certificate instead of
// recomputing them.
__global__ void __launch_bounds__(kScoreThreads) __attribute__((amdgpu_waves_per_eu(2, 8)))
centroid_scores_kernel(const uint16_t* __restrict__ qc, const uint16_t* __restrict__ kc, int qn, int kn,
                       float inv_sqrt_d, int defer, uint16_t* __restrict__ out) {
  const int b = blockIdx.y, kt = blockIdx.x;
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave, h = lane / 32, l32 = lane % 32;
  const int qtiles = (qn + 31) / 32;
  const int jrow = min(kt * 32 + l32, kn - 1);
  const uint16_t* kbase = kc + (size_t)b * kn * 128;
  const uint16_t* qbase = qc + (size_t)b * qn * 128;
  u32x4_t ka[8];
  uint32_t ksub = 0;
  {
    const u32x4_t* src = (const u32x4_t*)(kbase + (size_t)jrow * 128) + 8 * h;
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      ka[st] = src[st];
      ksub |= has_subnormal(ka[st]);
    }
  }
  // key rows (of this tile) holding a subnormal, as a bit mask over l32
  const uint64_t kmask64 = __ballot(ksub != 0);
  const uint32_t kmask = (uint32_t)kmask64 | (uint32_t)(kmask64 >> 32);
  const u32x4_t absm = {0x7fff7fffu, 0x7fff7fffu, 0x7fff7fffu, 0x7fff7fffu};
  const float half_width = 0x1p-24f * (float)(32 * kStepsPerPartial);
  __shared__ uint16_t redo_list[kScoreThreads / kWave][kWave * 16];
  for (int qt = wave; qt < qtiles; qt += kScoreThreads / kWave) {
    const int i = qt * 32 + l32, irow = min(i, qn - 1);
    u32x4_t qb[8];
    uint32_t qsub = 0;
    {
      const u32x4_t* src = (const u32x4_t*)(qbase + (size_t)irow * 128) + 8 * h;
#pragma unroll
      for (int st = 0; st < 8; ++st) {
        qb[st] = src[st];
        qsub |= has_subnormal(qb[st]);
      }
    }
    // this lane's query row holds a subnormal (either half)
    const auto qsw = __builtin_amdgcn_permlane32_swap(qsub, qsub, false, false);
    const uint32_t qsub_row = qsw[0] | qsw[1];
    // partials of kStepsPerPartial k-steps each, summed in fp64 as they come
    double sd[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) sd[r] = 0.0;
#pragma unroll
    for (int p0 = 0; p0 < 8; p0 += kStepsPerPartial) {
      f32x16_t part = f32x16_t{};
#pragma unroll
      for (int st = p0; st < p0 + kStepsPerPartial; ++st)
        part = mfma32x32x16(as_bf16x8(ka[st]), as_bf16x8(qb[st]), part);
#pragma unroll
      for (int r = 0; r < 16; ++r) sd[r] += (double)part[r];
    }
    f32x16_t asum = f32x16_t{};
#pragma unroll
    for (int st = 0; st < 8; ++st)
      asum = mfma32x32x16(as_bf16x8(ka[st] & absm), as_bf16x8(qb[st] & absm), asum);
    // entries whose certificate fails: bit r of `redo`
    uint32_t redo = 0;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      uint32_t packed[2] = {0u, 0u};
      const int j0 = kt * 32 + g * 8 + 4 * h;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = 4 * g + e;
        const float rs = (float)sd[r];
        const float a = asum[r];
        const float err = fmaf(a, half_width, 0x1p-118f);
        const uint16_t sb = f32_to_bf16(rs - err);
        const bool sub = ((kmask >> (g * 8 + 4 * h + e)) & 1u) != 0 || qsub_row != 0;
        uint32_t tb = f32_to_bf16(bf16_to_f32(sb) * inv_sqrt_d);
        if (sub || !(a <= 3.0e38f) || sb != f32_to_bf16(rs + err)) {
          redo |= 1u << r;
          if (defer) tb = kDeferredScore;
        }
        packed[e / 2] |= tb << (16 * (e % 2));
      }
      if (i < qn) {
        uint16_t* dst = out + ((size_t)b * qn + i) * kn + j0;
        if (j0 + 3 < kn && (kn % 4) == 0)
          *(uint2*)dst = make_uint2(packed[0], packed[1]);
        else
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (j0 + e < kn) dst[e] = (uint16_t)(packed[e / 2] >> (16 * (e % 2)));
      }
    }
    // The failed entries again, exactly in fp64, four at a time by groups of 16 lanes (listed in this wave's
    // LDS slice as lane << 4 | r); their stores come after the first ones, in the same wave.
    if (!defer) {
      if (i >= qn) redo = 0;
      const int nmine = __builtin_popcount(redo);
      int pos = nmine;
#pragma unroll
      for (int o = 1; o < kWave; o <<= 1) {
        const int n = __shfl_up(pos, o);
        if (lane >= o) pos += n;
      }
      const int total = __shfl(pos, kWave - 1);
      pos -= nmine;
      uint16_t* list = redo_list[wave];
      while (redo) {
        const int r = __builtin_ctz(redo);
        redo &= redo - 1;
        list[pos++] = (uint16_t)((lane << 4) | r);
      }
      __builtin_amdgcn_wave_barrier();
      for (int base = 0; base < total; base += 4) {
        const int slot = base + lane / 16;
        const bool valid = slot < total;
        int ii = 0, jj = 0;
        if (valid) {
          const int ent = list[slot], ln = ent >> 4, r = ent & 15;
          ii = qt * 32 + (ln % 32);
          jj = kt * 32 + (r / 4) * 8 + 4 * (ln / 32) + (r % 4);
        }
        const bool ok = valid && jj < kn;
        const double dot = group16_dot128(qbase + (size_t)ii * 128, kbase + (size_t)min(jj, kn - 1) * 128, ok);
        if (ok && lane % 16 == 0)
          out[((size_t)b * qn + ii) * kn + jj] = f32_to_bf16(bf16_to_f32(f32_to_bf16((float)dot)) * inv_sqrt_d);
      }
      __builtin_amdgcn_wave_barrier();
    }
  }
}

// ------------------------------------------------------------------------------------------ block mask
// The sort keys are the bf16 bits of p (p >= 0, so they order as unsigned integers like the values):
// bin = key >> 7 (the exponent), sub-bin = key & 127 (the mantissa), so a sub-bin holds one value.
constexpr int kBins = 128;

// bf16(f32(x * 2^-60)) <= p_st for a fixed-point prefix x (monotone in x)
__device__ __forceinline__ bool prefix_within(long long x, float p_st) {
  return bf16_round_f32((float)((double)x * 0x1p-60)) <= p_st;
}

// floor(p * 2^60) of a bf16 probability key
__device__ __forceinline__ long long fixed60(uint32_t key) {
  const float p = bf16_to_f32((uint16_t)key);
  return p > 0.0f ? (long long)ldexp((double)p, 60) : 0ll;
}

// Inclusive scans over the 64 lanes of a wave.
__device__ __forceinline__ long long wave_incl_scan_i64(long long v) {
  const int l = threadIdx.x % kWave;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const long long n = __shfl_up(v, o);
    if (l >= o) v += n;
  }
  return v;
}
__device__ __forceinline__ int wave_incl_scan_i32(int v) {
  const int l = threadIdx.x % kWave;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int n = __shfl_up(v, o);
    if (l >= o) v += n;
  }
  return v;
}

// Thread t owns entries j = E t .. E t + E - 1.  The kept set is the first L clusters in the order (p desc,
// j asc); instead of sorting, the kernel finds where that order crosses the top-p threshold and where it
// reaches L from histograms of the keys:
//   level 1: count and fixed-point mass per exponent bin; a scan over the bins (descending) finds the bin in
//            which the prefix first leaves the threshold;
//   level 2: counts per mantissa (one value each, so its mass is count * fx) inside that bin; a scan finds
//            the value, and within it (equal values, index order) the crossing position follows from
//            base + (r + 1) * fx by a binary search;
// the same two levels by count find the key and the rank among equal keys of position L - 1, and a scan of
// the equal-key indicator in index order gives each entry its rank.
template <int KP>
__global__ void __launch_bounds__(kMaskThreads) block_mask_kernel(uint16_t* __restrict__ scores,
                                                                  const uint16_t* __restrict__ qc,
                                                                  const uint16_t* __restrict__ kc,
                                                                  const int32_t* __restrict__ ksz,
                                                                  const int32_t* __restrict__ preserve,
                                                                  const int32_t* __restrict__ cap, int h, int qn,
                                                                  int kn, float inv_sqrt_d, float p_st,
                                                                  uint8_t* __restrict__ map,
                                                                  int32_t* __restrict__ lengths) {
  constexpr int E = KP / kMaskThreads;  // entries per thread
  __shared__ uint32_t cnt1[kBins], ccum1[kBins], cnt2[kBins];
  __shared__ unsigned long long mass1[kBins];
  __shared__ double red_d[kMaskThreads / kWave];
  __shared__ float red_f[kMaskThreads / kWave];
  __shared__ long long red_l[kMaskThreads / kWave];
  __shared__ long long bc[4];  // broadcast slots
  __shared__ uint16_t dlist[KP], tfix[KP];
  __shared__ int ndef;

  const int bh = blockIdx.y, i = blockIdx.x, tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const int head = bh % h;
  const size_t row = (size_t)bh * qn + i;
  uint8_t* mrow = map + row * kn;
  uint16_t* trow = scores + row * kn;
  const uint16_t* qrow = qc + row * 128;
  const uint16_t* kb = kc + (size_t)bh * kn * 128;

  // Scores.  The entries the score kernel could not certify are listed, computed exactly here (16 at a time,
  // 16 lanes each) and written back; then the row max.
  if (tid == 0) ndef = 0;
  __syncthreads();
  uint16_t tb[E];
  uint32_t deferred = 0;
#pragma unroll
  for (int u = 0; u < E; ++u) {
    const int j = tid * E + u;
    tb[u] = j < kn ? trow[j] : 0;
    if (j < kn && tb[u] == kDeferredScore) {
      deferred |= 1u << u;
      dlist[atomicAdd(&ndef, 1)] = (uint16_t)j;
    }
  }
  __syncthreads();
  const int nd = ndef;
  if (nd > 0) {
    for (int base = 0; base < nd; base += kMaskThreads / 16) {
      const int slot = base + tid / 16;
      const bool valid = slot < nd;
      const int j = valid ? dlist[slot] : 0;
      const double dot = group16_dot128(qrow, kb + (size_t)j * 128, valid);
      if (valid && tid % 16 == 0) {
        const uint16_t bits = f32_to_bf16(bf16_to_f32(f32_to_bf16((float)dot)) * inv_sqrt_d);
        tfix[j] = bits;
        trow[j] = bits;
      }
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < E; ++u)
      if (deferred & (1u << u)) tb[u] = tfix[tid * E + u];
  }
  float tv[E];
  float lmax = -INFINITY;
#pragma unroll
  for (int u = 0; u < E; ++u) {
    tv[u] = tid * E + u < kn ? bf16_to_f32(tb[u]) : -INFINITY;
    lmax = fmaxf(lmax, tv[u]);
  }
  const float m = block_max_f32<kMaskThreads>(lmax, red_f);

  // Weighted softmax in fp64 -> bf16 probability keys.
  const int32_t* wrow = ksz + (size_t)bh * kn;
  double we[E];
  double lsum = 0.0;
#pragma unroll
  for (int u = 0; u < E; ++u) {
    const int j = tid * E + u;
    we[u] = 0.0;
    if (j < kn) {
      we[u] = (double)wrow[j] * exp((double)tv[u] - (double)m);
      lsum += we[u];
    }
  }
  const double den = fmax(block_sum_f64<kMaskThreads>(lsum, red_d), 1e-12);
  uint32_t key[E];
#pragma unroll
  for (int u = 0; u < E; ++u) key[u] = f32_to_bf16((float)(we[u] / den));

  // Level 1: counts and masses per exponent bin.
  if (tid < kBins) {
    cnt1[tid] = 0;
    mass1[tid] = 0;
  }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < E; ++u) {
    if (tid * E + u < kn) {
      // (a NaN key, from NaN scores, lands in the top bin instead of outside the table)
      atomicAdd(&cnt1[(key[u] >> 7) & (kBins - 1)], 1u);
      atomicAdd(&mass1[(key[u] >> 7) & (kBins - 1)], (unsigned long long)fixed60(key[u]));
    }
  }
  __syncthreads();
  // Wave 0 scans the bins in descending order (lane l: positions 2l, 2l + 1 = bins 127 - 2l, 126 - 2l) and
  // finds the first bin whose inclusive prefix leaves the threshold.
  if (wave == 0) {
    const int b0 = kBins - 1 - 2 * lane, b1 = b0 - 1;
    const int c0 = (int)cnt1[b0], c1 = (int)cnt1[b1];
    const long long m0 = (long long)mass1[b0], m1 = (long long)mass1[b1];
    const int ci = wave_incl_scan_i32(c0 + c1);
    const long long mi = wave_incl_scan_i64(m0 + m1);
    const int ce = ci - c0 - c1;
    const long long me = mi - m0 - m1;
    ccum1[2 * lane] = (uint32_t)(ce + c0);
    ccum1[2 * lane + 1] = (uint32_t)ci;
    const bool out0 = !prefix_within(me + m0, p_st), out1 = !prefix_within(mi, p_st);
    const uint64_t any = __ballot(out0 || out1);
    if (any == 0) {
      if (lane == 0) bc[0] = -1;
    } else if (lane == __builtin_ctzll(any)) {
      const bool first = out0;
      bc[0] = first ? 2 * lane : 2 * lane + 1;   // position of the bin
      bc[1] = first ? me : me + m0;              // mass before it
      bc[2] = first ? ce : ce + c0;              // entries before it
    }
  }
  __syncthreads();
  const int dstar = (int)bc[0];
  long long T = kn;  // leading positions whose prefix stays within the threshold
  if (dstar >= 0) {
    const int bstar = kBins - 1 - dstar;
    // Level 2 inside that bin: counts per mantissa.
    if (tid < kBins) cnt2[tid] = 0;
    __syncthreads();
#pragma unroll
    for (int u = 0; u < E; ++u)
      if (tid * E + u < kn && (int)((key[u] >> 7) & (kBins - 1)) == bstar) atomicAdd(&cnt2[key[u] & 127], 1u);
    __syncthreads();
    if (wave == 0) {
      const long long base_m = bc[1], base_c = bc[2];
      const int s0 = kBins - 1 - 2 * lane, s1 = s0 - 1;
      const uint32_t k0 = ((uint32_t)bstar << 7) | (uint32_t)s0, k1 = ((uint32_t)bstar << 7) | (uint32_t)s1;
      const int c0 = (int)cnt2[s0], c1 = (int)cnt2[s1];
      const long long f0 = fixed60(k0), f1 = fixed60(k1);
      const long long m0 = (long long)c0 * f0, m1 = (long long)c1 * f1;
      const int ci = wave_incl_scan_i32(c0 + c1);
      const long long mi = wave_incl_scan_i64(m0 + m1);
      const int ce = ci - c0 - c1;
      const long long me = mi - m0 - m1;
      const bool out0 = !prefix_within(base_m + me + m0, p_st), out1 = !prefix_within(base_m + mi, p_st);
      const uint64_t any = __ballot(out0 || out1);
      if (any != 0 && lane == __builtin_ctzll(any)) {
        const bool first = out0;
        const long long mb = base_m + (first ? me : me + m0);
        const long long fx = first ? f0 : f1;
        const int cnt = first ? c0 : c1;
        // smallest r in [0, cnt) with the prefix mb + (r + 1) fx outside the threshold
        int lo = 0, hi = cnt - 1;
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          if (!prefix_within(mb + (long long)(mid + 1) * fx, p_st))
            hi = mid;
          else
            lo = mid + 1;
        }
        bc[3] = base_c + (first ? ce : ce + c0) + lo;
      }
    }
    __syncthreads();
    T = bc[3];
  }
  int len = 1 + (int)min(T, (long long)(kn - 1));
  len = max(len, (int)preserve[head]);
  if (cap[head] > 0) len = min(len, (int)cap[head]);
  len = min(len, kn);

  // The key and the rank among equal keys of position len - 1.
  uint32_t key_l = 0;
  int rank_l = 0;
  if (len < kn) {
    __syncthreads();  // bc and cnt2 are read above
    if (wave == 0) {
      const bool r0 = (int)ccum1[2 * lane] >= len, r1 = (int)ccum1[2 * lane + 1] >= len;
      const uint64_t any = __ballot(r0 || r1);
      if (lane == __builtin_ctzll(any)) {
        const int d = r0 ? 2 * lane : 2 * lane + 1;
        bc[0] = d;
        bc[1] = d > 0 ? (long long)ccum1[d - 1] : 0;
      }
    }
    __syncthreads();
    const int dl = (int)bc[0];
    const int bl = kBins - 1 - dl;
    if (dl != dstar) {  // block-uniform: rebuild the level-2 counts for this bin
      if (tid < kBins) cnt2[tid] = 0;
      __syncthreads();
#pragma unroll
      for (int u = 0; u < E; ++u)
        if (tid * E + u < kn && (int)((key[u] >> 7) & (kBins - 1)) == bl) atomicAdd(&cnt2[key[u] & 127], 1u);
      __syncthreads();
    }
    if (wave == 0) {
      const long long base_c = bc[1];
      const int s0 = kBins - 1 - 2 * lane, s1 = s0 - 1;
      const int c0 = (int)cnt2[s0], c1 = (int)cnt2[s1];
      const int ci = wave_incl_scan_i32(c0 + c1);
      const int ce = ci - c0 - c1;
      const bool r0 = base_c + ce + c0 >= len, r1 = base_c + ci >= len;
      const uint64_t any = __ballot(r0 || r1);
      if (lane == __builtin_ctzll(any)) {
        const bool first = r0;
        bc[2] = ((long long)bl << 7) | (first ? s0 : s1);
        bc[3] = len - 1 - (base_c + (first ? ce : ce + c0));
      }
    }
    __syncthreads();
    key_l = (uint32_t)bc[2];
    rank_l = (int)bc[3];
  }

  // Rank of each entry among the entries with key key_l, in index order; kept = ahead of position len - 1.
  int eq = 0;
#pragma unroll
  for (int u = 0; u < E; ++u) eq += (tid * E + u < kn && key[u] == key_l) ? 1 : 0;
  long long tot;
  int rank = (int)block_exclusive_scan_i64<kMaskThreads>(eq, red_l, &tot);
  uint32_t word = 0;
#pragma unroll
  for (int u = 0; u < E; ++u) {
    bool keep = true;
    if (len < kn) {
      keep = key[u] > key_l;
      if (key[u] == key_l) keep = rank++ <= rank_l;
    }
    if (tid * E + u < kn && keep) word |= 1u << (8 * (u % 4));
    if (u % 4 == 3 || u == E - 1) {
      const int j0 = tid * E + (u / 4) * 4;
      if ((kn & 3) == 0 && E >= 4) {
        if (j0 < kn) *(uint32_t*)(mrow + j0) = word;
      } else {
        for (int e = 0; e <= u % 4; ++e)
          if (j0 + e < kn) mrow[j0 + e] = (uint8_t)(word >> (8 * e));
      }
      word = 0;
    }
  }
  if (tid == 0 && lengths) lengths[row] = len;
}

// All-true map rows (top_p >= 1, svoo/co_clustering.py:575-576).
__global__ void __launch_bounds__(kMaskThreads) full_mask_kernel(uint8_t* __restrict__ map, int qn, int kn,
                                                                 int32_t* __restrict__ lengths) {
  const size_t row = (size_t)blockIdx.y * qn + blockIdx.x;
  uint8_t* mrow = map + row * kn;
  for (int j = threadIdx.x; j < kn; j += kMaskThreads) mrow[j] = 1;
  if (threadIdx.x == 0 && lengths) lengths[row] = kn;
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

extern "C" int svoo_centroid_scores(const uint16_t* qc, const uint16_t* kc, int bh, int qn, int kn, int d,
                                    uint16_t* scores, void* stream) {
  SVOO_REQUIRE(qc && kc && scores, SVOO_ERR_INVALID_ARG, "svoo_centroid_scores: null pointer");
  SVOO_REQUIRE(bh > 0 && qn > 0 && kn > 0, SVOO_ERR_INVALID_ARG, "svoo_centroid_scores: bad dims");
  SVOO_REQUIRE_HEAD_DIM(d, "svoo_centroid_scores");
  SVOO_REQUIRE(bh <= 65535 && kn <= (1 << 26), SVOO_ERR_UNSUPPORTED, "svoo_centroid_scores: grid too large");
  const float inv = 1.0f / (float)sqrt((double)d);
  hipLaunchKernelGGL(centroid_scores_kernel, dim3((kn + 31) / 32, bh), dim3(kScoreThreads), 0, (hipStream_t)stream,
                     qc, kc, qn, kn, inv, 0, scores);
  return check_launch("svoo_centroid_scores");
}

extern "C" int svoo_block_mask(const uint16_t* qc, const uint16_t* kc, const int32_t* k_sizes,
                               const int32_t* preserve, const int32_t* cap, int b, int h, int qn, int kn, int d,
                               float p_storage, int full, uint8_t* map, int32_t* lengths, uint16_t* scores,
                               void* stream) {
  SVOO_REQUIRE(map && (full || (qc && kc && k_sizes && preserve && cap && scores)), SVOO_ERR_INVALID_ARG,
               "svoo_block_mask: null pointer");
  SVOO_REQUIRE(b > 0 && h > 0 && qn > 0 && kn > 0, SVOO_ERR_INVALID_ARG, "svoo_block_mask: bad dims");
  SVOO_REQUIRE_HEAD_DIM(d, "svoo_block_mask");
  SVOO_REQUIRE(kn <= 4096, SVOO_ERR_UNSUPPORTED, "svoo_block_mask: Kc=%d exceeds 4096", kn);
  SVOO_REQUIRE(qn <= 65535 && (long long)b * h <= 65535, SVOO_ERR_UNSUPPORTED, "svoo_block_mask: grid too large");
  dim3 grid(qn, b * h);
  hipStream_t s = (hipStream_t)stream;
  if (full) {
    hipLaunchKernelGGL(full_mask_kernel, grid, dim3(kMaskThreads), 0, s, map, qn, kn, lengths);
    return check_launch("svoo_block_mask");
  }
  const float inv = 1.0f / (float)sqrt((double)d);
  // scores with the uncertified entries deferred to the mask kernel, which computes them exactly
  hipLaunchKernelGGL(centroid_scores_kernel, dim3((kn + 31) / 32, b * h), dim3(kScoreThreads), 0, s, qc, kc, qn, kn,
                     inv, 1, scores);
  if (int rc = check_launch("svoo_block_mask (scores)")) return rc;
#define SVOO_MASK_LAUNCH(KP)                                                                                     \
  hipLaunchKernelGGL(block_mask_kernel<KP>, grid, dim3(kMaskThreads), 0, s, scores, qc, kc, k_sizes, preserve, cap, \
                     h, qn, kn, inv, p_storage, map, lengths)
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
