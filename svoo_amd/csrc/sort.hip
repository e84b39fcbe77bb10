// Stable counting sort of cluster labels (per batch-head row).
//
// Three HBM-light passes over labels[BH][N] (int32):
//   1. hist:    per 1024-token chunk, an LDS histogram -> counts[b][chunk][k]   (chunk-major, so the
//               write of a chunk's histogram and the scatter's read of its bases are contiguous)
//   2. scan:    per row, exclusive scan of counts in (cluster, chunk) order      -> chunk bases,
//               sizes[b][k] and offsets[b][k]; one thread per cluster sums its chunks, a block
//               scan gives the cluster offsets, and the thread walks its chunks again
//   3. scatter: one wave per chunk walks its tokens in order, 64 at a time; the lanes holding the
//               same label are found with one ballot per label bit (ceil(log2 K) ballots), and
//               ranked by lane order (popcount of the lower lanes), so equal labels keep their
//               original token order (stable).  A cluster's output lines collect one or two tokens
//               from each of ~70 chunks (K = 1000, N = 75600): with a head's chunks on one XCD the
//               4-byte writes merge in that XCD's L2 (81 -> 58 us per key-side sort at C3).
// A launch of the three passes sorts the rows of one or two independent sorts (SortSide), so that the
// co-clustering's two final sorts share their launches.
#include "svoo_common.h"

namespace svoo {

constexpr int kSortChunk = 1024;
constexpr int kMaxSortClusters = 16384;

// One sort of a launch: a launch sorts the rows of one or two of them (rows [0, bh_a) the first, the rest the
// second), so that two independent sorts share their three launches.
struct SortSide {
  const int32_t* labels;
  int32_t* counts;
  int32_t* sizes;
  int32_t* offsets;
  int32_t* sorted_idx;
  int32_t* sorted_labels;
  int k, kbits;
};

// With zs the blocks also clear zn doubles at zs (grid-stride; the sums a recount then accumulates into).
__global__ void __launch_bounds__(256) sort_hist_kernel(SortSide sa, SortSide sb, int bh_a, int n, int nchunks,
                                                        int32_t* __restrict__ err, const int32_t* __restrict__ guard,
                                                        int limit, double* __restrict__ zs, long long zn) {
  if (guard && *guard <= limit) return;
  if (zs) {
    const long long step = (long long)gridDim.x * gridDim.y * blockDim.x;
    for (long long i = ((long long)blockIdx.y * gridDim.x + blockIdx.x) * blockDim.x + threadIdx.x; i < zn; i += step)
      zs[i] = 0.0;
  }
  extern __shared__ int32_t hist[];
  const bool second = (int)blockIdx.y >= bh_a;
  const SortSide& S = second ? sb : sa;
  const int b = second ? blockIdx.y - bh_a : blockIdx.y, c = blockIdx.x, k = S.k;
  int32_t* counts = S.counts;
  for (int i = threadIdx.x; i < k; i += blockDim.x) hist[i] = 0;
  __syncthreads();
  const int32_t* lab = S.labels + (size_t)b * n;
  const int s = c * kSortChunk, e = min(n, s + kSortChunk);
  bool bad = false;
  for (int t = s + threadIdx.x; t < e; t += blockDim.x) {
    const int l = lab[t];
    if ((unsigned)l < (unsigned)k)
      atomicAdd(&hist[l], 1);
    else
      bad = true;
  }
  if (bad && err) atomicOr(err, 1);
  __syncthreads();
  int32_t* out = counts + (size_t)b * k * nchunks;
  for (int i = threadIdx.x; i < k; i += blockDim.x) out[(size_t)c * k + i] = hist[i];  // [chunk][cluster]
}

constexpr int kScanWaves = 16;

__device__ __forceinline__ int wave_inclusive_scan(int v, int lane) {
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int n = __shfl_up(v, o);
    if (lane >= o) v += n;
  }
  return v;
}

// counts [chunk][cluster] -> bases (in place): base of (chunk c, cluster i) = offset of cluster i + the counts of
// cluster i in chunks before c, which is the stable order (cluster, then token).  One thread per cluster, 1024
// clusters per pass; every access of a chunk row is contiguous over the threads.
__global__ void __launch_bounds__(kScanWaves * kWave) sort_scan_kernel(SortSide sa, SortSide sb, int bh_a, int nchunks,
                                                                       const int32_t* __restrict__ guard, int limit) {
  if (guard && *guard <= limit) return;
  __shared__ int wsum[kScanWaves];
  const bool second = (int)blockIdx.x >= bh_a;
  const SortSide& S = second ? sb : sa;
  const int k = S.k;
  int32_t* counts = S.counts;
  int32_t* sizes = S.sizes;
  int32_t* offsets = S.offsets;
  const int b = second ? blockIdx.x - bh_a : blockIdx.x, tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  int32_t* cnt = counts + (size_t)b * k * nchunks;
  int carry = 0;  // clusters of the earlier passes
  for (int i0 = 0; i0 < k; i0 += kScanWaves * kWave) {
    const int i = i0 + tid;
    int tot = 0;
    if (i < k) {
#pragma unroll 8
      for (int c = 0; c < nchunks; ++c) tot += cnt[(size_t)c * k + i];
    }
    const int inc = wave_inclusive_scan(tot, lane);
    if (lane == kWave - 1) wsum[wave] = inc;
    __syncthreads();
    int before = 0, all = 0;
#pragma unroll
    for (int w = 0; w < kScanWaves; ++w) {
      before += w < wave ? wsum[w] : 0;
      all += wsum[w];
    }
    if (i < k) {
      const int start = carry + before + inc - tot;
      offsets[(size_t)b * k + i] = start;
      sizes[(size_t)b * k + i] = tot;
      int run = start;
#pragma unroll 8
      for (int c = 0; c < nchunks; ++c) {
        const int v = cnt[(size_t)c * k + i];
        cnt[(size_t)c * k + i] = run;
        run += v;
      }
    }
    carry += all;
    __syncthreads();  // wsum is rewritten by the next pass
  }
}

__global__ void __launch_bounds__(64) sort_scatter_kernel(SortSide sa, SortSide sb, int bh_a, int rows, int n,
                                                          int nchunks, const int32_t* __restrict__ guard, int limit) {
  if (guard && *guard <= limit) return;
  extern __shared__ int32_t base[];
  // XCD-aware order: workgroup L runs on XCD L % 8, so with the row count a multiple of 8 row y's chunks all go
  // to XCD y % 8 and the scattered writes of a cluster's output lines merge in one L2
  int y, c;
  const int L = blockIdx.x, lane = threadIdx.x;
  if (rows % 8 == 0) {
    const int xcd = L % 8, sl = L / 8;
    y = (sl / nchunks) * 8 + xcd;
    c = sl % nchunks;
  } else {
    y = L / nchunks;
    c = L % nchunks;
  }
  const bool second = y >= bh_a;
  const SortSide& S = second ? sb : sa;
  const int b = second ? y - bh_a : y, k = S.k, kbits = S.kbits;
  const int32_t* bs = S.counts + (size_t)b * k * nchunks;
  for (int i = lane; i < k; i += kWave) base[i] = bs[(size_t)c * k + i];
  __syncthreads();
  const int32_t* lab = S.labels + (size_t)b * n;
  int32_t* out = S.sorted_idx + (size_t)b * n;
  int32_t* outl = S.sorted_labels ? S.sorted_labels + (size_t)b * n : nullptr;
  const int s = c * kSortChunk, e = min(n, s + kSortChunk);
  const unsigned long long below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int t0 = s; t0 < e; t0 += kWave) {
    const int t = t0 + lane;
    int l = t < e ? lab[t] : -1;
    if ((unsigned)l >= (unsigned)k) l = -1;  // out-of-range labels were flagged by the hist pass
    // Lanes with the same label: one ballot per label bit.
    unsigned long long same = __ballot(l >= 0);
    for (int bit = 0; bit < kbits; ++bit) {
      const bool on = (l >> bit) & 1;
      const unsigned long long bal = __ballot(on);
      same &= on ? bal : ~bal;
    }
    if (l >= 0) {
      const int rank = __popcll(same & below);
      const int cnt = __popcll(same);
      const int bval = base[l];
      const int pos = bval + rank;
      if ((unsigned)pos < (unsigned)n) {  // always true for consistent bases; guards memory anyway
        out[pos] = t;
        if (outl) outl[pos] = l;
      }
      if (rank == cnt - 1) base[l] = bval + cnt;
    }
    __builtin_amdgcn_wave_barrier();
  }
}

}  // namespace svoo

using namespace svoo;

static inline int sort_nchunks(int n) { return (n + kSortChunk - 1) / kSortChunk; }

extern "C" size_t svoo_cluster_sort_workspace_size(int bh, int n, int k) {
  if (bh <= 0 || n <= 0 || k <= 0) return 256;
  return ((size_t)bh * k * sort_nchunks(n) * sizeof(int32_t) + 255) / 256 * 256 + 256;
}

// Internal entry used by the co-clustering driver: the workspace pointer is already sized.
// With a guard the three kernels do their work only when *guard > limit (a count on the device; the
// co-clustering's choice between a full recount and the incremental update); then the histogram pass also
// clears zn doubles at zero_sums when given.
static SortSide sort_side(const int32_t* labels, int k, int32_t* sorted_idx, int32_t* sizes, int32_t* offsets,
                          int32_t* sorted_labels, int32_t* counts) {
  int kbits = 0;
  while ((1 << kbits) < k) ++kbits;
  return SortSide{labels, counts, sizes, offsets, sorted_idx, sorted_labels, k, kbits};
}

static int sort_launch(const SortSide& sa, const SortSide& sb, int bh_a, int bh_b, int n, int32_t* err,
                       hipStream_t stream, const int32_t* guard, int limit, double* zero_sums, long long zero_n) {
  const int nch = sort_nchunks(n), rows = bh_a + bh_b, kmax = max(sa.k, bh_b ? sb.k : 0);
  SVOO_REQUIRE((long long)kmax * nch < (1ll << 31), SVOO_ERR_UNSUPPORTED,
               "svoo_cluster_sort: k=%d x %d chunks too large", kmax, nch);
  hipLaunchKernelGGL(sort_hist_kernel, dim3(nch, rows), dim3(256), kmax * sizeof(int32_t), stream, sa, sb, bh_a, n,
                     nch, err, guard, limit, zero_sums, zero_n);
  hipLaunchKernelGGL(sort_scan_kernel, dim3(rows), dim3(kScanWaves * kWave), 0, stream, sa, sb, bh_a, nch, guard,
                     limit);
  hipLaunchKernelGGL(sort_scatter_kernel, dim3(nch * rows), dim3(64), kmax * sizeof(int32_t), stream, sa, sb, bh_a,
                     rows, n, nch, guard, limit);
  return check_launch("svoo_cluster_sort");
}

// Internal entry used by the co-clustering driver: the workspace pointer is already sized.
// With a guard the three kernels do their work only when *guard > limit (a count on the device; the
// co-clustering's choice between a full recount and the incremental update); then the histogram pass also
// clears zn doubles at zero_sums when given.
int svoo_cluster_sort_impl(const int32_t* labels, int bh, int n, int k, int32_t* sorted_idx, int32_t* sizes,
                           int32_t* offsets, int32_t* sorted_labels, int32_t* counts, int32_t* err,
                           hipStream_t stream, const int32_t* guard, int limit, double* zero_sums, long long zero_n) {
  const SortSide sa = sort_side(labels, k, sorted_idx, sizes, offsets, sorted_labels, counts);
  return sort_launch(sa, sa, bh, 0, n, err, stream, guard, limit, zero_sums, zero_n);
}

// Two independent sorts of bh rows each (their own counts workspaces) in one set of three launches.
int svoo_cluster_sort2_impl(const int32_t* labels_a, int k_a, int32_t* sorted_idx_a, int32_t* sizes_a,
                            int32_t* offsets_a, int32_t* sorted_labels_a, int32_t* counts_a, const int32_t* labels_b,
                            int k_b, int32_t* sorted_idx_b, int32_t* sizes_b, int32_t* offsets_b,
                            int32_t* sorted_labels_b, int32_t* counts_b, int bh, int n, hipStream_t stream) {
  const SortSide sa = sort_side(labels_a, k_a, sorted_idx_a, sizes_a, offsets_a, sorted_labels_a, counts_a);
  const SortSide sb = sort_side(labels_b, k_b, sorted_idx_b, sizes_b, offsets_b, sorted_labels_b, counts_b);
  return sort_launch(sa, sb, bh, bh, n, nullptr, stream, nullptr, 0, nullptr, 0);
}

extern "C" int svoo_cluster_sort(const int32_t* labels, int bh, int n, int k, int32_t* sorted_idx, int32_t* sizes,
                                 int32_t* offsets, int32_t* sorted_labels, void* workspace, size_t ws_bytes,
                                 void* stream) {
  SVOO_REQUIRE(labels && sorted_idx && sizes && offsets, SVOO_ERR_INVALID_ARG, "svoo_cluster_sort: null pointer");
  SVOO_REQUIRE(bh > 0 && n > 0 && k > 0, SVOO_ERR_INVALID_ARG, "svoo_cluster_sort: bad dims bh=%d n=%d k=%d", bh,
               n, k);
  SVOO_REQUIRE(k <= kMaxSortClusters, SVOO_ERR_UNSUPPORTED, "svoo_cluster_sort: k=%d exceeds %d", k,
               kMaxSortClusters);
  SVOO_REQUIRE((long long)bh * n < (1ll << 31), SVOO_ERR_UNSUPPORTED, "svoo_cluster_sort: bh*n too large");
  const size_t need = svoo_cluster_sort_workspace_size(bh, n, k);
  SVOO_REQUIRE(workspace && ws_bytes >= need, SVOO_ERR_WORKSPACE, "svoo_cluster_sort: workspace %zu < %zu",
               ws_bytes, need);
  return svoo_cluster_sort_impl(labels, bh, n, k, sorted_idx, sizes, offsets, sorted_labels, (int32_t*)workspace,
                                nullptr, (hipStream_t)stream, nullptr, 0, nullptr, 0);
}
