// Centroid update over cluster-sorted tokens.
//
// accumulate: each wave owns 128 consecutive sorted positions.  Labels are non-decreasing along
//   sorted positions, so the wave walks its rows in order, keeping two fp64 partial sums per lane
//   (lane l owns dims 2l, 2l+1 of a 128-dim row) and flushing them with one fp64 atomicAdd per
//   lane whenever the label changes.  A sum of bf16 values is exact in fp64 while, per cluster and
//   dimension, the members' exponent span (largest exponent minus smallest nonzero one) plus
//   log2(member count) stays within 53 - 8 = 45 bits (about 28 binades at N = 75600); then the result
//   does not depend on the order of the atomics.  Beyond that the fp64 sums round and the last bits can
//   depend on that order.  The wave's indices and labels arrive in two vector loads; rows are then
//   fetched 16 at a time, one batch ahead of the accumulation.
// finalize: centroid = bf16(f32(sum) / f32(size)), size 0 keeps the old centroid (four elements of a row per
//   thread: 16-byte sum loads, one 8-byte store); the sum buffer
//   is cleared on the way out so the next update starts from zero (or kept, for the delta update).
// delta: the co-clustering's later iterations move only the rows whose label changed: each wave walks a
//   piece of the change list, subtracts the rows from their old clusters' sums and adds them to the new
//   ones' (runs of equal labels summed in registers, then fp64 atomics) and moves the counts.  Under the
//   exponent-span condition above every partial sum is exact, so the sums equal a full recount bit for bit;
//   beyond it they can differ in the last fp64 bits.
// move: one launch for an incremental iteration that runs the delta or, with too many changed tokens, the
//   accumulation over the freshly sorted labels, chosen on the device from the change count.
#include "svoo_common.h"

namespace svoo {

constexpr int kCentPosPerWave = 128;  // two index words per lane
constexpr int kCentBatch = 16;        // rows in flight per wave (double buffered)

// The accumulation of block (bx, b) of the (positions / 512, heads) grid, 4 waves of 256 threads.
__device__ __forceinline__ void accumulate_rows(const uint32_t* __restrict__ x, const int32_t* __restrict__ sorted_idx,
                                                const int32_t* __restrict__ sorted_labels, double* __restrict__ sums,
                                                int n, int k, int bx, int b) {
  // D = 128 fixed: a row is 64 uint32 words (bf16 pairs), one per lane.
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int p0 = (bx * 4 + wave) * kCentPosPerWave;
  if (p0 >= n) return;
  const int cnt = min(n - p0, kCentPosPerWave);
  const int32_t* si = sorted_idx + (size_t)b * n + p0;
  const int32_t* sl = sorted_labels + (size_t)b * n + p0;
  const uint32_t* xb = x + (size_t)b * n * 64;
  double* sb = sums + (size_t)b * k * 128;
  // The wave's 128 (index, label) pairs in two vector loads; positions past the end read as
  // index -1 (contributes 0) and the last valid label (no flush).
  int idx2[2], lab2[2];
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    const int u = half * kWave + lane;
    idx2[half] = u < cnt ? si[u] : -1;
    lab2[half] = sl[min(u, cnt - 1)];
  }
  auto fetch = [&](uint32_t* w, int base) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < kCentBatch; ++u) {
      const int pos = base + u;  // compile-time after unrolling of the batch loop
      const int src = __builtin_amdgcn_readlane(idx2[pos / kWave], pos % kWave);
      // unconditional load (row 0 stands in for an invalid index) so that the loads of a batch
      // stay counted in order; the value is masked after it arrives
      const uint32_t v = xb[(size_t)((unsigned)src < (unsigned)n ? src : 0) * 64 + lane];
      w[u] = ((unsigned)src < (unsigned)n) ? v : 0u;
    }
  };
  int cur = __builtin_amdgcn_readlane(lab2[0], 0);
  double a0 = 0.0, a1 = 0.0;
  uint32_t wb[2][kCentBatch];
  fetch(wb[0], 0);
#pragma unroll
  for (int bt = 0; bt < kCentPosPerWave / kCentBatch; ++bt) {
    if (bt + 1 < kCentPosPerWave / kCentBatch) fetch(wb[(bt + 1) & 1], (bt + 1) * kCentBatch);
#pragma unroll
    for (int u = 0; u < kCentBatch; ++u) {
      const int pos = bt * kCentBatch + u;
      const int lab = __builtin_amdgcn_readlane(lab2[pos / kWave], pos % kWave);
      if (lab != cur) {
        if ((unsigned)cur < (unsigned)k) {
          atomicAdd(&sb[(size_t)cur * 128 + 2 * lane], a0);
          atomicAdd(&sb[(size_t)cur * 128 + 2 * lane + 1], a1);
        }
        a0 = 0.0;
        a1 = 0.0;
        cur = lab;
      }
      const uint32_t w = wb[bt & 1][u];
      a0 += (double)bf16_to_f32((uint16_t)(w & 0xffffu));
      a1 += (double)bf16_to_f32((uint16_t)(w >> 16));
    }
  }
  if ((unsigned)cur < (unsigned)k) {
    atomicAdd(&sb[(size_t)cur * 128 + 2 * lane], a0);
    atomicAdd(&sb[(size_t)cur * 128 + 2 * lane + 1], a1);
  }
}

__global__ void __launch_bounds__(256) centroid_accumulate_kernel(const uint32_t* __restrict__ x,
                                                                  const int32_t* __restrict__ sorted_idx,
                                                                  const int32_t* __restrict__ sorted_labels,
                                                                  double* __restrict__ sums, int n, int k) {
  accumulate_rows(x, sorted_idx, sorted_labels, sums, n, k, blockIdx.x, blockIdx.y);
}

// The finalize also clears zn int32 words at zp (the co-clustering's per-pass counters, which the next
// pass's prep needs at zero): one launch less per pass.
__global__ void __launch_bounds__(256) centroid_finalize_kernel(double* __restrict__ sums,
                                                                const int32_t* __restrict__ sizes,
                                                                const uint16_t* old_c, uint16_t* new_c,
                                                                long long total, int d, int keep_sums,
                                                                int32_t* __restrict__ reset, int32_t* __restrict__ zp,
                                                                long long zn) {
  // four consecutive elements of one row per thread (d is a multiple of 4)
  const long long t = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (reset && t == 0) *reset = 0;  // the delta list's counter, consumed by now
  if (zp && t < zn) zp[t] = 0;
  const long long i = 4 * t;
  if (i >= total) return;
  const long long row = i / d;
  const int cnt = sizes[row];
  double2* sp = (double2*)(sums + i);
  const double2 s01 = sp[0], s23 = sp[1];
  if (!keep_sums) {
    sp[0] = make_double2(0.0, 0.0);
    sp[1] = make_double2(0.0, 0.0);
  }
  uint2 out;
  if (cnt > 0) {
    const float c = (float)cnt;
    out.x = f32_to_bf16((float)s01.x / c) | ((uint32_t)f32_to_bf16((float)s01.y / c) << 16);
    out.y = f32_to_bf16((float)s23.x / c) | ((uint32_t)f32_to_bf16((float)s23.y / c) << 16);
  } else {
    out = *(const uint2*)(old_c + i);
  }
  *(uint2*)(new_c + i) = out;
}

__global__ void zero_f64_kernel(double* __restrict__ p, long long n) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.0;
}

__global__ void zero_i32_kernel(int32_t* __restrict__ p, long long n) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

constexpr int kDeltaBlocks = 1024;  // waves split the change list (its length is on the device) into pieces
constexpr int kDeltaBatch = 8;      // rows gathered at once per wave

// Each wave takes one contiguous piece of the change list.  The producers write it in runs: a wave of the
// assignment appends its tokens together, and the key side's candidate pass handles tokens in label order, so
// neighbouring entries often leave the same cluster or join the same one.  A wave sums a run of equal old (new)
// labels in registers and adds it with one atomic per element (under the exponent-span condition above every
// partial sum is exact, so grouping the additions changes nothing).
// Wave w0 of nw takes its piece of the change list (total entries).
__device__ __forceinline__ void delta_rows(const uint32_t* __restrict__ x, const int2* __restrict__ changes, int total,
                                           double* __restrict__ sums, int32_t* __restrict__ sizes, int n, int k, int w0,
                                           int nw) {
  const int lane = threadIdx.x % kWave;
  const int per = (total + nw - 1) / nw;
  const int e0 = w0 * per, e1 = min(total, e0 + per);
  long long kn = -1, ko = -1;  // cluster rows (head * k + label) of the open runs
  double n0 = 0.0, n1 = 0.0, o0 = 0.0, o1 = 0.0;
  int cn = 0, co = 0;
  auto flush = [&](long long row, double v0, double v1, int cnt) {
    if (row < 0) return;
    double* sp = sums + (size_t)row * 128 + 2 * lane;
    atomicAdd(sp, v0);
    atomicAdd(sp + 1, v1);
    if (lane == 0) atomicAdd(&sizes[row], cnt);
  };
  for (int e = e0; e < e1; e += kDeltaBatch) {
    int2 c[kDeltaBatch];
    uint32_t w[kDeltaBatch];
#pragma unroll
    for (int i = 0; i < kDeltaBatch; ++i) c[i] = e + i < e1 ? changes[e + i] : make_int2(-1, 0);
#pragma unroll
    for (int i = 0; i < kDeltaBatch; ++i) w[i] = c[i].x >= 0 ? x[(size_t)c[i].x * 64 + lane] : 0u;
#pragma unroll
    for (int i = 0; i < kDeltaBatch; ++i) {
      if (c[i].x < 0) break;  // the same for every lane
      const long long b = c[i].x / n;
      const long long rn = b * k + (c[i].y & 0xffff), ro = b * k + (c[i].y >> 16);
      const double v0 = (double)bf16_to_f32((uint16_t)(w[i] & 0xffffu));
      const double v1 = (double)bf16_to_f32((uint16_t)(w[i] >> 16));
      if (rn != kn) {
        flush(kn, n0, n1, cn);
        kn = rn, n0 = 0.0, n1 = 0.0, cn = 0;
      }
      n0 += v0, n1 += v1, ++cn;
      if (ro != ko) {
        flush(ko, o0, o1, co);
        ko = ro, o0 = 0.0, o1 = 0.0, co = 0;
      }
      o0 -= v0, o1 -= v1, --co;
    }
  }
  flush(kn, n0, n1, cn);
  flush(ko, o0, o1, co);
}

// An incremental iteration's update: with at most `limit` changed tokens the blocks below kDeltaBlocks move
// them (delta), else the blocks below nbx * bh recount every cluster from the sorted labels (accumulate; the
// sort and the cleared sums come from the guarded sort launched before).  One launch instead of two guarded
// ones.
__global__ void __launch_bounds__(256) centroid_move_kernel(const uint32_t* __restrict__ x,
                                                            const int32_t* __restrict__ sorted_idx,
                                                            const int32_t* __restrict__ sorted_labels,
                                                            const int2* __restrict__ changes,
                                                            const int32_t* __restrict__ nchanges,
                                                            double* __restrict__ sums, int32_t* __restrict__ sizes,
                                                            int n, int k, int limit, int nbx, int bh) {
  const int total = *nchanges;
  const int bid = blockIdx.x;
  if (total > limit) {
    if (bid < nbx * bh) accumulate_rows(x, sorted_idx, sorted_labels, sums, n, k, bid % nbx, bid / nbx);
  } else if (bid < kDeltaBlocks) {
    delta_rows(x, changes, total, sums, sizes, n, k, bid * 4 + (int)threadIdx.x / kWave, kDeltaBlocks * 4);
  }
}

}  // namespace svoo

using namespace svoo;

int svoo_zero_f64(double* p, long long n, hipStream_t stream) {
  if (n <= 0) return SVOO_OK;
  hipLaunchKernelGGL(zero_f64_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, p, n);
  return check_launch("zero_f64");
}

int svoo_zero_i32(int32_t* p, long long n, hipStream_t stream) {
  if (n <= 0) return SVOO_OK;
  hipLaunchKernelGGL(zero_i32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, p, n);
  return check_launch("zero_i32");
}

// An incremental iteration's centroid update (the co-clustering's later passes): the move kernel (delta or
// recount, chosen on the device from *nchanges against limit), then the centroids; *nchanges is cleared by the
// finalize, which also clears zn int32 words at zp.
int svoo_centroid_move_impl(const uint16_t* x, const int32_t* sorted_idx, const int32_t* sorted_labels,
                            const int2* changes, int32_t* nchanges, double* sums, int32_t* sizes, const uint16_t* old_c,
                            uint16_t* new_c, int bh, int n, int k, int limit, hipStream_t stream, int32_t* zp,
                            long long zn) {
  const int nbx = (n + 4 * kCentPosPerWave - 1) / (4 * kCentPosPerWave);
  const int blocks = max(nbx * bh, kDeltaBlocks);
  hipLaunchKernelGGL(centroid_move_kernel, dim3(blocks), dim3(256), 0, stream, (const uint32_t*)x, sorted_idx,
                     sorted_labels, changes, nchanges, sums, sizes, n, k, limit, nbx, bh);
  const long long total = (long long)bh * k * 128;
  const long long fthreads = max(total / 4, zp ? zn : 0ll);
  hipLaunchKernelGGL(centroid_finalize_kernel, dim3((unsigned)((fthreads + 255) / 256)), dim3(256), 0, stream, sums,
                     sizes, old_c, new_c, total, 128, 1, nchanges, zp, zn);
  return check_launch("svoo_centroid_move");
}

// sums must be zero on entry; it is zero again on return unless keep_sums.  The finalize also clears zn int32
// words at zp.
int svoo_centroid_update_impl(const uint16_t* x, const int32_t* sorted_idx, const int32_t* sorted_labels,
                              const int32_t* sizes, const uint16_t* old_c, uint16_t* new_c, int bh, int n, int k,
                              double* sums, hipStream_t stream, int keep_sums, int32_t* zp, long long zn) {
  const int waves_per_block = 4;
  const int pos_per_block = waves_per_block * kCentPosPerWave;
  dim3 grid((n + pos_per_block - 1) / pos_per_block, bh);
  hipLaunchKernelGGL(centroid_accumulate_kernel, grid, dim3(256), 0, stream, (const uint32_t*)x, sorted_idx,
                     sorted_labels, sums, n, k);
  const long long total = (long long)bh * k * 128;
  const long long fthreads = max(total / 4, zp ? zn : 0ll);
  hipLaunchKernelGGL(centroid_finalize_kernel, dim3((unsigned)((fthreads + 255) / 256)), dim3(256), 0, stream, sums,
                     sizes, old_c, new_c, total, 128, keep_sums, (int32_t*)nullptr, zp, zn);
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
  SVOO_REQUIRE_HEAD_DIM(d, "svoo_centroid_update");
  SVOO_REQUIRE(bh <= 65535, SVOO_ERR_UNSUPPORTED, "svoo_centroid_update: bh too large");
  const size_t need = svoo_centroid_update_workspace_size(bh, k, d);
  SVOO_REQUIRE(workspace && ws_bytes >= need, SVOO_ERR_WORKSPACE, "svoo_centroid_update: workspace %zu < %zu",
               ws_bytes, need);
  hipStream_t s = (hipStream_t)stream;
  double* sums = (double*)workspace;
  if (int rc = svoo_zero_f64(sums, (long long)bh * k * d, s)) return rc;
  return svoo_centroid_update_impl(x, sorted_idx, sorted_labels, sizes, old_c, new_c, bh, n, k, sums, s, 0, nullptr,
                                   0);
}
