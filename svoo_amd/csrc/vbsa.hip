// Variable-block-sparse attention (VBSA) over cluster-contiguous tokens, gfx950 MFMA.
//
// Plan (one block per batch-head, on device, no host round trip):
//   qoff/koff = exclusive prefix of the cluster sizes (validated to sum to S), and a work list of
//   (q-cluster, q-tile) items, kQTile queries each, the query clusters with the longest KV streams first.
// Order (one block): heads by estimated work, heaviest first, and the grid's work list, head after head.
// Attention (one block of 8 waves per work item of 256 queries, 32 queries per wave):
//   * the block compacts its map row into a list of active key segments (start, length) in LDS;
//     the KV stream is their concatenation (ascending cluster), cut into 64-key tiles that span
//     segment boundaries, so padding happens once per work item instead of once per cluster;
//   * K and V tiles are double buffered in LDS and filled by LDS DMA (global_load_lds_dwordx4);
//     two waves resolve the token rows of upcoming tiles into a small LDS table;
//   * S^T = K Q^T with v_mfma_f32_32x32x16_bf16 (keys on M, queries on N), so each lane holds 16
//     keys of one query: the row max needs one cross-half exchange and the online-softmax rescale
//     is a per-lane scalar;  O^T += V^T P^T reuses the S^T accumulators as the B operand directly,
//     with the V^T operand gathered by gfx950's transposing LDS read (ds_read_b64_tr_b16);
//   * ping-pong: the two waves sharing a SIMD belong to two groups that alternate, one half-step
//     apart, between the MFMA work of a tile and the softmax of the next, so matrix and vector
//     units are busy at the same time;
//   * fp32 online softmax (exp2 with the scale folded in), P rounded to bf16 for the PV MFMA, as
//     the reference's Triton kernel does; rows of a cluster with no active keys are written as 0.
// Fused variant (IDX): Q, K and V stay in token order; the kernel reads them through the clusters'
// sorted indices (query rows when loaded, key rows when the row tables are resolved) and writes each
// output row to its token's place in [B, S, H, D], so the permutes and the inverse permutation around
// the attention are not separate passes.
// EAR variant (centroid compensation): the KV stream continues after the active tokens with the
// (key, value) centroids of the inactive clusters, each scored q . kc_j / sqrt(D) + log(|K_j| + 1e-6),
// so one online softmax covers both (the reference's token attention + log-sum-exp merge).
#include <mutex>
#include <type_traits>

#include "svoo_common.h"

namespace svoo {

constexpr int kVWaves = 8;
constexpr int kKT = 64;          // keys per tile
constexpr int kPlanThreads = 1024;  // plan kernel
constexpr int kOrderThreads = 256;  // order kernel
constexpr int kPlanSortMax = 4096;  // heads with at most this many query clusters get their items longest first
constexpr int kPlanBuckets = 4096;
constexpr int kMaxKN = 4096;

template <int QB>
struct VbsaCfg {
  static constexpr int kQTile = kVWaves * 32 * QB;
};

// ------------------------------------------------------------------------------------------ plan
__global__ void __launch_bounds__(kPlanThreads) vbsa_plan_kernel(const int32_t* __restrict__ qs,
                                                                 const int32_t* __restrict__ ks,
                                                                 const uint8_t* __restrict__ map, int ear,
                                                                 int32_t* __restrict__ work, int s, int qn, int kn,
                                                                 int qtile, int cap, int half_ok,
                                                                 int32_t* __restrict__ qoff,
                                                                 int32_t* __restrict__ koff,
                                                                 int32_t* __restrict__ items,
                                                                 int32_t* __restrict__ nitems,
                                                                 int32_t* __restrict__ status) {
  __shared__ long long red[kPlanThreads / kWave];
  __shared__ int bad;
  const int b = blockIdx.x, tid = threadIdx.x;
  if (tid == 0) bad = 0;
  __syncthreads();
  const int32_t* qsb = qs + (size_t)b * qn;
  const int32_t* ksb = ks + (size_t)b * kn;
  int32_t* qo = qoff + (size_t)b * (qn + 1);
  int32_t* ko = koff + (size_t)b * (kn + 1);
  // koff
  {
    const int per = (kn + kPlanThreads - 1) / kPlanThreads;
    const int j0 = min(kn, tid * per), j1 = min(kn, j0 + per);
    long long loc = 0;
    for (int j = j0; j < j1; ++j) {
      const int v = ksb[j];
      if (v < 0) bad = 1;
      loc += v;
    }
    long long tot;
    long long run = block_exclusive_scan_i64<kPlanThreads>(loc, red, &tot);
    for (int j = j0; j < j1; ++j) {
      ko[j] = (int32_t)run;
      run += ksb[j];
    }
    if (tid == 0) {
      ko[kn] = (int32_t)tot;
      if (tot != s) bad = 1;
    }
  }
  // qoff and the tile counts (packed: tiles << 32 | rows)
  bool ok;
  {
    const int per = (qn + kPlanThreads - 1) / kPlanThreads;
    const int i0 = min(qn, tid * per), i1 = min(qn, i0 + per);
    long long loc = 0;
    for (int i = i0; i < i1; ++i) {
      const int v = qsb[i];
      if (v < 0) bad = 1;
      const long long t = v > 0 ? (v + qtile - 1) / qtile : 0;
      loc += (t << 32) | (long long)(uint32_t)v;
    }
    long long tot;
    long long run = block_exclusive_scan_i64<kPlanThreads>(loc, red, &tot);
    __syncthreads();
    ok = !bad && (int)(tot & 0xffffffffll) == s && (int)(tot >> 32) <= cap;
    for (int i = i0; i < i1; ++i) {
      const int v = qsb[i];
      qo[i] = (int32_t)(run & 0xffffffffll);
      const int t0 = (int)(run >> 32);
      const int nt = v > 0 ? (v + qtile - 1) / qtile : 0;
      // a last tile of at most qtile / 2 queries is a half item (flag 0x8000) when the kernel has
      // the LDS for a second KV stream
      const int rem = v - (nt - 1) * qtile;
      // last tile: a half item (0x8000) up to qtile / 2 queries, B-chunked (bit 31) up to 3 qtile / 4
      const uint32_t hflag = !half_ok ? 0u : 2 * rem <= qtile ? 0x8000u : 4 * rem <= 3 * qtile ? 0x80000000u : 0u;
      if (ok && qn > kPlanSortMax)
        for (int t = 0; t < nt; ++t)
          items[(size_t)b * cap + t0 + t] = (int32_t)(((uint32_t)i << 16) | (uint32_t)t | (t == nt - 1 ? hflag : 0u));
      run += ((long long)nt << 32) | (long long)(uint32_t)v;
    }
    if (tid == 0) {
      qo[qn] = (int32_t)(tot & 0xffffffffll);
      // -1 marks a head whose sizes do not sum to S: the attention fills its rows with NaN
      nitems[b] = ok ? (int32_t)(tot >> 32) : -1;
      if (!ok && status) atomicOr(status, 1);
    }
  }
  // Work of the head in KV tiles (the attention's launch order runs heavy heads first): a wave sums the
  // stream length of a query cluster's map row (active keys, plus the inactive centroids for EAR) and
  // weighs it by the cluster's query tiles.  The pass is bound by load latency, not bytes: a wave keeps
  // four rows (i + r * kPW) in flight and reads a row 4 bytes per lane and load when its rows start 4-byte
  // aligned, with the key sizes from LDS.
  {
    __shared__ __attribute__((aligned(16))) int32_t s_ks[kMaxKN];
    __shared__ int32_t s_tiles[kPlanSortMax];  // KV tiles of each query cluster's stream
    for (int j = tid; j < kn; j += kPlanThreads) s_ks[j] = ksb[j];
    __syncthreads();
    constexpr int kPW = kPlanThreads / kWave;
    const int wave = tid / kWave, lane = tid % kWave;
    const bool words = kn % 4 == 0 && (uintptr_t)map % 4 == 0;
    long long wsum = 0;
    for (int i = wave; i < qn; i += 4 * kPW) {
      int act[4] = {0, 0, 0, 0};
      const uint8_t* mr[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) mr[r] = map + ((size_t)b * qn + min(i + r * kPW, qn - 1)) * kn;
      if (words) {
#pragma unroll 4
        for (int w = lane; w < kn / 4; w += kWave) {
          uint32_t m4[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) m4[r] = ((const uint32_t*)mr[r])[w];
          const int4 k4 = *(const int4*)&s_ks[4 * w];
#pragma unroll
          for (int r = 0; r < 4; ++r)
            act[r] += ((m4[r] & 0xffu) ? k4.x : ear) + ((m4[r] & 0xff00u) ? k4.y : ear) +
                      ((m4[r] & 0xff0000u) ? k4.z : ear) + ((m4[r] >> 24) ? k4.w : ear);
        }
      } else {
#pragma unroll 8
        for (int j = lane; j < kn; j += kWave) {
          const int kv = s_ks[j];
#pragma unroll
          for (int r = 0; r < 4; ++r) act[r] += mr[r][j] ? kv : ear;
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        int a = act[r];
#pragma unroll
        for (int o = kWave / 2; o > 0; o >>= 1) a += __shfl_xor(a, o);
        const int row = i + r * kPW;
        const int v = row < qn ? qsb[row] : 0;
        if (v > 0) wsum += (long long)((v + qtile - 1) / qtile) * (1 + (a + kKT - 1) / kKT);
        if (lane == 0 && row < qn && qn <= kPlanSortMax) s_tiles[row] = (a + kKT - 1) / kKT;
      }
    }
    __syncthreads();  // the scans above are done with red
    if (lane == 0) red[wave] = wsum;
    __syncthreads();
    if (tid == 0) {
      long long w = 0;
      for (int i = 0; i < kPlanThreads / kWave; ++i) w += red[i];
      work[b] = (int32_t)min(w, 0x7fffffffll);
    }
    // The head's work items, longest first: an item's length is its cluster's KV stream in tiles, 0.72 of it for
    // a half item; a cluster's full items stay together (they read the same keys), its half item goes with the
    // other half items of its length.  A counting sort over kPlanBuckets lengths (longer ones share the last
    // bucket); the order of equal lengths is free.  Heads with more than kPlanSortMax clusters keep the cluster
    // order (written above).
    if (ok && qn <= kPlanSortMax) {
      __shared__ int32_t s_bk[kPlanBuckets];
      auto bk = [&](int tl) { return kPlanBuckets - 1 - min(tl, kPlanBuckets - 1); };
      for (int e = tid; e < kPlanBuckets; e += kPlanThreads) s_bk[e] = 0;
      __syncthreads();
      for (int i = tid; i < qn; i += kPlanThreads) {
        const int v = qsb[i];
        if (v <= 0) continue;
        const int nt = (v + qtile - 1) / qtile, rem = v - (nt - 1) * qtile;
        const bool hl = half_ok && 2 * rem <= qtile;
        if (nt - (hl ? 1 : 0) > 0) atomicAdd(&s_bk[bk(s_tiles[i])], nt - (hl ? 1 : 0));
        if (hl) atomicAdd(&s_bk[bk((s_tiles[i] * 23) / 32)], 1);
      }
      __syncthreads();
      constexpr int kPer = kPlanBuckets / kPlanThreads;
      int c[kPer];
      long long loc = 0;
#pragma unroll
      for (int e = 0; e < kPer; ++e) {
        c[e] = s_bk[tid * kPer + e];
        loc += c[e];
      }
      long long tot;
      long long run = block_exclusive_scan_i64<kPlanThreads>(loc, red, &tot);  // its barriers follow the reads
#pragma unroll
      for (int e = 0; e < kPer; ++e) {
        s_bk[tid * kPer + e] = (int32_t)run;
        run += c[e];
      }
      __syncthreads();
      for (int i = tid; i < qn; i += kPlanThreads) {
        const int v = qsb[i];
        if (v <= 0) continue;
        const int nt = (v + qtile - 1) / qtile, rem = v - (nt - 1) * qtile;
        const bool hl = half_ok && 2 * rem <= qtile;
        const int nf = nt - (hl ? 1 : 0);
        if (nf > 0) {
          const int pos = atomicAdd(&s_bk[bk(s_tiles[i])], nf);
          const uint32_t bflag = (half_ok && 4 * rem <= 3 * qtile) ? 0x80000000u : 0u;  // B-chunked last tile
          for (int t = 0; t < nf; ++t)
            items[(size_t)b * cap + pos + t] = (int32_t)(((uint32_t)i << 16) | (uint32_t)t | (t == nt - 1 ? bflag : 0u));
        }
        if (hl) items[(size_t)b * cap + atomicAdd(&s_bk[bk((s_tiles[i] * 23) / 32)], 1)] = (i << 16) | (nt - 1) | 0x8000;
      }
    }
  }
}

// The grid's work list.  Heads in launch order: by work, heaviest first (ties by index), so the last work
// items of the grid are short ones (bh above kOrderMax keeps the natural order).  The list holds, head after
// head in that order, one entry (head << 15 | item slot) per work item of the head: its nitems slots, or for a
// head whose sizes do not sum to S one NaN-filling slot per qtile token rows; -1 fills the rest of its
// bh * cap entries.  A dense list gives every XCD an equal share of the real items: with per-head slot ranges
// the unused slots at the end of each head's range fall on the same XCDs head after head.
constexpr int kOrderMax = 4096;
__global__ void __launch_bounds__(kOrderThreads) vbsa_order_kernel(const int32_t* __restrict__ work,
                                                                  const int32_t* __restrict__ nitems, int bh, int cap,
                                                                  int nan_slots, int32_t* __restrict__ list) {
  __shared__ int32_t w[kOrderMax], rk[kOrderMax];  // work and rank of each head, then the head of each rank
  __shared__ long long red[kOrderThreads / kWave];
  __shared__ int32_t c_head[kOrderThreads], c_n[kOrderThreads], c_base[kOrderThreads];
  const int tid = threadIdx.x;
  const bool ranked = bh <= kOrderMax;
  if (ranked) {
    for (int h = tid; h < bh; h += kOrderThreads) w[h] = work[h];
    __syncthreads();
    for (int h = tid; h < bh; h += kOrderThreads) {
      const int wh = w[h];
      int rank = 0;
      for (int g = 0; g < bh; ++g) rank += (w[g] > wh || (w[g] == wh && g < h)) ? 1 : 0;
      rk[h] = rank;
    }
    __syncthreads();  // every thread is done reading the work values
    for (int h = tid; h < bh; h += kOrderThreads) w[rk[h]] = h;
    __syncthreads();
  }
  long long run = 0;
  for (int r0 = 0; r0 < bh; r0 += kOrderThreads) {
    const int r = r0 + tid;
    int n = 0, h = 0;
    if (r < bh) {
      h = ranked ? w[r] : r;
      const int ni = nitems[h];
      n = ni >= 0 ? ni : nan_slots;
    }
    long long tot;
    const long long ex = block_exclusive_scan_i64<kOrderThreads>(n, red, &tot);
    c_head[tid] = h;
    c_n[tid] = n;
    c_base[tid] = (int32_t)(run + ex);
    __syncthreads();
    const int m = min(kOrderThreads, bh - r0);
    for (int i = 0; i < m; ++i) {
      const int32_t tag = c_head[i] << 15, base = c_base[i];
      for (int j = tid; j < c_n[i]; j += kOrderThreads) list[base + j] = tag | j;
    }
    __syncthreads();  // the chunk's tables are read before the next chunk writes them
    run += tot;
  }
  for (long long i = run + tid; i < (long long)bh * cap; i += kOrderThreads) list[i] = -1;
}

// Compacts the active key clusters of one map row into (start, cumulative length) segments in
// LDS.  Returns the segment count; *total receives the number of keys.
__device__ __forceinline__ int build_segments(const uint8_t* __restrict__ mrow, const int32_t* __restrict__ ko,
                                              const int32_t* __restrict__ ksb, int kn, int32_t* seg_start,
                                              int32_t* seg_cum, long long* red, int* total) {
  const int tid = threadIdx.x, nt = blockDim.x;
  const int per = (kn + nt - 1) / nt;
  const int j0 = min(kn, tid * per), j1 = min(kn, j0 + per);
  long long loc = 0;
  for (int j = j0; j < j1; ++j) {
    const int len = ksb[j];
    if (mrow[j] && len > 0) loc += (1ll << 32) | (long long)len;
  }
  long long tot;
  long long run = block_exclusive_scan_i64<kVWaves * kWave>(loc, red, &tot);
  int idx = (int)(run >> 32);
  int cum = (int)(run & 0xffffffffll);
  for (int j = j0; j < j1; ++j) {
    const int len = ksb[j];
    if (mrow[j] && len > 0) {
      seg_start[idx] = ko[j];
      seg_cum[idx] = cum;
      ++idx;
      cum += len;
    }
  }
  const int nseg = (int)(tot >> 32);
  if (tid == 0) seg_cum[nseg] = (int)(tot & 0xffffffffll);
  __syncthreads();
  *total = (int)(tot & 0xffffffffll);
  return nseg;
}

// EAR: compacts the inactive key clusters of one map row (ascending) with their score bias
// log2(e) * log(|K_j| + 1e-6) into LDS.  Returns their count.
__device__ __forceinline__ int build_centroids(const uint8_t* __restrict__ mrow, const int32_t* __restrict__ ksb,
                                               int kn, int32_t* cent_idx, float* cent_bias, long long* red) {
  const int tid = threadIdx.x, nt = blockDim.x;
  const int per = (kn + nt - 1) / nt;
  const int j0 = min(kn, tid * per), j1 = min(kn, j0 + per);
  long long loc = 0;
  for (int j = j0; j < j1; ++j) loc += mrow[j] ? 0 : 1;
  long long tot;
  int idx = (int)block_exclusive_scan_i64<kVWaves * kWave>(loc, red, &tot);
  for (int j = j0; j < j1; ++j) {
    if (!mrow[j]) {
      cent_idx[idx] = j;
      cent_bias[idx] = 1.4426950408889634f * logf((float)ksb[j] + 1e-6f);
      ++idx;
    }
  }
  __syncthreads();
  return (int)tot;
}

// Segment containing stream position p (seg_cum ascending, seg_cum[0] == 0).
__device__ __forceinline__ int find_segment(const int32_t* seg_cum, int nseg, int p) {
  int lo = 0, hi = nseg - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (seg_cum[mid] <= p)
      lo = mid;
    else
      hi = mid - 1;
  }
  return lo;
}

// XCD-aware block -> work-item map: workgroups are dispatched round-robin over the 8 XCDs
// (bid % 8), so runs of kXcdRun consecutive items (the q-tiles of one query cluster, which read
// the same keys) are given to one XCD and start together, sharing that XCD's L2.
constexpr int kXcdRun = 8;
__device__ __forceinline__ long long xcd_item(long long bid) {
  const long long x = bid % 8, j = bid / 8;
  return (j / kXcdRun) * (8 * kXcdRun) + x * kXcdRun + (j % kXcdRun);
}

// ------------------------------------------------------------------------------------------ attention
// Position cursor over the segmented KV stream: row = off + p while p < next.
struct KvCursor {
  int seg, off, next;
};
__device__ __forceinline__ void cursor_init(KvCursor& c, const int32_t* seg_start, const int32_t* seg_cum, int nseg,
                                            int p) {
  c.seg = find_segment(seg_cum, nseg, p);
  c.off = seg_start[c.seg] - seg_cum[c.seg];
  c.next = seg_cum[c.seg + 1];
}
__device__ __forceinline__ int cursor_row(KvCursor& c, const int32_t* seg_start, const int32_t* seg_cum, int p) {
  while (p >= c.next) {
    ++c.seg;
    c.off = seg_start[c.seg] - seg_cum[c.seg];
    c.next = seg_cum[c.seg + 1];
  }
  return c.off + p;
}

// Block = kVWaves waves x 32 queries of one query cluster; K and V tiles of 64 keys are double
// buffered in LDS with one barrier per tile.  Iteration t holds the scores S(t) in registers and
//   * issues the global loads of K(t+2) and V(t+1) (registers), then
//   * computes S(t+1) = K(t+1) Q^T (MFMA, A = K rows via ds_read_b128, B = Q in registers) next to
//     the softmax of S(t) (VALU): P = exp2(S * scale * log2e - m) with a lazily updated running max
//     m (rescale only when the tile max exceeds m by more than 8, i.e. P <= 2^8), bf16 P,
//   * O^T += V(t)^T P^T (MFMA, A = V columns via the transposing LDS read, B = the score
//     accumulators' registers, whose key order the V read follows),
//   * stores K(t+2) and V(t+1) into the buffers freed by K(t) and V(t-1).
// Ping-pong block: 8 waves in two groups of 4 (group A = waves 0-3, group B = waves 4-7), each
// wave 32 queries (query tile 256: A owns queries 0-127, B 128-255).  The waves of a SIMD come
// from different groups and alternate between an MFMA phase M(t) = {O += V(t)^T P(t)^T, S(t+1) =
// K(t+1) Q^T} and a VALU phase V(t) = {softmax of S(t) -> P(t)}; group B runs one half-step behind
// group A, so in every half-step one wave per SIMD does MFMA work while the other does VALU work.
// Group B also issues the LDS DMA of the next K/V tiles; waves 0 and 1 resolve their token rows into
// the row tables during group A's softmax half-step.
// Half items (HC kernels only: a second set of K/V buffers in LDS): a last tile of at most 128
// queries is taken by both groups, each wave of a group holding the same 32 queries as its partner
// in the other group; group A walks the even tiles of the KV stream (stream 0), group B the odd
// ones (stream 1), on the same half-step schedule, and the two online-softmax states are merged
// through LDS at the end, so such an item costs about half the time of a full one.
// B-chunked items (HC kernels: a last tile of 129 to 192 queries, so group B holds at most 64): group B's
// waves wg and wg + 2 hold the same 32 queries and take the first and the second 32 keys of every tile (16
// MFMAs and 16 exponentials per wave and tile), group B resolves the row tables (waves 4 and 5) in place of
// waves 0 and 1, and the two states of a query merge through LDS at the end.
// Half items: each group copies
// its own stream's tiles during its softmax, and group A's waves resolve the four row tables (one
// each) at the start of their MFMA half-step, where they would otherwise wait at the barrier for
// group B's longer softmax with copies.
template <int QB, bool EAR, bool IDX, bool HC>
__global__ void __launch_bounds__(kVWaves * kWave) __attribute__((amdgpu_waves_per_eu(2, 2))) vbsa_attn_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc,
    const uint8_t* __restrict__ map, const int32_t* __restrict__ ks, uint16_t* __restrict__ o, int s, int qn, int kn,
    int cap, long long total_items, const int32_t* __restrict__ qoff, const int32_t* __restrict__ koff,
    const int32_t* __restrict__ items, const int32_t* __restrict__ nitems, float scale_log2,
    const int32_t* __restrict__ q_idx, const int32_t* __restrict__ k_idx, int heads,
    const int32_t* __restrict__ list) {
  constexpr int kQTile = VbsaCfg<QB>::kQTile;
  constexpr int kThreads = kVWaves * kWave;
  constexpr int kDmaIt = kKT / (4 * 4);  // 4-row DMA groups per group-B wave per tile and matrix
  __shared__ __attribute__((aligned(16))) uint16_t k_s0[kKT * 128], k_s1[kKT * 128];
  __shared__ __attribute__((aligned(16))) uint16_t v_s0[kKT * 128], v_s1[kKT * 128];
  // stream 1 of a half item
  constexpr int kS1 = HC ? kKT * 128 : 8;
  __shared__ __attribute__((aligned(16))) uint16_t k1_s0[kS1], k1_s1[kS1], v1_s0[kS1], v1_s1[kS1];
  __shared__ long long red[kVWaves];
  __shared__ int32_t rowtab[HC ? 2 : 1][2][2][kKT];  // [stream][K/V][slot][tile position] -> token row
  extern __shared__ int32_t seg_mem[];  // seg_start[kn], seg_cum[kn + 1] (EAR: cent_idx[kn], cent_bias[kn])

  const long long item = xcd_item(blockIdx.x);
  if (item >= total_items) return;
  const int32_t entry = list[item];
  if (entry < 0) return;  // past the last work item
  const int b = entry >> 15, local = entry & 0x7fff;
  if (nitems[b] < 0) {
    // Sizes of this head do not sum to S (the reference asserts, svoo/co_clustering.py:1138-1139):
    // slot `local` (one of ceil(S / kQTile)) writes NaN over token rows [local * kQTile, +kQTile) of the
    // head, so the failure is visible in the output instead of leaving the buffer's old contents.  Rows
    // are addressed by token (not through the sorted indices, which may be as inconsistent as the sizes).
    const int r0 = local * kQTile, r1 = min(s, r0 + kQTile);
    const u32x4_t nan4 = {0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u};
    for (int idx = threadIdx.x; idx < (r1 - r0) * 16; idx += kVWaves * kWave) {
      const int t = r0 + idx / 16;
      uint16_t* row = IDX ? o + (((size_t)(b / heads) * s + t) * heads + (b % heads)) * 128
                          : o + ((size_t)b * s + t) * 128;
      ((u32x4_t*)row)[idx % 16] = nan4;
    }
    return;
  }
  const uint32_t packed = (uint32_t)items[(size_t)b * cap + local];
  const int ci = (int)((packed >> 16) & 0x7fff), tile = (int)(packed & 0x7fff);
  const bool half = HC && (packed & 0x8000u) != 0;
  const bool bchunk = HC && (packed >> 31) != 0;  // a full item whose group B holds at most 64 queries
  const int32_t* qo = qoff + (size_t)b * (qn + 1);
  const int q0 = qo[ci] + tile * kQTile;
  const int q1 = min(qo[ci + 1], q0 + kQTile);

  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave, h = lane / 32, l32 = lane % 32;
  const int grp = lane / 16, gl = lane % 16;  // transposed-read group and lane within it
  const bool group_b = wave >= 4;
  const int wg = wave & 3;
  const size_t head = (size_t)b * s * 128;
  const uint16_t* qb = q + head;
  const uint16_t* kb = k + head;
  const uint16_t* vb = v + head;
  uint16_t* ob = o + head;
  // IDX: sorted position -> token row of this head, and the output row of a sorted query position
  const int32_t* qix = IDX ? q_idx + (size_t)b * s : nullptr;
  const int32_t* kix = IDX ? k_idx + (size_t)b * s : nullptr;
  auto out_row = [&](int r) __attribute__((always_inline)) -> uint16_t* {
    if constexpr (IDX)
      return o + (((size_t)(b / heads) * s + qix[r]) * heads + (b % heads)) * 128;
    else
      return ob + (size_t)r * 128;
  };
  // EAR: the centroid rows are addressed from the token base of the head, as rows at a signed offset
  // (the host checks that the buffers are 256-byte congruent and that every row index fits int32), so
  // the DMA path is the same as for token rows.
  int crow_k = 0, crow_v = 0;
  if constexpr (EAR) {
    crow_k = (int)(((long long)(uintptr_t)(kc + (size_t)b * kn * 128) - (long long)(uintptr_t)kb) / 256);
    crow_v = (int)(((long long)(uintptr_t)(vc + (size_t)b * kn * 128) - (long long)(uintptr_t)vb) / 256);
  }

  int32_t* seg_start = seg_mem;
  int32_t* seg_cum = seg_mem + kn;
  int32_t* cent_idx = seg_cum + kn + 1;
  float* cent_bias = (float*)(cent_idx + kn);
  int total = 0;
  const uint8_t* mrow = map + ((size_t)b * qn + ci) * kn;
  const int nseg_v = build_segments(mrow, koff + (size_t)b * (kn + 1), ks + (size_t)b * kn, kn, seg_start, seg_cum,
                                    red, &total);
  // Segment count and stream length are block-uniform: keep them scalar so tile-loop branches are uniform.
  const int nseg = __builtin_amdgcn_readfirstlane(nseg_v);
  total = __builtin_amdgcn_readfirstlane(total);
  const int total_tok = total;  // keys of the active clusters; EAR appends the inactive centroids
  if constexpr (EAR) {
    const int ncent = build_centroids(mrow, ks + (size_t)b * kn, kn, cent_idx, cent_bias, red);
    total = __builtin_amdgcn_readfirstlane(total_tok + ncent);
  }

  if (total == 0) {
    // Empty row: zero output (reference semantics, svoo/co_clustering.py:1102-1104).
    for (int idx = tid; idx < (q1 - q0) * 16; idx += kThreads) {
      const int r = idx / 16, c = idx % 16;
      ((u32x4_t*)out_row(q0 + r))[c] = u32x4_t{0u, 0u, 0u, 0u};
    }
    return;
  }
  // full item: group A owns queries 0-127, group B 128-255; half item: both own queries 0-127
  const int qrow0 = q0 + ((group_b && !half) ? 128 : 0) + ((bchunk && group_b) ? (wg & 1) : wg) * 32;
  const bool active = qrow0 < q1;

  u32x4_t qop[8];
  {
    const int row = min(qrow0 + l32, q1 - 1);
    const u32x4_t* src = (const u32x4_t*)(qb + (size_t)(IDX ? qix[row] : row) * 128);
#pragma unroll
    for (int ks2 = 0; ks2 < 8; ++ks2) qop[ks2] = src[ks2 * 2 + h];
  }
  f32x16_t acc[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) acc[db] = f32x16_t{};
  float m_run = -INFINITY, l_run = 0.0f;

  // Row tables (lane = tile position): in a full item wave 0 resolves K tiles and wave 1 V tiles; in a
  // half item waves 0 and 1 resolve stream 0 (even tiles), waves 2 and 3 stream 1 (odd tiles).
  // Rows past the stream repeat its last token row (0 when an EAR row has no active tokens); EAR
  // centroid j of the K (V) table is row crow_k + j (crow_v + j).
  int last_row = nseg > 0 ? seg_start[nseg - 1] + (total_tok - 1 - seg_cum[nseg - 1]) : 0;
  if constexpr (IDX) last_row = kix[last_row];
  KvCursor cursor;
  const bool resolver = (half ? wave < 4 : bchunk ? (wave == 4 || wave == 5) : wave < 2) && nseg > 0;
  const int p_first = (half && wave >= 2 ? kKT : 0) + lane;  // this lane's row in the wave's first tile
  if (resolver) cursor_init(cursor, seg_start, seg_cum, nseg, min(p_first, total_tok - 1));
  // IDX: the token index of this lane's row in the next tile the wave resolves, loaded one call
  // ahead so that the global load's latency is off the resolving wave's path
  int pend = 0;
  if constexpr (IDX) {
    if (resolver && p_first < total_tok) pend = kix[cursor_row(cursor, seg_start, seg_cum, p_first)];
  }
  const int crow = (wave & 1) ? crow_v : crow_k;  // the resolving waves: even for K, odd for V
  // Table of tile t; the wave's next table is tile t + step (full items 1, half items 2).
  auto resolve = [&](int32_t* tab, int t, int step) __attribute__((always_inline)) {
    const int p = t * kKT + lane;
    if (p < total_tok) {
      if constexpr (IDX)
        tab[lane] = pend;
      else
        tab[lane] = cursor_row(cursor, seg_start, seg_cum, p);
    }
    else if (EAR && p < total)
      tab[lane] = crow + cent_idx[p - total_tok];
    else
      tab[lane] = last_row;
    if constexpr (IDX) {
      const int pn = p + step * kKT;
      if (pn < total_tok) pend = kix[cursor_row(cursor, seg_start, seg_cum, pn)];
    }
  };
  // DMA mapping (group B): wave 4+w, group j moves tile rows 4(kDmaIt w + j) + lane/16.
  const int prow = lane / 16, pch = lane % 16;
  auto dma = [&](const uint16_t* src, const int32_t* tab, uint16_t* buf) __attribute__((always_inline)) {
    int rows[kDmaIt];  // all table reads first: one LDS wait for the group
#pragma unroll
    for (int j = 0; j < kDmaIt; ++j) rows[j] = tab[4 * (kDmaIt * wg + j) + prow];
#pragma unroll
    for (int j = 0; j < kDmaIt; ++j) {
      const int r = 4 * (kDmaIt * wg + j) + prow;
      if constexpr (EAR) {
        // negative rows for EAR centroid rows below the token buffer
        lds_dma16(src + (long long)rows[j] * 128 + swz(r, pch) * 8, buf + 4 * (kDmaIt * wg + j) * 128);
      } else {
        // a head's rows are < 2^24: a 32-bit byte offset from the wave-uniform base (SGPR-based addressing)
        const uint32_t off = (uint32_t)rows[j] * 256u + (uint32_t)swz(r, pch) * 16u;
        lds_dma16((const char*)src + off, buf + 4 * (kDmaIt * wg + j) * 128);
      }
    }
  };
  // The same copies one group at a time (full items: interleaved with group B's softmax), with the
  // wave's four table rows read ahead into registers.
  auto dma_rows = [&](const int32_t* tab) __attribute__((always_inline)) -> int4 {
    const int o = 4 * kDmaIt * wg + prow;
    return make_int4(tab[o], tab[o + 4], tab[o + 8], tab[o + 12]);
  };
  auto dma_one = [&](const uint16_t* src, int row, int j, uint16_t* buf) __attribute__((always_inline)) {
    const int r = 4 * (kDmaIt * wg + j) + prow;
    if constexpr (EAR) {
      lds_dma16(src + (long long)row * 128 + swz(r, pch) * 8, buf + 4 * (kDmaIt * wg + j) * 128);
    } else {
      const uint32_t off = (uint32_t)row * 256u + (uint32_t)swz(r, pch) * 16u;
      lds_dma16((const char*)src + off, buf + 4 * (kDmaIt * wg + j) * 128);
    }
  };
  auto dma_all = [&](int4 rk4, uint16_t* kdst, int4 rv4, uint16_t* vdst) __attribute__((always_inline)) {
    const int rka[4] = {rk4.x, rk4.y, rk4.z, rk4.w}, rva[4] = {rv4.x, rv4.y, rv4.z, rv4.w};
#pragma unroll
    for (int j = 0; j < kDmaIt; ++j) dma_one(kb, rka[j], j, kdst);
#pragma unroll
    for (int j = 0; j < kDmaIt; ++j) dma_one(vb, rva[j], j, vdst);
  };

  int koffs[8], voffs[2][4];
#pragma unroll
  for (int ks2 = 0; ks2 < 8; ++ks2) koffs[ks2] = l32 * 128 + swz(l32, ks2 * 2 + h) * 8;
  {
    const int r0 = 4 * (grp / 2) + gl / 4;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      const int c = 4 * db + 2 * (grp % 2) + (gl % 4) / 2, e0 = 4 * (gl % 2);
      voffs[0][db] = r0 * 128 + swz(r0, c) * 8 + e0;
      voffs[1][db] = (r0 + 8) * 128 + swz(r0 + 8, c) * 8 + e0;
    }
  }

  const int ntiles = (total + kKT - 1) / kKT;
  f32x16_t sacc[2];
  u32x4_t pop[2][2];

  auto scores = [&](const uint16_t* kt) __attribute__((always_inline)) {
    sacc[0] = f32x16_t{};
    sacc[1] = f32x16_t{};
#pragma unroll
    for (int ks2 = 0; ks2 < 8; ++ks2) {
#pragma unroll
      for (int kb2 = 0; kb2 < 2; ++kb2) {
        const bf16x8_t a = as_bf16x8(*(const u32x4_t*)(&kt[kb2 * 32 * 128 + koffs[ks2]]));
        sacc[kb2] = mfma32x32x16(a, as_bf16x8(qop[ks2]), sacc[kb2]);
      }
    }
  };
  // MFMA phase M(t): O += V(t)^T P(t)^T, then S(t+1).  The 32 MFMAs run as one software pipeline whose
  // operand reads are issued two MFMAs ahead into three rotating buffers (the order is pinned with
  // scheduling barriers).  S(t+1) is also computed after the last tile, on stale LDS, and not used.
  auto mop = [&](int i, const uint16_t* vt, const uint16_t* knext) __attribute__((always_inline)) -> u32x4_t {
    if (i < 16) {
      const int kb2 = i / 8, st = (i / 4) % 2, db = i % 4;
      const int rb = (kb2 * 32 + st * 16) * 128;
      const uint2 lo = ds_read_tr16_b64(&vt[rb + voffs[0][db]]);
      const uint2 hi = ds_read_tr16_b64(&vt[rb + voffs[1][db]]);
      return u32x4_t{lo.x, lo.y, hi.x, hi.y};
    }
    const int j = i - 16, ks2 = j / 2, kb2 = j % 2;
    return *(const u32x4_t*)(&knext[kb2 * 32 * 128 + koffs[ks2]]);
  };
  auto mphase = [&](int t, const uint16_t* vt, const uint16_t* knext) __attribute__((always_inline)) {
    u32x4_t buf[3];
    buf[0] = mop(0, vt, knext);
    buf[1] = mop(1, vt, knext);
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
    auto mm = [&](int i) __attribute__((always_inline)) {
      if (i < 16) {
        const int kb2 = i / 8, st = (i / 4) % 2, db = i % 4;
        acc[db] = mfma32x32x16(as_bf16x8(buf[i % 3]), as_bf16x8(pop[kb2][st]), acc[db]);
      } else {
        const int j = i - 16, ks2 = j / 2, kb2 = j % 2;
        if (j < 2) sacc[kb2] = f32x16_t{};
        sacc[kb2] = mfma32x32x16(as_bf16x8(buf[i % 3]), as_bf16x8(qop[ks2]), sacc[kb2]);
      }
    };
#pragma unroll
    for (int i = 0; i < 14; ++i) {
      buf[(i + 2) % 3] = mop(i + 2, vt, knext);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      mm(i);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    }
#pragma unroll
    for (int i = 14; i < 30; ++i) {
      buf[(i + 2) % 3] = mop(i + 2, vt, knext);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      mm(i);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    }
    mm(30);
    mm(31);
    (void)t;
  };
  // VALU phase V(t): online softmax of S(t) -> bf16 P(t) (per lane: one query, 32 of 64 keys).  With
  // dmaon the eight copy groups of this wave (rows rk4 into kdst, rv4 into vdst) are issued between the
  // exponentials, one per four scores, so the vector-memory path sees them spread over the phase.
  auto vphase = [&](int t, bool dmaon = false, int4 rk4 = int4{}, uint16_t* kdst = nullptr, int4 rv4 = int4{},
                    uint16_t* vdst = nullptr) __attribute__((always_inline)) {
    // sl: the factor from sacc to log2-domain logits (1 once an EAR tile is pre-scaled and biased)
    float sl = scale_log2;
    if constexpr (EAR) {
      if ((t + 1) * kKT > total_tok) {
        const int tbase = t * kKT;
#pragma unroll
        for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int p = tbase + kb2 * 32 + (r / 4) * 8 + h * 4 + (r % 4);
            float xv = sacc[kb2][r] * scale_log2;
            if (p >= total)
              xv = -INFINITY;
            else if (p >= total_tok)
              xv += cent_bias[p - total_tok];
            sacc[kb2][r] = xv;
          }
        sl = 1.0f;
      }
    } else {
      if ((t + 1) * kKT > total) {
        const int tbase = t * kKT;
#pragma unroll
        for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = kb2 * 32 + (r / 4) * 8 + h * 4 + (r % 4);
            if (tbase + key >= total) sacc[kb2][r] = -INFINITY;
          }
      }
    }
    // P against the running max m_run.  The lane's row sum over its 32 values bounds each of them, so
    // the maximum is only needed when the sum leaves [0, 2^13]: a value more than 13 (log2) above
    // m_run, or the first tile (m_run = -inf gives inf / NaN).  Then m_run moves to the tile maximum,
    // O and l are rescaled and P is recomputed.  The row sum adds the fp32 values (as the reference's
    // kernel does) in four chains.
    auto pexp = [&](bool dm) __attribute__((always_inline)) -> float {
      const float mneg = -m_run;
      const int rka[4] = {rk4.x, rk4.y, rk4.z, rk4.w}, rva[4] = {rv4.x, rv4.y, rv4.z, rv4.w};
      float la[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int kb2 = 0; kb2 < 2; ++kb2) {
        float pv[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          pv[r] = __builtin_amdgcn_exp2f(fmaf(sacc[kb2][r], sl, mneg));
          if (dm && r % 4 == 3) {
            const int j = (kb2 * 16 + r) / 4;
            __builtin_amdgcn_sched_group_barrier(0x002, 12, 0);
            if (j < kDmaIt)
              dma_one(kb, rka[j], j, kdst);
            else
              dma_one(vb, rva[j - kDmaIt], j - kDmaIt, vdst);
            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
          }
        }
#pragma unroll
        for (int st = 0; st < 2; ++st)
#pragma unroll
          for (int e = 0; e < 4; ++e) pop[kb2][st][e] = cvt_pk_bf16(pv[8 * st + 2 * e], pv[8 * st + 2 * e + 1]);
#pragma unroll
        for (int r = 0; r < 16; ++r) la[r % 4] += pv[r];
      }
      return (la[0] + la[1]) + (la[2] + la[3]);
    };
    float lsum = dmaon ? pexp(true) : pexp(false);
    if (__any(!(lsum <= 8192.0f))) {
      float mx = sacc[0][0];
#pragma unroll
      for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[kb2][r]);
      mx = xhalf_max(mx) * sl;
      const float m_new = fmaxf(m_run, mx);
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[db][r] *= alpha;
      lsum = pexp(false);
    }
    l_run += lsum;
  };
  // B-chunked items: group B's phases on the wave's 32-key chunk of a tile (its rows 32 rows further in
  // every K and V buffer; the swizzle depends on the row mod 16, so the chunk's rows read as rows 0-31),
  // with the scores and P of the chunk in sacc[0] and pop[0].
  const int chunk = (bchunk && group_b) ? (wg >> 1) : 0;
  if (chunk) {
    // the chunk's rows start 32 rows into every K and V buffer: folded into the lane offsets once
#pragma unroll
    for (int ks2 = 0; ks2 < 8; ++ks2) koffs[ks2] += 32 * 128;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      voffs[0][db] += 32 * 128;
      voffs[1][db] += 32 * 128;
    }
  }
  auto scores_q = [&](const uint16_t* kt) __attribute__((always_inline)) {
    sacc[0] = f32x16_t{};
#pragma unroll
    for (int ks2 = 0; ks2 < 8; ++ks2)
      sacc[0] = mfma32x32x16(as_bf16x8(*(const u32x4_t*)(&kt[koffs[ks2]])), as_bf16x8(qop[ks2]), sacc[0]);
  };
  auto mop_q = [&](int i, const uint16_t* vt, const uint16_t* knext) __attribute__((always_inline)) -> u32x4_t {
    if (i < 8) {
      const int st = i / 4, db = i % 4;
      const int rb = st * 16 * 128;
      const uint2 lo = ds_read_tr16_b64(&vt[rb + voffs[0][db]]);
      const uint2 hi = ds_read_tr16_b64(&vt[rb + voffs[1][db]]);
      return u32x4_t{lo.x, lo.y, hi.x, hi.y};
    }
    return *(const u32x4_t*)(&knext[koffs[i - 8]]);
  };
  auto mphase_q = [&](const uint16_t* vt, const uint16_t* knext) __attribute__((always_inline)) {
    u32x4_t buf[3];
    buf[0] = mop_q(0, vt, knext);
    buf[1] = mop_q(1, vt, knext);
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
    auto mm = [&](int i) __attribute__((always_inline)) {
      if (i < 8) {
        const int st = i / 4, db = i % 4;
        acc[db] = mfma32x32x16(as_bf16x8(buf[i % 3]), as_bf16x8(pop[0][st]), acc[db]);
      } else {
        if (i == 8) sacc[0] = f32x16_t{};
        sacc[0] = mfma32x32x16(as_bf16x8(buf[i % 3]), as_bf16x8(qop[i - 8]), sacc[0]);
      }
    };
#pragma unroll
    for (int i = 0; i < 6; ++i) {
      buf[(i + 2) % 3] = mop_q(i + 2, vt, knext);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      mm(i);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    }
#pragma unroll
    for (int i = 6; i < 14; ++i) {
      buf[(i + 2) % 3] = mop_q(i + 2, vt, knext);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      mm(i);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    }
    mm(14);
    mm(15);
  };
  // Softmax of the chunk of tile t; the eight copies of a copying wave go out one per two exponentials.
  // Only called for a chunk that holds a key (so the running maximum is finite after the first call).
  auto vphase_q = [&](int t, bool dmaon = false, int4 rk4 = int4{}, uint16_t* kdst = nullptr, int4 rv4 = int4{},
                      uint16_t* vdst = nullptr) __attribute__((always_inline)) {
    const int tbase = t * kKT + chunk * 32;
    if (tbase + 32 > total) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = (r / 4) * 8 + h * 4 + (r % 4);
        if (tbase + key >= total) sacc[0][r] = -INFINITY;
      }
    }
    auto pexp = [&](bool dm) __attribute__((always_inline)) -> float {
      const float mneg = -m_run;
      const int rka[4] = {rk4.x, rk4.y, rk4.z, rk4.w}, rva[4] = {rv4.x, rv4.y, rv4.z, rv4.w};
      float la[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      float pv[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        pv[r] = __builtin_amdgcn_exp2f(fmaf(sacc[0][r], scale_log2, mneg));
        if (dm && r % 2 == 1) {
          const int j = r / 2;
          __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
          if (j < kDmaIt)
            dma_one(kb, rka[j], j, kdst);
          else
            dma_one(vb, rva[j - kDmaIt], j - kDmaIt, vdst);
          __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
        }
      }
#pragma unroll
      for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int e = 0; e < 4; ++e) pop[0][st][e] = cvt_pk_bf16(pv[8 * st + 2 * e], pv[8 * st + 2 * e + 1]);
#pragma unroll
      for (int r = 0; r < 16; ++r) la[r % 4] += pv[r];
      return (la[0] + la[1]) + (la[2] + la[3]);
    };
    float lsum = dmaon ? pexp(true) : pexp(false);
    if (__any(!(lsum <= 8192.0f))) {
      float mx = sacc[0][0];
#pragma unroll
      for (int r = 1; r < 16; ++r) mx = fmaxf(mx, sacc[0][r]);
      mx = xhalf_max(mx) * scale_log2;
      const float m_new = fmaxf(m_run, mx);
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[db][r] *= alpha;
      lsum = pexp(false);
    }
    l_run += lsum;
  };
  if (!half) {
    // B-chunked items (kB): group B's waves wg and wg + 2 hold the same 32 queries and take the two 32-key
    // halves of every tile (its phases half as long), and group B resolves the row tables (waves 4 and 5, after
    // its MFMA phase) in place of waves 0 and 1.  The loop in two copies, one per item kind.
    const int nt1 = total > 32 ? (total - 32 + kKT - 1) / kKT : 0;  // tiles with a key in their second half
    const int nvb = __builtin_amdgcn_readfirstlane(chunk == 1 ? nt1 : ntiles);  // tiles of a B wave's chunk
    auto full_loop = [&](auto bchunk_tag) __attribute__((always_inline)) -> bool {
      constexpr bool kB = decltype(bchunk_tag)::value;
      constexpr int rw0 = kB ? 4 : 0, rw1 = kB ? 5 : 1;  // the resolving waves
      auto bvph = [&](int t, int4 rk4, uint16_t* kdst, int4 rv4, uint16_t* vdst) __attribute__((always_inline)) {
        if constexpr (kB)
          vphase_q(t, true, rk4, kdst, rv4, vdst);
        else
          vphase(t, true, rk4, kdst, rv4, vdst);
      };
      auto bmph = [&](const uint16_t* vt, const uint16_t* knext) __attribute__((always_inline)) {
        if constexpr (kB)
          mphase_q(vt, knext);
        else
          mphase(0, vt, knext);
      };
      // Prologue: tables K(0), K(1), V(0), V(1) (a table past the stream holds the last row, so copies
      // of tiles past the end stay inside this head); DMA K(0), V(0) -> buffers 0, K(1) -> K buffer 1;
      // S(0) everywhere, V(0) in group A; tables K(2), K(3), V(2); group B reads the rows of its first
      // copies (K(2), V(1)).
      if (wave == rw0) {
        resolve(rowtab[0][0][0], 0, 1);
        resolve(rowtab[0][0][1], 1, 1);
      }
      if (wave == rw1) {
        resolve(rowtab[0][1][0], 0, 1);
        resolve(rowtab[0][1][1], 1, 1);
      }
      __syncthreads();
      if (group_b) {
        dma(kb, rowtab[0][0][0], k_s0);
        dma(vb, rowtab[0][1][0], v_s0);
        if (ntiles > 1) dma(kb, rowtab[0][0][1], k_s1);
        __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
      }
      __syncthreads();
      if constexpr (kB) {
        if (!group_b) {
          if (active) {
            scores(k_s0);
            vphase(0);
          }
        } else if (active && nvb > 0) {
          scores_q(k_s0);
        }
      } else {
        if (active) scores(k_s0);
        if (active && !group_b) vphase(0);
      }
      if (wave == rw0) {
        resolve(rowtab[0][0][0], 2, 1);
        resolve(rowtab[0][0][1], 3, 1);
      }
      if (wave == rw1) resolve(rowtab[0][1][0], 2, 1);
      __syncthreads();
      int4 rk = make_int4(0, 0, 0, 0), rv = make_int4(0, 0, 0, 0);
      if (group_b) {
        rk = dma_rows(rowtab[0][0][0]);
        rv = dma_rows(rowtab[0][1][1]);
      }

      // Half-steps h = 0 .. 2T-1 (unrolled by 4: tile parity fixes the buffers).
      //   A: h = 2t -> M(t);  h = 2t+1 -> V(t+1), tables K(t+4) and V(t+3) (waves 0, 1)
      //   B: h = 2t -> V(t) with the copies of K(t+2) and V(t+1) spread through it;
      //      h = 2t+1 -> M(t), rows of the next copies K(t+3) and V(t+2), wait for the copies.
      // Copies run for tiles past the end too (rows from the tables), so the phases carry no branches.
      for (int t = 0; t < ntiles; t += 2) {
        // tile t (even): V(t) in v_s0, K(t+1) in k_s1
        if (!group_b) {
          if (active) mphase(t, v_s0, k_s1);
        } else {
          if (active && (!kB || t < nvb))
            bvph(t, rk, k_s0, rv, v_s1);
          else
            dma_all(rk, k_s0, rv, v_s1);
        }
        __syncthreads();
        if (!group_b) {
          if (active && t + 1 < ntiles) vphase(t + 1);
          if constexpr (!kB) {
            if (wave == 0 && t + 4 < ntiles) resolve(rowtab[0][0][t & 1], t + 4, 1);
            if (wave == 1 && t + 3 < ntiles) resolve(rowtab[0][1][(t + 1) & 1], t + 3, 1);
          }
        } else {
          if (active && (!kB || t < nvb)) bmph(v_s0, k_s1);
          if constexpr (kB) {
            if (wave == 4 && t + 4 < ntiles) resolve(rowtab[0][0][t & 1], t + 4, 1);
            if (wave == 5 && t + 3 < ntiles) resolve(rowtab[0][1][(t + 1) & 1], t + 3, 1);
          }
          rk = dma_rows(rowtab[0][0][(t + 1) & 1]);
          rv = dma_rows(rowtab[0][1][t & 1]);
          __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        __syncthreads();
        if (t + 1 >= ntiles) break;
        // tile t+1 (odd): V(t+1) in v_s1, K(t+2) in k_s0
        if (!group_b) {
          if (active) mphase(t + 1, v_s1, k_s0);
        } else {
          if (active && (!kB || t + 1 < nvb))
            bvph(t + 1, rk, k_s1, rv, v_s0);
          else
            dma_all(rk, k_s1, rv, v_s0);
        }
        __syncthreads();
        if (!group_b) {
          if (active && t + 2 < ntiles) vphase(t + 2);
          if constexpr (!kB) {
            if (wave == 0 && t + 5 < ntiles) resolve(rowtab[0][0][(t + 1) & 1], t + 5, 1);
            if (wave == 1 && t + 4 < ntiles) resolve(rowtab[0][1][t & 1], t + 4, 1);
          }
        } else {
          if (active && (!kB || t + 1 < nvb)) bmph(v_s1, k_s0);
          if constexpr (kB) {
            if (wave == 4 && t + 5 < ntiles) resolve(rowtab[0][0][(t + 1) & 1], t + 5, 1);
            if (wave == 5 && t + 4 < ntiles) resolve(rowtab[0][1][t & 1], t + 4, 1);
          }
          rk = dma_rows(rowtab[0][0][t & 1]);
          rv = dma_rows(rowtab[0][1][(t + 1) & 1]);
          __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        __syncthreads();
      }

      // B-chunked: the chunk-1 waves' states (queries 128 + 32 (wg & 1) ..) merge into the chunk-0 waves'
      // (every wave takes part in the barriers; the K/V buffers are free after the loop's last barrier)
      if constexpr (kB) {
        float* ob_lds[4] = {(float*)k_s0, (float*)k_s1, (float*)v_s0, (float*)v_s1};
        float2* ml_lds = (float2*)k1_s0;
        const int sl = (wg & 1) * kWave + lane;
        if (group_b && active && chunk == 1) {
#pragma unroll
          for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4)
              ((f32x4_t*)ob_lds[db])[r4 * 256 + sl] =
                  f32x4_t{acc[db][4 * r4], acc[db][4 * r4 + 1], acc[db][4 * r4 + 2], acc[db][4 * r4 + 3]};
          ml_lds[sl] = make_float2(m_run, l_run);
        }
        __syncthreads();
        if (group_b && active && chunk == 0) {
          const float2 mlb = ml_lds[sl];
          const float m = fmaxf(m_run, mlb.x);
          // chunk 0 holds tile 0's first key, so m is finite; an empty chunk 1 has m = -inf and weight 0
          const float wa = __builtin_amdgcn_exp2f(m_run - m), wb = __builtin_amdgcn_exp2f(mlb.x - m);
          l_run = l_run * wa + mlb.y * wb;
#pragma unroll
          for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
              const f32x4_t o2 = ((const f32x4_t*)ob_lds[db])[r4 * 256 + sl];
#pragma unroll
              for (int e = 0; e < 4; ++e) acc[db][4 * r4 + e] = acc[db][4 * r4 + e] * wa + o2[e] * wb;
            }
        }
        return !(group_b && chunk == 1);
      }
      return true;
    };
    const bool keep = bchunk ? full_loop(std::true_type{}) : full_loop(std::false_type{});
    if (!keep) return;
  } else if constexpr (HC) {
    // Half item: local tile u of stream x is global tile 2u + x; stream 0 (n0 tiles) lives in the
    // k_s / v_s buffers and is used by group A, stream 1 (n1 tiles) in k1_s / v1_s, used by group B.
    // Each group copies its own stream's tiles during its softmax; waves 0-3 resolve the four tables.
    const int n0 = (ntiles + 1) / 2, n1 = ntiles / 2;
    // Tables of step u (waves 0-3, before group A's MFMA half-step): K(u+3) and V(u+2) of each stream.
    auto resolve2 = [&](int u) __attribute__((always_inline)) {
      if (wave == 0 && u + 3 < n0) resolve(rowtab[0][0][(u + 1) & 1], 2 * (u + 3), 2);
      if (wave == 1 && u + 2 < n0) resolve(rowtab[0][1][u & 1], 2 * (u + 2), 2);
      if (wave == 2 && u + 3 < n1) resolve(rowtab[1][0][(u + 1) & 1], 2 * (u + 3) + 1, 2);
      if (wave == 3 && u + 2 < n1) resolve(rowtab[1][1][u & 1], 2 * (u + 2) + 1, 2);
    };
    // Rows of the copies of K(u+2) and V(u+1) of a stream with n tiles (tables of slot u & 1 and (u + 1) & 1).
    // A tile past the stream takes row 0 of the head: the copy lands in a buffer that is not read for it.
    auto rows2 = [&](int x, int u, int n, int4& rk, int4& rv) __attribute__((always_inline)) {
      rk = u + 2 < n ? dma_rows(rowtab[x][0][u & 1]) : make_int4(0, 0, 0, 0);
      rv = u + 1 < n ? dma_rows(rowtab[x][1][(u + 1) & 1]) : make_int4(0, 0, 0, 0);
    };
    if (wave == 0) {
      resolve(rowtab[0][0][0], 0, 2);
      if (n0 > 1) resolve(rowtab[0][0][1], 2, 2);
    }
    if (wave == 1) {
      resolve(rowtab[0][1][0], 0, 2);
      if (n0 > 1) resolve(rowtab[0][1][1], 2, 2);
    }
    if (wave == 2 && n1 > 0) {
      resolve(rowtab[1][0][0], 1, 2);
      if (n1 > 1) resolve(rowtab[1][0][1], 3, 2);
    }
    if (wave == 3 && n1 > 0) {
      resolve(rowtab[1][1][0], 1, 2);
      if (n1 > 1) resolve(rowtab[1][1][1], 3, 2);
    }
    __syncthreads();
    if (group_b) {
      dma(kb, rowtab[0][0][0], k_s0);
      dma(vb, rowtab[0][1][0], v_s0);
      if (n0 > 1) dma(kb, rowtab[0][0][1], k_s1);
      if (n1 > 0) {
        dma(kb, rowtab[1][0][0], k1_s0);
        dma(vb, rowtab[1][1][0], v1_s0);
        if (n1 > 1) dma(kb, rowtab[1][0][1], k1_s1);
      }
      __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    __syncthreads();
    if (active) {
      if (!group_b) {
        scores(k_s0);
        vphase(0);
      } else if (n1 > 0) {
        scores(k1_s0);
      }
    }
    if (wave == 0 && n0 > 2) resolve(rowtab[0][0][0], 4, 2);
    if (wave == 2 && n1 > 2) resolve(rowtab[1][0][0], 5, 2);
    __syncthreads();
    //   A: h = 2u -> M(u), h = 2u+1 -> V(u+1) with the copies of stream 0's K(u+2), V(u+1) spread through it;
    //   B: h = 2u -> V(u) with the copies of stream 1's K(u+2), V(u+1) spread through it and the tables,
    //   h = 2u+1 -> M(u).  Each group's copies land in buffers the other group does not read, by the barrier
    //   that ends the half-step; group B runs out of tiles first (n1 <= n0) and then only copies.
    for (int u = 0; u < n0; u += 2) {
      int4 rk, rv;
      if (!group_b) {
        resolve2(u);
        if (active) mphase(u, v_s0, k_s1);
      } else {
        rows2(1, u, n1, rk, rv);
        if (active && u < n1)
          vphase(2 * u + 1, true, rk, k1_s0, rv, v1_s1);
        else
          dma_all(rk, k1_s0, rv, v1_s1);
      }
      __syncthreads();
      if (!group_b) {
        rows2(0, u, n0, rk, rv);
        if (active && u + 1 < n0)
          vphase(2 * u + 2, true, rk, k_s0, rv, v_s1);
        else
          dma_all(rk, k_s0, rv, v_s1);
      } else {
        if (active && u < n1) mphase(u, v1_s0, k1_s1);
      }
      __syncthreads();
      if (u + 1 >= n0) break;
      if (!group_b) {
        resolve2(u + 1);
        if (active) mphase(u + 1, v_s1, k_s0);
      } else {
        rows2(1, u + 1, n1, rk, rv);
        if (active && u + 1 < n1)
          vphase(2 * u + 3, true, rk, k1_s1, rv, v1_s0);
        else
          dma_all(rk, k1_s1, rv, v1_s0);
      }
      __syncthreads();
      if (!group_b) {
        rows2(0, u + 1, n0, rk, rv);
        if (active && u + 2 < n0)
          vphase(2 * u + 4, true, rk, k_s1, rv, v_s0);
        else
          dma_all(rk, k_s1, rv, v_s0);
      } else {
        if (active && u + 1 < n1) mphase(u + 1, v1_s1, k1_s0);
      }
      __syncthreads();
    }
    // Merge: group B leaves (m, l, O) in the stream-0 buffers (no tile is read any more and no copy
    // is in flight); group A rescales both states to the common maximum and adds them.  Layout
    // [db][r / 4][wave][lane] of 16-byte chunks for O, [wave][lane] of (m, l) pairs.
    float* ob_lds[4] = {(float*)k_s0, (float*)k_s1, (float*)v_s0, (float*)v_s1};
    float2* ml_lds = (float2*)k1_s0;
    const int slot = wg * kWave + lane;
    if (group_b && active) {
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4)
          ((f32x4_t*)ob_lds[db])[r4 * 256 + slot] =
              f32x4_t{acc[db][4 * r4], acc[db][4 * r4 + 1], acc[db][4 * r4 + 2], acc[db][4 * r4 + 3]};
      ml_lds[slot] = make_float2(m_run, l_run);
    }
    __syncthreads();
    if (group_b) return;
    if (active) {
      const float2 mlb = ml_lds[slot];
      const float m = fmaxf(m_run, mlb.x);
      // stream 0 holds tile 0, so m is finite; an empty stream 1 has m = -inf and weight 0
      const float wa = __builtin_amdgcn_exp2f(m_run - m), wb = __builtin_amdgcn_exp2f(mlb.x - m);
      l_run = l_run * wa + mlb.y * wb;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const f32x4_t o2 = ((const f32x4_t*)ob_lds[db])[r4 * 256 + slot];
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[db][4 * r4 + e] = acc[db][4 * r4 + e] * wa + o2[e] * wb;
        }
    }
  }

  if (!active) return;
  // Normalise and store: lane holds d = db*32 + (r/4)*8 + 4h + r%4 of query l32.
  const float lt = xhalf_sum(l_run);
  const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
  const int row = qrow0 + l32;
  if (row < q1) {
    uint16_t* dst = out_row(row);
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = db * 32 + g * 8 + h * 4;
        uint2 w;
        w.x = cvt_pk_bf16(acc[db][4 * g] * inv, acc[db][4 * g + 1] * inv);
        w.y = cvt_pk_bf16(acc[db][4 * g + 2] * inv, acc[db][4 * g + 3] * inv);
        *(uint2*)(dst + d0) = w;
      }
  }
}

// ------------------------------------------------------------------------------------------ segments (diagnostic)
__global__ void __launch_bounds__(kVWaves * kWave) vbsa_segments_kernel(const uint8_t* __restrict__ map,
                                                                        const int32_t* __restrict__ ks, int qn, int kn,
                                                                        int32_t* __restrict__ out_start,
                                                                        int32_t* __restrict__ out_len,
                                                                        int32_t* __restrict__ out_count) {
  __shared__ long long red[kVWaves];
  extern __shared__ int32_t seg_mem[];  // koff[kn + 1], seg_start[kn], seg_cum[kn + 1]
  const int b = blockIdx.y, i = blockIdx.x, tid = threadIdx.x;
  int32_t* ko = seg_mem;
  int32_t* seg_start = seg_mem + kn + 1;
  int32_t* seg_cum = seg_start + kn;
  const int32_t* ksb = ks + (size_t)b * kn;
  if (tid == 0) {
    int run = 0;
    for (int j = 0; j < kn; ++j) {
      ko[j] = run;
      run += ksb[j];
    }
    ko[kn] = run;
  }
  __syncthreads();
  int total = 0;
  const int nseg = build_segments(map + ((size_t)b * qn + i) * kn, ko, ksb, kn, seg_start, seg_cum, red, &total);
  const size_t row = (size_t)b * qn + i;
  for (int c = tid; c < nseg; c += blockDim.x) {
    out_start[row * kn + c] = seg_start[c];
    out_len[row * kn + c] = seg_cum[c + 1] - seg_cum[c];
  }
  if (tid == 0) out_count[row] = nseg;
}

}  // namespace svoo

using namespace svoo;

namespace {
constexpr int kDefaultQB = 1;
struct VbsaWs {
  size_t qoff, koff, items, nitems, work, list, total;
  int cap;
};
VbsaWs vbsa_layout(int bh, int s, int qn, int kn) {
  auto al = [](size_t v) { return (v + 255) / 256 * 256; };
  VbsaWs w;
  const int qtile = VbsaCfg<kDefaultQB>::kQTile;
  w.cap = (s + qtile - 1) / qtile + qn;
  w.qoff = 0;
  w.koff = w.qoff + al((size_t)bh * (qn + 1) * 4);
  w.items = w.koff + al((size_t)bh * (kn + 1) * 4);
  w.nitems = w.items + al((size_t)bh * w.cap * 4);
  w.work = w.nitems + al((size_t)bh * 4);
  w.list = w.work + al((size_t)bh * 4);
  w.total = w.list + al((size_t)bh * w.cap * 4);
  return w;
}
}  // namespace

extern "C" size_t svoo_vbsa_workspace_size(int bh, int s, int qn, int kn) {
  if (bh <= 0 || s <= 0 || qn <= 0 || kn <= 0) return 256;
  return vbsa_layout(bh, s, qn, kn).total;
}

namespace {
template <bool EAR, bool IDX = false>
int vbsa_launch(const char* name, const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* kc,
                const uint16_t* vc, const uint8_t* map, const int32_t* q_sizes, const int32_t* k_sizes, uint16_t* o,
                int bh, int s, int d, int qn, int kn, void* workspace, size_t ws_bytes, int32_t* status,
                void* stream, const int32_t* q_idx = nullptr, const int32_t* k_idx = nullptr, int heads = 1) {
  SVOO_REQUIRE(q && k && v && map && q_sizes && k_sizes && o && (!EAR || (kc && vc)), SVOO_ERR_INVALID_ARG,
               "%s: null pointer", name);
  SVOO_REQUIRE_HEAD_DIM(d, name);
  SVOO_REQUIRE(bh > 0 && s > 0 && qn > 0 && kn > 0, SVOO_ERR_INVALID_ARG, "%s: bad dims", name);
  SVOO_REQUIRE(kn <= kMaxKN && qn < 32768, SVOO_ERR_UNSUPPORTED, "%s: qn=%d kn=%d above limits", name, qn, kn);
  // a work-list entry is head << 15 | slot
  SVOO_REQUIRE(bh < 65536, SVOO_ERR_UNSUPPORTED, "%s: bh=%d above 65535", name, bh);
  SVOO_REQUIRE((long long)bh * s * 128 < (1ll << 40), SVOO_ERR_UNSUPPORTED, "%s: too large", name);
  SVOO_REQUIRE(s < (1 << 24), SVOO_ERR_UNSUPPORTED, "%s: S=%d above 2^24 tokens per head", name, s);
  const VbsaWs lay = vbsa_layout(bh, s, qn, kn);
  // the tile index of a work item is 15 bits (bit 15 flags a half item)
  SVOO_REQUIRE(lay.cap < 32768, SVOO_ERR_UNSUPPORTED, "%s: too many q tiles per head", name);
  SVOO_REQUIRE(workspace && ws_bytes >= lay.total, SVOO_ERR_WORKSPACE, "%s: workspace %zu < %zu", name, ws_bytes,
               lay.total);
  if (EAR) {
    // centroid rows are addressed as signed int32 row offsets from the token buffers
    const long long dk = (long long)(uintptr_t)kc - (long long)(uintptr_t)k;
    const long long dv = (long long)(uintptr_t)vc - (long long)(uintptr_t)v;
    SVOO_REQUIRE(dk % 256 == 0 && dv % 256 == 0, SVOO_ERR_INVALID_ARG,
                 "%s: centroid buffers must be 256-byte congruent with k and v", name);
    const long long lim = (1ll << 31) - 1 - (long long)bh * (s + kn);
    SVOO_REQUIRE(llabs(dk / 256) < lim && llabs(dv / 256) < lim, SVOO_ERR_UNSUPPORTED,
                 "%s: centroid buffers too far from k / v for int32 row offsets", name);
  }
  hipStream_t st = (hipStream_t)stream;
  char* base = (char*)workspace;
  int32_t* qoff = (int32_t*)(base + lay.qoff);
  int32_t* koff = (int32_t*)(base + lay.koff);
  int32_t* items = (int32_t*)(base + lay.items);
  int32_t* nitems = (int32_t*)(base + lay.nitems);
  int32_t* work = (int32_t*)(base + lay.work);
  int32_t* list = (int32_t*)(base + lay.list);
  constexpr int qtile = VbsaCfg<kDefaultQB>::kQTile;
  const size_t smem = (size_t)((EAR ? 4 : 2) * kn + 1) * sizeof(int32_t);
  // Half items need the kernel with a second set of K/V buffers (130 KB of static LDS with the row
  // tables), which leaves 28 KB of the 160 KB LDS for the segment tables.  The EAR kernel (64-bit copy
  // addresses for the centroid rows) runs full items only: with both paths it exceeds 256 registers.
  const bool half_ok = !EAR && smem <= (size_t)28 * 1024;
  hipLaunchKernelGGL(vbsa_plan_kernel, dim3(bh), dim3(kPlanThreads), 0, st, q_sizes, k_sizes, map, EAR ? 1 : 0, work,
                     s, qn, kn, qtile, lay.cap, half_ok ? 1 : 0, qoff, koff, items, nitems, status);
  if (int rc = check_launch(name)) return rc;
  hipLaunchKernelGGL(vbsa_order_kernel, dim3(1), dim3(kOrderThreads), 0, st, work, nitems, bh, lay.cap,
                     (s + qtile - 1) / qtile, list);
  if (int rc = check_launch(name)) return rc;
  const long long total_items = (long long)bh * lay.cap;
  const long long nblocks = (total_items + 8 * kXcdRun - 1) / (8 * kXcdRun) * (8 * kXcdRun);
  SVOO_REQUIRE(nblocks < (1ll << 31), SVOO_ERR_UNSUPPORTED, "%s: too many work items", name);
  const float scale_log2 = (float)(1.4426950408889634 / sqrt((double)d));
  if (!EAR && half_ok)
    hipLaunchKernelGGL((vbsa_attn_kernel<kDefaultQB, EAR, IDX, !EAR>), dim3((unsigned)nblocks), dim3(kVWaves * kWave),
                       smem, st, q, k, v, kc, vc, map, k_sizes, o, s, qn, kn, lay.cap, total_items, qoff, koff, items,
                       nitems, scale_log2, q_idx, k_idx, heads, list);
  else
    hipLaunchKernelGGL((vbsa_attn_kernel<kDefaultQB, EAR, IDX, false>), dim3((unsigned)nblocks), dim3(kVWaves * kWave),
                       smem, st, q, k, v, kc, vc, map, k_sizes, o, s, qn, kn, lay.cap, total_items, qoff, koff, items,
                       nitems, scale_log2, q_idx, k_idx, heads, list);
  return check_launch(name);
}
}  // namespace

extern "C" int svoo_vbsa_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint8_t* map,
                             const int32_t* q_sizes, const int32_t* k_sizes, uint16_t* o, int bh, int s, int d, int qn,
                             int kn, void* workspace, size_t ws_bytes, int32_t* status, void* stream) {
  return vbsa_launch<false>("svoo_vbsa_fwd", q, k, v, nullptr, nullptr, map, q_sizes, k_sizes, o, bh, s, d, qn, kn,
                            workspace, ws_bytes, status, stream);
}

extern "C" int svoo_vbsa_fused_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v, const int32_t* q_sorted_idx,
                                   const int32_t* k_sorted_idx, const uint8_t* map, const int32_t* q_sizes,
                                   const int32_t* k_sizes, uint16_t* o_bshd, int bh, int heads, int s, int d, int qn,
                                   int kn, void* workspace, size_t ws_bytes, int32_t* status, void* stream) {
  SVOO_REQUIRE(q_sorted_idx && k_sorted_idx, SVOO_ERR_INVALID_ARG, "svoo_vbsa_fused_fwd: null index");
  SVOO_REQUIRE(heads > 0 && bh % heads == 0, SVOO_ERR_INVALID_ARG, "svoo_vbsa_fused_fwd: bh=%d not a multiple of H=%d",
               bh, heads);
  return vbsa_launch<false, true>("svoo_vbsa_fused_fwd", q, k, v, nullptr, nullptr, map, q_sizes, k_sizes, o_bshd, bh,
                                  s, d, qn, kn, workspace, ws_bytes, status, stream, q_sorted_idx, k_sorted_idx, heads);
}

// ------------------------------------------------------------------------------------------ allocation-free entry
// svoo_vbsa_fused_fwd_noalloc keeps the plan (cluster offsets, work items, work list) in this file-scope
// device array instead of a caller workspace.  Each device holds its own copy; host code must use the
// address hipGetSymbolAddress returns for the current device, never the array's name.
static __device__ __align__(256) unsigned char scratch[SVOO_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};

// Address of `scratch` on the current device, resolved once per device.
int scratch_on_current_device(const char* name, void** out) {
  int dev = -1;
  const hipError_t e = hipGetDevice(&dev);
  SVOO_REQUIRE(e == hipSuccess, SVOO_ERR_HIP, "%s: hipGetDevice failed: %s", name, hipGetErrorString(e));
  SVOO_REQUIRE(dev >= 0 && dev < kMaxScratchDevices, SVOO_ERR_UNSUPPORTED, "%s: device %d above %d", name, dev,
               kMaxScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t es = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    SVOO_REQUIRE(es == hipSuccess && p, SVOO_ERR_HIP, "%s: hipGetSymbolAddress(scratch) on device %d failed: %s",
                 name, dev, hipGetErrorString(es));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return SVOO_OK;
}
}  // namespace

extern "C" int svoo_vbsa_fused_fwd_noalloc(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                           const int32_t* q_sorted_idx, const int32_t* k_sorted_idx,
                                           const uint8_t* map, const int32_t* q_sizes, const int32_t* k_sizes,
                                           uint16_t* o_bshd, int bh, int heads, int s, int d, int qn, int kn,
                                           int32_t* status, void* stream) {
  static const char* name = "svoo_vbsa_fused_fwd_noalloc";
  SVOO_REQUIRE(bh > 0 && s > 0 && qn > 0 && kn > 0, SVOO_ERR_INVALID_ARG, "%s: bad dims", name);
  const size_t need = vbsa_layout(bh, s, qn, kn).total;
  SVOO_REQUIRE(need <= (size_t)SVOO_NOALLOC_SCRATCH_BYTES, SVOO_ERR_WORKSPACE,
               "%s: plan needs %zu bytes, above the static scratch of %zu bytes (use svoo_vbsa_fused_fwd with a "
               "workspace)", name, need, (size_t)SVOO_NOALLOC_SCRATCH_BYTES);
  SVOO_REQUIRE(q_sorted_idx && k_sorted_idx, SVOO_ERR_INVALID_ARG, "%s: null index", name);
  SVOO_REQUIRE(heads > 0 && bh % heads == 0, SVOO_ERR_INVALID_ARG, "%s: bh=%d not a multiple of H=%d", name, bh,
               heads);
  void* ws = nullptr;
  if (int rc = scratch_on_current_device(name, &ws)) return rc;
  return vbsa_launch<false, true>(name, q, k, v, nullptr, nullptr, map, q_sizes, k_sizes, o_bshd, bh, s, d, qn, kn,
                                  ws, (size_t)SVOO_NOALLOC_SCRATCH_BYTES, status, stream, q_sorted_idx, k_sorted_idx,
                                  heads);
}

extern "C" int svoo_vbsa_ear_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* k_cent,
                                 const uint16_t* v_cent, const uint8_t* map, const int32_t* q_sizes,
                                 const int32_t* k_sizes, uint16_t* o, int bh, int s, int d, int qn, int kn,
                                 void* workspace, size_t ws_bytes, int32_t* status, void* stream) {
  return vbsa_launch<true>("svoo_vbsa_ear_fwd", q, k, v, k_cent, v_cent, map, q_sizes, k_sizes, o, bh, s, d, qn, kn,
                           workspace, ws_bytes, status, stream);
}

extern "C" int svoo_vbsa_segments(const uint8_t* map, const int32_t* k_sizes, int bh, int qn, int kn,
                                  int32_t* seg_start, int32_t* seg_len, int32_t* seg_count, void* stream) {
  SVOO_REQUIRE(map && k_sizes && seg_start && seg_len && seg_count, SVOO_ERR_INVALID_ARG,
               "svoo_vbsa_segments: null pointer");
  SVOO_REQUIRE(bh > 0 && qn > 0 && kn > 0 && kn <= kMaxKN && qn <= 65535 && bh <= 65535, SVOO_ERR_INVALID_ARG,
               "svoo_vbsa_segments: bad dims");
  const size_t smem = (size_t)(3 * kn + 2) * sizeof(int32_t);
  hipLaunchKernelGGL(vbsa_segments_kernel, dim3(qn, bh), dim3(kVWaves * kWave), smem, (hipStream_t)stream, map,
                     k_sizes, qn, kn, seg_start, seg_len, seg_count);
  return check_launch("svoo_vbsa_segments");
}
