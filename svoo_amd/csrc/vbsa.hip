// Variable-block-sparse attention (VBSA) over cluster-contiguous tokens, gfx950 MFMA.
//
// Plan (one block per batch-head, on device, no host round trip):
//   qoff/koff = exclusive prefix of the cluster sizes (validated to sum to S), and a work list of
//   (q-cluster, q-tile) items, kQTile queries each.
// Attention (one block per work item, 4 waves, each wave owns 32*QB queries):
//   * the block compacts its map row into a list of active key segments (start, length) in LDS;
//     the KV stream is their concatenation (ascending cluster), cut into 64-key tiles that span
//     segment boundaries, so padding happens once per work item instead of once per cluster;
//   * per tile: K and V are staged row-major in LDS; the next tile's rows are fetched into
//     registers while the current tile computes;
//   * S^T = K Q^T with v_mfma_f32_32x32x16_bf16 (keys on M, queries on N), so each lane holds 16
//     keys of one query: the row max needs one cross-half exchange and the online-softmax rescale
//     is a per-lane scalar;  O^T += V^T P^T reuses the S^T accumulators as the B operand directly,
//     with the V^T operand gathered by gfx950's transposing LDS read (ds_read_b64_tr_b16);
//   * fp32 online softmax (exp2 with the scale folded in), P rounded to bf16 for the PV MFMA, as
//     the reference's Triton kernel does; rows of a cluster with no active keys are written as 0.
#include "svoo_common.h"

namespace svoo {

constexpr int kVWaves = 4;
constexpr int kKT = 64;          // keys per tile
constexpr int kKStride = 136;    // bf16 per staged K row (128 + 8 pad)
constexpr int kVStride = 160;    // bf16 per staged V row (128 + 32 pad: conflict-free transposed reads)
constexpr int kPlanThreads = 256;
constexpr int kMaxKN = 4096;

template <int QB>
struct VbsaCfg {
  static constexpr int kQTile = kVWaves * 32 * QB;
};

// ------------------------------------------------------------------------------------------ plan
__global__ void __launch_bounds__(kPlanThreads) vbsa_plan_kernel(const int32_t* __restrict__ qs,
                                                                 const int32_t* __restrict__ ks, int s, int qn, int kn,
                                                                 int qtile, int cap, int32_t* __restrict__ qoff,
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
    const bool ok = !bad && (int)(tot & 0xffffffffll) == s && (int)(tot >> 32) <= cap;
    for (int i = i0; i < i1; ++i) {
      const int v = qsb[i];
      qo[i] = (int32_t)(run & 0xffffffffll);
      const int t0 = (int)(run >> 32);
      const int nt = v > 0 ? (v + qtile - 1) / qtile : 0;
      if (ok)
        for (int t = 0; t < nt; ++t) items[(size_t)b * cap + t0 + t] = (i << 16) | t;
      run += ((long long)nt << 32) | (long long)(uint32_t)v;
    }
    if (tid == 0) {
      qo[qn] = (int32_t)(tot & 0xffffffffll);
      nitems[b] = ok ? (int32_t)(tot >> 32) : 0;
      if (!ok && status) atomicOr(status, 1);
    }
  }
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
// Block = 4 waves x 32 queries of one query cluster.  Per 64-key tile:
//   S^T = K Q^T   (A = K rows from LDS via ds_read_b128, B = Q held in registers), 16 MFMAs/wave;
//   P = exp2(S * scale * log2e - m)  with a lazily updated running max m (rescale only when the
//       tile max exceeds m by more than 8, i.e. P <= 2^8), P rounded to bf16 in registers;
//   O^T += V^T P^T  (A = V columns read transposed from row-major LDS with ds_read_b64_tr_b16,
//       B = the S^T accumulators' registers, whose key order the V read follows), 16 MFMAs/wave.
template <int QB>
__global__ void __launch_bounds__(kVWaves * kWave) __attribute__((amdgpu_waves_per_eu(2, 2))) vbsa_attn_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const uint8_t* __restrict__ map, const int32_t* __restrict__ ks, uint16_t* __restrict__ o, int s, int qn, int kn,
    int cap, long long total_items, const int32_t* __restrict__ qoff, const int32_t* __restrict__ koff,
    const int32_t* __restrict__ items, const int32_t* __restrict__ nitems, float scale_log2) {
  constexpr int kQTile = VbsaCfg<QB>::kQTile;
  __shared__ __attribute__((aligned(16))) uint16_t k_s[kKT * kKStride];
  __shared__ __attribute__((aligned(16))) uint16_t v_s[kKT * kVStride];
  __shared__ long long red[kVWaves];
  extern __shared__ int32_t seg_mem[];  // seg_start[kn], seg_cum[kn + 1]

  const long long item = xcd_item(blockIdx.x);
  if (item >= total_items) return;
  const int b = (int)(item / cap), local = (int)(item % cap);
  if (local >= nitems[b]) return;
  const int packed = items[(size_t)b * cap + local];
  const int ci = packed >> 16, tile = packed & 0xffff;
  const int32_t* qo = qoff + (size_t)b * (qn + 1);
  const int q0 = qo[ci] + tile * kQTile;
  const int q1 = min(qo[ci + 1], q0 + kQTile);

  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave, h = lane / 32, l32 = lane % 32;
  const int grp = lane / 16, gl = lane % 16;  // transposed-read group and lane within it
  const size_t head = (size_t)b * s * 128;
  const uint16_t* qb = q + head;
  const uint16_t* kb = k + head;
  const uint16_t* vb = v + head;
  uint16_t* ob = o + head;

  int32_t* seg_start = seg_mem;
  int32_t* seg_cum = seg_mem + kn;
  int total = 0;
  const int nseg = build_segments(map + ((size_t)b * qn + ci) * kn, koff + (size_t)b * (kn + 1), ks + (size_t)b * kn,
                                  kn, seg_start, seg_cum, red, &total);

  if (total == 0) {
    // Empty row: zero output (reference semantics, svoo/co_clustering.py:1102-1104).
    for (int idx = tid; idx < (q1 - q0) * 16; idx += kVWaves * kWave) {
      const int r = idx / 16, c = idx % 16;
      ((u32x4_t*)(ob + (size_t)(q0 + r) * 128))[c] = u32x4_t{0u, 0u, 0u, 0u};
    }
    return;
  }

  // Q operands (B of S^T = K Q^T): lane holds 8 consecutive d of its query per 16-wide k-step.
  u32x4_t qop[QB][8];
#pragma unroll
  for (int qbk = 0; qbk < QB; ++qbk) {
    const int row = min(q0 + wave * 32 * QB + qbk * 32 + l32, q1 - 1);
    const u32x4_t* src = (const u32x4_t*)(qb + (size_t)row * 128);
#pragma unroll
    for (int ks2 = 0; ks2 < 8; ++ks2) qop[qbk][ks2] = src[ks2 * 2 + h];
  }

  f32x16_t acc[QB][4];
#pragma unroll
  for (int qbk = 0; qbk < QB; ++qbk)
#pragma unroll
    for (int db = 0; db < 4; ++db) acc[qbk][db] = f32x16_t{};
  float m_run[QB], l_run[QB];
#pragma unroll
  for (int qbk = 0; qbk < QB; ++qbk) {
    m_run[qbk] = -INFINITY;
    l_run[qbk] = 0.0f;
  }

  // Each thread moves 4 rows x 16 bytes of K and of V per tile: rows r_u = tid/16 + 16u, piece tid%16.
  const int piece = tid % 16, rbase = tid / 16;
  int cur[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) cur[u] = find_segment(seg_cum, nseg, min(rbase + 16 * u, total - 1));
  u32x4_t kreg[4], vreg[4];
  auto fetch = [&](int t0) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int p = t0 + rbase + 16 * u;
      if (p < total) {
        while (cur[u] + 1 < nseg && seg_cum[cur[u] + 1] <= p) ++cur[u];
        const int row = seg_start[cur[u]] + (p - seg_cum[cur[u]]);
        kreg[u] = ((const u32x4_t*)(kb + (size_t)row * 128))[piece];
        vreg[u] = ((const u32x4_t*)(vb + (size_t)row * 128))[piece];
      } else {
        kreg[u] = u32x4_t{0u, 0u, 0u, 0u};
        vreg[u] = u32x4_t{0u, 0u, 0u, 0u};
      }
    }
  };

  const int ntiles = (total + kKT - 1) / kKT;
  fetch(0);
  for (int t = 0; t < ntiles; ++t) {
    __syncthreads();
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int r = rbase + 16 * u;
      *(u32x4_t*)(&k_s[r * kKStride + piece * 8]) = kreg[u];
      *(u32x4_t*)(&v_s[r * kVStride + piece * 8]) = vreg[u];
    }
    __syncthreads();
    if (t + 1 < ntiles) fetch((t + 1) * kKT);

    // S^T = K Q^T for the two 32-key blocks of the tile.
    f32x16_t sacc[QB][2];
#pragma unroll
    for (int qbk = 0; qbk < QB; ++qbk) {
      sacc[qbk][0] = f32x16_t{};
      sacc[qbk][1] = f32x16_t{};
    }
#pragma unroll
    for (int ks2 = 0; ks2 < 8; ++ks2) {
#pragma unroll
      for (int kb2 = 0; kb2 < 2; ++kb2) {
        const bf16x8_t a = as_bf16x8(*(const u32x4_t*)(&k_s[(kb2 * 32 + l32) * kKStride + ks2 * 16 + h * 8]));
#pragma unroll
        for (int qbk = 0; qbk < QB; ++qbk) sacc[qbk][kb2] = mfma32x32x16(a, as_bf16x8(qop[qbk][ks2]), sacc[qbk][kb2]);
      }
    }

    // Online softmax (per lane: one query, 32 of the tile's 64 keys).
    const bool tail = (t + 1) * kKT > total;
    u32x4_t pop[QB][2][2];
#pragma unroll
    for (int qbk = 0; qbk < QB; ++qbk) {
      if (tail) {
        const int tbase = t * kKT;
#pragma unroll
        for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = kb2 * 32 + (r / 4) * 8 + h * 4 + (r % 4);
            if (tbase + key >= total) sacc[qbk][kb2][r] = -INFINITY;
          }
      }
      float mx = sacc[qbk][0][0];
#pragma unroll
      for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[qbk][kb2][r]);
      mx = fmaxf(mx, __shfl_xor(mx, 32)) * scale_log2;
      if (__any(mx > m_run[qbk] + 8.0f)) {
        const float m_new = fmaxf(m_run[qbk], mx);
        const float alpha = __builtin_amdgcn_exp2f(m_run[qbk] - m_new);
        m_run[qbk] = m_new;
        l_run[qbk] *= alpha;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[qbk][db][r] *= alpha;
      }
      const float mneg = -m_run[qbk];
      float ls = 0.0f;
#pragma unroll
      for (int kb2 = 0; kb2 < 2; ++kb2) {
        float pv[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          pv[r] = __builtin_amdgcn_exp2f(fmaf(sacc[qbk][kb2][r], scale_log2, mneg));
          ls += pv[r];
        }
#pragma unroll
        for (int st = 0; st < 2; ++st)
#pragma unroll
          for (int e = 0; e < 4; ++e) pop[qbk][kb2][st][e] = cvt_pk_bf16(pv[8 * st + 2 * e], pv[8 * st + 2 * e + 1]);
      }
      l_run[qbk] += ls;
    }

    // O^T += V^T P^T.  P^T operand element e of lane (query, h) is tile key 16st + 8(e/4) + 4h + e%4
    // (the S^T accumulator layout); the V operand reads those keys' rows transposed: group grp
    // gathers rows key0 + gl/4 (key0 = 32kb2 + 16st + 4(grp/2), +8 for elements 4..7), columns
    // 32db + 16(grp%2) + 4(gl%4).
#pragma unroll
    for (int kb2 = 0; kb2 < 2; ++kb2) {
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        const int key0 = kb2 * 32 + st * 16 + 4 * (grp / 2) + gl / 4;
#pragma unroll
        for (int db = 0; db < 4; ++db) {
          const int col = db * 32 + 16 * (grp % 2) + 4 * (gl % 4);
          const uint2 lo = ds_read_tr16_b64(&v_s[key0 * kVStride + col]);
          const uint2 hi = ds_read_tr16_b64(&v_s[(key0 + 8) * kVStride + col]);
          const bf16x8_t a = as_bf16x8(u32x4_t{lo.x, lo.y, hi.x, hi.y});
#pragma unroll
          for (int qbk = 0; qbk < QB; ++qbk) acc[qbk][db] = mfma32x32x16(a, as_bf16x8(pop[qbk][kb2][st]), acc[qbk][db]);
        }
      }
    }
  }

  // Normalise and store: lane holds d = db*32 + (r/4)*8 + 4h + r%4 of query l32.
#pragma unroll
  for (int qbk = 0; qbk < QB; ++qbk) {
    const float lt = l_run[qbk] + __shfl_xor(l_run[qbk], 32);
    const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
    const int row = q0 + wave * 32 * QB + qbk * 32 + l32;
    if (row < q1) {
      uint16_t* dst = ob + (size_t)row * 128;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d0 = db * 32 + g * 8 + h * 4;
          uint2 w;
          w.x = cvt_pk_bf16(acc[qbk][db][4 * g] * inv, acc[qbk][db][4 * g + 1] * inv);
          w.y = cvt_pk_bf16(acc[qbk][db][4 * g + 2] * inv, acc[qbk][db][4 * g + 3] * inv);
          *(uint2*)(dst + d0) = w;
        }
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
  size_t qoff, koff, items, nitems, total;
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
  w.total = w.nitems + al((size_t)bh * 4);
  return w;
}
}  // namespace

extern "C" size_t svoo_vbsa_workspace_size(int bh, int s, int qn, int kn) {
  if (bh <= 0 || s <= 0 || qn <= 0 || kn <= 0) return 256;
  return vbsa_layout(bh, s, qn, kn).total;
}

extern "C" int svoo_vbsa_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint8_t* map,
                             const int32_t* q_sizes, const int32_t* k_sizes, uint16_t* o, int bh, int s, int d, int qn,
                             int kn, void* workspace, size_t ws_bytes, int32_t* status, void* stream) {
  SVOO_REQUIRE(q && k && v && map && q_sizes && k_sizes && o, SVOO_ERR_INVALID_ARG, "svoo_vbsa_fwd: null pointer");
  SVOO_REQUIRE(d == 128, SVOO_ERR_UNSUPPORTED, "svoo_vbsa_fwd: D=%d (only 128 supported)", d);
  SVOO_REQUIRE(bh > 0 && s > 0 && qn > 0 && kn > 0, SVOO_ERR_INVALID_ARG, "svoo_vbsa_fwd: bad dims");
  SVOO_REQUIRE(kn <= kMaxKN && qn < 32768, SVOO_ERR_UNSUPPORTED, "svoo_vbsa_fwd: qn=%d kn=%d above limits", qn, kn);
  SVOO_REQUIRE((long long)bh * s * 128 < (1ll << 40), SVOO_ERR_UNSUPPORTED, "svoo_vbsa_fwd: too large");
  const VbsaWs lay = vbsa_layout(bh, s, qn, kn);
  SVOO_REQUIRE(lay.cap < 65536, SVOO_ERR_UNSUPPORTED, "svoo_vbsa_fwd: too many q tiles per head");
  SVOO_REQUIRE(workspace && ws_bytes >= lay.total, SVOO_ERR_WORKSPACE, "svoo_vbsa_fwd: workspace %zu < %zu", ws_bytes,
               lay.total);
  hipStream_t st = (hipStream_t)stream;
  char* base = (char*)workspace;
  int32_t* qoff = (int32_t*)(base + lay.qoff);
  int32_t* koff = (int32_t*)(base + lay.koff);
  int32_t* items = (int32_t*)(base + lay.items);
  int32_t* nitems = (int32_t*)(base + lay.nitems);
  constexpr int qtile = VbsaCfg<kDefaultQB>::kQTile;
  hipLaunchKernelGGL(vbsa_plan_kernel, dim3(bh), dim3(kPlanThreads), 0, st, q_sizes, k_sizes, s, qn, kn, qtile, lay.cap,
                     qoff, koff, items, nitems, status);
  if (int rc = check_launch("svoo_vbsa_fwd(plan)")) return rc;
  const long long total_items = (long long)bh * lay.cap;
  const long long nblocks = (total_items + 8 * kXcdRun - 1) / (8 * kXcdRun) * (8 * kXcdRun);
  SVOO_REQUIRE(nblocks < (1ll << 31), SVOO_ERR_UNSUPPORTED, "svoo_vbsa_fwd: too many work items");
  const float scale_log2 = (float)(1.4426950408889634 / sqrt((double)d));
  const size_t smem = (size_t)(2 * kn + 1) * sizeof(int32_t);
  hipLaunchKernelGGL(vbsa_attn_kernel<kDefaultQB>, dim3((unsigned)nblocks), dim3(kVWaves * kWave), smem, st, q, k, v,
                     map, k_sizes, o, s, qn, kn, lay.cap, total_items, qoff, koff, items, nitems, scale_log2);
  return check_launch("svoo_vbsa_fwd");
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
