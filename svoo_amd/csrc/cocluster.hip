// Profile-space co-clustering (QK k-means) on device.
//
// The reference assigns token x to argmin_j 2 - 2 (x C^T / ||x C^T||) . P_j with P the row-normalised
// centroid profiles.  ||x C^T|| is a positive per-token constant, so the label is
// argmax_j x . E_j with E = P C ([J x D]).  That turns the assignment into one [N x D] x [D x J]
// GEMM with an argmax epilogue, instead of recomputing x C^T for every tile of J.
//
// prep:   P = l2norm(bf16(A B^T)) with exact (fp64) dots, E = P B, written as two bf16 matrices
//         E_hi + E_lo (the bf16 MFMA then sees E to ~16 significant bits) and as a scaled fp16 copy E16
//         with the per-head error maxima of that copy.
// assign16: one fp16 MFMA pass over E16 with a rigorous score-error bound; a token whose best score
//         beats the second by more than twice the bound has the exact argmax label, the others go to a
//         per-head list.
// assign: 4 waves x 128 tokens per block (all tokens, or the listed ones); token rows stay in registers
//         as the MFMA B operand, E_hi and E_lo stream through LDS in 64-row chunks (double buffered,
//         LDS DMA), and each lane keeps a running argmax over the 16 cluster rows it holds of every 32x32
//         tile.
// From the second iteration on the passes list the tokens whose label changed, and the centroid sums
// are updated from that list alone (fp64; equal to a full recount while the sums are exact, see
// centroid.hip), or recounted when many labels changed.
// candidate pass (key side, second iteration on, at least 1000 key clusters): the triangle inequality in
// profile space around each token's current label bounds which clusters can beat it; only those are scored
// (radius, lists and score kernels below), the same labels as a full pass.
#include <stdlib.h>

#include "svoo_common.h"

namespace svoo {

constexpr int kPrepMaxLds = 52 * 1024;  // LDS budget of the prep kernel's profile rows
constexpr int kAssignChunk = 64;   // E rows staged in LDS per step
// Shared counters (per-head fallback counts, the two change counters) sit 256 bytes apart, each on a cache
// line of its own, and every wave reserves all the slots it needs with one atomic: thousands of waves adding
// one by one to counters on one line serialise in the L2.
constexpr int kCounterStride = 64;  // int32 elements

// One atomicAdd per wave on `counter` for `count` slots (wave-uniform); the base slot in every lane.
__device__ __forceinline__ int wave_reserve(int32_t* counter, int count) {
  int base = 0;
  if (count > 0 && (threadIdx.x % kWave) == 0) base = atomicAdd(counter, count);
  return __shfl(base, 0);
}
// Rank of this lane among the set lanes of a wave mask below it.
__device__ __forceinline__ int mask_rank(uint64_t m) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0));
}

// --------------------------------------------------------------------------------------- prep
// kPrepRows rows of A per block: 8 when there are many rows (the key side) and the profile width
// is at most 1664 (LDS), else 2 (more blocks for the few, long query-side rows).
template <int kPrepRows>
__global__ void __launch_bounds__(256) cocluster_prep_kernel(const uint16_t* __restrict__ a,
                                                             const uint16_t* __restrict__ bmat,
                                                             uint16_t* __restrict__ e_hi, uint16_t* __restrict__ e_lo,
                                                             float* __restrict__ profile, int j, int kp, int jpad) {
  extern __shared__ unsigned char smem[];
  double* arow = (double*)smem;                                 // [kPrepRows][128]
  double* inv = arow + kPrepRows * 128;                         // [kPrepRows]
  float* praw = (float*)(inv + kPrepRows);                      // [kPrepRows][kp]
  const int bidx = blockIdx.y;
  const int r0 = blockIdx.x * kPrepRows;
  const int tid = threadIdx.x;
  const uint16_t* ab = a + (size_t)bidx * j * 128;
  const uint16_t* bb = bmat + (size_t)bidx * kp * 128;
  // Rows r0 .. r0 + nrows - 1 are computed; padding rows (j <= row < jpad) repeat row j - 1, so
  // that a padding row can only tie with row j - 1 in the assignment's argmax.
  const int nrows = max(0, min(kPrepRows, jpad - r0));
  const int nreal = max(0, min(kPrepRows, j - r0));

  for (int t = tid; t < kPrepRows * 128; t += 256) {
    const int r = t / 128, dd = t % 128;
    arow[t] = (r < nrows) ? (double)bf16_to_f32(ab[(size_t)min(r0 + r, j - 1) * 128 + dd]) : 0.0;
  }
  __syncthreads();

  // Phase 1: exact dots A_r . B_k, rounded like a bf16 matmul output (fp32 then bf16).
  if (nrows > 0) {
    for (int k = tid; k < kp; k += 256) {
      double acc[kPrepRows];
#pragma unroll
      for (int r = 0; r < kPrepRows; ++r) acc[r] = 0.0;
      const u32x4_t* brow = (const u32x4_t*)(bb + (size_t)k * 128);
#pragma unroll 2
      for (int c = 0; c < 16; ++c) {
        const u32x4_t w = brow[c];
        double bv[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          bv[2 * e] = (double)bf16_to_f32((uint16_t)(w[e] & 0xffffu));
          bv[2 * e + 1] = (double)bf16_to_f32((uint16_t)(w[e] >> 16));
        }
#pragma unroll
        for (int r = 0; r < kPrepRows; ++r) {
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[r] = fma(arow[r * 128 + c * 8 + e], bv[e], acc[r]);
        }
      }
#pragma unroll
      for (int r = 0; r < kPrepRows; ++r) praw[r * kp + k] = bf16_round_f32((float)acc[r]);
    }
  }
  __syncthreads();

  // Phase 2: row norms (one wave per row), inv = 1 / sqrt(sum + 1e-8).
  const int wave = tid / kWave, lane = tid % kWave;
  for (int r = wave; r < kPrepRows; r += 4) {
    double s = 0.0;
    for (int k = lane; k < kp; k += kWave) {
      const double v = praw[r * kp + k];
      s += v * v;
    }
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
    if (lane == 0) inv[r] = 1.0 / sqrt(s + 1e-8);
  }
  __syncthreads();

  if (profile) {
    float* pb = profile + (size_t)bidx * j * kp;
    for (int t = tid; t < nreal * kp; t += 256) {
      const int r = t / kp, k = t % kp;
      pb[(size_t)(r0 + r) * kp + k] = (float)((double)praw[r * kp + k] * inv[r]);
    }
  }

  // Phase 3: E[r][dd] = inv_r * sum_k praw[r][k] * B[k][dd] (fp64), split into bf16 hi + lo.
  const int dd = tid % 128, g = tid / 128;
  double acc[kPrepRows / 2];
#pragma unroll
  for (int q = 0; q < kPrepRows / 2; ++q) acc[q] = 0.0;
  if (nrows > 0) {
#pragma unroll 4
    for (int k = 0; k < kp; ++k) {
      const double bv = (double)bf16_to_f32(bb[(size_t)k * 128 + dd]);
#pragma unroll
      for (int q = 0; q < kPrepRows / 2; ++q) acc[q] = fma((double)praw[(2 * q + g) * kp + k], bv, acc[q]);
    }
  }
  uint16_t* hb = e_hi + (size_t)bidx * jpad * 128;
  uint16_t* lb = e_lo + (size_t)bidx * jpad * 128;
#pragma unroll
  for (int q = 0; q < kPrepRows / 2; ++q) {
    const int r = 2 * q + g;
    if (r0 + r >= jpad) continue;
    uint16_t hi = 0, lo = 0;
    if (r < nrows) {
      const double e = acc[q] * inv[r];
      hi = f32_to_bf16((float)e);
      lo = f32_to_bf16((float)(e - (double)bf16_to_f32(hi)));
    }
    hb[(size_t)(r0 + r) * 128 + dd] = hi;
    lb[(size_t)(r0 + r) * 128 + dd] = lo;
  }
}

// --------------------------------------------------------------------------------------- prep (MFMA)
// The same three phases for 16 rows of A per block, for profile widths up to kPmMaxKp.
//   phase 1: praw = bf16(A B^T) on v_mfma_f64_16x16x4_f64 tile by tile (16 columns per MFMA tile, the
//            waves take every 4th tile): products of bf16 values are exact in fp64 and so is the sum of
//            128 of them, so praw is the correctly rounded bf16 of the exact dot, as in the vector kernel;
//            the contraction is permuted so that lane quarter q covers d in [32q, 32q+32) and every lane
//            loads 64 contiguous bytes of its A and B rows;
//   phase 2: row norms of praw (kept in LDS as bf16, which it is exactly), fp64;
//   phase 3: E = inv * (praw B) on v_mfma_f32_32x32x16_bf16 (exact products, fp32 sums over the profile
//            width; fp64 on the 16x16x4 MFMA cost as much as phase 1 again), with B staged through LDS in
//            64-row chunks of 144-element rows, each requested from memory two chunks ahead.
constexpr int kPmRows = 16;
constexpr int kPmChunk = 64;
constexpr int kPmChunkStride = 144;
constexpr int kPmMaxKp = 1408;

static inline __host__ __device__ int pm_kpp(int kp) { return (kp + kPmChunk - 1) / kPmChunk * kPmChunk; }
static inline __host__ __device__ size_t pm_praw_bytes(int kp) {
  return (size_t)kPmRows * (pm_kpp(kp) + 8) * sizeof(uint16_t);
}
static inline size_t pm_smem(int kp) {
  return pm_praw_bytes(kp) + kPmRows * sizeof(double) + (size_t)kPmChunk * kPmChunkStride * sizeof(uint16_t);
}

// Element offset of E16[row][col] within a head: 32-row tiles of 8 KB, each [k-step 0..7][lane 0..63][8],
// where lane 32 hh + r holds columns 16 ks + 8 hh .. + 7 of tile row r.  The A operand of one k-step of
// v_mfma_f32_32x32x16_f16 is then 1 KB of consecutive bytes, lane i at 16 i.
__host__ __device__ __forceinline__ size_t e16_offset(int row, int col) {
  return (size_t)(row >> 5) * 4096 + (col >> 4) * 512 + (((col >> 3) & 1) * 32 + (row & 31)) * 8 + (col & 7);
}

__device__ __forceinline__ double bf16_half_f64(uint32_t w, int hi) {
  return (double)bf16_to_f32((uint16_t)(hi ? (w >> 16) : (w & 0xffffu)));
}

__global__ void __launch_bounds__(256) cocluster_prep_mfma_kernel(const uint16_t* __restrict__ a,
                                                                  const uint16_t* __restrict__ bmat,
                                                                  uint16_t* __restrict__ e_hi,
                                                                  uint16_t* __restrict__ e_lo,
                                                                  float* __restrict__ profile, int j, int kp,
                                                                  int jpad, uint16_t* __restrict__ e16,
                                                                  uint32_t* __restrict__ err_max,
                                                                  uint32_t* __restrict__ norm_max,
                                                                  double* __restrict__ e_old,
                                                                  float* __restrict__ delta,
                                                                  uint32_t* __restrict__ delta_max,
                                                                  int32_t* __restrict__ t_out, int have_old,
                                                                  uint16_t* __restrict__ praw_out,
                                                                  double* __restrict__ inv_out,
                                                                  float* __restrict__ nrm_out) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int kpp = pm_kpp(kp), ps = kpp + 8;
  uint16_t* praw = (uint16_t*)smem;                             // [16][ps] bf16
  double* inv = (double*)(smem + pm_praw_bytes(kp));           // [16]
  uint16_t* bch = (uint16_t*)(inv + kPmRows);                   // [64][144] bf16
  const int bidx = blockIdx.y, r0 = blockIdx.x * kPmRows;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave, li = lane % 16, q = lane / 16;
  const uint16_t* ab = a + (size_t)bidx * j * 128;
  const uint16_t* bb = bmat + (size_t)bidx * kp * 128;

  // Phase 3's B chunks of 64 rows: this thread's four 16-byte pieces (rows tid / 16 + 16 i, piece tid % 16).
  // The first two are requested here, before phase 1, and each later one two chunks ahead of its use.
  auto chunk_load = [&](u32x4_t(&r)[4], int c) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      r[i] = *((const u32x4_t*)(bb + (size_t)min(c + tid / 16 + 16 * i, kp - 1) * 128) + tid % 16);
  };
  u32x4_t pre0[4], pre1[4];
  chunk_load(pre0, 0);
  if (kPmChunk < kpp) chunk_load(pre1, kPmChunk);

  // Phase 1.  Rows past j repeat row j - 1 (padding rows of E), columns past kp are zero.  The B rows of the
  // wave's next column tile are requested before the MFMAs of the current one.
  u32x4_t afr[4];
  {
    const u32x4_t* src = (const u32x4_t*)(ab + (size_t)min(r0 + li, j - 1) * 128) + 4 * q;
#pragma unroll
    for (int t = 0; t < 4; ++t) afr[t] = src[t];
  }
  auto tile_load = [&](u32x4_t(&r)[4], int ct) {
    const u32x4_t* bsrc = (const u32x4_t*)(bb + (size_t)min(ct * 16 + li, kp - 1) * 128) + 4 * q;
#pragma unroll
    for (int t = 0; t < 4; ++t) r[t] = bsrc[t];
  };
  const int ntile = kpp / 16;
  u32x4_t bfr[4];
  if (wave < ntile) tile_load(bfr, wave);
  for (int ct = wave; ct < ntile; ct += 4) {
    const int col = ct * 16 + li;
    u32x4_t bnx[4];
    if (ct + 4 < ntile) tile_load(bnx, ct + 4);
    f64x4_t acc = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int st = 0; st < 32; ++st) {
      const int t = st / 8, w = (st % 8) / 2, hf = st % 2;
      acc = mfma16x16x4_f64(bf16_half_f64(afr[t][w], hf), bf16_half_f64(bfr[t][w], hf), acc);
    }
#pragma unroll
    for (int v = 0; v < 4; ++v)  // D row 4 v + q, column li
      praw[(4 * v + q) * ps + col] = col < kp ? f32_to_bf16((float)acc[v]) : (uint16_t)0;
    if (ct + 4 < ntile) {
#pragma unroll
      for (int t = 0; t < 4; ++t) bfr[t] = bnx[t];
    }
  }
  __syncthreads();

  // Phase 2: inv = 1 / sqrt(sum + 1e-8), 16 threads per row.
  {
    const int r = tid / 16, sub = tid % 16;
    double sq = 0.0;
    for (int k = sub; k < kp; k += 16) {
      const double v = (double)bf16_to_f32(praw[r * ps + k]);
      sq += v * v;
    }
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) sq += __shfl_xor(sq, o);
    if (sub == 0) {
      inv[r] = 1.0 / sqrt(sq + 1e-8);
      // profile rows for the key side's candidate pass (kp <= 128): 1 / |praw| and |P|^2 = sq / (sq + 1e-8)
      if (inv_out && r0 + r < jpad) {
        inv_out[(size_t)bidx * jpad + r0 + r] = inv[r];
        nrm_out[(size_t)bidx * jpad + r0 + r] = (float)(sq / (sq + 1e-8));
      }
    }
  }
  __syncthreads();
  if (praw_out) {
    // praw (exactly bf16) as [jpad][128] rows, zero past kp
    for (int t = tid; t < kPmRows * 16; t += 256) {
      const int r = t / 16, c = t % 16;
      if (r0 + r < jpad)
        *((u32x4_t*)(praw_out + ((size_t)bidx * jpad + r0 + r) * 128) + c) =
            c * 8 < kpp ? *(const u32x4_t*)(praw + r * ps + c * 8) : u32x4_t{0u, 0u, 0u, 0u};
    }
  }
  if (profile) {
    const int nreal = max(0, min(kPmRows, j - r0));
    float* pb = profile + (size_t)bidx * j * kp;
    for (int t = tid; t < nreal * kp; t += 256) {
      const int r = t / kp, k = t % kp;
      pb[(size_t)(r0 + r) * kp + k] = (float)((double)bf16_to_f32(praw[r * ps + k]) * inv[r]);
    }
  }

  // Phase 3 on v_mfma_f32_32x32x16_bf16: the E^T tile [32 columns dd][32 n] += B^T[dd][k] praw^T[k][n], with
  // the 16 rows of praw as n (n and n + 16 the same row).  Wave w takes columns [32 w, 32 w + 32).  The B^T
  // operand comes from the staged B chunk through the transposing LDS read (group g of 16 lanes reads columns
  // 16 (g % 2) .., chunk rows 8 (g / 2) .. + 8 in two halves of four), the praw operand is 16 contiguous bytes
  // of a row.  Products of bf16 values are exact in fp32; the sums over k are fp32.
  f32x16_t acc3 = {};
  const int dd0 = 32 * wave, grp = lane / 16, s16 = lane % 16;
  const int toff = (8 * (grp / 2) + s16 / 4) * kPmChunkStride + dd0 + 16 * (grp % 2) + 4 * (s16 % 4);
  const int poff = (lane % 16) * ps + 8 * (lane / 32);
  uint32_t bmax = 0;  // max |B| as bf16 magnitude bits (they order like the values)
  // Stage the chunk held in r (rows c ..), request chunk c + 2 * kPmChunk into r, then the chunk's MFMAs.
  auto chunk_step = [&](u32x4_t(&r)[4], int c) {
    __syncthreads();  // the previous chunk is consumed
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      *(u32x4_t*)(bch + (tid / 16 + 16 * i) * kPmChunkStride + (tid % 16) * 8) = r[i];
#pragma unroll
      for (int e = 0; e < 4; ++e) bmax = max(bmax, max(r[i][e] & 0x7fffu, (r[i][e] >> 16) & 0x7fffu));
    }
    if (c + 2 * kPmChunk < kpp) chunk_load(r, c + 2 * kPmChunk);
    __syncthreads();
#pragma unroll
    for (int st = 0; st < kPmChunk / 16; ++st) {
      const uint16_t* tb = bch + st * 16 * kPmChunkStride + toff;
      const uint2 lo = ds_read_tr16_b64(tb);
      const uint2 hi = ds_read_tr16_b64(tb + 4 * kPmChunkStride);
      const u32x4_t bt = {lo.x, lo.y, hi.x, hi.y};
      const u32x4_t pr = *(const u32x4_t*)(praw + poff + c + 16 * st);
      acc3 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(bt), as_bf16x8(pr), acc3, 0, 0, 0);
    }
  };
  for (int c = 0; c < kpp; c += 2 * kPmChunk) {
    chunk_step(pre0, c);
    if (c + kPmChunk < kpp) chunk_step(pre1, c + kPmChunk);
  }
  uint16_t* hb = e_hi + (size_t)bidx * jpad * 128;
  uint16_t* lb = e_lo + (size_t)bidx * jpad * 128;
  // fp16 copy for the certified single-pass assignment: E * 2^t with one power of two per head, chosen
  // from an a-priori bound so that no element overflows (|E_ji| <= |P_j| |B_.i| <= sqrt(kp) max|B|, and
  // |P_j| <= 1): every block of the head derives the same t from max|B|.
  int t_scale = 0;
  if (e16) {
    __syncthreads();  // every thread is done with bch
    uint32_t* red = (uint32_t*)bch;
    for (int o = 32; o > 0; o >>= 1) bmax = max(bmax, (uint32_t)__shfl_xor((int)bmax, o));
    if (lane == 0) red[wave] = bmax;
    __syncthreads();
    bmax = max(max(red[0], red[1]), max(red[2], red[3]));
    __syncthreads();
    if (bmax) {
      int ex;
      frexp(sqrt((double)kp) * (double)bf16_to_f32((uint16_t)bmax), &ex);  // bound < 2^ex
      t_scale = 15 - ex;
    }
    if (t_out && tid == 0) t_out[bidx] = t_scale;  // the same value from every block of the head
  }
  // Lane l with l % 32 < 16 holds row r = l % 16 at columns dd0 + 8 (v / 4) + 4 (l / 32) + v % 4 (v = 0..15).
  float err2 = 0.0f, nrm2 = 0.0f, dl2 = 0.0f;
  const int rr = lane % 16, row = r0 + rr;
  // Slots 4q .. 4q + 3 are four consecutive columns: each array gets one 8-byte store per group (the fp64 copy
  // two 16-byte accesses) instead of four 2-byte (8-byte) ones.
  if ((lane % 32) < 16 && row < jpad) {
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int dd = dd0 + 8 * q4 + 4 * (lane / 32);
      uint16_t hi[4], lo[4], h16b[4];
      double ev[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const double e = (double)acc3[4 * q4 + i] * inv[rr];
        ev[i] = e;
        hi[i] = f32_to_bf16((float)e);
        lo[i] = f32_to_bf16((float)(e - (double)bf16_to_f32(hi[i])));
      }
      *(uint2*)(hb + (size_t)row * 128 + dd) =
          make_uint2(hi[0] | ((uint32_t)hi[1] << 16), hi[2] | ((uint32_t)hi[3] << 16));
      *(uint2*)(lb + (size_t)row * 128 + dd) =
          make_uint2(lo[0] | ((uint32_t)lo[1] << 16), lo[2] | ((uint32_t)lo[3] << 16));
      if (e16) {
        double old[4];
        double* eo = e_old ? e_old + ((size_t)bidx * jpad + row) * 128 + dd : nullptr;
        if (eo && have_old) {
          const double2 o01 = *(const double2*)eo, o23 = *(const double2*)(eo + 2);
          old[0] = o01.x, old[1] = o01.y, old[2] = o23.x, old[3] = o23.y;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          // padding rows (row >= j) are zero in the fp16 copy: their score is exactly 0
          const double es = row < j ? ldexp(ev[i], t_scale) : 0.0;
          const _Float16 h16 = (_Float16)(float)es;
          const double err = es - (double)(float)h16;  // exact
          err2 += (float)(err * err);
          nrm2 += (float)((double)(float)h16 * (double)(float)h16);
          h16b[i] = __builtin_bit_cast(uint16_t, h16);
          if (eo && have_old) {
            // change of E since the previous call on this buffer (for the pruning bounds)
            const double df = ev[i] - old[i];
            dl2 += (float)(df * df);
          }
        }
        *(uint2*)(e16 + (size_t)bidx * jpad * 128 + e16_offset(row, dd)) =
            make_uint2(h16b[0] | ((uint32_t)h16b[1] << 16), h16b[2] | ((uint32_t)h16b[3] << 16));
        if (eo) {  // keep this E
          *(double2*)eo = make_double2(ev[0], ev[1]);
          *(double2*)(eo + 2) = make_double2(ev[2], ev[3]);
        }
      }
    }
  }
  if (e16) {
    // Per-row |2^t E_j - E16_j| and |E16_j| (rows of real clusters only), then the head's maxima.  A row's 128
    // columns are spread over lanes r and r + 32 of each of the 4 waves.
    err2 += __shfl_xor(err2, 32);
    nrm2 += __shfl_xor(nrm2, 32);
    dl2 += __shfl_xor(dl2, 32);
    float* part = (float*)bch;  // [wave][row][3]
    __syncthreads();            // every wave is done with bch
    if (lane < 16) {
      part[(wave * 16 + lane) * 3] = err2;
      part[(wave * 16 + lane) * 3 + 1] = nrm2;
      part[(wave * 16 + lane) * 3 + 2] = dl2;
    }
    __syncthreads();
    if (tid < 16) {
      const int i = tid;
      float er = 0.0f, nr = 0.0f, dl = 0.0f;
      if (r0 + i < j)
        for (int w = 0; w < 4; ++w) {
          er += part[(w * 16 + i) * 3];
          nr += part[(w * 16 + i) * 3 + 1];
          dl += part[(w * 16 + i) * 3 + 2];
        }
      // rounded-to-nearest fp32 sums of at most 128 squares: 2^-17 relative slack covers their rounding
      er = sqrtf(er * (1.0f + 0x1p-16f)) * (1.0f + 0x1p-20f);
      nr = sqrtf(nr * (1.0f + 0x1p-16f)) * (1.0f + 0x1p-20f);
      dl = sqrtf(dl * (1.0f + 0x1p-16f)) * (1.0f + 0x1p-20f);
      if (e_old && have_old && r0 + i < jpad) delta[(size_t)bidx * jpad + r0 + i] = dl;
#pragma unroll
      for (int o = 8; o > 0; o >>= 1) {
        er = fmaxf(er, __shfl_xor(er, o));
        nr = fmaxf(nr, __shfl_xor(nr, o));
        dl = fmaxf(dl, __shfl_xor(dl, o));
      }
      if (tid == 0) {
        atomicMax(err_max + bidx, __float_as_uint(er));
        atomicMax(norm_max + bidx, __float_as_uint(nr));
        if (e_old && have_old) atomicMax(delta_max + bidx, __float_as_uint(dl));
      }
    }
  }
}

// --------------------------------------------------------------------------------------- assign
// Block = 4 waves x 32 NCB tokens (NCB MFMA column blocks of 32 per wave); the token rows stay in
// registers as the MFMA B operand for the whole pass.  E_hi and E_lo stream through LDS in chunks
// of 64 rows, double buffered and filled by LDS DMA (unpadded rows, XOR-swizzled 16-byte chunks),
// one barrier per chunk.  Each lane keeps a running argmax over the 16 cluster rows it holds of
// each 32x32 accumulator tile: one max over the scores with their slot in the low 4 mantissa bits,
// then a tile-level compare (ties resolve to the lowest cluster index; scores within 2^-19 of each
// other, below the rounding of the hi + lo sums, are ordered by slot, and for negative scores the
// higher slot of a tile wins such a near-tie).
constexpr int kAsgTokWave = 128;
constexpr int kAsgTok = 4 * kAsgTokWave;

// With LIST the block's tokens are entries [T x, T x + T) of the head's token list (T = 128 NCB; list[bidx][.],
// count[bidx] entries; blocks past the count exit at once): the tokens the certified fp16 pass or the
// candidate pass could not settle.  Every block streams all of E, so a short list runs fastest on one column
// block per wave (more blocks, each a quarter of the MFMA work): the candidate passes leave about 0.6% of the
// keys at C3 from a warm start, one 512-token block per head with four column blocks (80-87 us per pass
// against 38-41 us with one).  The certified pass's longer lists keep four.
template <bool LIST, int NCB>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
cocluster_assign_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ e_hi,
                        const uint16_t* __restrict__ e_lo, int32_t* __restrict__ labels, int n, int j, int jpad,
                        int2* __restrict__ changes, int32_t* __restrict__ nchanges,
                        const int32_t* __restrict__ list, const int32_t* __restrict__ list_count) {
  __shared__ __attribute__((aligned(16))) uint16_t s_e[2][2][kAssignChunk * 128];  // [buffer][hi, lo]
  const int bidx = blockIdx.y;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int h = lane / 32, l32 = lane % 32;
  constexpr int kTokWave = 32 * NCB, kTokBlock = 4 * kTokWave;
  const int tok0 = blockIdx.x * kTokBlock + wave * kTokWave;
  const int ntok = LIST ? list_count[(size_t)bidx * kCounterStride] : n;  // positions < ntok hold tokens
  if (LIST && (int)blockIdx.x * kTokBlock >= ntok) return;
  const int32_t* lst = LIST ? list + (size_t)bidx * n : nullptr;
  // token at position p of this block's range (positions past the range load a valid row, unused)
  auto token_at = [&](int pos) __attribute__((always_inline)) -> int {
    if constexpr (LIST)
      return lst[min(pos, ntok - 1)];
    else
      return min(pos, n - 1);
  };
  const uint16_t* xb = x + (size_t)bidx * n * 128;
  const uint16_t* hb = e_hi + (size_t)bidx * jpad * 128;
  const uint16_t* lb = e_lo + (size_t)bidx * jpad * 128;
  const int nchunks = jpad / kAssignChunk;

  // DMA of chunk c into buffer bf: wave w moves rows 16 w .. 16 w + 15 of both matrices, 4 rows
  // (1 KB) per instruction; lane i fills LDS chunk i%16 of row 4 g + i/16 from its logical chunk.
  const int prow = lane / 16, pch = lane % 16;
  auto issue = [&](int c, int bf) __attribute__((always_inline)) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int r = 16 * wave + 4 * g + prow;
      const size_t src = (size_t)(c * kAssignChunk + r) * 128 + swz(r, pch) * 8;
      lds_dma16(hb + src, &s_e[bf][0][(16 * wave + 4 * g) * 128]);
      lds_dma16(lb + src, &s_e[bf][1][(16 * wave + 4 * g) * 128]);
    }
  };
  issue(0, 0);

  // Token operands: B[k = d][n = token], lane provides 8 consecutive d of token l32 per k-step.
  u32x4_t xop[NCB][8];
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    const int row = token_at(tok0 + cb * 32 + l32);
    const u32x4_t* src = (const u32x4_t*)(xb + (size_t)row * 128);
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) xop[cb][ks] = src[ks * 2 + h];
  }
  // LDS element offset of A-operand k-step ks in row l32: swz(l32, 2 ks + h) * 8, written as
  // 16 (ks ^ g) + 8 e so that it costs one xor per use instead of eight live registers.
  const int sw = swz(l32, 0), g = sw >> 1;
  const int abase = l32 * 128 + 8 * (h ^ (sw & 1));
#define AOFF(ks) (abase + 16 * ((ks) ^ g))

  float best_v[NCB], best_s[NCB];  // tagged, without the tag
  int best_j[NCB];                 // tile base row
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    best_v[cb] = -INFINITY;
    best_s[cb] = -INFINITY;
    best_j[cb] = 0;
  }

  for (int c = 0; c < nchunks; ++c) {
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (c + 1 < nchunks) issue(c + 1, (c + 1) & 1);
    const uint16_t* sh = s_e[c & 1][0];
    const uint16_t* sl = s_e[c & 1][1];
    // A operands one k-step ahead of the MFMAs that use them
    u32x4_t ah = *(const u32x4_t*)(sh + AOFF(0));
    u32x4_t al = *(const u32x4_t*)(sl + AOFF(0));
#pragma unroll
    for (int rb = 0; rb < kAssignChunk / 32; ++rb) {
      f32x16_t acc[NCB] = {};
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        const u32x4_t ch = ah, cl = al;
        if (ks < 7 || rb + 1 < kAssignChunk / 32) {
          const int nrb = ks < 7 ? rb : rb + 1, nks = (ks + 1) % 8;
          ah = *(const u32x4_t*)(sh + nrb * 32 * 128 + AOFF(nks));
          al = *(const u32x4_t*)(sl + nrb * 32 * 128 + AOFF(nks));
        }
        // keep the next k-step's LDS reads ahead of this step's eight MFMAs
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb) acc[cb] = mfma32x32x16(as_bf16x8(ch), as_bf16x8(xop[cb][ks]), acc[cb]);
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb) acc[cb] = mfma32x32x16(as_bf16x8(cl), as_bf16x8(xop[cb][ks]), acc[cb]);
      }
      // Argmax over the lane's 16 values of each tile: the low 4 mantissa bits of each score are
      // replaced by 15 - r (a change of at most 2^-19 of the score, below the rounding of the hi + lo
      // sums), so one max over the tagged values gives the tile's best score and, on equal scores, the
      // lowest slot; across tiles the scores are compared without the tags (ties keep the earlier tile).
      // Row of slot r is jb + (r/4)*8 + r%4 + 4h, decoded at the end.
      const int jb = c * kAssignChunk + rb * 32;
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) {
        float t[16];
#pragma unroll
        for (int r = 0; r < 16; ++r)
        {
          const float av = acc[cb][r];
          t[r] = __uint_as_float((__float_as_uint(av) & ~15u) | (uint32_t)(15 - r));
        }
        auto max3 = [](float a, float b, float c) { return fmaxf(fmaxf(a, b), c); };
        const float m = fmaxf(max3(max3(t[0], t[1], t[2]), max3(t[3], t[4], t[5]), max3(t[6], t[7], t[8])),
                              max3(max3(t[9], t[10], t[11]), max3(t[12], t[13], t[14]), t[15]));
        const float ms = __uint_as_float(__float_as_uint(m) & ~15u);
        const bool up = ms > best_s[cb];
        best_s[cb] = up ? ms : best_s[cb];
        best_v[cb] = up ? m : best_v[cb];
        best_j[cb] = up ? jb : best_j[cb];
      }
    }
  }
#undef AOFF
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    const int r = 15 - (int)(__float_as_uint(best_v[cb]) & 15u);
    best_j[cb] += (r / 4) * 8 + (r % 4) + h * 4;
  }
  int lab[NCB], oldl[NCB], tokv[NCB];
  uint64_t chm[NCB];
  int nch_wave = 0;
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    // the two halves of a token: larger score, then lower row
    const float ov = __shfl_xor(best_s[cb], 32);
    const int oj = __shfl_xor(best_j[cb], 32);
    if (ov > best_s[cb] || (ov == best_s[cb] && oj < best_j[cb])) {
      best_s[cb] = ov;
      best_j[cb] = oj;
    }
    const int pos = tok0 + cb * 32 + l32;
    const bool mine = h == 0 && pos < ntok;
    tokv[cb] = mine ? token_at(pos) : -1;
    // padding rows repeat row j - 1: a padding winner stands for row j - 1
    lab[cb] = min(best_j[cb], j - 1);
    // labels holds the previous iteration's labels when the changes are listed
    oldl[cb] = (mine && nchanges) ? labels[(size_t)bidx * n + tokv[cb]] : lab[cb];
    chm[cb] = __ballot(mine && oldl[cb] != lab[cb]);
    nch_wave += (int)__popcll(chm[cb]);
  }
  const int cbase = nchanges ? wave_reserve(nchanges, nch_wave) : 0;
  int cpre = 0;
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    if (tokv[cb] >= 0) {
      if (oldl[cb] != lab[cb])
        changes[cbase + cpre + mask_rank(chm[cb])] = make_int2(bidx * n + tokv[cb], (oldl[cb] << 16) | lab[cb]);
      labels[(size_t)bidx * n + tokv[cb]] = lab[cb];
    }
    cpre += (int)__popcll(chm[cb]);
  }
}

// --------------------------------------------------------------------------------------- certified fp16 assign
// One MFMA pass in fp16 instead of the two bf16 passes (E_hi, E_lo), with a rigorous error bound.
//   * Token x is scaled by a power of two 2^u (its largest |component| into [2^14, 2^15)) and rounded
//     to fp16 with round-toward-zero: bf16 values in that range are exact in fp16, and components below
//     2^-17 (scaled) move by less than 2^-24 each.  E16 = fp16(2^t E) (prep; one t per head).
//   * s~_j = x~ . E16_j on v_mfma_f32_32x32x16_f16 (exact fp16 products, fp32 sums).  For the scaled exact
//     score S_j = 2^(u+t) x . E_j:  |S_j - s~_j| <= |x~| (D + 2^-17 Emax) + 2^-20 (Emax + D)
//     with D = max_j |2^t E_j - E16_j| and Emax = max_j |E16_j| (prep measures both per head), the fp32
//     sum bound 128 * 2^-24 |x~||E16_j| and the token rounding |2^u x - x~| < 2^-20.5.  The tag in the
//     low 4 mantissa bits moves a score by < 2^-19 |s~|.  With |x~| >= 2^14 all of it is below
//     B = |x~| (D + 2^-15 Emax).
//   * The label is certified when the best score exceeds the second by more than 2 B: then it is the
//     exact argmax of x . E (no tie is possible).  Other tokens (near-equal top scores, a zero token) go
//     to the head's fallback list for the hi + lo kernel, which also applies its tie rule.
// Each lane keeps the top two tagged scores of its cluster rows (updated two scores at a time) and the tile
// of the best.  Padding rows (j .. jpad-1) are zero in E16, so they score exactly 0: as the runner-up such a
// row only tightens the test, and a token whose best row is padding goes to the fallback.
// E16 is stored in MFMA operand order (e16_offset) and streams through LDS in 16 KB chunks by LDS DMA
// issued from inline assembly; measured with per-wave cycle stamps at C3's key side, the main loop runs at
// the MFMA rate of two waves per SIMD (about 61 cycles per 32-cycle MFMA and wave), and the token
// conversion before it and the certification after it take a quarter of a block's time.
// NCB token blocks of 32 per wave: four for many cluster rows (two waves per SIMD), two for at most 128 rows
// (the query side, where the pass streams the tokens more than it multiplies: three waves per SIMD, the
// chunk's two tiles alternating between the accumulator pairs; 196 -> 186 us for the first pass at C3 and
// 127 -> 121 us per pruned pass).
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));
// Through a by-value parameter: this compiler's __builtin_bit_cast of a vector element operand (v[e], v.y)
// reads element 0 whatever the index.
__device__ __forceinline__ f16x2_t as_f16x2(uint32_t w) { return __builtin_bit_cast(f16x2_t, w); }
__device__ __forceinline__ f16x8_t as_f16x8(u32x4_t v) { return __builtin_bit_cast(f16x8_t, v); }
__device__ __forceinline__ f32x16_t mfma32x32x16_f16(f16x8_t a, f16x8_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// With bnd (planes [3][bh][n]: lower bound on the label's exact score x . E_label, upper bound on every other
// cluster's, upper bound on |x|; unscaled) the pass also records, per token, what the pruning test of the
// next pass needs: certified tokens get their bounds, the others -inf / +inf.  With LIST the block's tokens
// are entries [512 x, 512 x + 512) of the head's list (list[bidx][.], list_count[bidx * kCounterStride]
// entries; blocks past the count exit at once).
template <bool LIST, int NCB>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(NCB == 4 ? 2 : 3, NCB == 4 ? 2 : 3)))
cocluster_assign16_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ e16,
                          const uint32_t* __restrict__ err_max, const uint32_t* __restrict__ norm_max,
                          int32_t* __restrict__ labels, int n, int j, int jpad, int2* __restrict__ changes,
                          int32_t* __restrict__ nchanges, int32_t* __restrict__ fb_list,
                          int32_t* __restrict__ fb_count, float* __restrict__ bnd, const int32_t* __restrict__ t_head,
                          const int32_t* __restrict__ list, const int32_t* __restrict__ list_count) {
  // two chunk buffers of 16 KB, each two 32-row tiles in the layout of e16_offset
  __shared__ __attribute__((aligned(16))) uint16_t s_e[2 * kAssignChunk * 128];
  const int bidx = blockIdx.y;
  const int tid = threadIdx.x, lane = tid % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int h = lane / 32, l32 = lane % 32;
  static_assert(NCB == 2 || NCB == 4, "two or four column blocks per wave");
  constexpr int kTokWave = 32 * NCB, kTokBlock = 4 * kTokWave;
  const int tok0 = blockIdx.x * kTokBlock + wave * kTokWave;
  const int ntok = LIST ? list_count[(size_t)bidx * kCounterStride] : n;  // positions < ntok hold tokens
  if (LIST && (int)blockIdx.x * kTokBlock >= ntok) return;
  const int32_t* lst = LIST ? list + (size_t)bidx * n : nullptr;
  // token at position p of this block's range (positions past the range load a valid row, unused)
  auto token_at = [&](int pos) __attribute__((always_inline)) -> int {
    if constexpr (LIST)
      return lst[min(pos, ntok - 1)];
    else
      return min(pos, n - 1);
  };
  const uint16_t* xb = x + (size_t)bidx * n * 128;
  const char* eb = (const char*)(e16 + (size_t)bidx * jpad * 128);
  const int nchunks = jpad / kAssignChunk;

  // A chunk is 16 KB contiguous in e16 and in LDS: wave w copies bytes [4 KB w, 4 KB w + 4 KB), 1 KB per
  // instruction (inline-assembly DMA, waited for before each chunk's barrier).
  const uint32_t voff = wave * 4096 + lane * 16;
  const uint32_t lds0 = lds_addr(s_e) + wave * 4096;
  auto issue = [&](int c, int bf) __attribute__((always_inline)) {
    const char* src = eb + (size_t)c * (kAssignChunk * 256);
#pragma unroll
    for (int g = 0; g < 4; ++g) lds_dma16_asm(src, voff + g * 1024, lds0 + bf * (kAssignChunk * 256) + g * 1024);
  };
  issue(0, 0);

  // Tokens: fp16, scaled per token.  The previous labels, compared at the end when the changes are listed,
  // are loaded here so that their latency is spent under the pass.
  int tokv[NCB], prevl[NCB], uexp[NCB];
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    const int pos = tok0 + cb * 32 + l32;
    tokv[cb] = (h == 0 && pos < ntok) ? token_at(pos) : -1;  // -1: no token of this lane
    prevl[cb] = (nchanges && tokv[cb] >= 0) ? labels[(size_t)bidx * n + tokv[cb]] : -1;
  }
  u32x4_t xop[NCB][8];
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    const int row = token_at(tok0 + cb * 32 + l32);
    const u32x4_t* src = (const u32x4_t*)(xb + (size_t)row * 128);
    u32x4_t raw[8];
    // largest magnitude bits of the lane's 64 components, two halves at a time (packed 16-bit max)
    u16x2_t m2 = {0, 0};
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      raw[ks] = src[ks * 2 + h];
#pragma unroll
      for (int e = 0; e < 4; ++e) m2 = __builtin_elementwise_max(m2, __builtin_bit_cast(u16x2_t, raw[ks][e] & 0x7fff7fffu));
    }
    uint32_t mbits = max((uint32_t)m2[0], (uint32_t)m2[1]);
    mbits = max(mbits, (uint32_t)__shfl_xor((int)mbits, 32));
    // biased exponent of the largest component (subnormals count as exponent -126)
    const int be = max(1, (int)(mbits >> 7));
    const int u = mbits ? 14 - (be - 127) : 0;
    uexp[cb] = u;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float lo = __builtin_amdgcn_ldexpf(bf16_to_f32((uint16_t)(raw[ks][e] & 0xffffu)), u);
        const float hi = __builtin_amdgcn_ldexpf(bf16_to_f32((uint16_t)(raw[ks][e] >> 16)), u);
        xop[cb][ks][e] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo, hi));
      }
  }
  // A operand of k-step ks of a tile: 16 bytes per lane at tile + 1 KB ks + 16 lane (immediate offsets)
  const uint16_t* alane = s_e + lane * 8;
#define AOFF(ks) ((ks) * 512)

  float top1[NCB], top2[NCB];
  int tbase[NCB];
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    top1[cb] = -INFINITY;
    top2[cb] = -INFINITY;
    tbase[cb] = 0;
  }
  f32x16_t acc[4];
  // Top-two update of token block cb with tile jb: per score a tag, a median of three and a max (the IEEE
  // maximum builtin: fmaxf on bit-cast values would add a NaN-quieting instruction per score).
  auto epi = [&](int ai, int cb, int jb) __attribute__((always_inline)) {
    const float prev = top1[cb];
#pragma unroll
    for (int r = 0; r < 16; r += 2) {
      const float ta = __uint_as_float((__float_as_uint(acc[ai][r]) & ~15u) | (uint32_t)(15 - r));
      const float tb = __uint_as_float((__float_as_uint(acc[ai][r + 1]) & ~15u) | (uint32_t)(14 - r));
      const float mid = __builtin_amdgcn_fmed3f(top1[cb], ta, tb);
      top1[cb] = __builtin_elementwise_maximum(__builtin_elementwise_maximum(top1[cb], ta), tb);
      top2[cb] = __builtin_elementwise_maximum(top2[cb], mid);
    }
    tbase[cb] = top1[cb] != prev ? jb : tbase[cb];
  };
  // Two token blocks' MFMAs, their accumulator chains interleaved (a chain's next MFMA waits on the previous),
  // with the A operands (E16 rows of the 32-row tile) read from LDS two k-steps ahead into a ring of three.
  // (accumulators a0, a0 + 1 from the token blocks x0, x0 + 1)
  auto mfmas2 = [&](int a0, int x0, const uint16_t* tile) __attribute__((always_inline)) {
    u32x4_t ring[4];
    ring[0] = *(const u32x4_t*)(tile + AOFF(0));
    ring[1] = *(const u32x4_t*)(tile + AOFF(1));
    ring[2] = *(const u32x4_t*)(tile + AOFF(2));
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      acc[a0] = mfma32x32x16_f16(as_f16x8(ring[ks % 4]), as_f16x8(xop[x0][ks]), ks ? acc[a0] : f32x16_t{});
      if (ks + 3 < 8) ring[(ks + 3) % 4] = *(const u32x4_t*)(tile + AOFF(ks + 3));
      acc[a0 + 1] =
          mfma32x32x16_f16(as_f16x8(ring[ks % 4]), as_f16x8(xop[x0 + 1][ks]), ks ? acc[a0 + 1] : f32x16_t{});
    }
  };
  // Software pipeline within the wave: the MFMAs of blocks {0, 1} run while the VALU updates the top two of
  // blocks {2, 3} of the previous 32-row tile, then the MFMAs of {2, 3} beside the updates of {0, 1}; per k-step
  // an MFMA, six VALU instructions, the LDS read two k-steps ahead, an MFMA, six VALU instructions.
  auto interleave = [&]() __attribute__((always_inline)) {
    __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);
      if (i + 3 < 8) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);
    }
  };
  // Before the first tile the pending updates of blocks 2 and 3 see scores of -FLT_MAX, below every real score
  // (|s~| < 2^38), so they change nothing that survives; the update needs no branch (a branch would split the
  // scheduling region and keep the VALU work away from the MFMAs).
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    acc[2][r] = -3.402823466e38f;
    acc[3][r] = -3.402823466e38f;
  }
  int pend_jb = 0;
  for (int c = 0; c < nchunks; ++c) {
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    // The last step copies the last chunk again into the free buffer: no branch around the copy.
    issue(min(c + 1, nchunks - 1), (c + 1) & 1);
    const uint16_t* se = alane + (c & 1) * (kAssignChunk * 128);
    if constexpr (NCB == 4) {
#pragma unroll
      for (int rb = 0; rb < kAssignChunk / 32; ++rb) {
        const uint16_t* tile = se + rb * 32 * 128;
        const int jb = c * kAssignChunk + rb * 32;
        __builtin_amdgcn_sched_barrier(0);
        mfmas2(0, 0, tile);
        epi(2, 2, pend_jb);
        epi(3, 3, pend_jb);
        interleave();
        __builtin_amdgcn_sched_barrier(0);
        mfmas2(2, 2, tile);
        epi(0, 0, jb);
        epi(1, 1, jb);
        interleave();
        __builtin_amdgcn_sched_barrier(0);
        pend_jb = jb;
      }
    } else {
      // two column blocks: the chunk's two tiles alternate between accumulators {0, 1} and {2, 3}, so a tile's
      // MFMAs still run beside the top-two updates of the tile before it, in tile order
      static_assert(kAssignChunk == 64, "two tiles per chunk");
      const int jb0 = c * kAssignChunk;
      __builtin_amdgcn_sched_barrier(0);
      mfmas2(0, 0, se);
      epi(2, 0, pend_jb);
      epi(3, 1, pend_jb);
      interleave();
      __builtin_amdgcn_sched_barrier(0);
      mfmas2(2, 0, se + 32 * 128);
      epi(0, 0, jb0);
      epi(1, 1, jb0);
      interleave();
      __builtin_amdgcn_sched_barrier(0);
      pend_jb = jb0 + 32;
    }
  }
  if constexpr (NCB == 4) {
    epi(2, 2, pend_jb);
    epi(3, 3, pend_jb);
  } else {
    epi(2, 0, pend_jb);
    epi(3, 1, pend_jb);
  }
#undef AOFF
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the extra copy lands before the block ends
  const float dd = __uint_as_float(err_max[bidx]), em = __uint_as_float(norm_max[bidx]);
  const float slack = dd + 0x1p-15f * em;
  int lab[4], oldl[4];
  bool certv[4], minev[4];
  uint64_t fbm[4], chm[4];
  int nfb = 0, nch_wave = 0;
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    // |x~| of the fp16 operands themselves: fp32 sums of exact fp16 squares, two per v_dot2_f32_f16 (at most
    // two roundings per step over 64 steps; 1.001 below covers them)
    float n2 = 0.0f;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const f16x2_t hv = as_f16x2(xop[cb][ks][e]);
        n2 = __builtin_amdgcn_fdot2(hv, hv, n2, false);
      }
    n2 += __shfl_xor(n2, 32);
    const float xnorm = sqrtf(n2);
    const int r = 15 - (int)(__float_as_uint(top1[cb]) & 15u);
    const int jbest = tbase[cb] + (r / 4) * 8 + (r % 4) + h * 4;
    const float s1 = __uint_as_float(__float_as_uint(top1[cb]) & ~15u);
    const float s2 = __uint_as_float(__float_as_uint(top2[cb]) & ~15u);
    const float o1 = __shfl_xor(s1, 32), o2 = __shfl_xor(s2, 32);
    const int oj = __shfl_xor(jbest, 32);
    const float best = fmaxf(s1, o1);
    const float second = fmaxf(fminf(s1, o1), fmaxf(s2, o2));
    lab[cb] = s1 >= o1 ? jbest : oj;
    const float bound = xnorm * slack * 1.001f;
    // a padding row (score 0) as the second only makes the test stricter; as the best it is not a label
    certv[cb] = (best - second) > 2.0f * bound && lab[cb] < j;  // false for NaN
    minev[cb] = tokv[cb] >= 0;
    if (bnd && minev[cb]) {
      // unscaled bounds: the exact scaled scores are within `bound` of the fp16 ones (1.01 covers the fp32
      // rounding of the sums here), |2^u x| <= |x~| + 2^-20
      const size_t plane = (size_t)gridDim.y * n, o = (size_t)bidx * n + tokv[cb];
      const int sc = uexp[cb] + t_head[bidx];
      bnd[o] = certv[cb] ? __builtin_amdgcn_ldexpf(best - 1.01f * bound, -sc) : -INFINITY;
      bnd[plane + o] = certv[cb] ? __builtin_amdgcn_ldexpf(second + 1.01f * bound, -sc) : INFINITY;
      bnd[2 * plane + o] = __builtin_amdgcn_ldexpf(xnorm * 1.001f + 0x1p-20f, -uexp[cb]);
    }
    fbm[cb] = __ballot(minev[cb] && !certv[cb]);
    // labels holds the previous iteration's labels when the changes are listed
    oldl[cb] = (minev[cb] && certv[cb] && nchanges) ? prevl[cb] : lab[cb];
    chm[cb] = __ballot(minev[cb] && certv[cb] && oldl[cb] != lab[cb]);
    nfb += (int)__popcll(fbm[cb]);
    nch_wave += (int)__popcll(chm[cb]);
  }
  // One reservation per block and list: the four waves' counts meet in LDS, lane 0 of wave 0 reserves the
  // fallback slots and lane 0 of wave 1 the change slots (side by side), and each wave takes its share in
  // wave order.  Tens of thousands of per-wave atomics on the one change counter serialise in the L2.
  __shared__ int s_cnt[2][4], s_base[2];
  if (lane == 0) {
    s_cnt[0][wave] = nfb;
    s_cnt[1][wave] = nch_wave;
  }
  __syncthreads();
  if (lane == 0 && wave < 2) {
    const int tot = s_cnt[wave][0] + s_cnt[wave][1] + s_cnt[wave][2] + s_cnt[wave][3];
    int base = 0;
    if (tot > 0 && wave == 0) base = atomicAdd(fb_count + (size_t)bidx * kCounterStride, tot);
    if (tot > 0 && wave == 1 && nchanges) base = atomicAdd(nchanges, tot);
    s_base[wave] = base;
  }
  __syncthreads();
  int fbase = s_base[0], cbase = s_base[1];
  for (int w = 0; w < wave; ++w) {
    fbase += s_cnt[0][w];
    cbase += s_cnt[1][w];
  }
  int fpre = 0, cpre = 0;
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    const int tok = tokv[cb];
    if (minev[cb] && !certv[cb]) fb_list[(size_t)bidx * n + fbase + fpre + mask_rank(fbm[cb])] = tok;
    if (minev[cb] && certv[cb]) {
      if (oldl[cb] != lab[cb])
        changes[cbase + cpre + mask_rank(chm[cb])] = make_int2(bidx * n + tok, (oldl[cb] << 16) | lab[cb]);
      labels[(size_t)bidx * n + tok] = lab[cb];
    }
    fpre += (int)__popcll(fbm[cb]);
    cpre += (int)__popcll(chm[cb]);
  }
}

// --------------------------------------------------------------------------------------- prune
// Exact pruning of an assignment pass (Hamerly-style bounds).  For token x with label a and the bounds the
// previous pass left (L <= x . E_a, U >= x . E_j for every j != a, |x| <= X, all against that pass's E), the
// new E moves each row by at most delta_j, so x . E'_a >= L - X delta_a and x . E'_j <= U + X max_j delta_j.
// When the first exceeds the second, a is still the unique argmax: the token keeps its label and the carried
// bounds, and the assignment skips it.  The others go to the head's list for the pass.  fp32 rounding of the
// update is covered by a relative margin of 2^-20 of the magnitudes (and 2^-120 absolute for subnormal bounds).
// One list reservation per block of 2048 tokens (the four waves' counts meet in LDS): per-block atomics on
// the head's counter serialise in the L2.
constexpr int kPruneSub = 8;  // 256-token groups per block: one list reservation per 2048 tokens
__global__ void __launch_bounds__(256) cocluster_prune_kernel(const int32_t* __restrict__ labels,
                                                              float* __restrict__ bnd,
                                                              const float* __restrict__ delta,
                                                              const uint32_t* __restrict__ delta_max, int n, int jpad,
                                                              int32_t* __restrict__ list,
                                                              int32_t* __restrict__ list_count) {
  const int bidx = blockIdx.y, tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const size_t plane = (size_t)gridDim.y * n;
  const float dmax = __uint_as_float(delta_max[bidx]) * (1.0f + 0x1p-20f);
  uint64_t m[kPruneSub];
  int cnt = 0;
#pragma unroll
  for (int sub = 0; sub < kPruneSub; ++sub) {
    const int t = (blockIdx.x * kPruneSub + sub) * 256 + tid;
    const size_t o = (size_t)bidx * n + t;
    bool need = false;
    if (t < n) {
      const float lo = bnd[o], hi = bnd[plane + o], xn = bnd[2 * plane + o];
      const float da = xn * delta[(size_t)bidx * jpad + labels[o]] * (1.0f + 0x1p-20f);
      const float dm = xn * dmax;
      const float lo2 = lo - da, hi2 = hi + dm;
      const float margin = 0x1p-20f * (fabsf(lo) + fabsf(hi) + da + dm) + 0x1p-120f;
      need = !(lo2 - hi2 > margin);  // also for inf / NaN bounds
      if (!need) {
        bnd[o] = lo2;
        bnd[plane + o] = hi2;
      }
    }
    m[sub] = __ballot(need);
    cnt += (int)__popcll(m[sub]);
  }
  __shared__ int s_cnt[4], s_base;
  if (lane == 0) s_cnt[wave] = cnt;
  __syncthreads();
  if (tid == 0) {
    const int tot = s_cnt[0] + s_cnt[1] + s_cnt[2] + s_cnt[3];
    s_base = tot ? atomicAdd(list_count + (size_t)bidx * kCounterStride, tot) : 0;
  }
  __syncthreads();
  int base = s_base;
  for (int w = 0; w < wave; ++w) base += s_cnt[w];
#pragma unroll
  for (int sub = 0; sub < kPruneSub; ++sub) {
    if ((m[sub] >> lane) & 1) list[(size_t)bidx * n + base + mask_rank(m[sub])] = (blockIdx.x * kPruneSub + sub) * 256 + tid;
    base += (int)__popcll(m[sub]);
  }
}

// --------------------------------------------------------------------------------------- candidate pass
// Exact pruning of a key-side pass by the triangle inequality in profile space.  The score of token x and
// cluster j is x . E_j = P_j . y with y = C x (C the other side's centroids, kp <= 128 of them) and P_j the
// profile rows, unit vectors up to |P_j|^2 = n_j = sq / (sq + 1e-8).  With u = y / |y|, d_a = |u - P_a| for
// the token's current label a (its anchor) and D_aj = |P_a - P_j|:
//   D_aj >= 2 d_a + m   implies   u . P_a - u . P_j >= (m^2 - nu) / 2,   nu >= max_j n_j - n_a,
// so such a cluster scores at least |y| (m^2 - nu) / 2 below the anchor.  m is chosen per token so that this
// exceeds twice |x| eps_E, the difference between the exact score and the one the prep's E defines (fp32
// sums in its phase 3, eps_E <= 2^-16 ||C||_F): those clusters are then strictly below the anchor in the
// scores that define the label.  Three kernels per pass:
//   radius: per token T = 2 d_a + m from |y| (y on the MFMA) and the anchor's score, as rigorous upper
//           bounds; the cluster's radius is the maximum over its tokens;
//   lists:  per cluster a, the clusters with D_aj below its radius (D from the exactly-bf16 raw profiles on
//           the MFMA, lowered by 2^-14 against the fp32 sums), at most kCandList of them;
//   score:  per 64 label-sorted tokens (one wave, few anchors), the union of their anchors' lists scored on
//           the hi + lo MFMA (within e = 2^-15 |x| Emax of x . E); the best is certified when it beats the
//           second by more than 2 e: it is then the exact argmax of x . E, the label every other pass of this
//           file gives such a token.  The others (near ties, long lists, a zero y) go to the head's fallback
//           list for the hi + lo kernel.
constexpr int kCandList = 32;   // list entries per cluster
constexpr int kCandUnion = 128; // clusters a wave scores (4 tiles of 32)
constexpr int kCandMaxJ = 4096; // clusters per side (the library's limit)

// Upper bound on the radius T = 2 d_a + m of one token (both lanes of the token call it with the same
// arguments); -1 when the token cannot be bounded (no anchor, y too small, a non-finite value).
__device__ __forceinline__ float cand_radius(float s_a, float yn, float xnu, float cfro, float emax, float n_a,
                                             float nu) {
  const float etok = 0x1p-15f * xnu * emax;  // |s~_a - x . E_a|
  const float epsx = 0x1p-16f * cfro * xnu;   // |x| eps_E, and |y~ - y| without the norm's rounding
  const float epsy = epsx + 0x1p-17f * yn;
  const float yl = yn - epsy, yu = yn + epsy;
  const float slo = s_a - etok - epsx;  // lower bound on P_a . y
  float ratio = slo >= 0.0f ? slo / yu : slo / yl;
  ratio -= 0x1p-20f * fabsf(ratio) + 0x1p-40f;
  const float d2 = (1.0f + n_a - 2.0f * ratio) * (1.0f + 0x1p-20f) + 0x1p-40f;
  const float dup = sqrtf(fmaxf(d2, 0.0f)) * (1.0f + 0x1p-20f);
  const float m = sqrtf((4.0f * epsx / yl + nu) * (1.0f + 0x1p-20f) + 0x1p-40f) * (1.0f + 0x1p-20f);
  const float t = 2.0f * dup + m;
  return (yl > 0.0f && t < INFINITY) ? t : -1.0f;  // -1 also for NaN
}

// bf16 pairs: a.x b.x + a.y b.y + c on v_dot2_f32_bf16 (exact products, fp32 sums)
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c, false);
}

// Token operands of TB 32-token blocks (lane l and l + 32 hold the halves of token l of a block), |x|^2.
template <int TB>
__device__ __forceinline__ void cand_tokens(const uint16_t* xb, const int32_t* tok, int h, u32x4_t (*xop)[8],
                                            float* xn2) {
#pragma unroll
  for (int cb = 0; cb < TB; ++cb) {
    const u32x4_t* src = (const u32x4_t*)(xb + (size_t)tok[cb] * 128);
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) xop[cb][ks] = src[ks * 2 + h];
  }
#pragma unroll
  for (int cb = 0; cb < TB; ++cb) {
    float q2 = 0.0f;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
#pragma unroll
      for (int e = 0; e < 4; ++e) q2 = dot2_bf16(xop[cb][ks][e], xop[cb][ks][e], q2);
    xn2[cb] = q2 + __shfl_xor(q2, 32);
  }
}

// Upper bound on E's row norms: |2^t E_j| <= |E16_j| + |2^t E_j - E16_j|.
__device__ __forceinline__ float cand_emax(const uint32_t* norm_max, const uint32_t* err_max, const int32_t* t_head,
                                           int bidx) {
  return __builtin_amdgcn_ldexpf(__uint_as_float(norm_max[bidx]) + __uint_as_float(err_max[bidx]), -t_head[bidx]) *
         (1.0f + 0x1p-20f);
}

// Value of token slot `lane` of a wave (lanes 0-31: block 0, lanes 32-63: block 1 when TB == 2); the two
// lanes of a token hold the same value.
template <int TB, typename T>
__device__ __forceinline__ T cand_slot(const T* v, int h, int l32) {
  if constexpr (TB == 1) {
    return v[0];
  } else {
    const T v1 = __shfl(v[1], l32);
    return h == 0 ? v[0] : v1;
  }
}

constexpr int kCandTB = 1;                  // token blocks of 32 per wave
constexpr int kCandWaveTok = 32 * kCandTB;  // label-sorted positions per wave
constexpr int kCandBlockTok = 4 * kCandWaveTok;

// radius: one wave per kCandWaveTok consecutive positions of the head's label-sorted order.  The anchor of a
// position is pos_anc (the sorted labels of the last sort, moved along by the score kernel's certified
// labels).  Writes, per position, the radius (or -1) and the cluster maxima to trad (float bits, zero on
// entry), one atomic per distinct anchor of a wave.  C is staged in LDS once per block (16-byte chunk c of
// row r at chunk swz(r, c)) by DMA issued beside the position loads, the anchor rows are requested before the
// barrier that publishes C, and the kernel runs four waves per SIMD (112 registers, the LDS allows four
// blocks per CU): 293 -> 264 us per launch at C3 for the first two, 230 us with the third.
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4, 4))) cocluster_radius_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ cother, const uint16_t* __restrict__ e_hi,
    const uint16_t* __restrict__ e_lo, const float* __restrict__ nrm, const uint32_t* __restrict__ nu_bits,
    const uint32_t* __restrict__ err_max, const uint32_t* __restrict__ norm_max, const int32_t* __restrict__ t_head,
    const int32_t* __restrict__ sorted_idx, const int32_t* __restrict__ pos_anc, int n, int j, int jpad, int ko,
    float* __restrict__ pos_t, uint32_t* __restrict__ trad) {
  constexpr int TB = kCandTB;
  __shared__ __attribute__((aligned(16))) uint16_t s_c[128 * 128];
  const int bidx = blockIdx.y, tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave, h = lane / 32,
            l32 = lane % 32;
  const int p0 = blockIdx.x * kCandBlockTok + wave * kCandWaveTok;
  const uint16_t* cb_base = cother + (size_t)bidx * ko * 128;
  int tok[TB], anc[TB];
  bool inpos[TB], vt[TB];
#pragma unroll
  for (int cb = 0; cb < TB; ++cb) {
    inpos[cb] = p0 + cb * 32 + l32 < n;
    const size_t o = (size_t)bidx * n + min(p0 + cb * 32 + l32, n - 1);
    tok[cb] = sorted_idx[o];
    anc[cb] = pos_anc[o];
  }
  // C into LDS by DMA beside the position loads (as in the score kernel): wave w fills rows 32 w .. 32 w + 31,
  // rows past ko are written as zeros; waited for before the barrier that publishes C
  {
    const uint32_t sbase = lds_addr(s_c);
    const int wu = __builtin_amdgcn_readfirstlane(wave);
    const int prow = lane / 16, pch = lane % 16;
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      const int r = 32 * wave + 4 * g + prow;
      if (r < ko)
        lds_dma16_asm(cb_base, (uint32_t)(r * 128 + swz(r, pch) * 8) * 2u, sbase + (32 * wu + 4 * g) * 256);
      else
        *(u32x4_t*)(s_c + r * 128 + pch * 8) = u32x4_t{0u, 0u, 0u, 0u};
    }
  }
#pragma unroll
  for (int cb = 0; cb < TB; ++cb) {
    vt[cb] = inpos[cb] && anc[cb] >= 0 && anc[cb] < j;
    if (!vt[cb]) anc[cb] = 0;
  }
  u32x4_t xop[TB][8];
  float xn2[TB];
  cand_tokens<TB>(x + (size_t)bidx * n * 128, tok, h, xop, xn2);
  // anchor scores on v_dot2_f32_bf16: the lane's 64 components of x against E_hi + E_lo of the anchor (before
  // the barrier, so the anchor rows' latency overlaps the token rows')
  float sa[TB];
#pragma unroll
  for (int cb = 0; cb < TB; ++cb) {
    const u32x4_t* hr = (const u32x4_t*)(e_hi + ((size_t)bidx * jpad + anc[cb]) * 128);
    const u32x4_t* lr = (const u32x4_t*)(e_lo + ((size_t)bidx * jpad + anc[cb]) * 128);
    float acc = 0.0f;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      const u32x4_t wh = hr[ks * 2 + h], wl = lr[ks * 2 + h];
#pragma unroll
      for (int e = 0; e < 4; ++e) acc = dot2_bf16(xop[cb][ks][e], wl[e], dot2_bf16(xop[cb][ks][e], wh[e], acc));
    }
    sa[cb] = acc + __shfl_xor(acc, 32);
  }
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's C rows have landed
  __syncthreads();
  if (p0 >= n) return;
  float csq = 0.0f;  // ||C||_F^2 from the |y| loop's reads (each wave reads all of C once)
  // |y|^2 on the MFMA (C rows past ko are zero)
  float ysq[TB];
#pragma unroll
  for (int cb = 0; cb < TB; ++cb) ysq[cb] = 0.0f;
  for (int ct = 0; ct * 32 < ko; ++ct) {
    const int crow = ct * 32 + l32;
    u32x4_t ca[8];
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) ca[ks] = *(const u32x4_t*)(s_c + crow * 128 + swz(crow, ks * 2 + h) * 8);
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
#pragma unroll
      for (int e = 0; e < 4; ++e) csq = dot2_bf16(ca[ks][e], ca[ks][e], csq);
#pragma unroll
    for (int cb = 0; cb < TB; ++cb) {
      f32x16_t acc = {};
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) acc = mfma32x32x16(as_bf16x8(ca[ks]), as_bf16x8(xop[cb][ks]), acc);
#pragma unroll
      for (int r = 0; r < 16; ++r) ysq[cb] = fmaf(acc[r], acc[r], ysq[cb]);
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) csq += __shfl_xor(csq, o);
  const float cfro = sqrtf(csq * (1.0f + 0x1p-16f)) * (1.0f + 0x1p-20f);
  const float emax = cand_emax(norm_max, err_max, t_head, bidx);
  const float nu = __uint_as_float(nu_bits[bidx]);
  float tr[TB];
#pragma unroll
  for (int cb = 0; cb < TB; ++cb) {
    const float yn = sqrtf(ysq[cb] + __shfl_xor(ysq[cb], 32));
    const float xnu = sqrtf(xn2[cb] * (1.0f + 0x1p-16f)) * (1.0f + 0x1p-20f);
    tr[cb] = vt[cb] ? cand_radius(sa[cb], yn, xnu, cfro, emax, nrm[(size_t)bidx * jpad + anc[cb]], nu) : -1.0f;
    if (inpos[cb] && h == 0) pos_t[(size_t)bidx * n + p0 + cb * 32 + l32] = tr[cb];
  }
  // cluster maxima: one atomic per distinct anchor of the wave
  const int myanc = cand_slot<TB>(anc, h, l32);
  const float myt0 = cand_slot<TB>(tr, h, l32);
  const float myt = (TB == 1 && h == 1) ? -1.0f : myt0;
  uint64_t todo = __ballot(myt > 0.0f);
  while (todo) {
    const int first = __builtin_ctzll(todo);
    const int a = __shfl(myanc, first);
    const uint64_t same = __ballot(myt > 0.0f && myanc == a);
    float mx = (same >> lane) & 1 ? myt : 0.0f;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    if (lane == first) atomicMax(trad + (size_t)bidx * jpad + a, __float_as_uint(mx));
    todo &= ~same;
  }
}

// lists: one block per 32-row strip of a head; each wave keeps the strip's raw-profile operand and takes every
// 4th 32-column tile: D_aj^2 >= n_a + n_j - 2 inv_a inv_j (praw_a . praw_j) - 2^-14, and cluster j joins a's
// list when that is below a's squared radius (trad * tmul + tadd, also written to tused).  A list that would
// be longer than kCandList keeps its count.
__global__ void __launch_bounds__(256) cocluster_lists_kernel(const uint16_t* __restrict__ praw,
                                                              const double* __restrict__ inv,
                                                              const float* __restrict__ nrm,
                                                              const uint32_t* __restrict__ trad, float tmul,
                                                              float tadd, int j, int jpad,
                                                              int16_t* __restrict__ lists,
                                                              int32_t* __restrict__ list_n,
                                                              uint32_t* __restrict__ tused,
                                                              uint32_t* __restrict__ tzero) {
  __shared__ int cnt[32];
  __shared__ int16_t lst[32][kCandList];
  const int bidx = blockIdx.y, ta = blockIdx.x, tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave,
            h = lane / 32, l32 = lane % 32;
  const int nt = jpad / 32;
  if (tid < 32) cnt[tid] = 0;
  const uint16_t* pb = praw + (size_t)bidx * jpad * 128;
  const double* ib = inv + (size_t)bidx * jpad;
  const float* nb = nrm + (size_t)bidx * jpad;
  u32x4_t aop[8];
  const u32x4_t* arow = (const u32x4_t*)(pb + (size_t)(ta * 32 + l32) * 128);
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) aop[ks] = arow[ks * 2 + h];
  double ia[16];
  float na[16], th[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int a = ta * 32 + (r / 4) * 8 + h * 4 + r % 4;
    ia[r] = ib[a];
    na[r] = nb[a];
    const float t0 = __uint_as_float(trad[(size_t)bidx * jpad + a]);
    const float t = t0 > 0.0f ? fmaf(t0, tmul, tadd) : 0.0f;
    th[r] = a < j ? t * t : 0.0f;
  }
  __syncthreads();
  // the wave's column tiles tj = wave, wave + 4, ...; the next tile's rows are requested before this one's MFMAs
  auto tile_load = [&](u32x4_t(&r)[8], int tj) __attribute__((always_inline)) {
    const u32x4_t* brow = (const u32x4_t*)(pb + (size_t)(tj * 32 + l32) * 128);
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) r[ks] = brow[ks * 2 + h];
  };
  // The column constants travel with their tile's rows, one tile ahead: a load issued after the MFMAs and used
  // at once would also wait for the next tile's rows (loads complete in order), which undid the prefetch.
  u32x4_t bop[8];
  double ij = 0.0;
  float njf = 0.0f;
  if (wave < nt) {
    tile_load(bop, wave);
    ij = ib[wave * 32 + l32];
    njf = nb[wave * 32 + l32];
  }
  for (int tj = wave; tj < nt; tj += 4) {
    u32x4_t bnx[8];
    double ij_n = 0.0;
    float nj_n = 0.0f;
    if (tj + 4 < nt) {
      tile_load(bnx, tj + 4);
      ij_n = ib[(tj + 4) * 32 + l32];
      nj_n = nb[(tj + 4) * 32 + l32];
    }
    f32x16_t acc = {};
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) acc = mfma32x32x16(as_bf16x8(aop[ks]), as_bf16x8(bop[ks]), acc);
    const int jj = tj * 32 + l32;
    const double nj = (double)njf;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float d2 = (float)((double)na[r] + nj - 2.0 * ((double)acc[r] * ia[r] * ij) - 0x1p-14);
      if (jj < j && d2 < th[r]) {
        const int al = (r / 4) * 8 + h * 4 + r % 4;
        const int slot = atomicAdd(&cnt[al], 1);
        if (slot < kCandList) lst[al][slot] = (int16_t)jj;
      }
    }
    if (tj + 4 < nt) {
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) bop[ks] = bnx[ks];
      ij = ij_n;
      njf = nj_n;
    }
  }
  __syncthreads();
  for (int t = tid; t < 32 * kCandList; t += 256) {
    const int al = t / kCandList, e = t % kCandList;
    const int a = ta * 32 + al;
    lists[((size_t)bidx * jpad + a) * kCandList + e] = e < cnt[al] ? lst[al][e] : (int16_t)-1;
  }
  if (tid < 32) {
    const size_t o = (size_t)bidx * jpad + ta * 32 + tid;
    list_n[o] = cnt[tid];
    const float t0 = __uint_as_float(trad[o]);
    tused[o] = __float_as_uint(t0 > 0.0f ? fmaf(t0, tmul, tadd) : 0.0f);  // the radius the list was built for
    if (tzero) tzero[o] = 0u;  // the radii the score kernel is about to record
  }
}

// nu of each head: twice the largest |1 - n_a| over its real rows (nu_bits zero on entry).
__global__ void __launch_bounds__(256) cocluster_nu_kernel(const float* __restrict__ nrm, int j, int jpad,
                                                           uint32_t* __restrict__ nu_bits) {
  const int bidx = blockIdx.y;
  float dv = 0.0f;
  for (int a = threadIdx.x; a < j; a += 256) dv = fmaxf(dv, fabsf(1.0f - nrm[(size_t)bidx * jpad + a]));
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) dv = fmaxf(dv, __shfl_xor(dv, o));
  if (threadIdx.x % kWave == 0) atomicMax(nu_bits + bidx, __float_as_uint(2.0f * dv * (1.0f + 0x1p-20f) + 0x1p-40f));
}

// score: one wave per kCandWaveTok consecutive label-sorted positions, as in the radius kernel: the same
// anchors, the radii it wrote.  A certified label also becomes the position's anchor for the next pass.  The
// wave's distinct anchors (usually one or two) bring their lists; the union (a bitmap in the wave's LDS, then
// compacted in cluster order) is scored on the hi + lo MFMA 32 clusters at a time.  One reservation per block
// and list.  With SELF, C reaches LDS by DMA issued beside the position loads, so its latency overlaps theirs
// (a register load, wait and LDS store ahead of them cost a round trip per block: 403 against 370 us per
// launch at C3), and ||C||_F comes from the reads of the |y| loop.  The |y| MFMAs run once the union is
// known, while the first tile's E_hi rows are in flight (after the scores they cost ~6% more per launch);
// C is read one k-step at a time there, which keeps the kernel at four waves per SIMD.
template <bool SELF>
__global__ void __launch_bounds__(256) cocluster_score_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ e_hi, const uint16_t* __restrict__ e_lo,
    const int16_t* __restrict__ lists, const int32_t* __restrict__ list_n, const float* __restrict__ pos_t,
    int32_t* __restrict__ pos_anc, const uint32_t* __restrict__ err_max, const uint32_t* __restrict__ norm_max,
    const int32_t* __restrict__ t_head, const int32_t* __restrict__ sorted_idx, int32_t* __restrict__ labels, int n,
    int j, int jpad, int2* __restrict__ changes, int32_t* __restrict__ nchanges, int32_t* __restrict__ fb_list,
    int32_t* __restrict__ fb_count, const uint16_t* __restrict__ cother, int ko, const float* __restrict__ nrm,
    const uint32_t* __restrict__ nu_bits, const uint32_t* __restrict__ tused, uint32_t* __restrict__ trec) {
  constexpr int TB = kCandTB;
  __shared__ uint32_t s_bm[4][kCandMaxJ / 32];
  __shared__ int16_t s_u[4][kCandUnion];
  __shared__ int s_cnt[2][4], s_base[2];
  constexpr int kCRows = SELF ? 128 : 1;
  __shared__ __attribute__((aligned(16))) uint16_t s_c[kCRows * 128];
  const int bidx = blockIdx.y, tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave, h = lane / 32,
            l32 = lane % 32;
  const int p0 = blockIdx.x * kCandBlockTok + wave * kCandWaveTok;
  const bool wv = p0 < n;  // the wave has positions (the block's reservations below need every wave)
  uint32_t* bm = s_bm[wave];
  int16_t* ul = s_u[wave];
  const int nw = (j + 31) / 32;  // bitmap words in use
  for (int w = lane; w < nw; w += kWave) bm[w] = 0u;
  int tok[TB], anc[TB];
  bool inpos[TB], vt[TB];
#pragma unroll
  for (int cb = 0; cb < TB; ++cb) {
    const int pos = p0 + cb * 32 + l32;
    inpos[cb] = pos < n;
    const size_t o = (size_t)bidx * n + min(pos, n - 1);
    tok[cb] = sorted_idx[o];
    anc[cb] = pos_anc[o];
    vt[cb] = inpos[cb] && anc[cb] >= 0 && anc[cb] < j && (SELF || pos_t[o] > 0.0f);
    if (!vt[cb]) anc[cb] = 0;
  }
  float nrm_a[TB], tu_a[TB];  // the anchor's profile norm and list radius, requested early
  if constexpr (SELF) {
    // C into LDS by DMA (16-byte chunk c of row r at chunk swz(r, c)): wave w fills rows 32 w .. 32 w + 31,
    // 4 rows (1 KB) per instruction, lane i chunk i % 16 of row 4 g + i / 16 from logical chunk swz(r, i % 16);
    // rows past ko are written as zeros.  Completion is waited for before the barrier that publishes C.
    const uint16_t* cb_base = cother + (size_t)bidx * ko * 128;
    const uint32_t sbase = lds_addr(s_c);
    const int wu = __builtin_amdgcn_readfirstlane(wave);
    const int prow = lane / 16, pch = lane % 16;
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      const int r = 32 * wave + 4 * g + prow;
      if (r < ko)
        lds_dma16_asm(cb_base, (uint32_t)(r * 128 + swz(r, pch) * 8) * 2u, sbase + (32 * wu + 4 * g) * 256);
      else
        *(u32x4_t*)(s_c + r * 128 + pch * 8) = u32x4_t{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int cb = 0; cb < TB; ++cb) {
      nrm_a[cb] = nrm[(size_t)bidx * jpad + anc[cb]];
      tu_a[cb] = __uint_as_float(tused[(size_t)bidx * jpad + anc[cb]]);
    }
  }
  // distinct anchors: lane k < nd holds the k-th
  const int myanc = cand_slot<TB>(anc, h, l32);
  const bool myv0 = cand_slot<TB>(vt, h, l32);
  const bool myv = myv0 && !(TB == 1 && h == 1);
  uint64_t todo = __ballot(myv);
  int da = -1, nd = 0;
  while (todo) {
    const int first = __builtin_ctzll(todo);
    const int a = __shfl(myanc, first);
    if (lane == nd) da = a;
    ++nd;
    todo &= ~__ballot(myv && myanc == a);
  }
  int ln = 0;
  int16_t ent[kCandList];
  if (da >= 0) {
    ln = list_n[(size_t)bidx * jpad + da];
    const int16_t* lp = lists + ((size_t)bidx * jpad + da) * kCandList;
#pragma unroll
    for (int e = 0; e < kCandList; e += 8) *(u32x4_t*)&ent[e] = *(const u32x4_t*)&lp[e];
  }
  u32x4_t xop[TB][8];
  float xn2[TB];
  int old[TB];  // the token's label before this pass (the anchor unless the fallback kernel moved it)
#pragma unroll
  for (int cb = 0; cb < TB; ++cb) old[cb] = wv ? labels[(size_t)bidx * n + tok[cb]] : 0;
  if (wv) cand_tokens<TB>(x + (size_t)bidx * n * 128, tok, h, xop, xn2);
  // the anchors' lists into the bitmap (a list longer than kCandList leaves its tokens to the fallback)
  __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the bitmap is clear
  if (da >= 0 && ln <= kCandList) {
#pragma unroll
    for (int e = 0; e < kCandList; ++e)
      if (e < ln) atomicOr(&bm[ent[e] >> 5], 1u << (ent[e] & 31));
  }
  // per token: its anchor's list fitted
  bool lok[TB];
  {
    const uint64_t longm = __ballot(da >= 0 && ln > kCandList);
#pragma unroll
    for (int cb = 0; cb < TB; ++cb) {
      bool bad = false;
      uint64_t m = longm;
      while (m) {
        const int dk = __shfl(da, __builtin_ctzll(m));  // every lane takes part in the exchange
        bad = bad || anc[cb] == dk;
        m &= m - 1;
      }
      lok[cb] = !bad;
    }
  }
  __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the bitmap is complete
  // compact the union in cluster order
  int nu = 0;
  {
    const uint32_t w0 = 2 * lane < nw ? bm[2 * lane] : 0u, w1 = 2 * lane + 1 < nw ? bm[2 * lane + 1] : 0u;
    const int c = __popc(w0) + __popc(w1);
    int inc = c;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      const int u = __shfl_up(inc, o);
      if (lane >= o) inc += u;
    }
    nu = __shfl(inc, kWave - 1);
    int idx = inc - c;
    for (uint32_t w = w0, base = 64 * lane; w; w &= w - 1) {
      if (idx < kCandUnion) ul[idx] = (int16_t)(base + __builtin_ctz(w));
      ++idx;
    }
    for (uint32_t w = w1, base = 64 * lane + 32; w; w &= w - 1) {
      if (idx < kCandUnion) ul[idx] = (int16_t)(base + __builtin_ctz(w));
      ++idx;
    }
  }
  __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  const bool uover = nu > kCandUnion;
  float b1[TB], b2[TB], sav[TB];  // sav: the anchor's score, in the lane that holds its row
  int c1[TB];
  bool fin[TB];
#pragma unroll
  for (int cb = 0; cb < TB; ++cb) {
    b1[cb] = -INFINITY;
    b2[cb] = -INFINITY;
    sav[cb] = -INFINITY;
    c1[cb] = -1;
    fin[cb] = true;
  }
  const bool scoring = wv && !uover;
  const uint16_t* eh = e_hi + (size_t)bidx * jpad * 128;
  const uint16_t* el = e_lo + (size_t)bidx * jpad * 128;
  u32x4_t ph[8], pl[8];
  auto tile_row = [&](int ut) __attribute__((always_inline)) {
    const int ui = ut * 32 + l32;
    return (int)ul[ui < nu ? ui : 0];
  };
  auto load_hi = [&](int crow) __attribute__((always_inline)) {
    const u32x4_t* hrow = (const u32x4_t*)(eh + (size_t)crow * 128) + h;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) ph[ks] = hrow[ks * 2];
  };
  auto load_lo = [&](int crow) __attribute__((always_inline)) {
    const u32x4_t* lrow = (const u32x4_t*)(el + (size_t)crow * 128) + h;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) pl[ks] = lrow[ks * 2];
  };
  float ysq[TB];
  float csq = 0.0f;  // SELF: ||C||_F^2 from the |y| loop's reads (each wave reads all of C once)
#pragma unroll
  for (int cb = 0; cb < TB; ++cb) ysq[cb] = 0.0f;
  if constexpr (SELF) {
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's C rows (and token rows) have landed
    __syncthreads();                                        // C is in LDS
    // the first tile's E_hi rows arrive under the |y| work; an empty union (every anchor's list too long)
    // has no tile, and ul holds nothing written by this block
    if (scoring && nu > 0) load_hi(tile_row(0));
    if (wv) {
      static_assert(TB == 1, "one token block");
      for (int ct = 0; ct * 32 < ko; ++ct) {
        const int crow = ct * 32 + l32;
        f32x16_t acc = {};
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
          const u32x4_t ca = *(const u32x4_t*)(s_c + crow * 128 + swz(crow, ks * 2 + h) * 8);
#pragma unroll
          for (int e = 0; e < 4; ++e) csq = dot2_bf16(ca[e], ca[e], csq);
          acc = mfma32x32x16(as_bf16x8(ca), as_bf16x8(xop[0][ks]), acc);
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) ysq[0] = fmaf(acc[r], acc[r], ysq[0]);
      }
    }
  }
  if (scoring) {
    for (int ut = 0; ut * 32 < nu; ++ut) {
      const int crow_t = tile_row(ut);
      if (!SELF || ut > 0) load_hi(crow_t);
      load_lo(crow_t);
#pragma unroll
      for (int cb = 0; cb < TB; ++cb) {
        f32x16_t acc = {};
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
          acc = mfma32x32x16(as_bf16x8(ph[ks]), as_bf16x8(xop[cb][ks]), acc);
          acc = mfma32x32x16(as_bf16x8(pl[ks]), as_bf16x8(xop[cb][ks]), acc);
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = ut * 32 + (r / 4) * 8 + h * 4 + r % 4;
          const float sv = acc[r];
          if (row < nu) {
            const int cl = ul[row];
            fin[cb] = fin[cb] && (sv > -INFINITY && sv < INFINITY);
            if (SELF && cl == anc[cb]) sav[cb] = sv;
            if (sv > b1[cb]) {
              b2[cb] = b1[cb];
              b1[cb] = sv;
              c1[cb] = cl;
            } else if (sv > b2[cb]) {
              b2[cb] = sv;
            }
          }
        }
      }
    }
  }
  const float emax = cand_emax(norm_max, err_max, t_head, bidx);
  // SELF: the token's radius from this pass's y and anchor score must fit in the one its anchor's list was
  // built for; the radii are recorded (cluster maxima) for the next pass's lists
  bool rok[TB];
#pragma unroll
  for (int cb = 0; cb < TB; ++cb) rok[cb] = true;
  if constexpr (SELF) {
    const float nu = __uint_as_float(nu_bits[bidx]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) csq += __shfl_xor(csq, o);
    const float cfro = sqrtf(csq * (1.0f + 0x1p-16f)) * (1.0f + 0x1p-20f);
    float tr[TB];
#pragma unroll
    for (int cb = 0; cb < TB; ++cb) {
      const float yn = sqrtf(ysq[cb] + __shfl_xor(ysq[cb], 32));
      const float sa = fmaxf(sav[cb], __shfl_xor(sav[cb], 32));
      const float xnu = wv ? sqrtf(xn2[cb] * (1.0f + 0x1p-16f)) * (1.0f + 0x1p-20f) : 0.0f;
      tr[cb] = (vt[cb] && sa > -INFINITY) ? cand_radius(sa, yn, xnu, cfro, emax, nrm_a[cb], nu) : -1.0f;
      rok[cb] = tr[cb] > 0.0f && tr[cb] <= tu_a[cb];
    }
    // record: one atomic per distinct anchor of the wave
    const int myanc2 = cand_slot<TB>(anc, h, l32);
    const float myt0 = cand_slot<TB>(tr, h, l32);
    const float myt = (TB == 1 && h == 1) ? -1.0f : myt0;
    uint64_t todo2 = __ballot(myt > 0.0f);
    while (todo2) {
      const int first = __builtin_ctzll(todo2);
      const int a = __shfl(myanc2, first);
      const uint64_t same = __ballot(myt > 0.0f && myanc2 == a);
      float mx = (same >> lane) & 1 ? myt : 0.0f;
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
      if (lane == first) atomicMax(trec + (size_t)bidx * jpad + a, __float_as_uint(mx));
      todo2 &= ~same;
    }
  }
  int lab[TB];
  bool cert[TB];
  uint64_t fbm[TB], chm[TB];
  int nfb = 0, nch = 0;
#pragma unroll
  for (int cb = 0; cb < TB; ++cb) {
    const float o1 = __shfl_xor(b1[cb], 32), o2 = __shfl_xor(b2[cb], 32);
    const int oc = __shfl_xor(c1[cb], 32);
    const bool ofin = __shfl_xor((int)fin[cb], 32) != 0;
    const float best = fmaxf(b1[cb], o1);
    const float second = fmaxf(fminf(b1[cb], o1), fmaxf(b2[cb], o2));
    lab[cb] = b1[cb] > o1 ? c1[cb] : oc;
    const float xnu = wv ? sqrtf(xn2[cb] * (1.0f + 0x1p-16f)) * (1.0f + 0x1p-20f) : 0.0f;
    const float etok = 0x1p-15f * xnu * emax;
    // b1 == o1 is a tie of two clusters (second == best): not certified
    cert[cb] = vt[cb] && rok[cb] && lok[cb] && !uover && fin[cb] && ofin && (best - second) > 2.0f * etok &&
               lab[cb] >= 0;
    const bool mine = inpos[cb] && h == 0;
    fbm[cb] = __ballot(mine && !cert[cb]);
    chm[cb] = __ballot(mine && cert[cb] && lab[cb] != old[cb]);
    nfb += (int)__popcll(fbm[cb]);
    nch += (int)__popcll(chm[cb]);
  }
  if (lane == 0) {
    s_cnt[0][wave] = nfb;
    s_cnt[1][wave] = nch;
  }
  __syncthreads();
  if (lane == 0 && wave < 2) {
    const int tot = s_cnt[wave][0] + s_cnt[wave][1] + s_cnt[wave][2] + s_cnt[wave][3];
    int base = 0;
    if (tot > 0 && wave == 0) base = atomicAdd(fb_count + (size_t)bidx * kCounterStride, tot);
    if (tot > 0 && wave == 1) base = atomicAdd(nchanges, tot);
    s_base[wave] = base;
  }
  __syncthreads();
  int fbase = s_base[0], cbase = s_base[1];
  for (int w = 0; w < wave; ++w) {
    fbase += s_cnt[0][w];
    cbase += s_cnt[1][w];
  }
#pragma unroll
  for (int cb = 0; cb < TB; ++cb) {
    const bool mine = inpos[cb] && h == 0;
    if (mine && !cert[cb]) fb_list[(size_t)bidx * n + fbase + mask_rank(fbm[cb])] = tok[cb];
    if (mine && cert[cb]) {
      if (lab[cb] != old[cb])
        changes[cbase + mask_rank(chm[cb])] = make_int2(bidx * n + tok[cb], (old[cb] << 16) | lab[cb]);
      labels[(size_t)bidx * n + tok[cb]] = lab[cb];
      pos_anc[(size_t)bidx * n + p0 + cb * 32 + l32] = lab[cb];
    }
    fbase += (int)__popcll(fbm[cb]);
    cbase += (int)__popcll(chm[cb]);
  }
}

}  // namespace svoo

using namespace svoo;

// Forward declarations of the other translation units' internal entry points.
int svoo_cluster_sort_impl(const int32_t* labels, int bh, int n, int k, int32_t* sorted_idx, int32_t* sizes,
                           int32_t* offsets, int32_t* sorted_labels, int32_t* counts, int32_t* err,
                           hipStream_t stream, const int32_t* guard = nullptr, int limit = 0,
                           double* zero_sums = nullptr, long long zero_n = 0);
int svoo_cluster_sort2_impl(const int32_t* labels_a, int k_a, int32_t* sorted_idx_a, int32_t* sizes_a,
                            int32_t* offsets_a, int32_t* sorted_labels_a, int32_t* counts_a, const int32_t* labels_b,
                            int k_b, int32_t* sorted_idx_b, int32_t* sizes_b, int32_t* offsets_b,
                            int32_t* sorted_labels_b, int32_t* counts_b, int bh, int n, hipStream_t stream);
extern "C" size_t svoo_cluster_sort_workspace_size(int bh, int n, int k);
int svoo_centroid_update_impl(const uint16_t* x, const int32_t* sorted_idx, const int32_t* sorted_labels,
                              const int32_t* sizes, const uint16_t* old_c, uint16_t* new_c, int bh, int n, int k,
                              double* sums, hipStream_t stream, int keep_sums, int32_t* zp, long long zn);
int svoo_centroid_move_impl(const uint16_t* x, const int32_t* sorted_idx, const int32_t* sorted_labels,
                            const int2* changes, int32_t* nchanges, double* sums, int32_t* sizes, const uint16_t* old_c,
                            uint16_t* new_c, int bh, int n, int k, int limit, hipStream_t stream, int32_t* zp,
                            long long zn);
int svoo_zero_i32(int32_t* p, long long n, hipStream_t stream);
int svoo_zero_f64(double* p, long long n, hipStream_t stream);

static inline int pad_to(int v, int m) { return (v + m - 1) / m * m; }

static size_t prep_smem(int rows, int kp) {
  return (size_t)rows * 128 * sizeof(double) + rows * sizeof(double) + (size_t)rows * kp * sizeof(float);
}

// With e16 (only for kp <= kPmMaxKp, the fp64-MFMA kernel) also the fp16 copy and the per-head error maxima
// (err_max / norm_max must be zero on entry).
// With e_old (fp64 E of the previous call on the same buffers, replaced by this one) and have_old, also the
// per-row change delta and its head maximum delta_max (zero on entry), for the pruning test; t_out receives
// the head's power-of-two scale of the fp16 copy.
static int prep_launch(const uint16_t* a, const uint16_t* b, uint16_t* e_hi, uint16_t* e_lo, float* profile, int bh,
                       int j, int kp, int jpad, hipStream_t stream, uint16_t* e16 = nullptr,
                       uint32_t* err_max = nullptr, uint32_t* norm_max = nullptr, double* e_old = nullptr,
                       float* delta = nullptr, uint32_t* delta_max = nullptr, int32_t* t_out = nullptr,
                       int have_old = 0, uint16_t* praw_out = nullptr, double* inv_out = nullptr,
                       float* nrm_out = nullptr) {
  if (kp <= kPmMaxKp) {
    hipLaunchKernelGGL(cocluster_prep_mfma_kernel, dim3(jpad / kPmRows, bh), dim3(256), pm_smem(kp), stream, a, b,
                       e_hi, e_lo, profile, j, kp, jpad, e16, err_max, norm_max, e_old, delta, delta_max, t_out,
                       have_old, praw_out, inv_out, nrm_out);
    return check_launch("svoo_cocluster_prep");
  }
  // Wide profiles: the vector kernel.  Few rows -> 2 rows per block for more blocks; many -> 8.
  if (j >= 512 && (size_t)8 * kp * sizeof(float) <= (size_t)kPrepMaxLds) {
    hipLaunchKernelGGL(cocluster_prep_kernel<8>, dim3(jpad / 8, bh), dim3(256), prep_smem(8, kp), stream, a, b, e_hi,
                       e_lo, profile, j, kp, jpad);
  } else {
    hipLaunchKernelGGL(cocluster_prep_kernel<2>, dim3(jpad / 2, bh), dim3(256), prep_smem(2, kp), stream, a, b, e_hi,
                       e_lo, profile, j, kp, jpad);
  }
  return check_launch("svoo_cocluster_prep");
}

// short_list: the list is expected to hold a small share of the tokens (the candidate pass's leftovers): one
// column block per wave.
static int assign_launch(const uint16_t* x, const uint16_t* e_hi, const uint16_t* e_lo, int32_t* labels, int bh, int n,
                         int j, int jpad, hipStream_t stream, int2* changes = nullptr, int32_t* nchanges = nullptr,
                         const int32_t* list = nullptr, const int32_t* list_count = nullptr, bool short_list = false) {
  if (list && short_list)
    hipLaunchKernelGGL((cocluster_assign_kernel<true, 1>), dim3((n + 127) / 128, bh), dim3(256), 0, stream, x, e_hi,
                       e_lo, labels, n, j, jpad, changes, nchanges, list, list_count);
  else if (list)
    hipLaunchKernelGGL((cocluster_assign_kernel<true, 4>), dim3((n + kAsgTok - 1) / kAsgTok, bh), dim3(256), 0, stream,
                       x, e_hi, e_lo, labels, n, j, jpad, changes, nchanges, list, list_count);
  else
    hipLaunchKernelGGL((cocluster_assign_kernel<false, 4>), dim3((n + kAsgTok - 1) / kAsgTok, bh), dim3(256), 0,
                       stream, x, e_hi, e_lo, labels, n, j, jpad, changes, nchanges, nullptr, nullptr);
  return check_launch("svoo_cocluster_assign");
}

// The certified fp16 pass, then the hi + lo kernel on the tokens it left (fb_count must be zero on entry).
// With bnd (and t_head) the pass records the pruning bounds; with list it runs on the listed tokens only.
static int assign16_launch(const uint16_t* x, const uint16_t* e16, const uint16_t* e_hi, const uint16_t* e_lo,
                           const uint32_t* err_max, const uint32_t* norm_max, int32_t* labels, int bh, int n, int j,
                           int jpad, int32_t* fb_list, int32_t* fb_count, hipStream_t stream, int2* changes,
                           int32_t* nchanges, float* bnd = nullptr, const int32_t* t_head = nullptr,
                           const int32_t* list = nullptr, const int32_t* list_count = nullptr) {
  // few cluster rows (the query side): two column blocks per wave and four waves per SIMD
  if (jpad <= 128) {
    dim3 grid((n + 255) / 256, bh);
    if (list)
      hipLaunchKernelGGL((cocluster_assign16_kernel<true, 2>), grid, dim3(256), 0, stream, x, e16, err_max, norm_max,
                         labels, n, j, jpad, changes, nchanges, fb_list, fb_count, bnd, t_head, list, list_count);
    else
      hipLaunchKernelGGL((cocluster_assign16_kernel<false, 2>), grid, dim3(256), 0, stream, x, e16, err_max,
                         norm_max, labels, n, j, jpad, changes, nchanges, fb_list, fb_count, bnd, t_head, nullptr,
                         nullptr);
  } else {
    dim3 grid((n + kAsgTok - 1) / kAsgTok, bh);
    if (list)
      hipLaunchKernelGGL((cocluster_assign16_kernel<true, 4>), grid, dim3(256), 0, stream, x, e16, err_max, norm_max,
                         labels, n, j, jpad, changes, nchanges, fb_list, fb_count, bnd, t_head, list, list_count);
    else
      hipLaunchKernelGGL((cocluster_assign16_kernel<false, 4>), grid, dim3(256), 0, stream, x, e16, err_max,
                         norm_max, labels, n, j, jpad, changes, nchanges, fb_list, fb_count, bnd, t_head, nullptr,
                         nullptr);
  }
  if (int rc = check_launch("svoo_co_cluster (fp16 assign)")) return rc;
  return assign_launch(x, e_hi, e_lo, labels, bh, n, j, jpad, stream, changes, nchanges, fb_list, fb_count);
}

static const int kMaxClusters = 4096;
// Pruning per side.  Measured on the C3 workload (one head, warm start, exact scores on the CPU): from the
// second iteration on the test settles 95-99% of the query tokens (100 clusters) and 4-8% of the key tokens
// (1000 clusters, whose top-two gaps are small against the centroid moves).
// SVOO_QUERY_PRUNE=0 in the environment switches the query side's pruning off (comparisons and tests).  A pruned
// token keeps its label, which is then the exact argmax of x.E; an unpruned pass gives the hi + lo kernel's label,
// which can differ from the exact argmax only where two scores lie within that kernel's rounding.
static const bool kPruneKeys = false;
static bool query_prune_enabled() {
  const char* v = getenv("SVOO_QUERY_PRUNE");
  return !(v && v[0] == '0' && v[1] == 0);
}
// The key side's candidate pass (radius, lists and score kernels) replaces the full pass from the second
// iteration on when the query centroids fit one 128-row operand and there are at least kCandMinKc key clusters.
// Its cost hardly depends on the cluster count while the full pass's grows with it; measured at the Wan shapes
// (same labels either way, warm start): 500 key clusters, 1.31 ms full against 1.39 ms with it per 5-iteration
// clustering; 1000 key clusters, 6.4-6.5 against 5.6 ms.  SVOO_KEY_CANDIDATES=0 / 1 in the environment switches it off / on
// whatever the shape (comparisons and tests).
static const int kCandMaxKp = 128;
static const int kCandMinKc = 1000;
// Later candidate passes build each cluster's list for its last measured radius times kCandRadiusGrowth plus
// kCandRadiusPad (profile space, radii up to 2); a token whose new radius exceeds that goes to the fallback.
// Measured at C3 (warm start): 1.05 / 0.005 and 1.1 / 0 leave as many tokens to the fallback as the measuring
// pass does; 1.25 / 0.02 leaves about 10% more (longer lists overflow), 1.5 / 0.04 five times more.
static const float kCandRadiusGrowth = 1.05f;
static const float kCandRadiusPad = 0.005f;
static bool key_candidates_enabled(int qc, int kc) {
  if (qc > kCandMaxKp) return false;
  const char* v = getenv("SVOO_KEY_CANDIDATES");
  if (v && v[0] == '0' && v[1] == 0) return false;
  if (v && v[0] == '1' && v[1] == 0) return true;
  return kc >= kCandMinKc;
}

extern "C" int svoo_cocluster_prep(const uint16_t* a, const uint16_t* b, uint16_t* e_hi, uint16_t* e_lo,
                                   float* profile, int bh, int j, int kp, int d, int jpad, void* stream) {
  SVOO_REQUIRE(a && b && e_hi && e_lo, SVOO_ERR_INVALID_ARG, "svoo_cocluster_prep: null pointer");
  SVOO_REQUIRE_HEAD_DIM(d, "svoo_cocluster_prep");
  SVOO_REQUIRE(bh > 0 && bh <= 65535 && j > 0 && kp > 0, SVOO_ERR_INVALID_ARG, "svoo_cocluster_prep: bad dims");
  SVOO_REQUIRE(j <= kMaxClusters && kp <= kMaxClusters, SVOO_ERR_UNSUPPORTED,
               "svoo_cocluster_prep: cluster counts above %d", kMaxClusters);
  SVOO_REQUIRE(jpad >= j && jpad % kAssignChunk == 0, SVOO_ERR_INVALID_ARG,
               "svoo_cocluster_prep: jpad=%d must be >= j and a multiple of %d", jpad, kAssignChunk);
  return prep_launch(a, b, e_hi, e_lo, profile, bh, j, kp, jpad, (hipStream_t)stream);
}

extern "C" int svoo_cocluster_assign(const uint16_t* x, const uint16_t* e_hi, const uint16_t* e_lo, int32_t* labels,
                                     int bh, int n, int j, int jpad, int d, void* stream) {
  SVOO_REQUIRE(x && e_hi && e_lo && labels, SVOO_ERR_INVALID_ARG, "svoo_cocluster_assign: null pointer");
  SVOO_REQUIRE_HEAD_DIM(d, "svoo_cocluster_assign");
  SVOO_REQUIRE(bh > 0 && bh <= 65535 && n > 0 && j > 0, SVOO_ERR_INVALID_ARG, "svoo_cocluster_assign: bad dims");
  SVOO_REQUIRE(jpad >= j && jpad % kAssignChunk == 0, SVOO_ERR_INVALID_ARG,
               "svoo_cocluster_assign: jpad=%d must be >= j and a multiple of %d", jpad, kAssignChunk);
  return assign_launch(x, e_hi, e_lo, labels, bh, n, j, jpad, (hipStream_t)stream);
}

// Workspace layout of svoo_co_cluster (each region 256-byte aligned):
//   e_hi, e_lo   [bh][jpad_max][128] bf16
//   counts       [bh][nchunks][kmax] int32   (cluster-sort scratch)
//   sums_k       [bh][kc][128] fp64          (key-centroid sums, kept across iterations)
//   sorted_lab   [bh][n] int32
//   sums_q       [bh][qc][128] fp64          (query-centroid sums)
//   changes      [bh * n] int2               (label changes of one assignment: token, old << 16 | new)
//   nchanges     2 int32, 256 bytes apart    (change counters, key and query side)
//   e16          [bh][jpad_max][128] fp16    (the certified single-pass copy of E)
//   fb_list      [bh][n] int32               (tokens the fp16 pass left to the hi + lo kernel)
//   stats        2 x [bh] x 256 B + 4 x [bh] (fallback and pruning-list counts 256 bytes apart, max |2^t E -
//                                            E16|, max |E16|, max row change of E, the fp16 scale t)
//   eold_k/q     [bh][jpad_k/q][128] fp64    (E of the previous pass of each side, for the pruning test)
//   delta_k/q    [bh][jpad_k/q] fp32         (per-row change of E since that pass)
//   bnd_k/q      [3][bh][n] fp32             (per-token pruning bounds of each side)
//   plist        [bh][n] int32               (tokens the pruning test left to the assignment pass)
// and for the key side's candidate pass (qc <= 128 only; bnd_k's first plane holds the radius of each
// label-sorted position):
//   praw_k       [bh][jpad_k][128] bf16      (raw key-centroid profiles)
//   inv_k        [bh][jpad_k] fp64, nrm_k [bh][jpad_k] fp32   (1 / |praw|, |P|^2)
//   trad_k       [bh][jpad_k] fp32 bits      (cluster radii)
//   lists_k      [bh][jpad_k][kCandList] int16, list_n_k [bh][jpad_k] int32   (candidate lists)
//   kslab        [bh][n] int32               (the key side's sorted labels, the candidate pass's anchors)
//   trad2_k, tused_k [bh][jpad_k] fp32 bits  (radii recorded by a pass; the radius each list was built for)
struct CoClusterWs {
  size_t e_off, counts_off, sums_off, slab_off, sums_q_off, changes_off, nchanges_off, e16_off, fb_off, stats_off,
      eold_k_off, eold_q_off, delta_k_off, delta_q_off, bnd_k_off, bnd_q_off, plist_off, praw_off, inv_off, nrm_off,
      trad_off, lists_off, listn_off, kslab_off, trad2_off, tused_off, total;
};

static CoClusterWs co_cluster_layout(int bh, int n, int qc, int kc) {
  auto al = [](size_t v) { return (v + 255) / 256 * 256; };
  const int kmax = qc > kc ? qc : kc;
  const int jpad = pad_to(kmax, kAssignChunk);
  const int nch = (n + 1023) / 1024;
  CoClusterWs w;
  w.e_off = 0;
  size_t e_bytes = al((size_t)bh * jpad * 128 * sizeof(uint16_t));
  w.counts_off = 2 * e_bytes;
  w.sums_off = w.counts_off + al((size_t)bh * kmax * nch * sizeof(int32_t));
  w.slab_off = w.sums_off + al((size_t)bh * kc * 128 * sizeof(double));
  w.sums_q_off = w.slab_off + al((size_t)bh * n * sizeof(int32_t));
  w.changes_off = w.sums_q_off + al((size_t)bh * qc * 128 * sizeof(double));
  w.nchanges_off = w.changes_off + al((size_t)bh * n * sizeof(int2));
  w.e16_off = w.nchanges_off + al(2 * kCounterStride * sizeof(int32_t));
  w.fb_off = w.e16_off + e_bytes;
  w.stats_off = w.fb_off + al((size_t)bh * n * sizeof(int32_t));
  const int jk = pad_to(kc, kAssignChunk), jq = pad_to(qc, kAssignChunk);
  w.eold_k_off = w.stats_off + al((size_t)(2 * kCounterStride + 5) * bh * sizeof(uint32_t));
  w.eold_q_off = w.eold_k_off + al((size_t)bh * jk * 128 * sizeof(double));
  w.delta_k_off = w.eold_q_off + al((size_t)bh * jq * 128 * sizeof(double));
  w.delta_q_off = w.delta_k_off + al((size_t)bh * jk * sizeof(float));
  w.bnd_k_off = w.delta_q_off + al((size_t)bh * jq * sizeof(float));
  w.bnd_q_off = w.bnd_k_off + al((size_t)3 * bh * n * sizeof(float));
  w.plist_off = w.bnd_q_off + al((size_t)3 * bh * n * sizeof(float));
  w.praw_off = w.plist_off + al((size_t)bh * n * sizeof(int32_t));
  const bool cand = qc <= kCandMaxKp;
  w.inv_off = w.praw_off + (cand ? al((size_t)bh * jk * 128 * sizeof(uint16_t)) : 0);
  w.nrm_off = w.inv_off + (cand ? al((size_t)bh * jk * sizeof(double)) : 0);
  w.trad_off = w.nrm_off + (cand ? al((size_t)bh * jk * sizeof(float)) : 0);
  w.lists_off = w.trad_off + (cand ? al((size_t)bh * jk * sizeof(uint32_t)) : 0);
  w.listn_off = w.lists_off + (cand ? al((size_t)bh * jk * kCandList * sizeof(int16_t)) : 0);
  w.kslab_off = w.listn_off + (cand ? al((size_t)bh * jk * sizeof(int32_t)) : 0);
  w.trad2_off = w.kslab_off + (cand ? al((size_t)bh * n * sizeof(int32_t)) : 0);
  w.tused_off = w.trad2_off + (cand ? al((size_t)bh * jk * sizeof(uint32_t)) : 0);
  w.total = w.tused_off + (cand ? al((size_t)bh * jk * sizeof(uint32_t)) : 0);
  return w;
}

extern "C" size_t svoo_co_cluster_workspace_size(int bh, int n, int qc, int kc, int d) {
  (void)d;
  if (bh <= 0 || n <= 0 || qc <= 0 || kc <= 0) return 256;
  return co_cluster_layout(bh, n, qc, kc).total;
}

extern "C" int svoo_co_cluster(const uint16_t* q, const uint16_t* k, int bh, int n, int d, int qc, int kc,
                               int max_iters, uint16_t* q_cent, uint16_t* k_cent, int32_t* q_labels,
                               int32_t* k_labels, int32_t* q_sizes, int32_t* k_sizes, int32_t* q_sorted_idx,
                               int32_t* k_sorted_idx, int32_t* q_offsets, int32_t* k_offsets, void* workspace,
                               size_t ws_bytes, void* stream) {
  SVOO_REQUIRE(q && k && q_cent && k_cent && q_labels && k_labels && q_sizes && k_sizes && q_sorted_idx &&
                   k_sorted_idx && q_offsets && k_offsets,
               SVOO_ERR_INVALID_ARG, "svoo_co_cluster: null pointer");
  SVOO_REQUIRE_HEAD_DIM(d, "svoo_co_cluster");
  SVOO_REQUIRE(bh > 0 && bh <= 65535 && n > 0 && qc > 0 && kc > 0, SVOO_ERR_INVALID_ARG,
               "svoo_co_cluster: bad dims bh=%d n=%d qc=%d kc=%d", bh, n, qc, kc);
  SVOO_REQUIRE(qc <= kMaxClusters && kc <= kMaxClusters, SVOO_ERR_UNSUPPORTED,
               "svoo_co_cluster: cluster counts above %d", kMaxClusters);
  SVOO_REQUIRE(max_iters >= 1, SVOO_ERR_INVALID_ARG, "svoo_co_cluster: max_iters=%d must be >= 1", max_iters);
  SVOO_REQUIRE((long long)bh * n * 128 < (1ll << 40) && (long long)bh * n < (1ll << 31), SVOO_ERR_UNSUPPORTED,
               "svoo_co_cluster: too large");
  const CoClusterWs lay = co_cluster_layout(bh, n, qc, kc);
  SVOO_REQUIRE(workspace && ws_bytes >= lay.total, SVOO_ERR_WORKSPACE, "svoo_co_cluster: workspace %zu < %zu",
               ws_bytes, lay.total);
  hipStream_t s = (hipStream_t)stream;
  char* base = (char*)workspace;
  const size_t e_bytes = (lay.counts_off) / 2;
  uint16_t* e_hi = (uint16_t*)(base + lay.e_off);
  uint16_t* e_lo = (uint16_t*)(base + lay.e_off + e_bytes);
  int32_t* counts = (int32_t*)(base + lay.counts_off);
  double* sums_k = (double*)(base + lay.sums_off);
  double* sums_q = (double*)(base + lay.sums_q_off);
  int32_t* slab = (int32_t*)(base + lay.slab_off);
  int2* changes = (int2*)(base + lay.changes_off);
  int32_t* nch = (int32_t*)(base + lay.nchanges_off);
  uint16_t* e16 = (uint16_t*)(base + lay.e16_off);
  int32_t* fb_list = (int32_t*)(base + lay.fb_off);
  uint32_t* stats = (uint32_t*)(base + lay.stats_off);
  int32_t* fb_count = (int32_t*)stats;  // head b at fb_count[b * kCounterStride]
  int32_t* list_count = fb_count + (size_t)kCounterStride * bh;
  uint32_t* err_max = stats + (size_t)2 * kCounterStride * bh;
  uint32_t* norm_max = err_max + bh;
  uint32_t* delta_max = norm_max + bh;
  int32_t* t_head = (int32_t*)(delta_max + bh);
  uint32_t* nu_bits = (uint32_t*)(t_head + bh);
  const size_t stats_words = (size_t)(2 * kCounterStride + 5) * bh;
  double* eold_k = (double*)(base + lay.eold_k_off);
  double* eold_q = (double*)(base + lay.eold_q_off);
  float* delta_k = (float*)(base + lay.delta_k_off);
  float* delta_q = (float*)(base + lay.delta_q_off);
  float* bnd_k = (float*)(base + lay.bnd_k_off);
  float* bnd_q = (float*)(base + lay.bnd_q_off);
  int32_t* plist = (int32_t*)(base + lay.plist_off);
  uint16_t* praw_k = (uint16_t*)(base + lay.praw_off);
  double* inv_k = (double*)(base + lay.inv_off);
  float* nrm_k = (float*)(base + lay.nrm_off);
  uint32_t* trad_k = (uint32_t*)(base + lay.trad_off);
  int16_t* lists_k = (int16_t*)(base + lay.lists_off);
  int32_t* listn_k = (int32_t*)(base + lay.listn_off);
  int32_t* kslab = (int32_t*)(base + lay.kslab_off);
  uint32_t* trad2_k = (uint32_t*)(base + lay.trad2_off);
  uint32_t* tused_k = (uint32_t*)(base + lay.tused_off);
  // the key side's candidate passes: the first measures the radii (radius kernel); later ones build their lists
  // from the radii the previous pass recorded, widened by kCandRadiusGrowth
  int key_cand_pass = 0;
  uint32_t* t_prev = trad_k;
  uint32_t* t_rec = trad2_k;
  const bool key_cand = key_candidates_enabled(qc, kc);
  const bool prune_q = query_prune_enabled();
  // changed tokens above which an iteration recounts every cluster instead of moving the changed ones
  const int limit = (int)((long long)bh * n / 32);
  const int jpad_k = pad_to(kc, kAssignChunk), jpad_q = pad_to(qc, kAssignChunk);
  int rc = svoo_zero_f64(sums_k, (long long)bh * kc * 128, s);
  if (!rc) rc = svoo_zero_f64(sums_q, (long long)bh * qc * 128, s);
  if (!rc) rc = svoo_zero_i32(nch, 2 * kCounterStride, s);
  // the per-pass counters start at zero; each side's finalize clears them again for the next side's prep
  if (!rc) rc = svoo_zero_i32((int32_t*)stats, (long long)stats_words, s);
  // One side of an iteration: profiles of x's tokens live in the other side's centroid space.
  // A full iteration sorts the labels and sums every cluster (sums zero on entry, kept on exit); an
  // incremental one lists the tokens whose label changed and moves only their rows between the kept fp64
  // sums (the finalize resets the counter).
  // With prune (fp16 path only) the side keeps per-token bounds: from its second pass on, the tokens whose
  // label provably cannot change are skipped (cocluster_prune_kernel) and the pass runs on the rest.
  auto side = [&](const uint16_t* x, uint16_t* cent, const uint16_t* other, int32_t* labels, int32_t* sizes,
                  int32_t* sorted_idx, int32_t* offsets, double* sums, int kx, int ko, int jpad, int32_t* cnt,
                  bool first, bool prune, double* eold, float* delta, float* bnd, bool cand) -> int {
    int r;
    // sorted labels of this side's sorts; the key side keeps its own while the candidate pass runs (they are
    // its anchors)
    int32_t* sl = cand ? kslab : slab;
    // The certified fp16 pass needs the fp16 copy of E, which the fp64-MFMA prep writes (profile widths up
    // to kPmMaxKp); wider profiles run the hi + lo kernel on every token.
    const bool fp16 = ko <= kPmMaxKp;
    const bool pr = fp16 && prune;
    // candidate pass: from the second iteration on, over the label order of the last sort
    const bool cp = cand && fp16 && ko <= kCandMaxKp && !first;
    if ((r = prep_launch(cent, other, e_hi, e_lo, nullptr, bh, kx, ko, jpad, s, fp16 ? e16 : nullptr, err_max,
                         norm_max, pr ? eold : nullptr, delta, delta_max, t_head, first ? 0 : 1,
                         cp ? praw_k : nullptr, cp ? inv_k : nullptr, cp ? nrm_k : nullptr)))
      return r;
    int2* chg = first ? nullptr : changes;
    int32_t* nc = first ? nullptr : cnt;
    if (cp) {
      const dim3 tgrid((n + kCandBlockTok - 1) / kCandBlockTok, bh);
      float* pos_t = bnd;  // plane 0
      // nu in a launch of its own: from the prep's blocks, 10^4 atomics on one word per head cost ~50 us
      hipLaunchKernelGGL(cocluster_nu_kernel, dim3(1, bh), dim3(256), 0, s, nrm_k, kx, jpad, nu_bits);
      if ((r = check_launch("svoo_co_cluster (nu)"))) return r;
      const bool measure = key_cand_pass++ == 0;
      if (measure) {
        if ((r = svoo_zero_i32((int32_t*)t_prev, (long long)bh * jpad, s))) return r;
        hipLaunchKernelGGL(cocluster_radius_kernel, tgrid, dim3(256), 0, s, x, other, e_hi, e_lo, nrm_k, nu_bits,
                           err_max, norm_max, t_head, sorted_idx, sl, n, kx, jpad, ko, pos_t, t_prev);
        if ((r = check_launch("svoo_co_cluster (radius)"))) return r;
      }
      hipLaunchKernelGGL(cocluster_lists_kernel, dim3(jpad / 32, bh), dim3(256), 0, s, praw_k, inv_k, nrm_k, t_prev,
                         measure ? 1.0f : kCandRadiusGrowth, measure ? 0.0f : kCandRadiusPad, kx, jpad, lists_k,
                         listn_k, tused_k, measure ? nullptr : t_rec);
      if ((r = check_launch("svoo_co_cluster (lists)"))) return r;
      if (measure) {
        hipLaunchKernelGGL(cocluster_score_kernel<false>, tgrid, dim3(256), 0, s, x, e_hi, e_lo, lists_k, listn_k, pos_t,
                           sl, err_max, norm_max, t_head, sorted_idx, labels, n, kx, jpad, changes, cnt, fb_list,
                           fb_count, other, ko, nrm_k, nu_bits, tused_k, t_rec);
      } else {
        hipLaunchKernelGGL(cocluster_score_kernel<true>, tgrid, dim3(256), 0, s, x, e_hi, e_lo, lists_k, listn_k, pos_t,
                           sl, err_max, norm_max, t_head, sorted_idx, labels, n, kx, jpad, changes, cnt, fb_list,
                           fb_count, other, ko, nrm_k, nu_bits, tused_k, t_rec);
        std::swap(t_prev, t_rec);
      }
      if ((r = check_launch("svoo_co_cluster (candidates)"))) return r;
      r = assign_launch(x, e_hi, e_lo, labels, bh, n, kx, jpad, s, changes, cnt, fb_list, fb_count, true);
    } else if (pr && !first) {
      hipLaunchKernelGGL(cocluster_prune_kernel, dim3((n + 256 * kPruneSub - 1) / (256 * kPruneSub), bh), dim3(256),
                         0, s, labels, bnd, delta, delta_max, n, jpad, plist, list_count);
      if ((r = check_launch("svoo_co_cluster (prune)"))) return r;
      r = assign16_launch(x, e16, e_hi, e_lo, err_max, norm_max, labels, bh, n, kx, jpad, fb_list, fb_count, s, chg,
                          nc, bnd, t_head, plist, list_count);
    } else if (fp16) {
      r = assign16_launch(x, e16, e_hi, e_lo, err_max, norm_max, labels, bh, n, kx, jpad, fb_list, fb_count, s, chg,
                          nc, pr ? bnd : nullptr, t_head);
    } else {
      r = assign_launch(x, e_hi, e_lo, labels, bh, n, kx, jpad, s, chg, nc);
    }
    if (r) return r;
    if (first) {
      if ((r = svoo_cluster_sort_impl(labels, bh, n, kx, sorted_idx, sizes, offsets, sl, counts, nullptr, s)))
        return r;
      return svoo_centroid_update_impl(x, sorted_idx, sl, sizes, cent, cent, bh, n, kx, sums, s, 1,
                                       (int32_t*)stats, (long long)stats_words);
    }
    // More changed tokens than `limit` (a share of all the tokens at which both updates take about the same
    // time at the Wan shapes): recount every cluster from the sorted labels (the guarded sort, which returns at
    // once otherwise, also clears the sums); else move the changed tokens.  The choice is made on the device
    // from the count, by the sort's kernels and inside the one move launch.
    if ((r = svoo_cluster_sort_impl(labels, bh, n, kx, sorted_idx, sizes, offsets, sl, counts, nullptr, s, cnt,
                                    limit, sums, (long long)bh * kx * 128)))
      return r;
    return svoo_centroid_move_impl(x, sorted_idx, sl, changes, cnt, sums, sizes, cent, cent, bh, n, kx, limit, s,
                                   (int32_t*)stats, (long long)stats_words);
  };
  // Iteration 1 recounts every cluster from the sorted labels.  Later iterations list the tokens whose label
  // changed; with more than `limit` of them (after a random start, iteration 2 moves 30-90% of the tokens at the
  // Wan2.1-14B 720p shape, which the per-token fp64 atomics of the incremental update handle ten times slower)
  // the sorted recount runs instead, chosen on the device.
  for (int it = 0; it < max_iters && rc == SVOO_OK; ++it) {
    if ((rc = side(k, k_cent, q_cent, k_labels, k_sizes, k_sorted_idx, k_offsets, sums_k, kc, qc, jpad_k, nch,
                   it == 0, kPruneKeys, eold_k, delta_k, bnd_k, key_cand)))
      break;
    if ((rc = side(q, q_cent, k_cent, q_labels, q_sizes, q_sorted_idx, q_offsets, sums_q, qc, kc, jpad_q,
                   nch + kCounterStride, it == 0, prune_q, eold_q, delta_q, bnd_q, false)))
      break;
  }
  // The stable sort of the final labels (the first iteration's sort already is when max_iters == 1).
  // The two sides' final sorts are independent: one set of three launches, the query side's counts in the change
  // list's buffer (consumed by now); their sorted labels are not needed.
  if (rc == SVOO_OK && max_iters > 1) {
    if (svoo_cluster_sort_workspace_size(bh, n, qc) <= (size_t)bh * n * sizeof(int2)) {
      rc = svoo_cluster_sort2_impl(k_labels, kc, k_sorted_idx, k_sizes, k_offsets, nullptr, counts, q_labels, qc,
                                   q_sorted_idx, q_sizes, q_offsets, nullptr, (int32_t*)changes, bh, n, s);
    } else {
      rc = svoo_cluster_sort_impl(k_labels, bh, n, kc, k_sorted_idx, k_sizes, k_offsets, nullptr, counts, nullptr, s);
      if (!rc)
        rc = svoo_cluster_sort_impl(q_labels, bh, n, qc, q_sorted_idx, q_sizes, q_offsets, nullptr, counts, nullptr, s);
    }
  }
  return rc;
}
