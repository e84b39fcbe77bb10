// Shared device helpers and host error plumbing for the SVOO HIP kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/svoo_hip.h"

namespace svoo {

constexpr int kWave = 64;

// ---------------------------------------------------------------- bf16 <-> f32
__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float(((uint32_t)b) << 16); }

// Round-to-nearest-even float32 -> bfloat16 bit pattern (NaN -> quiet NaN).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)0x7fc0u;
  uint32_t lsb = (u >> 16) & 1u;
  return (uint16_t)((u + 0x7fffu + lsb) >> 16);
}

__device__ __forceinline__ float bf16_round_f32(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// ---------------------------------------------------------------- vector types for MFMA
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bf16x8_t as_bf16x8(u32x4_t v) { return __builtin_bit_cast(bf16x8_t, v); }

// 32x32x16 bf16 MFMA, fp32 accumulate.  Operand layout (wave64):
//   A[m][k]: lane m + 32*(k/8), element k%8     B[k][n]: lane n + 32*(k/8), element k%8
//   C[m][n]: lane n + 32*((m/4)%2), element (m/8)*4 + m%4
__device__ __forceinline__ f32x16_t mfma32x32x16(bf16x8_t a, bf16x8_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// 16x16x32 bf16 MFMA.  A[m][k]: lane m + 16*(k/8); C[m][n]: lane n + 16*(m/4), element m%4.
__device__ __forceinline__ f32x4_t mfma16x16x32(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// 16x16x4 fp64 MFMA.  A[i][k]: lane i + 16 k; B[k][j]: lane j + 16 k; D[i][j]: lane j + 16 (i % 4),
// element i / 4 (measured by svoo_probe_mfma_f64_layout).
typedef double f64x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ f64x4_t mfma16x16x4_f64(double a, double b, f64x4_t c) {
  return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return (uint32_t)f32_to_bf16(lo) | ((uint32_t)f32_to_bf16(hi) << 16);
}

// Two floats -> packed bf16 pair with the gfx950 conversion instruction (v_cvt_pk_bf16_f32,
// round to nearest even); same values as pack_bf16x2 for every non-NaN input.
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t cvt_pk_bf16(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t));
}

// gfx950 transposing LDS read (ds_read_b64_tr_b16).  Within each group of 16 lanes, lane i of the
// group receives element e (e = 0..3) = element i%4 of the 8 bytes read by group lane 4e + i/4.
// With group lane s addressing row (r0 + s/4), columns (c0 + 4*(s%4) .. +3) of a row-major bf16
// matrix, lane i receives rows r0..r0+3 of column c0 + i.
typedef short i16x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint2 ds_read_tr16_b64(const uint16_t* lds_ptr) {
  const i16x4_t r =
      __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4_t*)(lds_ptr));
  return __builtin_bit_cast(uint2, r);
}

// Physical 16-byte chunk of logical chunk c in row r of an LDS tile of unpadded 256-byte rows.  The
// XOR pattern makes both read patterns used here conflict-free: 16 consecutive rows at one chunk
// (MFMA A-operand rows via ds_read_b128) and 4 consecutive rows x 4 consecutive chunks (the
// transposing reads).
__device__ __forceinline__ int swz(int r, int c) { return c ^ (((r & 3) << 2) | ((r >> 2) & 3)); }

// Direct global -> LDS copy of 16 bytes per lane: lane i writes lds_base + 16 i (gfx950 LDS DMA,
// global_load_lds_dwordx4).  lds_base must be wave-uniform; completion is tracked by vmcnt.
__device__ __forceinline__ void lds_dma16(const void* src, uint16_t* lds_base) {
  __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                   (__attribute__((address_space(3))) void*)lds_base, 16, 0, 0);
}

// The same copy issued from inline assembly: 16 bytes per lane from sbase + voff (bytes) to LDS byte address
// lds + 16 * lane (sbase and lds wave-uniform).  The compiler neither sees nor counts it, so its waits for the
// kernel's own LDS reads stay exact (it treats a visible LDS DMA as an LDS event that may complete out of
// order and answers every later LDS read with lgkmcnt(0)).  The caller waits for completion explicitly
// (s_waitcnt vmcnt) before the barrier that publishes the data.  M0 needs one wait state after its write.
__device__ __forceinline__ void lds_dma16_asm(const void* sbase, uint32_t voff, uint32_t lds) {
  __asm__ volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(lds)
                   : "memory", "m0");
}
// LDS byte address of a __shared__ object, wave-uniform.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p);
}

// Max / sum of a value and its partner lane (lane ^ 32), in both lanes: one v_permlane32_swap (a VALU
// op) instead of a ds_bpermute round trip through LDS.  The swap returns {lanes 0-31 of the first operand
// with lanes 0-31 of the second in the upper half, lanes 32-63 of the first in the lower half with lanes
// 32-63 of the second}; with both operands x, each lane sees x of itself and of its partner.
__device__ __forceinline__ float xhalf_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xhalf_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// ---------------------------------------------------------------- block reductions
template <int kThreads>
__device__ __forceinline__ double block_sum_f64(double v, double* scratch) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  const int w = threadIdx.x / kWave, l = threadIdx.x % kWave;
  __syncthreads();
  if (l == 0) scratch[w] = v;
  __syncthreads();
  double t = 0.0;
#pragma unroll
  for (int i = 0; i < kThreads / kWave; ++i) t += scratch[i];
  return t;
}

template <int kThreads>
__device__ __forceinline__ float block_max_f32(float v, float* scratch) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  const int w = threadIdx.x / kWave, l = threadIdx.x % kWave;
  __syncthreads();
  if (l == 0) scratch[w] = v;
  __syncthreads();
  float t = scratch[0];
#pragma unroll
  for (int i = 1; i < kThreads / kWave; ++i) t = fmaxf(t, scratch[i]);
  return t;
}

template <int kThreads>
__device__ __forceinline__ int block_sum_i32(int v, int* scratch) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  const int w = threadIdx.x / kWave, l = threadIdx.x % kWave;
  __syncthreads();
  if (l == 0) scratch[w] = v;
  __syncthreads();
  int t = 0;
#pragma unroll
  for (int i = 0; i < kThreads / kWave; ++i) t += scratch[i];
  return t;
}

// Exclusive prefix sum over the block (int64); returns this thread's exclusive prefix and writes the total.
template <int kThreads>
__device__ __forceinline__ long long block_exclusive_scan_i64(long long v, long long* scratch, long long* total) {
  const int w = threadIdx.x / kWave, l = threadIdx.x % kWave;
  long long inc = v;
  for (int o = 1; o < kWave; o <<= 1) {
    long long n = __shfl_up(inc, o);
    if (l >= o) inc += n;
  }
  __syncthreads();
  if (l == kWave - 1) scratch[w] = inc;
  __syncthreads();
  long long base = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < kThreads / kWave; ++i) {
    if (i < w) base += scratch[i];
    tot += scratch[i];
  }
  *total = tot;
  return base + inc - v;
}

// ---------------------------------------------------------------- host side
void set_error(const char* fmt, ...);
int check_launch(const char* what);

}  // namespace svoo

#define SVOO_REQUIRE(cond, code, ...)     \
  do {                                    \
    if (!(cond)) {                        \
      ::svoo::set_error(__VA_ARGS__);     \
      return (code);                      \
    }                                     \
  } while (0)

// Head dims: rows always hold 128 elements; d (1..128) is the head dim, elements d..127 of every row are zero.
#define SVOO_REQUIRE_HEAD_DIM(d, name)                                                                    \
  SVOO_REQUIRE((d) >= 1 && (d) <= 128, SVOO_ERR_UNSUPPORTED, "%s: D=%d (head dims 1..128, rows of 128)", \
               name, (d))
