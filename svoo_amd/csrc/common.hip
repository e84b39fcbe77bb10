// Error plumbing, version and the MFMA operand-layout probe.
#include <stdarg.h>
#include <stdio.h>

#include "svoo_common.h"

namespace svoo {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return SVOO_ERR_HIP;
  }
  return SVOO_OK;
}

// Two accumulating MFMAs on index-coded operands so that C[m][n] = 64*m + n (32x32x16) and
// C[m][n] = 16*m + n (16x16x32):
//   run 1: A[m][k] = m for every k, B[k][n] = 64 (16) for k == 0 and 0 otherwise  -> 64*m (16*m)
//   run 2: A[m][k] = 1 for k == 0 and 0 otherwise, B[k][n] = n                    -> n
// Every value is a small integer, so all products and sums are exact.  The host decodes (m, n)
// from each lane/register and checks it against the C layout documented in svoo_common.h.
__global__ void probe_kernel(float* out32, float* out16) {
  const int l = threadIdx.x;
  u32x4_t a1, b1, a2, b2;
  const int h = l / 32, m = l % 32;
  // element e of lane l corresponds to k = 8*h + e.
  uint16_t av[8], bv[8], av2[8], bv2[8];
  for (int e = 0; e < 8; ++e) {
    const int k = 8 * h + e;
    av[e] = f32_to_bf16((float)m);                 // A row index is lane % 32
    bv[e] = f32_to_bf16(k == 0 ? 64.0f : 0.0f);
    av2[e] = f32_to_bf16(k == 0 ? 1.0f : 0.0f);
    bv2[e] = f32_to_bf16((float)m);                // B column index is lane % 32
  }
  for (int i = 0; i < 4; ++i) {
    a1[i] = av[2 * i] | ((uint32_t)av[2 * i + 1] << 16);
    b1[i] = bv[2 * i] | ((uint32_t)bv[2 * i + 1] << 16);
    a2[i] = av2[2 * i] | ((uint32_t)av2[2 * i + 1] << 16);
    b2[i] = bv2[2 * i] | ((uint32_t)bv2[2 * i + 1] << 16);
  }
  f32x16_t c = {};
  c = mfma32x32x16(as_bf16x8(a1), as_bf16x8(b1), c);
  c = mfma32x32x16(as_bf16x8(a2), as_bf16x8(b2), c);
  for (int r = 0; r < 16; ++r) out32[l * 16 + r] = c[r];

  // 16x16x32: lane l: m = l%16, k = 8*(l/16) + e.
  const int q = l / 16, m16 = l % 16;
  for (int e = 0; e < 8; ++e) {
    const int k = 8 * q + e;
    av[e] = f32_to_bf16((float)m16);
    bv[e] = f32_to_bf16(k == 0 ? 16.0f : 0.0f);
    av2[e] = f32_to_bf16(k == 0 ? 1.0f : 0.0f);
    bv2[e] = f32_to_bf16((float)m16);
  }
  for (int i = 0; i < 4; ++i) {
    a1[i] = av[2 * i] | ((uint32_t)av[2 * i + 1] << 16);
    b1[i] = bv[2 * i] | ((uint32_t)bv[2 * i + 1] << 16);
    a2[i] = av2[2 * i] | ((uint32_t)av2[2 * i + 1] << 16);
    b2[i] = bv2[2 * i] | ((uint32_t)bv2[2 * i + 1] << 16);
  }
  f32x4_t c4 = {};
  c4 = mfma16x16x32(as_bf16x8(a1), as_bf16x8(b1), c4);
  c4 = mfma16x16x32(as_bf16x8(a2), as_bf16x8(b2), c4);
  for (int r = 0; r < 4; ++r) out16[l * 4 + r] = c4[r];
}

// fp64 16x16x4 MFMA, index-coded as above: D[i][j] = 64 i + j when A[i][k] sits in lane i + 16 k,
// B[k][j] in lane j + 16 k, and D[i][j] in lane j + 16 (i % 4), element i / 4.
__global__ void probe_f64_kernel(double* out) {
  const int l = threadIdx.x, i = l % 16, k = l / 16;
  const double a1 = k == 0 ? (double)i : 0.0, b1 = k == 0 ? 64.0 : 0.0;
  const double a2 = k == 0 ? 1.0 : 0.0, b2 = k == 0 ? (double)i : 0.0;
  f64x4_t c = {0.0, 0.0, 0.0, 0.0};
  c = mfma16x16x4_f64(a1, b1, c);
  c = mfma16x16x4_f64(a2, b2, c);
  for (int r = 0; r < 4; ++r) out[l * 4 + r] = c[r];
}

}  // namespace svoo

extern "C" int svoo_version(void) { return 100; }

extern "C" const char* svoo_last_error(void) { return svoo::g_last_error; }

extern "C" int svoo_probe_mfma_f64_layout(double* out, void* stream) {
  SVOO_REQUIRE(out, SVOO_ERR_INVALID_ARG, "svoo_probe_mfma_f64_layout: null output");
  hipLaunchKernelGGL(svoo::probe_f64_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, out);
  return svoo::check_launch("svoo_probe_mfma_f64_layout");
}

extern "C" int svoo_probe_mfma_layout(float* out32, float* out16, void* stream) {
  SVOO_REQUIRE(out32 && out16, SVOO_ERR_INVALID_ARG, "svoo_probe_mfma_layout: null output");
  hipLaunchKernelGGL(svoo::probe_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, out32, out16);
  return svoo::check_launch("svoo_probe_mfma_layout");
}
