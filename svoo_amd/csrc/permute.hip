// Row gather / scatter along the token axis.  Each row (256 B for D=128 bf16) is moved by 16 lanes
// with one 16-byte load and one 16-byte store each, so every row is a fully coalesced 256 B
// transaction; a 256-thread block moves 16 rows.  Pure HBM traffic: read once, write once, both
// non-temporal (streamed: neither side is read again by this pass).
#include "svoo_common.h"

namespace svoo {

// One step of 16 rows per block (more for rows under 256 B, one step of 256 threads): many small blocks keep more rows in flight across the chip than
// fewer blocks that loop (64 rows per block measured 8-12% slower at the C3 size).
constexpr int kRowsPerBlock = 16;

// y[b][s] = x[b][idx[b][s]]  for s < n_out (x has n_in rows per b).
__global__ void __launch_bounds__(256) permute_rows_kernel(const u32x4_t* __restrict__ x, const int32_t* __restrict__ idx,
                                                           u32x4_t* __restrict__ y, int n_in, int n_out, int vec_per_row,
                                                           int32_t* __restrict__ err) {
  const int b = blockIdx.y;
  const int rows_per_step = blockDim.x / vec_per_row;
  const int rpb = max(kRowsPerBlock, rows_per_step);  // rows of this block
  const int sub = threadIdx.x / vec_per_row, v = threadIdx.x % vec_per_row;
  const int r0 = blockIdx.x * rpb;
  const int32_t* ib = idx + (size_t)b * n_out;
  const u32x4_t* xb = x + (size_t)b * n_in * vec_per_row;
  u32x4_t* yb = y + (size_t)b * n_out * vec_per_row;
  if (sub >= rows_per_step) return;
  for (int r = r0 + sub; r < min(r0 + rpb, n_out); r += rows_per_step) {
    int src = ib[r];
    if ((unsigned)src >= (unsigned)n_in) {
      if (err) atomicOr(err, 1);
      src = 0;
    }
    __builtin_nontemporal_store(__builtin_nontemporal_load(&xb[(size_t)src * vec_per_row + v]), &yb[(size_t)r * vec_per_row + v]);
  }
}

__global__ void __launch_bounds__(256) permute_rows2_kernel(const u32x4_t* __restrict__ x0, const u32x4_t* __restrict__ x1,
                                                            const int32_t* __restrict__ idx, u32x4_t* __restrict__ y0,
                                                            u32x4_t* __restrict__ y1, int n, int vec_per_row,
                                                            int32_t* __restrict__ err) {
  const int b = blockIdx.y;
  const int rows_per_step = blockDim.x / vec_per_row;
  const int rpb = max(kRowsPerBlock, rows_per_step);  // rows of this block
  const int sub = threadIdx.x / vec_per_row, v = threadIdx.x % vec_per_row;
  const int r0 = blockIdx.x * rpb;
  const size_t base = (size_t)b * n * vec_per_row;
  const int32_t* ib = idx + (size_t)b * n;
  if (sub >= rows_per_step) return;
  for (int r = r0 + sub; r < min(r0 + rpb, n); r += rows_per_step) {
    int src = ib[r];
    if ((unsigned)src >= (unsigned)n) {
      if (err) atomicOr(err, 1);
      src = 0;
    }
    const size_t so = base + (size_t)src * vec_per_row + v, d = base + (size_t)r * vec_per_row + v;
    const u32x4_t a = __builtin_nontemporal_load(&x0[so]);
    const u32x4_t c = __builtin_nontemporal_load(&x1[so]);
    __builtin_nontemporal_store(a, &y0[d]);
    __builtin_nontemporal_store(c, &y1[d]);
  }
}

// x[b][idx[b][s]] = y[b][s]
__global__ void __launch_bounds__(256) unpermute_rows_kernel(const u32x4_t* __restrict__ y, const int32_t* __restrict__ idx,
                                                             u32x4_t* __restrict__ x, int n, int vec_per_row,
                                                             int32_t* __restrict__ err) {
  const int b = blockIdx.y;
  const int rows_per_step = blockDim.x / vec_per_row;
  const int rpb = max(kRowsPerBlock, rows_per_step);  // rows of this block
  const int sub = threadIdx.x / vec_per_row, v = threadIdx.x % vec_per_row;
  const int r0 = blockIdx.x * rpb;
  const size_t base = (size_t)b * n * vec_per_row;
  const int32_t* ib = idx + (size_t)b * n;
  if (sub >= rows_per_step) return;
  for (int r = r0 + sub; r < min(r0 + rpb, n); r += rows_per_step) {
    const int dst = ib[r];
    if ((unsigned)dst >= (unsigned)n) {
      if (err) atomicOr(err, 1);
      continue;
    }
    __builtin_nontemporal_store(__builtin_nontemporal_load(&y[base + (size_t)r * vec_per_row + v]), &x[base + (size_t)dst * vec_per_row + v]);
  }
}

// x[b / heads][idx[b][s]][b % heads] = y[b][s]: scatter into the [B, S, H, D] (= [B, S, H*D]) layout the
// attention processor returns, fusing the unpermute with the final transpose.
__global__ void __launch_bounds__(256) unpermute_rows_bshd_kernel(const u32x4_t* __restrict__ y,
                                                                  const int32_t* __restrict__ idx,
                                                                  u32x4_t* __restrict__ x, int n, int heads,
                                                                  int vec_per_row) {
  const int b = blockIdx.y;
  const int bb = b / heads, hh = b % heads;
  const int rows_per_step = blockDim.x / vec_per_row;
  const int rpb = max(kRowsPerBlock, rows_per_step);  // rows of this block
  const int sub = threadIdx.x / vec_per_row, v = threadIdx.x % vec_per_row;
  const int r0 = blockIdx.x * rpb;
  const int32_t* ib = idx + (size_t)b * n;
  const u32x4_t* yb = y + (size_t)b * n * vec_per_row;
  if (sub >= rows_per_step) return;
  for (int r = r0 + sub; r < min(r0 + rpb, n); r += rows_per_step) {
    const int dst = ib[r];
    if ((unsigned)dst >= (unsigned)n) continue;
    __builtin_nontemporal_store(__builtin_nontemporal_load(&yb[(size_t)r * vec_per_row + v]), &x[(((size_t)bb * n + dst) * heads + hh) * vec_per_row + v]);
  }
}

}  // namespace svoo

using namespace svoo;

static int row_blocks(int n, int row_bytes) {
  const int rpb = std::max(kRowsPerBlock, 256 / (row_bytes / 16));
  return (n + rpb - 1) / rpb;
}

static int check_rows(int bh, int n, int row_bytes, const char* what) {
  SVOO_REQUIRE(bh > 0 && n >= 0, SVOO_ERR_INVALID_ARG, "%s: bad dims bh=%d n=%d", what, bh, n);
  SVOO_REQUIRE(row_bytes > 0 && row_bytes % 16 == 0 && row_bytes / 16 <= 256 && 256 % (row_bytes / 16) == 0,
               SVOO_ERR_UNSUPPORTED, "%s: row_bytes=%d must be 16*2^i <= 4096", what, row_bytes);
  SVOO_REQUIRE(bh <= 65535, SVOO_ERR_UNSUPPORTED, "%s: bh=%d exceeds grid limit", what, bh);
  return SVOO_OK;
}

int svoo_permute_rows_err(const void* x, const int32_t* idx, void* y, int bh, int n_in, int n_out, int row_bytes,
                          int32_t* err, hipStream_t stream) {
  if (int rc = check_rows(bh, n_out, row_bytes, "svoo_permute_rows")) return rc;
  if (n_out == 0) return SVOO_OK;
  SVOO_REQUIRE(x && idx && y && n_in > 0, SVOO_ERR_INVALID_ARG, "svoo_permute_rows: null pointer or n_in=0");
  dim3 grid(row_blocks(n_out, row_bytes), bh);
  hipLaunchKernelGGL(permute_rows_kernel, grid, dim3(256), 0, stream, (const u32x4_t*)x, idx, (u32x4_t*)y, n_in,
                     n_out, row_bytes / 16, err);
  return check_launch("svoo_permute_rows");
}

extern "C" int svoo_permute_rows(const void* x, const int32_t* idx, void* y, int bh, int n_in, int n_out,
                                 int row_bytes, void* stream) {
  return svoo_permute_rows_err(x, idx, y, bh, n_in, n_out, row_bytes, nullptr, (hipStream_t)stream);
}

extern "C" int svoo_permute_rows2(const void* x0, const void* x1, const int32_t* idx, void* y0, void* y1, int bh,
                                  int n, int row_bytes, void* stream) {
  if (int rc = check_rows(bh, n, row_bytes, "svoo_permute_rows2")) return rc;
  if (n == 0) return SVOO_OK;
  SVOO_REQUIRE(x0 && x1 && idx && y0 && y1, SVOO_ERR_INVALID_ARG, "svoo_permute_rows2: null pointer");
  dim3 grid(row_blocks(n, row_bytes), bh);
  hipLaunchKernelGGL(permute_rows2_kernel, grid, dim3(256), 0, (hipStream_t)stream, (const u32x4_t*)x0,
                     (const u32x4_t*)x1, idx, (u32x4_t*)y0, (u32x4_t*)y1, n, row_bytes / 16, (int32_t*)nullptr);
  return check_launch("svoo_permute_rows2");
}

extern "C" int svoo_unpermute_rows(const void* y, const int32_t* idx, void* x, int bh, int n, int row_bytes,
                                   void* stream) {
  if (int rc = check_rows(bh, n, row_bytes, "svoo_unpermute_rows")) return rc;
  if (n == 0) return SVOO_OK;
  SVOO_REQUIRE(x && idx && y, SVOO_ERR_INVALID_ARG, "svoo_unpermute_rows: null pointer");
  dim3 grid(row_blocks(n, row_bytes), bh);
  hipLaunchKernelGGL(unpermute_rows_kernel, grid, dim3(256), 0, (hipStream_t)stream, (const u32x4_t*)y, idx,
                     (u32x4_t*)x, n, row_bytes / 16, (int32_t*)nullptr);
  return check_launch("svoo_unpermute_rows");
}

extern "C" int svoo_unpermute_rows_bshd(const void* y, const int32_t* idx, void* x, int bh, int n, int heads,
                                        int row_bytes, void* stream) {
  if (int rc = check_rows(bh, n, row_bytes, "svoo_unpermute_rows_bshd")) return rc;
  SVOO_REQUIRE(heads > 0 && bh % heads == 0, SVOO_ERR_INVALID_ARG, "svoo_unpermute_rows_bshd: bh=%d heads=%d", bh,
               heads);
  if (n == 0) return SVOO_OK;
  SVOO_REQUIRE(x && idx && y, SVOO_ERR_INVALID_ARG, "svoo_unpermute_rows_bshd: null pointer");
  dim3 grid(row_blocks(n, row_bytes), bh);
  hipLaunchKernelGGL(unpermute_rows_bshd_kernel, grid, dim3(256), 0, (hipStream_t)stream, (const u32x4_t*)y, idx,
                     (u32x4_t*)x, n, heads, row_bytes / 16);
  return check_launch("svoo_unpermute_rows_bshd");
}
