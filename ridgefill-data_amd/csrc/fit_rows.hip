// HBM-bound helpers of the closed-form fit: the row-block transpose that turns row-major samples
// [rows, cols] into the K-contiguous operand [cols, rows] of rf_gram_accumulate, with the columns'
// sums per 64-row tile as a by-product, and the fixed-order fp64 fold of those sums.
#include "rf_common.h"

namespace rf {
namespace {

constexpr int TT = 64;                            // transpose tile: 64 rows x 64 columns

// Block = one 64 x 64 tile, 256 threads. Load: thread t takes tile row t / 4, columns (t % 4) * 16 ..
// + 15 (two 16-byte loads). Store: thread t writes output row (source column) t / 4, source rows
// (t % 4) * 16 .. + 15. Rows at or past `rows` read as zeros, so padded output columns are zero.
__global__ __launch_bounds__(256) void k_transpose(const uint16_t* __restrict__ src, int64_t ld_src, int64_t rows,
                                                   int cols, uint16_t* __restrict__ dst, int64_t ld_dst,
                                                   float* __restrict__ partial) {
  __shared__ uint16_t tile[TT][TT + 2];
  const int t = threadIdx.x;
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * TT;
  const int c0 = blockIdx.y * TT;
  {
    const int r = t >> 2, c = (t & 3) * 16;
    uint4 a = make_uint4(0u, 0u, 0u, 0u), b = a;
    if (r0 + r < rows) {
      const uint4* p = reinterpret_cast<const uint4*>(src + (r0 + r) * ld_src + c0 + c);
      a = p[0];
      b = p[1];
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      tile[r][c + e] = lane_of(a, e);
      tile[r][c + 8 + e] = lane_of(b, e);
    }
  }
  __syncthreads();
  const int oc = t >> 2, rr = (t & 3) * 16;       // output row = source column c0 + oc
  uint16_t v[16];
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    v[e] = tile[rr + e][oc];
    s += bf2f(v[e]);
  }
  uint4* q = reinterpret_cast<uint4*>(dst + static_cast<int64_t>(c0 + oc) * ld_dst + r0 + rr);
  q[0] = make_uint4(pack2(v[0], v[1]), pack2(v[2], v[3]), pack2(v[4], v[5]), pack2(v[6], v[7]));
  q[1] = make_uint4(pack2(v[8], v[9]), pack2(v[10], v[11]), pack2(v[12], v[13]), pack2(v[14], v[15]));
  if (partial) {
    // the 4 threads of one column are adjacent lanes: fixed-order pairwise sum
    s += __shfl_xor(s, 1, 64);
    s += __shfl_xor(s, 2, 64);
    if ((t & 3) == 0) partial[static_cast<int64_t>(blockIdx.x) * cols + c0 + oc] = s;
  }
}

// sums[c] += sum over tiles j of partial[j, c], in fp64, in a fixed order: 16 threads per column, thread i
// sums tiles i, i + 16, i + 32, ... in order, then the 16 partial sums are added pairwise (i with i + 8,
// then + 4, + 2, + 1). A block of 256 threads covers 16 consecutive columns.
__global__ __launch_bounds__(256) void k_colsum_fold(const float* __restrict__ partial, int64_t ntiles, int cols,
                                                     double* __restrict__ sums) {
  __shared__ double red[16][17];
  const int t = threadIdx.x, cl = t & 15, i = t >> 4;
  const int c = blockIdx.x * 16 + cl;
  double s = 0.0;
  if (c < cols)
    for (int64_t j = i; j < ntiles; j += 16) s += static_cast<double>(partial[j * cols + c]);
  red[i][cl] = s;
  __syncthreads();
  for (int h = 8; h >= 1; h >>= 1) {
    if (i < h) red[i][cl] += red[i + h][cl];
    __syncthreads();
  }
  if (i == 0 && c < cols) sums[c] += red[0][cl];
}

// Read cosines of one late layer for one held-out document (code/scripts/fit_sweep.py:307-313). A work
// item is one head vector of one row: items 0 .. hkv - 1 of a row are its K heads, hkv .. 2 hkv - 1 its V
// heads (the [K | V] column layout of the reads GEMM). d / 8 lanes take one item, one 16-byte chunk each,
// and reduce dot and norms with xor butterflies (every lane ends with the same sums). A block covers
// COS_ROWS rows; each lane group walks its items in a fixed order, and the block's per-thread sums are
// folded by a fixed tree into partial[block] = (sum of K cosines, sum of V cosines).
constexpr int COS_ROWS = 16;

__global__ __launch_bounds__(256) void k_read_cosine(const uint16_t* __restrict__ pred, int64_t ldp,
                                                     const uint16_t* __restrict__ tru, int64_t ldt, int64_t rows,
                                                     int hkv, int d, const uint16_t* __restrict__ kgain,
                                                     int gain_kind, float2* __restrict__ partial) {
  __shared__ float red[2][256];
  const int t = threadIdx.x;
  const int g = d >> 3, sub = t & (g - 1), grp = t / g, ngrp = 256 / g;
  const int per_row = 2 * hkv, nitems = COS_ROWS * per_row;
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * COS_ROWS;
  float gn[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) gn[e] = kgain ? bf2f(kgain[sub * 8 + e]) + (gain_kind ? 1.0f : 0.0f) : 1.0f;
  float ak = 0.0f, av = 0.0f;
  for (int it = grp; it < nitems; it += ngrp) {
    const int64_t r = r0 + it / per_row;
    const int hv = it % per_row;
    if (r >= rows) break;                            // items run row-major: the rest of the walk is past `rows`
    const int64_t col = static_cast<int64_t>(hv) * d + sub * 8;
    const uint4 pv = *reinterpret_cast<const uint4*>(pred + r * ldp + col);
    const uint4 tv = *reinterpret_cast<const uint4*>(tru + r * ldt + col);
    const bool is_k = hv < hkv;
    float dot = 0.0f, n1 = 0.0f, n2 = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float s = is_k ? gn[e] : 1.0f;
      const float a = bf2f(lane_of(pv, e)) * s, b = bf2f(lane_of(tv, e)) * s;
      dot += a * b;
      n1 += a * a;
      n2 += b * b;
    }
    for (int m = g >> 1; m >= 1; m >>= 1) {
      dot += __shfl_xor(dot, m);
      n1 += __shfl_xor(n1, m);
      n2 += __shfl_xor(n2, m);
    }
    const float c = dot / (fmaxf(sqrtf(n1), 1e-8f) * fmaxf(sqrtf(n2), 1e-8f));
    if (sub == 0) {
      if (is_k) ak += c;
      else av += c;
    }
  }
  red[0][t] = ak;
  red[1][t] = av;
  __syncthreads();
  for (int h = 128; h >= 1; h >>= 1) {
    if (t < h) {
      red[0][t] += red[0][t + h];
      red[1][t] += red[1][t + h];
    }
    __syncthreads();
  }
  if (t == 0) partial[blockIdx.x] = make_float2(red[0][0], red[1][0]);
}

// out[0] += weight * sum_j partial[j].x, out[1] += weight * sum_j partial[j].y, in fp64 and a fixed order
// (thread i sums blocks i, i + 256, ... in order, then a fixed tree over the 256 threads).
__global__ __launch_bounds__(256) void k_cosine_fold(const float2* __restrict__ partial, int64_t nblk, double weight,
                                                     double* __restrict__ out) {
  __shared__ double red[2][256];
  const int t = threadIdx.x;
  double sk = 0.0, sv = 0.0;
  for (int64_t j = t; j < nblk; j += 256) {
    sk += static_cast<double>(partial[j].x);
    sv += static_cast<double>(partial[j].y);
  }
  red[0][t] = sk;
  red[1][t] = sv;
  __syncthreads();
  for (int h = 128; h >= 1; h >>= 1) {
    if (t < h) {
      red[0][t] += red[0][t + h];
      red[1][t] += red[1][t + h];
    }
    __syncthreads();
  }
  if (t == 0) {
    out[0] += weight * red[0][0];
    out[1] += weight * red[1][0];
  }
}

}  // namespace
}  // namespace rf

using namespace rf;

extern "C" int rf_transpose(const uint16_t* src, int64_t ld_src, int64_t rows, int64_t cols, uint16_t* dst,
                            int64_t ld_dst, float* partial, hipStream_t stream) {
  if (!src || !dst) return fail(RF_EINVAL_ARG, "rf_transpose: null pointer");
  const int64_t rows_out = (rows + TT - 1) / TT * TT;
  if (rows < 0 || cols <= 0 || cols % TT || cols > (1 << 24) || ld_src < cols || ld_src % 8 || ld_dst < rows_out ||
      ld_dst % 8 || rows_out / TT > (1ll << 31) - 1)
    return fail(RF_EINVAL_SHAPE, "rf_transpose: rows %lld, cols %lld (multiple of 64), ld_src %lld, ld_dst %lld "
                "(>= rows rounded up to 64)", (long long)rows, (long long)cols, (long long)ld_src, (long long)ld_dst);
  if (!aligned16(src) || !aligned16(dst)) return fail(RF_EINVAL_SHAPE, "rf_transpose: 16-byte alignment");
  if (rows == 0) return RF_OK;
  hipLaunchKernelGGL(k_transpose, dim3(static_cast<unsigned>(rows_out / TT), static_cast<unsigned>(cols / TT)),
                     dim3(256), 0, stream, src, ld_src, rows, static_cast<int>(cols), dst, ld_dst, partial);
  return check_launch("rf_transpose");
}

extern "C" int rf_colsum_fold(const float* partial, int64_t ntiles, int64_t cols, double* sums, hipStream_t stream) {
  if (!partial || !sums) return fail(RF_EINVAL_ARG, "rf_colsum_fold: null pointer");
  if (ntiles < 0 || cols <= 0 || cols > (1 << 30)) return fail(RF_EINVAL_SHAPE, "rf_colsum_fold: shape");
  if (ntiles == 0) return RF_OK;
  hipLaunchKernelGGL(k_colsum_fold, dim3(static_cast<unsigned>((cols + 15) / 16)), dim3(256), 0, stream, partial,
                     ntiles, static_cast<int>(cols), sums);
  return check_launch("rf_colsum_fold");
}

extern "C" int rf_read_cosine(const uint16_t* pred, int64_t ld_pred, const uint16_t* truth, int64_t ld_true,
                              int64_t rows, int hkv, int d, const uint16_t* kgain, int gain_kind, double weight,
                              double* out, void* workspace, size_t ws_bytes, hipStream_t stream) {
  if (!pred || !truth || !out) return fail(RF_EINVAL_ARG, "rf_read_cosine: null pointer");
  if (rows < 0 || hkv <= 0 || (d != 64 && d != 128 && d != 256) || ld_pred < 2ll * hkv * d ||
      ld_true < 2ll * hkv * d || ld_pred % 8 || ld_true % 8 || (gain_kind != 0 && gain_kind != 1))
    return fail(RF_EINVAL_SHAPE, "rf_read_cosine: rows %lld, hkv %d, d %d (64, 128 or 256), ld_pred %lld, "
                "ld_true %lld (>= 2 hkv d, multiples of 8), gain_kind %d", (long long)rows, hkv, d,
                (long long)ld_pred, (long long)ld_true, gain_kind);
  if (!aligned16(pred) || !aligned16(truth)) return fail(RF_EINVAL_SHAPE, "rf_read_cosine: 16-byte alignment");
  const int64_t nblk = (rows + COS_ROWS - 1) / COS_ROWS;
  if (nblk > (1ll << 31) - 1) return fail(RF_EINVAL_SHAPE, "rf_read_cosine: rows %lld", (long long)rows);
  if (rows == 0) return RF_OK;
  if (!workspace || ws_bytes < static_cast<size_t>(nblk) * sizeof(float2))
    return fail(RF_EINVAL_ARG, "rf_read_cosine: workspace %zu bytes, needs %lld", ws_bytes,
                (long long)(nblk * static_cast<int64_t>(sizeof(float2))));
  float2* part = static_cast<float2*>(workspace);
  hipLaunchKernelGGL(k_read_cosine, dim3(static_cast<unsigned>(nblk)), dim3(256), 0, stream, pred, ld_pred, truth,
                     ld_true, rows, hkv, d, kgain, gain_kind, part);
  if (int rc = check_launch("rf_read_cosine")) return rc;
  hipLaunchKernelGGL(k_cosine_fold, dim3(1), dim3(256), 0, stream, part, nblk, weight, out);
  return check_launch("rf_read_cosine");
}
