// HBM-bound helpers of the closed-form fit: the row-block transpose that turns row-major samples
// [rows, cols] into the K-contiguous operand [cols, rows] of rf_gram_accumulate, with the columns'
// sums per 64-row tile as a by-product, and the fixed-order fp64 fold of those sums.
#include "rf_common.h"

namespace rf {
namespace {

constexpr int TT = 64;                            // transpose tile: 64 rows x 64 columns

struct TransposeArgs {
  const uint16_t* src;
  int64_t ld_src, rows;
  int cols;
  uint16_t* dst;          // [cols, ld_dst]: output row c = source column c
  int64_t ld_dst;
  const float* shift;     // [cols] fp32 or null (no centring)
  const int* lo_row;      // [cols]: row of dst_lo receiving column c's middle part, or -1; null with shift null
  uint16_t* dst_lo;       // [2 n_centred, ld_dst]: middle parts in rows [0, n_centred), low parts after them
  int64_t lo_gap;         // n_centred: row offset of a column's low part from its middle part
  float* partial;         // [tiles, cols] column sums per 64-row tile, or null
  float* partial_sq;      // [tiles, cols] column sums of squares per 64-row tile, or null
};

// Block = 4 waves, wave w one 64 x 64 tile: source rows r0 .. r0 + 63, columns c0 = 256 blockIdx.y + 64 w ..
// + 63. Lane l = 8 i + j holds the 8 x 8 piece at rows 8 i .., columns 8 j .. in eight 16-byte registers and
// transposes it in registers (no LDS): its 8 output rows (source columns 8 j + c) get 16 bytes each (source
// rows 8 i .. + 7). A wave's loads and stores then move whole 128-byte lines: per instruction 8 source
// rows x 128 bytes, and 8 output rows x 128 bytes (the 8 lanes of one j). Rows at or past `rows` give
// zeros, so padded output columns are zero.
// Without a shift the values are copied bit for bit. With one, column c's value d = x - shift[c] (fp32)
// is written as hi = bf16(d) and, if lo_row[c] >= 0, mid = bf16(d - hi) into row lo_row[c] of dst_lo and
// lo = bf16(d - hi - mid) into row lo_row[c] + lo_gap: each remainder is exact in fp32 and the last one
// has at most 8 significant bits, so hi + mid + lo == d exactly and a Gram product over [hi rows; mid and
// lo rows] gives the products of the centred fp32 values. The sums (and squares) of d over a 64-row tile:
// each 16-row group in row order (lane 8 (2g + 1) + j continues the chain lane 8 (2g) + j began), then the
// four groups pairwise, ((g0 + g1) + (g2 + g3)).
template <bool SHIFT>
__global__ __launch_bounds__(256) void k_transpose(TransposeArgs a) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, i = lane >> 3, j = lane & 7;
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * TT;
  const int c0 = blockIdx.y * 4 * TT + w * TT;
  if (c0 >= a.cols) return;                       // wave-uniform; no barriers here
  const int cb = c0 + 8 * j;                      // the lane's first source column
  uint4 in[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int64_t r = r0 + 8 * i + k;
    in[k] = r < a.rows ? *reinterpret_cast<const uint4*>(a.src + r * a.ld_src + cb) : make_uint4(0u, 0u, 0u, 0u);
  }
  uint16_t v[8][8], mid[8][8], lo[8][8];          // [column][row]
  float dv[8][8];                                 // the values the sums take: d, or the copied value
  int lrow[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const float sh = SHIFT ? a.shift[cb + c] : 0.f;
    lrow[c] = SHIFT ? a.lo_row[cb + c] : -1;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint16_t x = lane_of(in[k], c);
      if constexpr (SHIFT) {
        const float d = (r0 + 8 * i + k < a.rows) ? bf2f(x) - sh : 0.f;
        v[c][k] = f2bf(d);
        const float r1 = d - bf2f(v[c][k]);
        mid[c][k] = f2bf(r1);
        lo[c][k] = f2bf(r1 - bf2f(mid[c][k]));
        dv[c][k] = d;
      } else {
        v[c][k] = x;
        dv[c][k] = bf2f(x);
      }
    }
  }
  if (a.partial) {
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      // the even row block's 8 values from zero; the odd one continues that chain with its own 8
      float es = 0.f, eq = 0.f;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        es += dv[c][k];
        eq = fmaf(dv[c][k], dv[c][k], eq);
      }
      float gs = __shfl_xor(es, 8, 64), gq = __shfl_xor(eq, 8, 64);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        gs += dv[c][k];
        gq = fmaf(dv[c][k], dv[c][k], gq);
      }
      // group g's sum now sits in the lanes of row block 2 g + 1: ((g0 + g1) + (g2 + g3))
      gs += __shfl_xor(gs, 16, 64);
      gq += __shfl_xor(gq, 16, 64);
      gs += __shfl_xor(gs, 32, 64);
      gq += __shfl_xor(gq, 32, 64);
      if (i == 1) {
        const int64_t at = static_cast<int64_t>(blockIdx.x) * a.cols + cb + c;
        a.partial[at] = gs;
        if (a.partial_sq) a.partial_sq[at] = gq;
      }
    }
  }
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const int64_t orow = cb + c;
    *reinterpret_cast<uint4*>(a.dst + orow * a.ld_dst + r0 + 8 * i) =
        make_uint4(pack2(v[c][0], v[c][1]), pack2(v[c][2], v[c][3]), pack2(v[c][4], v[c][5]), pack2(v[c][6], v[c][7]));
    if (SHIFT && lrow[c] >= 0) {
      *reinterpret_cast<uint4*>(a.dst_lo + static_cast<int64_t>(lrow[c]) * a.ld_dst + r0 + 8 * i) =
          make_uint4(pack2(mid[c][0], mid[c][1]), pack2(mid[c][2], mid[c][3]), pack2(mid[c][4], mid[c][5]),
                     pack2(mid[c][6], mid[c][7]));
      *reinterpret_cast<uint4*>(a.dst_lo + (static_cast<int64_t>(lrow[c]) + a.lo_gap) * a.ld_dst + r0 + 8 * i) =
          make_uint4(pack2(lo[c][0], lo[c][1]), pack2(lo[c][2], lo[c][3]), pack2(lo[c][4], lo[c][5]),
                     pack2(lo[c][6], lo[c][7]));
    }
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
// item is one vector of one row: items 0 .. na - 1 of a row are group a's vectors (an attention layer's K
// heads, scaled by the k_norm gain), na .. na + nb - 1 group b's (its V heads): the [K | V] column layout
// of the reads GEMM; a GDN layer's q | k, v and [b | a] column ranges are groups too. d / 8 lanes take one
// item, one 16-byte chunk each, and reduce dot and norms with xor butterflies (every lane ends with the
// same sums). A block covers COS_ROWS rows; each lane group walks its items in a fixed order, and the
// block's per-thread sums are folded by a fixed tree into partial[block] = (sum over group a, over group b).
constexpr int COS_ROWS = 16;

__global__ __launch_bounds__(256) void k_read_cosine(const uint16_t* __restrict__ pred, int64_t ldp,
                                                     const uint16_t* __restrict__ tru, int64_t ldt, int64_t rows,
                                                     int na, int nb, int d, const uint16_t* __restrict__ kgain,
                                                     int gain_kind, float2* __restrict__ partial) {
  __shared__ float red[2][256];
  const int t = threadIdx.x;
  const int g = d >> 3, sub = t & (g - 1), grp = t / g, ngrp = 256 / g;
  const int per_row = na + nb, nitems = COS_ROWS * per_row;
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
    const bool is_k = hv < na;
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

// out[0] += weight * sum_j partial[j].x, and if two, out[1] += weight * sum_j partial[j].y, in fp64 and a
// fixed order (thread i sums blocks i, i + 256, ... in order, then a fixed tree over the 256 threads).
__global__ __launch_bounds__(256) void k_cosine_fold(const float2* __restrict__ partial, int64_t nblk, double weight,
                                                     double* __restrict__ out, int two) {
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
    if (two) out[1] += weight * red[1][0];
  }
}

}  // namespace
}  // namespace rf

using namespace rf;

static int launch_transpose(const char* fn, const TransposeArgs& a, int64_t rows, int64_t cols, int64_t ld_src,
                            int64_t ld_dst, hipStream_t stream) {
  if (!a.src || !a.dst) return fail(RF_EINVAL_ARG, "%s: null pointer", fn);
  const int64_t rows_out = (rows + TT - 1) / TT * TT;
  if (rows < 0 || cols <= 0 || cols % TT || cols > (1 << 24) || ld_src < cols || ld_src % 8 || ld_dst < rows_out ||
      ld_dst % 8 || rows_out / TT > (1ll << 31) - 1)
    return fail(RF_EINVAL_SHAPE, "%s: rows %lld, cols %lld (multiple of 64), ld_src %lld, ld_dst %lld "
                "(>= rows rounded up to 64)", fn, (long long)rows, (long long)cols, (long long)ld_src, (long long)ld_dst);
  if (!aligned16(a.src) || !aligned16(a.dst) || (a.dst_lo && !aligned16(a.dst_lo)))
    return fail(RF_EINVAL_SHAPE, "%s: 16-byte alignment", fn);
  if (rows == 0) return RF_OK;
  const dim3 grid(static_cast<unsigned>(rows_out / TT), static_cast<unsigned>((cols + 4 * TT - 1) / (4 * TT)));
  if (a.shift) hipLaunchKernelGGL(k_transpose<true>, grid, dim3(256), 0, stream, a);
  else hipLaunchKernelGGL(k_transpose<false>, grid, dim3(256), 0, stream, a);
  return check_launch(fn);
}

extern "C" int rf_transpose(const uint16_t* src, int64_t ld_src, int64_t rows, int64_t cols, uint16_t* dst,
                            int64_t ld_dst, float* partial, hipStream_t stream) {
  const TransposeArgs a{src, ld_src, rows, static_cast<int>(cols), dst, ld_dst, nullptr, nullptr, nullptr, 0,
                        partial, nullptr};
  return launch_transpose("rf_transpose", a, rows, cols, ld_src, ld_dst, stream);
}

extern "C" int rf_transpose_centred(const uint16_t* src, int64_t ld_src, int64_t rows, int64_t cols,
                                    const float* shift, const int32_t* lo_row, int64_t n_centred, uint16_t* dst,
                                    int64_t ld_dst, uint16_t* dst_lo, float* partial, float* partial_sq,
                                    hipStream_t stream) {
  if ((shift == nullptr) != (lo_row == nullptr) || (shift && !dst_lo))
    return fail(RF_EINVAL_ARG, "rf_transpose_centred: shift, lo_row and dst_lo go together");
  if (n_centred < 0 || n_centred > cols)
    return fail(RF_EINVAL_ARG, "rf_transpose_centred: n_centred %lld", (long long)n_centred);
  const TransposeArgs a{src, ld_src, rows, static_cast<int>(cols), dst, ld_dst, shift, lo_row, dst_lo, n_centred,
                        partial, partial_sq};
  return launch_transpose("rf_transpose_centred", a, rows, cols, ld_src, ld_dst, stream);
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
                              int64_t rows, int na, int nb, int d, const uint16_t* kgain, int gain_kind, double weight,
                              double* out, void* workspace, size_t ws_bytes, hipStream_t stream) {
  if (!pred || !truth || !out) return fail(RF_EINVAL_ARG, "rf_read_cosine: null pointer");
  const bool d_ok = d >= 8 && d <= 256 && (d & (d - 1)) == 0;
  const int64_t width = static_cast<int64_t>(na) * d + static_cast<int64_t>(nb) * d;
  if (rows < 0 || na <= 0 || nb < 0 || na > 4096 || nb > 4096 || !d_ok || ld_pred < width || ld_true < width ||
      ld_pred % 8 || ld_true % 8 || (gain_kind != 0 && gain_kind != 1))
    return fail(RF_EINVAL_SHAPE, "rf_read_cosine: rows %lld, na %d, nb %d, d %d (a power of two, 8 to 256), "
                "ld_pred %lld, ld_true %lld (>= (na + nb) d, multiples of 8), gain_kind %d", (long long)rows, na, nb,
                d, (long long)ld_pred, (long long)ld_true, gain_kind);
  if (!aligned16(pred) || !aligned16(truth)) return fail(RF_EINVAL_SHAPE, "rf_read_cosine: 16-byte alignment");
  const int64_t nblk = (rows + COS_ROWS - 1) / COS_ROWS;
  if (nblk > (1ll << 31) - 1) return fail(RF_EINVAL_SHAPE, "rf_read_cosine: rows %lld", (long long)rows);
  if (rows == 0) return RF_OK;
  if (!workspace || ws_bytes < static_cast<size_t>(nblk) * sizeof(float2))
    return fail(RF_EINVAL_ARG, "rf_read_cosine: workspace %zu bytes, needs %lld", ws_bytes,
                (long long)(nblk * static_cast<int64_t>(sizeof(float2))));
  float2* part = static_cast<float2*>(workspace);
  hipLaunchKernelGGL(k_read_cosine, dim3(static_cast<unsigned>(nblk)), dim3(256), 0, stream, pred, ld_pred, truth,
                     ld_true, rows, na, nb, d, kgain, gain_kind, part);
  if (int rc = check_launch("rf_read_cosine")) return rc;
  hipLaunchKernelGGL(k_cosine_fold, dim3(1), dim3(256), 0, stream, part, nblk, weight, out, nb > 0 ? 1 : 0);
  return check_launch("rf_read_cosine");
}
