// The ridge solve of the closed-form fit on gfx950, all in fp64 (code/kva/ridge.py:80-105: RidgeFit solves
// W(lam) = (C + lam s I)^-1 Cxy with s = mean(diag C), by one eigendecomposition of C; this computes the same
// closed form through the inverse of C + lam s I).
//
//   k_dgemm       C = alpha A B + beta C, row-major fp64, v_mfma_f64_16x16x4f64. A workgroup of 4 wave64s
//                 computes a 128 x 128 tile over K in 16-deep blocks; each wave a 64 x 64 quarter as 4 x 4
//                 MFMA tiles (lane l feeds A[l % 16][l / 16] and B[l / 16][l % 16] and holds
//                 D[l / 16 + 4 i][l % 16] in its register pair i: the fp64 output's rows interleave, unlike the
//                 fp32 16x16x4 variant's 4 (l / 16) + i). Blocks are double-buffered in LDS (72 KB, so two
//                 workgroups share a CU and fill each other's barrier and LDS-latency gaps), the next block
//                 loaded into registers while the current one is multiplied. LDS strides: A rows of 18 doubles and B rows of 144 doubles, so
//                 the 16 rows x 2 k (A) and 16 columns x 2 k (B) of each half-wave's fragment reads fall in
//                 distinct banks. The k order of the sums is that of one pass over K in steps of 4.
//   k_spd_inv64   the inverse of a 64 x 64 symmetric positive definite block by in-place Gauss-Jordan
//                 elimination without pivoting (stable for SPD matrices), one workgroup, the matrix in
//                 registers and each step's pivot row and column exchanged through LDS.
//   the inverse   of an n x n SPD matrix (n a multiple of 64) by block recursion on [A11 A12; A21 A22]:
//                 X11 = A11^-1, T = A21 X11, S = A22 - T A12 (the Schur complement, SPD), X22 = S^-1,
//                 X21 = -X22 T, U = X11 A12 (= T^T), X11 -= U X21, X12 = X21^T -- every product a k_dgemm.
//   k_gemv_rows   out = init + alpha v M, rows summed by 4 waves in order (the bias's vector products).
//   rf_ridge_solve  per lambda: A = C + lam s I padded to a multiple of 64 with an identity block, X = A^-1,
//                 W = X[:d, :d] Cxy (k_dgemm, the dominant 2 d^2 R flops), bias = mean_y - (mean_x X) Cxy
//                 (= mean_y - mean_x W; one pass over Cxy for every lambda). Up to 8 lambdas go together:
//                 every launch of the recursion carries all of them in its grid.
#include <algorithm>

#include "rf_common.h"

namespace rf {
namespace {

typedef double f64x4 __attribute__((ext_vector_type(4)));

constexpr int DBM = 128, DBN = 128, DBK = 16;
constexpr int AST = DBK + 2;      // A block row stride in doubles (16-byte aligned rows, conflict-free reads)
constexpr int DLD = DBM * DBK / 2 / 256;   // double2 loads per thread per block and operand (A; B has the same)
constexpr int BST = DBN + 16;     // B block row stride in doubles

struct DgemmArgs {
  const double* A;
  int64_t lda;
  const double* B;
  int64_t ldb;
  double* C;
  int64_t ldc;
  int M, N, K;
  double alpha, beta;
  int64_t sa, sb, sc;     // element strides between the batch's matrices (blockIdx.y)
};

// Requires K and N even, lda / ldb even, A and B 16-byte aligned (checked by the host callers). Loads past
// M, N or K read a clamped in-bounds address and are replaced by zeros (no divergent branches in the loop).
__global__ __launch_bounds__(256, 2) void k_dgemm(DgemmArgs a) {
  __shared__ __align__(16) double As[2][DBM * AST];
  __shared__ __align__(16) double Bs[2][DBK * BST];
  const int t = threadIdx.x, lane = t & 63;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6), wm = w >> 1, wn = w & 1;
  // tile rows fastest: the blocks in flight share B's column panels (B is the large operand of the solve)
  const int tiles_m = (a.M + DBM - 1) / DBM;
  const int tn = blockIdx.x / tiles_m, tm = blockIdx.x - tn * tiles_m;
  const int m0 = tm * DBM, n0 = tn * DBN;
  const int64_t z = blockIdx.y;
  const double* __restrict__ Ag = a.A + z * a.sa;
  const double* __restrict__ Bg = a.B + z * a.sb;
  double* __restrict__ Cg = a.C + z * a.sc;
  // loader mapping: A chunk j = t + 256 i: row j / 8, k pair j % 8; B chunk j: k row j / 64, column pair j % 64
  // the zero masks are applied when the block is written to LDS, after the multiply that hides the loads
  double2 ra[DLD], rb[DLD];
  unsigned ok = 0;
  auto gload = [&](int k0) {
    ok = 0;
#pragma unroll
    for (int i = 0; i < DLD; ++i) {
      const int j = t + 256 * i;
      const int ar = j >> 3, ak = k0 + 2 * (j & 7);
      const int gr = m0 + ar;
      ok |= (gr < a.M && ak < a.K) ? 1u << i : 0u;
      ra[i] = *reinterpret_cast<const double2*>(Ag + static_cast<int64_t>(min(gr, a.M - 1)) * a.lda +
                                                min(ak, a.K - 2));
      const int bk = k0 + (j >> 6), bc = n0 + 2 * (j & 63);
      ok |= (bk < a.K && bc < a.N) ? 1u << (DLD + i) : 0u;
      rb[i] = *reinterpret_cast<const double2*>(Bg + static_cast<int64_t>(min(bk, a.K - 1)) * a.ldb +
                                                min(bc, a.N - 2));
    }
  };
  auto swrite = [&](int s) {
#pragma unroll
    for (int i = 0; i < DLD; ++i) {
      const int j = t + 256 * i;
      const bool ka = (ok >> i) & 1, kb = (ok >> (DLD + i)) & 1;
      const double2 va{ka ? ra[i].x : 0.0, ka ? ra[i].y : 0.0}, vb{kb ? rb[i].x : 0.0, kb ? rb[i].y : 0.0};
      *reinterpret_cast<double2*>(&As[s][(j >> 3) * AST + 2 * (j & 7)]) = va;
      *reinterpret_cast<double2*>(&Bs[s][(j >> 6) * BST + 2 * (j & 63)]) = vb;
    }
  };
  f64x4 acc[4][4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) acc[mt][nt] = f64x4{0.0, 0.0, 0.0, 0.0};
  const int nkb = (a.K + DBK - 1) / DBK;
  gload(0);
  swrite(0);
  __syncthreads();
  const int lr = lane & 15, lk = lane >> 4;
  for (int kb = 0; kb < nkb; ++kb) {
    const int s = kb & 1;
    if (kb + 1 < nkb) gload((kb + 1) * DBK);
    const double* as = As[s] + (wm * 64 + lr) * AST + lk;
    const double* bs = Bs[s] + lk * BST + wn * 64 + lr;
#pragma unroll
    for (int kk = 0; kk < DBK / 4; ++kk) {
      double af[4], bf[4];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) af[mt] = as[mt * 16 * AST + kk * 4];
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) bf[nt] = bs[kk * 4 * BST + nt * 16];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < 4; ++nt)
          acc[mt][nt] = __builtin_amdgcn_mfma_f64_16x16x4f64(af[mt], bf[nt], acc[mt][nt], 0, 0, 0);
    }
    if (kb + 1 < nkb) swrite(s ^ 1);                // stage s ^ 1 was last read before the previous barrier
    __syncthreads();
  }
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      const int col = n0 + wn * 64 + nt * 16 + lr;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t row = static_cast<int64_t>(m0) + wm * 64 + mt * 16 + lk + 4 * i;
        if (row < a.M && col < a.N) {
          double* c = Cg + row * a.ldc + col;
          double v = a.alpha * acc[mt][nt][i];
          if (a.beta != 0.0) v += a.beta * *c;
          *c = v;
        }
      }
    }
}

// X = A^-1 for a 64 x 64 SPD block: Gauss-Jordan elimination in place, thread t keeping row t / 4, columns
// 16 (t % 4) .. + 15 in registers. Step k: p = M[k][k]; row k /= p (M[k][k] = 1 / p); every other row i:
// M[i][j] -= M[i][k] M[k][j] (j != k), M[i][k] = -M[i][k] / p. Row k and column k as they were before the
// step are published in LDS (double-buffered by step parity, one barrier per step); the 64 steps are
// unrolled so that every register index is a constant.
__global__ __launch_bounds__(256) void k_spd_inv64(const double* __restrict__ A, int64_t lda, double* __restrict__ X,
                                                   int64_t ldx, int64_t sa, int64_t sx) {
  __shared__ double prow[2][64], pcol[2][64];
  const int t = threadIdx.x, r = t >> 2, q = t & 3, c0 = q * 16;
  A += static_cast<int64_t>(blockIdx.x) * sa;           // one block per matrix of the batch
  X += static_cast<int64_t>(blockIdx.x) * sx;
  double m[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) m[j] = A[static_cast<int64_t>(r) * lda + c0 + j];
#pragma unroll
  for (int k = 0; k < 64; ++k) {
    const int b = k & 1;
    if (r == k) {
#pragma unroll
      for (int j = 0; j < 16; ++j) prow[b][c0 + j] = m[j];
    }
    if (q == (k >> 4)) pcol[b][r] = m[k & 15];
    __syncthreads();
    const double rinv = 1.0 / prow[b][k];
    const double f = pcol[b][r];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const bool diag = q == (k >> 4) && j == (k & 15);
      const double p = diag ? rinv : prow[b][c0 + j] * rinv;
      if (r == k) m[j] = p;
      else m[j] = diag ? -f * rinv : m[j] - f * p;
    }
  }
#pragma unroll
  for (int j = 0; j < 16; ++j) X[static_cast<int64_t>(r) * ldx + c0 + j] = m[j];
}

// out_l[c] = init[c] + alpha sum_r v_l[r] M_l[r][c] for the batch's NL vectors v_l (sv apart) and matrices M_l
// (sm apart; sm 0: one matrix for all, read once), c < cols, r < rows. Block: 128 columns (a double2 per
// lane), its 4 waves summing row quarters in row order; the quarters are added in order (fixed bits).
template <int NL>
__global__ __launch_bounds__(256) void k_gemv_rows(const double* __restrict__ v, int64_t sv,
                                                   const double* __restrict__ M, int64_t ldm, int64_t sm, int rows,
                                                   int cols, const double* __restrict__ init, double alpha,
                                                   double* __restrict__ out, int64_t so) {
  __shared__ double2 part[4][NL][64];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int c = blockIdx.x * 128 + 2 * lane;
  const int l0 = NL == 1 ? blockIdx.y : 0;              // NL > 1: the shared matrix, every vector at once
  const double* __restrict__ Ml = M + static_cast<int64_t>(l0) * sm;
  const int per = (rows + 3) / 4, r0 = w * per, r1 = min(rows, r0 + per);
  double2 acc[NL];
#pragma unroll
  for (int l = 0; l < NL; ++l) acc[l] = double2{0.0, 0.0};
  if (c < cols) {
    const double* __restrict__ p = Ml + c;
    int r = r0;
    for (; r + 8 <= r1; r += 8) {
      double2 x[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) x[u] = *reinterpret_cast<const double2*>(p + static_cast<int64_t>(r + u) * ldm);
#pragma unroll
      for (int u = 0; u < 8; ++u)
#pragma unroll
        for (int l = 0; l < NL; ++l) {
          const double s = v[(l0 + l) * sv + r + u];
          acc[l].x += s * x[u].x;
          acc[l].y += s * x[u].y;
        }
    }
    for (; r < r1; ++r) {
      const double2 x = *reinterpret_cast<const double2*>(p + static_cast<int64_t>(r) * ldm);
#pragma unroll
      for (int l = 0; l < NL; ++l) {
        const double s = v[(l0 + l) * sv + r];
        acc[l].x += s * x.x;
        acc[l].y += s * x.y;
      }
    }
  }
#pragma unroll
  for (int l = 0; l < NL; ++l) part[w][l][lane] = acc[l];
  __syncthreads();
  if (w == 0 && c < cols) {
#pragma unroll
    for (int l = 0; l < NL; ++l) {
      double2 s = part[0][l][lane];
#pragma unroll
      for (int i = 1; i < 4; ++i) {
        s.x += part[i][l][lane].x;
        s.y += part[i][l][lane].y;
      }
      double2 o = init ? *reinterpret_cast<const double2*>(init + c) : double2{0.0, 0.0};
      o.x += alpha * s.x;
      o.y += alpha * s.y;
      *reinterpret_cast<double2*>(out + (l0 + l) * so + c) = o;
    }
  }
}

// dst[j][i] = src[i][j] for an rows x cols block (32 x 32 tiles through LDS).
__global__ __launch_bounds__(256) void k_dtranspose(const double* __restrict__ src, int64_t lds, double* __restrict__ dst,
                                                    int64_t ldd, int rows, int cols, int64_t ss, int64_t sd) {
  __shared__ double tile[32][33];
  src += static_cast<int64_t>(blockIdx.z) * ss;
  dst += static_cast<int64_t>(blockIdx.z) * sd;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  const int r0 = blockIdx.y * 32, c0 = blockIdx.x * 32;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = r0 + ty + 8 * i, c = c0 + tx;
    if (r < rows && c < cols) tile[ty + 8 * i][tx] = src[static_cast<int64_t>(r) * lds + c];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = c0 + ty + 8 * i, r = r0 + tx;
    if (r < rows && c < cols) dst[static_cast<int64_t>(c) * ldd + r] = tile[tx][ty + 8 * i];
  }
}

// dst[i][j] = src[i][j] + (i == j ? shift : 0) for i, j < n_src, and the identity on the padding up to n.
struct Shifts {
  double v[8];
};

__global__ __launch_bounds__(256) void k_dshift(const double* __restrict__ src, int64_t lds, int n_src,
                                                double* __restrict__ dst, int64_t ldd, int n, int64_t sd, Shifts sh) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const double shift = sh.v[blockIdx.y];
  dst += static_cast<int64_t>(blockIdx.y) * sd;
  if (idx >= static_cast<int64_t>(n) * n) return;
  const int i = static_cast<int>(idx / n), j = static_cast<int>(idx % n);
  double v;
  if (i < n_src && j < n_src) v = src[static_cast<int64_t>(i) * lds + j] + (i == j ? shift : 0.0);
  else v = (i == j) ? 1.0 : 0.0;
  dst[static_cast<int64_t>(i) * ldd + j] = v;
}

// dst = src for an rows x cols block; also the bias rows' initial mean_y (rows = 1).
__global__ __launch_bounds__(256) void k_dcopy(const double* __restrict__ src, int64_t lds, double* __restrict__ dst,
                                               int64_t ldd, int rows, int cols, int64_t ss, int64_t sd) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  src += static_cast<int64_t>(blockIdx.y) * ss;
  dst += static_cast<int64_t>(blockIdx.y) * sd;
  if (idx >= static_cast<int64_t>(rows) * cols) return;
  const int64_t i = idx / cols, j = idx % cols;
  dst[i * ldd + j] = src[i * lds + j];
}

// Launches on one stream for a batch of `nb` matrices laid out at fixed element strides (the lambdas of one
// solve): every matrix argument is the batch's first matrix and its stride.
struct Solver {
  hipStream_t stream;
  const char* fn;
  int nb;
  int rc = RF_OK;

  bool ok() {
    if (rc == RF_OK) rc = check_launch(fn);
    return rc == RF_OK;
  }
  void gemm(const double* A, int64_t lda, int64_t sa, const double* B, int64_t ldb, int64_t sb, double* C, int64_t ldc,
            int64_t sc, int M, int N, int K, double alpha, double beta) {
    if (rc != RF_OK || M <= 0 || N <= 0) return;
    const int tiles = ((M + DBM - 1) / DBM) * ((N + DBN - 1) / DBN);
    const DgemmArgs args{A, lda, B, ldb, C, ldc, M, N, K, alpha, beta, sa, sb, sc};
    hipLaunchKernelGGL(k_dgemm, dim3(tiles, nb), dim3(256), 0, stream, args);
    ok();
  }
  void transpose(const double* src, int64_t lds, int64_t ss, double* dst, int64_t ldd, int64_t sd, int rows, int cols) {
    if (rc != RF_OK) return;
    hipLaunchKernelGGL(k_dtranspose, dim3((cols + 31) / 32, (rows + 31) / 32, nb), dim3(256), 0, stream, src, lds, dst,
                       ldd, rows, cols, ss, sd);
    ok();
  }
  void copy(const double* src, int64_t lds, int64_t ss, double* dst, int64_t ldd, int64_t sd, int rows, int cols) {
    if (rc != RF_OK) return;
    const int64_t n = static_cast<int64_t>(rows) * cols;
    hipLaunchKernelGGL(k_dcopy, dim3(static_cast<unsigned>((n + 255) / 256), nb), dim3(256), 0, stream, src, lds, dst,
                       ldd, rows, cols, ss, sd);
    ok();
  }
  // X = A^-1 for each matrix of the batch (n x n SPD, n a multiple of 64; matrices sa / sx apart); work: each
  // matrix's own work_doubles(n) doubles, sw apart.
  void inverse(const double* A, int64_t lda, int64_t sa, double* X, int64_t ldx, int64_t sx, int n, double* work,
               int64_t sw) {
    if (rc != RF_OK) return;
    if (n == 64) {
      hipLaunchKernelGGL(k_spd_inv64, dim3(nb), dim3(256), 0, stream, A, lda, X, ldx, sa, sx);
      ok();
      return;
    }
    const int h = 64 * ((n + 127) / 128), h2 = n - h;
    const double* A12 = A + h;
    const double* A21 = A + static_cast<int64_t>(h) * lda;
    const double* A22 = A21 + h;
    double* X12 = X + h;
    double* X21 = X + static_cast<int64_t>(h) * ldx;
    double* X22 = X21 + h;
    double* T = work;                                   // [h2, h]
    double* S = work + static_cast<int64_t>(h2) * h;    // [h2, h2], later U [h, h2]
    double* deeper = S + static_cast<int64_t>(std::max(h2, h)) * std::max(h2, h);
    inverse(A, lda, sa, X, ldx, sx, h, work, sw);                              // X11 (T and S are not live yet)
    gemm(A21, lda, sa, X, ldx, sx, T, h, sw, h2, h, h, 1.0, 0.0);              // T = A21 X11
    copy(A22, lda, sa, S, h2, sw, h2, h2);
    gemm(T, h, sw, A12, lda, sa, S, h2, sw, h2, h2, h, -1.0, 1.0);             // S = A22 - T A12
    inverse(S, h2, sw, X22, ldx, sx, h2, deeper, sw);                          // X22 = S^-1
    gemm(X22, ldx, sx, T, h, sw, X21, ldx, sx, h2, h, h2, -1.0, 0.0);          // X21 = -X22 T
    gemm(X, ldx, sx, A12, lda, sa, S, h2, sw, h, h2, h, 1.0, 0.0);             // U = X11 A12 (into S's space)
    gemm(S, h2, sw, X21, ldx, sx, X, ldx, sx, h, h, h2, -1.0, 1.0);            // X11 -= U X21
    transpose(X21, ldx, sx, X12, ldx, sx, h2, h);                              // X12 = X21^T
  }
};

// doubles of work the recursion needs for n (T and S / U at this level, then the deeper levels)
int64_t work_doubles(int n) {
  if (n <= 64) return 0;
  const int h = 64 * ((n + 127) / 128), h2 = n - h;
  const int64_t mx = std::max(h2, h);
  return static_cast<int64_t>(h2) * h + mx * mx + std::max(work_doubles(h), work_doubles(h2));
}

int64_t padded(int64_t d) { return (d + 63) / 64 * 64; }

constexpr int MAX_LAMBDAS = 8;           // lambdas solved together (one batch of inverses)

size_t solve_workspace(int64_t d, int nlam) {
  const int64_t n = padded(d);
  const int nb = std::max(1, std::min(nlam, MAX_LAMBDAS));
  return static_cast<size_t>(nb) * (2 * n * n + work_doubles(static_cast<int>(n)) + n) * sizeof(double) + 256;
}

// out_l = init + alpha v_l M for l < nb with one matrix M shared by the batch (read once).
void gemv_shared(int nb, const double* v, int64_t sv, const double* M, int64_t ldm, int rows, int cols,
                 const double* init, double alpha, double* out, int64_t so, hipStream_t stream) {
  const dim3 grid((cols + 127) / 128), block(256);
  switch (nb) {
#define RF_GEMV(NL) \
  case NL: hipLaunchKernelGGL(k_gemv_rows<NL>, grid, block, 0, stream, v, sv, M, ldm, 0, rows, cols, init, alpha, out, so); break;
    RF_GEMV(1) RF_GEMV(2) RF_GEMV(3) RF_GEMV(4) RF_GEMV(5) RF_GEMV(6) RF_GEMV(7) RF_GEMV(8)
#undef RF_GEMV
    default: break;
  }
}

}  // namespace
}  // namespace rf

using namespace rf;

extern "C" int rf_ridge_solve_workspace_bytes(int64_t d, int nlam, size_t* bytes) {
  if (d <= 0 || d > 65536 || nlam <= 0 || !bytes)
    return fail(RF_EINVAL_ARG, "rf_ridge_solve_workspace_bytes: d %lld, nlam %d", (long long)d, nlam);
  *bytes = solve_workspace(d, nlam);
  return RF_OK;
}

extern "C" int rf_ridge_solve(const double* cxx, int64_t ldc, int64_t d, const double* cxy, int64_t ldb, int64_t R,
                              const double* mean_x, const double* mean_y, const double* lams, int nlam, double scale,
                              double* w, int64_t ldw, int64_t w_stride, double* bias, int64_t bias_stride,
                              void* workspace, size_t ws_bytes, hipStream_t stream) {
  const char* fn = "rf_ridge_solve";
  if (!cxx || !cxy || !lams || !w || !workspace) return fail(RF_EINVAL_ARG, "%s: null pointer", fn);
  if (bias && (!mean_x || !mean_y)) return fail(RF_EINVAL_ARG, "%s: the bias needs mean_x and mean_y", fn);
  if (d <= 0 || d > 65536 || R <= 0 || R > (1ll << 30) || R % 2 || d % 2 || ldc < d || ldb < R || ldb % 2 ||
      ldw < R || ldw % 2 || nlam <= 0 || (nlam > 1 && w_stride < d * ldw) || (bias && nlam > 1 && bias_stride < R))
    return fail(RF_EINVAL_SHAPE, "%s: d %lld, R %lld (even), ldc %lld, ldb %lld, ldw %lld (even, >= R), nlam %d, "
                "w_stride %lld, bias_stride %lld", fn, (long long)d, (long long)R, (long long)ldc, (long long)ldb,
                (long long)ldw, nlam, (long long)w_stride, (long long)bias_stride);
  if (!aligned16(cxy) || !aligned16(w) || !aligned16(workspace) || (mean_x && !aligned16(mean_x)) ||
      (bias && (!aligned16(bias) || !aligned16(mean_y) || (nlam > 1 && bias_stride % 2))))
    return fail(RF_EINVAL_SHAPE, "%s: cxy, w, mean_x, mean_y, bias and the workspace must be 16-byte aligned "
                "(bias_stride even)", fn);
  if (ws_bytes < solve_workspace(d, nlam))
    return fail(RF_EINVAL_ARG, "%s: workspace %zu bytes, needs %zu (rf_ridge_solve_workspace_bytes)", fn, ws_bytes,
                solve_workspace(d, nlam));
  for (int l = 0; l < nlam; ++l)
    if (!(lams[l] > 0.0) || !(scale > 0.0))
      return fail(RF_EINVAL_ARG, "%s: lambda %g, scale %g (both must be positive)", fn, lams[l], scale);
  const int n = static_cast<int>(padded(d));
  const int64_t nn = static_cast<int64_t>(n) * n, nw = work_doubles(n);
  double* A = static_cast<double*>(workspace);
  for (int l0 = 0; l0 < nlam; l0 += MAX_LAMBDAS) {        // up to MAX_LAMBDAS inverses as one batch
    const int nb = std::min(MAX_LAMBDAS, nlam - l0);
    double* X = A + nb * nn;
    double* work = X + nb * nn;
    Solver s{stream, fn, nb};
    Shifts sh{};
    for (int l = 0; l < nb; ++l) sh.v[l] = lams[l0 + l] * scale;
    hipLaunchKernelGGL(k_dshift, dim3(static_cast<unsigned>((nn + 255) / 256), nb), dim3(256), 0, stream, cxx, ldc,
                       static_cast<int>(d), A, static_cast<int64_t>(n), n, nn, sh);
    if (!s.ok()) return s.rc;
    s.inverse(A, n, nn, X, n, nn, n, work, nw);
    double* wl = w + l0 * w_stride;
    s.gemm(X, n, nn, cxy, ldb, 0, wl, ldw, w_stride, static_cast<int>(d), static_cast<int>(R), static_cast<int>(d),
           1.0, 0.0);
    if (bias && s.rc == RF_OK) {                       // mean_y - mean_x W = mean_y - (mean_x X) Cxy
      double* u = work + nb * nw;
      hipLaunchKernelGGL(k_gemv_rows<1>, dim3(static_cast<unsigned>((d + 127) / 128), nb), dim3(256), 0, stream,
                         mean_x, 0, X, static_cast<int64_t>(n), nn, static_cast<int>(d), static_cast<int>(d), nullptr,
                         1.0, u, static_cast<int64_t>(n));
      if (!s.ok()) return s.rc;
      gemv_shared(nb, u, n, cxy, ldb, static_cast<int>(d), static_cast<int>(R), mean_y, -1.0,
                  bias + l0 * bias_stride, bias_stride, stream);
      if (!s.ok()) return s.rc;
    }
    if (s.rc != RF_OK) return s.rc;
  }
  return RF_OK;
}
