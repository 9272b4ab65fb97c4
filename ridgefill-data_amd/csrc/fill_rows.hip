// Row-wise HBM-bound kernels of the fill: RMSNorm statistics of given inputs, the exact-row scatter and
// gather, the norm-gain fold, the RoPE table and the standalone RoPE + K / V cache write (fill_kv).
// The row-statistics kernels run one wave per row and form each 256-column group's sum of squares with
// row_partials (rf_common.h), in the order the GEMM epilogue uses; the others move 16-byte chunks.
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>

#include "rf_common.h"

namespace rf {

static thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(RF_EHIP, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
  return RF_OK;
}

namespace {

__global__ __launch_bounds__(256) void k_row_ssq(const uint16_t* __restrict__ x, int64_t ldx, float* __restrict__ ssq,
                                                 int64_t P, int nparts) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= P) return;
  const uint16_t* xr = x + row * ldx;
  row_partials([&](int64_t o) { return *reinterpret_cast<const uint2*>(xr + o); }, ssq + row * nparts, nparts,
               threadIdx.x & 63);
}

__global__ __launch_bounds__(256) void k_row_scatter(uint16_t* __restrict__ x, int64_t ldx, float* __restrict__ ssq,
                                                     int64_t P, int nparts, const int64_t* __restrict__ rows,
                                                     int64_t nrows, const uint16_t* __restrict__ hr, int64_t ldhr) {
  const int64_t j = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (j >= nrows) return;
  const int64_t row = rows[j];
  if (row < 0 || row >= P) return;
  const uint16_t* src = hr + j * ldhr;
  uint16_t* dst = x + row * ldx;
  row_partials([&](int64_t o) {
    const uint2 v = *reinterpret_cast<const uint2*>(src + o);
    *reinterpret_cast<uint2*>(dst + o) = v;
    return v;
  }, ssq + row * nparts, nparts, threadIdx.x & 63);
}

// out[j] = x[rows[j]] for j < nrows (bit-exact) and out's row partials; a row outside [0, P) gives zeros.
__global__ __launch_bounds__(256) void k_row_gather(const uint16_t* __restrict__ x, int64_t ldx, int64_t P,
                                                    int nparts, const int64_t* __restrict__ rows, int64_t nrows,
                                                    uint16_t* __restrict__ out, int64_t ldo, float* __restrict__ ssq) {
  const int64_t j = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (j >= nrows) return;
  const int64_t row = rows[j];
  const bool ok = row >= 0 && row < P;
  const uint16_t* src = x + (ok ? row : 0) * ldx;
  uint16_t* dst = out + j * ldo;
  row_partials([&](int64_t o) {
    const uint2 v = ok ? *reinterpret_cast<const uint2*>(src + o) : make_uint2(0u, 0u);
    *reinterpret_cast<uint2*>(dst + o) = v;
    return v;
  }, ssq + j * nparts, nparts, threadIdx.x & 63);
}

__global__ __launch_bounds__(256) void k_fold_norm(const uint16_t* __restrict__ w, const uint16_t* __restrict__ gain,
                                                   int kind, uint16_t* __restrict__ out, int64_t chunks, int64_t K) {
  const int64_t c = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (c >= chunks) return;
  const int64_t e0 = c * 8;
  const int64_t k0 = e0 % K;
  const uint4 v = *reinterpret_cast<const uint4*>(w + e0);
  const uint4 gv = *reinterpret_cast<const uint4*>(gain + k0);
  uint16_t o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float g = bf2f(lane_of(gv, e));
    o[e] = f2bf(bf2f(lane_of(v, e)) * (kind ? 1.0f + g : g));
  }
  *reinterpret_cast<uint4*>(out + e0) = make_uint4(pack2(o[0], o[1]), pack2(o[2], o[3]), pack2(o[4], o[5]), pack2(o[6], o[7]));
}

__global__ __launch_bounds__(256) void k_rope_table(const int64_t* __restrict__ pos, int64_t P,
                                                    const float* __restrict__ inv_freq, int half,
                                                    uint16_t* __restrict__ cs) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= P * half) return;
  const int64_t row = i / half;
  const int f = static_cast<int>(i - row * half);
  const float ang = static_cast<float>(pos[row]) * inv_freq[f];
  cs[row * 2 * half + f] = f2bf(cosf(ang));
  cs[row * 2 * half + half + f] = f2bf(sinf(ang));
}

// One 16-byte chunk per iteration: chunks [0, m hkv d/8) are K, the next as many are V; the cache writes
// are streaming (nontemporal) stores.
__device__ __forceinline__ void one_chunk(int64_t i, const uint16_t* __restrict__ k, int64_t ld_k,
                                          const uint16_t* __restrict__ v, int64_t ld_v, int64_t m, int hkv, int d,
                                          const uint16_t* __restrict__ cs, int rot, uint16_t* __restrict__ kbuf,
                                          uint16_t* __restrict__ vbuf, int64_t head_stride, int64_t row_stride,
                                          int64_t slot0) {
  const int cpr = hkv * (d >> 3);
  const int64_t per = m * cpr;
  if (i >= 2 * per) return;
  const bool is_k = i < per;
  const int64_t c = is_k ? i : i - per;
  const int64_t tok = c / cpr;
  const int rem = static_cast<int>(c - tok * cpr);
  const int head = rem / (d >> 3);
  const int j0 = (rem - head * (d >> 3)) * 8;
  uint16_t* dst = (is_k ? kbuf : vbuf) + head * head_stride + (slot0 + tok) * row_stride + j0;
  if (!is_k) {
    st_stream16(dst, *reinterpret_cast<const uint4*>(v + tok * ld_v + head * d + j0));
    return;
  }
  const uint16_t* src = k + tok * ld_k + head * d;
  const uint4 x = *reinterpret_cast<const uint4*>(src + j0);
  if (j0 >= rot) {
    st_stream16(dst, x);
    return;
  }
  const int half = rot >> 1;
  float f[8], pf[8], co[8], sn[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) f[e] = bf2f(lane_of(x, e));
  const uint16_t* t = cs + tok * rot;
  if (half >= 8) {
    const bool lo = j0 < half;
    const uint4 p = *reinterpret_cast<const uint4*>(src + (lo ? j0 + half : j0 - half));
    const int fi0 = lo ? j0 : j0 - half;            // 8 consecutive entries of each half of the table
    const uint4 cv = *reinterpret_cast<const uint4*>(t + fi0);
    const uint4 sv = *reinterpret_cast<const uint4*>(t + half + fi0);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      pf[e] = bf2f(lane_of(p, e));
      co[e] = bf2f(lane_of(cv, e));
      sn[e] = bf2f(lane_of(sv, e));
    }
  } else {                                          // rot == 8: one chunk holds both halves
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      pf[e] = f[e ^ 4];
      co[e] = bf2f(t[e & 3]);
      sn[e] = bf2f(t[4 + (e & 3)]);
    }
  }
  // x cos + rotate_half(x) sin with each product rounded to bf16, then the sum (code/kva/ops.py:66-77)
  float y[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float rh = j0 + e < half ? -pf[e] : pf[e];
    const uint32_t pr = bf16_pair(f[e] * co[e], rh * sn[e]);
    y[e] = bf_lo(pr) + bf_hi(pr);
  }
  st_stream16(dst, make_uint4(bf16_pair(y[0], y[1]), bf16_pair(y[2], y[3]), bf16_pair(y[4], y[5]), bf16_pair(y[6], y[7])));
}

// Grid-stride over the chunks (at most 8192 blocks of 256 threads).
__global__ __launch_bounds__(256) void k_rope_kv(const uint16_t* __restrict__ k, int64_t ld_k,
                                                 const uint16_t* __restrict__ v, int64_t ld_v, int64_t m, int hkv,
                                                 int d, const uint16_t* __restrict__ cs, int rot,
                                                 uint16_t* __restrict__ kbuf, uint16_t* __restrict__ vbuf,
                                                 int64_t head_stride, int64_t row_stride, int64_t slot0) {
  const int64_t n = 2 * m * hkv * (d >> 3);
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += stride)
    one_chunk(i, k, ld_k, v, ld_v, m, hkv, d, cs, rot, kbuf, vbuf, head_stride, row_stride, slot0);
}

int blocks(int64_t n, int per) { return static_cast<int>((n + per - 1) / per); }

}  // namespace
}  // namespace rf

using namespace rf;

extern "C" const char* rf_last_error(void) { return g_err; }

extern "C" int rf_version(void) { return 1; }

extern "C" int rf_row_ssq(const uint16_t* x, int64_t ldx, float* ssq, int64_t P, int64_t H, hipStream_t stream) {
  if (!x || !ssq) return fail(RF_EINVAL_ARG, "rf_row_ssq: null pointer");
  if (P < 0 || H <= 0 || H % SSQ_COLS || ldx < H || ldx % 8 || !aligned16(x))
    return fail(RF_EINVAL_SHAPE, "rf_row_ssq: P %lld, H %lld (multiple of 256), ldx %lld, 16-byte alignment",
                (long long)P, (long long)H, (long long)ldx);
  if (P == 0) return RF_OK;
  hipLaunchKernelGGL(k_row_ssq, dim3(blocks(P, 4)), dim3(256), 0, stream, x, ldx, ssq, P,
                     static_cast<int>(H / SSQ_COLS));
  return check_launch("rf_row_ssq");
}

extern "C" int rf_row_scatter(uint16_t* x, int64_t ldx, float* ssq, int64_t P, int64_t H, const int64_t* rows,
                              int64_t nrows, const uint16_t* hr, int64_t ldhr, hipStream_t stream) {
  if (!x || !ssq || (nrows > 0 && (!rows || !hr))) return fail(RF_EINVAL_ARG, "rf_row_scatter: null pointer");
  if (P < 0 || nrows < 0 || H <= 0 || H % SSQ_COLS || ldx < H || ldx % 8 || ldhr < H || ldhr % 8 ||
      !aligned16(x) || (hr && !aligned16(hr)))
    return fail(RF_EINVAL_SHAPE, "rf_row_scatter: P %lld, H %lld, ldx %lld, ldhr %lld", (long long)P,
                (long long)H, (long long)ldx, (long long)ldhr);
  if (nrows == 0) return RF_OK;
  hipLaunchKernelGGL(k_row_scatter, dim3(blocks(nrows, 4)), dim3(256), 0, stream, x, ldx, ssq, P,
                     static_cast<int>(H / SSQ_COLS), rows, nrows, hr, ldhr);
  return check_launch("rf_row_scatter");
}

extern "C" int rf_row_gather(const uint16_t* x, int64_t ldx, int64_t P, int64_t H, const int64_t* rows, int64_t nrows,
                             uint16_t* out, int64_t ldo, float* ssq, hipStream_t stream) {
  if (!x || !rows || !out || !ssq) return fail(RF_EINVAL_ARG, "rf_row_gather: null pointer");
  if (P < 0 || nrows < 0 || H <= 0 || H % SSQ_COLS || ldx < H || ldo < H || ldx % 4 || ldo % 4)
    return fail(RF_EINVAL_SHAPE, "rf_row_gather: P %lld, H %lld (multiple of 256), strides", (long long)P, (long long)H);
  if ((reinterpret_cast<uintptr_t>(x) & 7u) || (reinterpret_cast<uintptr_t>(out) & 7u))
    return fail(RF_EINVAL_SHAPE, "rf_row_gather: 8-byte alignment");
  if (nrows == 0) return RF_OK;
  hipLaunchKernelGGL(k_row_gather, dim3(blocks(nrows, 4)), dim3(256), 0, stream, x, ldx, P, static_cast<int>(H / SSQ_COLS),
                     rows, nrows, out, ldo, ssq);
  return check_launch("rf_row_gather");
}

extern "C" int rf_fold_norm(const uint16_t* w, const uint16_t* gain, int kind, uint16_t* w_out, int64_t N, int64_t K,
                            hipStream_t stream) {
  if (!w || !gain || !w_out) return fail(RF_EINVAL_ARG, "rf_fold_norm: null pointer");
  if (kind != 0 && kind != 1) return fail(RF_EINVAL_ARG, "rf_fold_norm: kind %d", kind);
  if (N <= 0 || K <= 0 || K % 8 || !aligned16(w) || !aligned16(gain) || !aligned16(w_out))
    return fail(RF_EINVAL_SHAPE, "rf_fold_norm: N %lld, K %lld (multiple of 8), 16-byte alignment", (long long)N,
                (long long)K);
  const int64_t chunks = N * K / 8;
  hipLaunchKernelGGL(k_fold_norm, dim3(blocks(chunks, 256)), dim3(256), 0, stream, w, gain, kind, w_out, chunks, K);
  return check_launch("rf_fold_norm");
}

extern "C" int rf_rope_table(const int64_t* pos, int64_t P, const float* inv_freq, int rot, uint16_t* cs,
                             hipStream_t stream) {
  if (!pos || !inv_freq || !cs) return fail(RF_EINVAL_ARG, "rf_rope_table: null pointer");
  if (P < 0 || rot <= 0 || rot % 2) return fail(RF_EINVAL_SHAPE, "rf_rope_table: P %lld, rot %d", (long long)P, rot);
  if (P == 0) return RF_OK;
  hipLaunchKernelGGL(k_rope_table, dim3(blocks(P * (rot / 2), 256)), dim3(256), 0, stream, pos, P, inv_freq, rot / 2,
                     cs);
  return check_launch("rf_rope_table");
}

extern "C" int rf_rope_kv_write(const uint16_t* k, int64_t ld_k, const uint16_t* v, int64_t ld_v, int64_t m, int hkv,
                                int d, const uint16_t* cs, int rot, uint16_t* kbuf, uint16_t* vbuf,
                                int64_t head_stride, int64_t row_stride, int64_t slot_begin, int64_t cap,
                                hipStream_t stream) {
  if (!k || !v || !cs || !kbuf || !vbuf) return fail(RF_EINVAL_ARG, "rf_rope_kv_write: null pointer");
  if (m < 0 || hkv <= 0 || d <= 0 || d % 8 || ld_k < hkv * d || ld_v < hkv * d || ld_k % 8 || ld_v % 8 ||
      head_stride % 8 || row_stride % 8 || row_stride < d)
    return fail(RF_EINVAL_SHAPE, "rf_rope_kv_write: m %lld, hkv %d, d %d, strides", (long long)m, hkv, d);
  if (rot <= 0 || rot > d || rot % 2 || ((rot / 2) % 8 && rot / 2 != 4))
    return fail(RF_EUNSUPPORTED, "rf_rope_kv_write: rotary dims %d of head_dim %d", rot, d);
  if (slot_begin < 0 || slot_begin + m > cap)
    return fail(RF_EINVAL_SHAPE, "rf_rope_kv_write: rows [%lld, %lld) exceed cache capacity %lld",
                (long long)slot_begin, (long long)(slot_begin + m), (long long)cap);
  if (!aligned16(k) || !aligned16(v) || !aligned16(kbuf) || !aligned16(vbuf) || !aligned16(cs))
    return fail(RF_EINVAL_SHAPE, "rf_rope_kv_write: pointers must be 16-byte aligned");
  if (m == 0) return RF_OK;
  const int64_t threads = 2 * m * hkv * (d / 8);
  hipLaunchKernelGGL(k_rope_kv, dim3(std::min(blocks(threads, 256), 8192)), dim3(256), 0, stream, k, ld_k, v, ld_v, m, hkv, d, cs,
                     rot, kbuf, vbuf, head_stride, row_stride, slot_begin);
  return check_launch("rf_rope_kv_write");
}
