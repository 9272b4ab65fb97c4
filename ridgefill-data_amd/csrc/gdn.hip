// Gated DeltaNet fill for gfx950: causal conv + SiLU, k l2-norm, gates and the chunked gated delta
// rule's state update over P rows of one layer, continuing a carried state (code/kva/model.py:452-484,
// ops.py:173-262 with need_out = False: the fill keeps only the final state and conv state).
//
// One workgroup (256 threads) per value head h walks the 64-row chunks in order. Thread t owns one
// conv channel (t < 128: the k channel t of key head h / (nv / nk); else the v channel t - 128 of
// head h) with its 3-row window in registers, and the state column c = t % 128, rows
// (t / 128) * 64 .. + 63, in registers. Per chunk, in LDS (fp32): k (l2-normed, row stride 132 so the
// 4 x 4-blocked K K^T reads spread over the banks), v then W, U then v_new, A then T = (I + A)^-1, the
// exchange of the state product's half sums, and the chunk's gates. All arithmetic is fp32, in the
// reference's order where it rounds differently (conv taps accumulated in order, no fused multiply-add
// there; bf16 rounding of the conv output and of sigmoid(b)).
#include "rf_common.h"

namespace rf {
namespace {

constexpr int DK = 128, DV = 128, CH = 64, NT = 256, KST = DK + 4;

struct GdnArgs {
  const uint16_t* pre;      // [P, ld] bf16: q | k | v channels, then b [nv], a [nv]
  int64_t ld, P;
  int nk, nv, C;            // C = 2 nk DK + nv DV
  const uint16_t* conv_w;   // [C, 4] bf16
  const uint16_t* conv_in;  // [3, C] bf16 or null (zeros)
  uint16_t* conv_out;       // [3, C] bf16
  const float* a_log;       // [nv]
  const float* dt_bias;     // [nv]
  float* state;             // [nv, DK, DV] fp32, updated in place
};

__device__ __forceinline__ float mul_rn(float a, float b) { return __fmul_rn(a, b); }
__device__ __forceinline__ float add_rn(float a, float b) { return __fadd_rn(a, b); }

__global__ __launch_bounds__(NT) void k_gdn_fill(GdnArgs a) {
  __shared__ float k_s[CH][KST];
  __shared__ float vw_s[CH][DV];
  __shared__ float u_s[CH][DV];
  __shared__ float x_s[CH][DV];
  __shared__ float t_s[CH][CH];
  __shared__ float beta_s[CH], g_s[CH], gam_s[CH], ed_s[CH];

  const int h = blockIdx.x, t = threadIdx.x;
  const int rep = a.nv / a.nk, kh = h / rep;
  const bool is_k = t < DK;
  const int ch = is_k ? a.nk * DK + kh * DK + t : 2 * a.nk * DK + h * DV + (t - DK);
  float w0 = bf2f(a.conv_w[ch * 4 + 0]), w1 = bf2f(a.conv_w[ch * 4 + 1]);
  float w2 = bf2f(a.conv_w[ch * 4 + 2]), w3 = bf2f(a.conv_w[ch * 4 + 3]);
  // window: x3 oldest .. x1 newest pre-conv input (bf16 values as fp32)
  float x3 = 0.f, x2 = 0.f, x1 = 0.f;
  if (a.conv_in) {
    x3 = bf2f(a.conv_in[0 * a.C + ch]);
    x2 = bf2f(a.conv_in[1 * a.C + ch]);
    x1 = bf2f(a.conv_in[2 * a.C + ch]);
  }
  const int c = t & (DV - 1), r0 = (t >> 7) * 64;
  float S[64];
  float* st = a.state + static_cast<int64_t>(h) * DK * DV;
#pragma unroll
  for (int r = 0; r < 64; ++r) S[r] = st[(r0 + r) * DV + c];
  const float negA = -expf(a.a_log[h]), dtb = a.dt_bias[h];
  const int boff = a.C + h, aoff = a.C + a.nv + h;

  for (int64_t p0 = 0; p0 < a.P; p0 += CH) {
    const int m = static_cast<int>(min(static_cast<int64_t>(CH), a.P - p0));
    // conv + SiLU (bf16 output) of this thread's channel over the chunk's rows
    for (int r = 0; r < CH; ++r) {
      float y = 0.f;
      if (r < m) {
        const float xin = bf2f(a.pre[(p0 + r) * a.ld + ch]);
        float acc = mul_rn(x3, w0);
        acc = add_rn(acc, mul_rn(x2, w1));
        acc = add_rn(acc, mul_rn(x1, w2));
        acc = add_rn(acc, mul_rn(xin, w3));
        y = bf2f(f2bf(acc / (1.0f + expf(-acc))));
        x3 = x2;
        x2 = x1;
        x1 = xin;
      }
      if (is_k) k_s[r][t] = y;
      else vw_s[r][t - DK] = y;
    }
    if (t < CH) {
      float beta = 0.f, g = 0.f;
      if (t < m) {
        const float b = bf2f(a.pre[(p0 + t) * a.ld + boff]);
        beta = bf2f(f2bf(1.0f / (1.0f + expf(-b))));
        const float av = bf2f(a.pre[(p0 + t) * a.ld + aoff]) + dtb;
        g = negA * (av > 20.0f ? av : log1pf(expf(av)));
      }
      beta_s[t] = beta;
      g_s[t] = g;
    }
    __syncthreads();
    {  // k rows l2-normalised: 4 threads per row
      const int row = t >> 2, q = (t & 3) * 32;
      float s = 0.f;
      for (int e = 0; e < 32; ++e) s = fmaf(k_s[row][q + e], k_s[row][q + e], s);
      s += __shfl_xor(s, 1, 64);
      s += __shfl_xor(s, 2, 64);
      const float inv = 1.0f / sqrtf(s + 1e-6f);
      for (int e = 0; e < 32; ++e) k_s[row][q + e] *= inv;
    }
    if (t == 0) {
      float acc = 0.f;
      for (int i = 0; i < CH; ++i) {
        acc += g_s[i];
        gam_s[i] = acc;
      }
    }
    __syncthreads();
    if (t < CH) ed_s[t] = expf(gam_s[CH - 1] - gam_s[t]);
    {  // t_s = -A, A = tril(beta_i (k_i . k_j) exp(gam_i - gam_j), -1): 4 x 4 blocks, lower half only
      const int bi = t >> 4, bj = t & 15;
      float acc[4][4] = {};
      if (bj <= bi) {
        for (int d = 0; d < DK; d += 4) {
          float4 ki[4], kj[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            ki[q] = *reinterpret_cast<const float4*>(&k_s[bi * 4 + q][d]);
            kj[q] = *reinterpret_cast<const float4*>(&k_s[bj * 4 + q][d]);
          }
#pragma unroll
          for (int p = 0; p < 4; ++p)
#pragma unroll
            for (int q = 0; q < 4; ++q)
              acc[p][q] = fmaf(ki[p].x, kj[q].x, fmaf(ki[p].y, kj[q].y, fmaf(ki[p].z, kj[q].z,
                               fmaf(ki[p].w, kj[q].w, acc[p][q]))));
        }
      }
#pragma unroll
      for (int p = 0; p < 4; ++p)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int i = bi * 4 + p, j = bj * 4 + q;
          t_s[i][j] = j < i ? -((beta_s[i] * acc[p][q]) * expf(gam_s[i] - gam_s[j])) : 0.f;
        }
    }
    __syncthreads();
    // T = (I + A)^-1 below the diagonal, row by row: t[i][j] = t0[i][j] + sum_{j<m<i} t0[i][m] t[m][j]
    for (int i = 2; i < CH; ++i) {
      float v = 0.f;
      if (t < i) {
        v = t_s[i][t];
        for (int mm = t + 1; mm < i; ++mm) v = fmaf(t_s[i][mm], t_s[mm][t], v);
      }
      __syncthreads();
      if (t < i) t_s[i][t] = v;
      __syncthreads();
    }
    // U = T (beta v), W = T (beta e^gam k): thread column c, rows (t / 128) * 32 .. + 31. T = t_s + I,
    // t_s zero on and above the diagonal, so every row sums all 64 columns (register arrays are only
    // ever indexed by compile-time constants) and adds its diagonal term from LDS.
    {
      const int i0 = (t >> 7) * 32;
      float bv[CH];
#pragma unroll
      for (int j = 0; j < CH; ++j) bv[j] = beta_s[j] * vw_s[j][c];
      for (int ii = 0; ii < 32; ++ii) {
        const int i = i0 + ii;
        float acc = beta_s[i] * vw_s[i][c];
#pragma unroll
        for (int j = 0; j < CH; ++j) acc = fmaf(t_s[i][j], bv[j], acc);
        u_s[i][c] = acc;
      }
#pragma unroll
      for (int j = 0; j < CH; ++j) bv[j] = (beta_s[j] * expf(gam_s[j])) * k_s[j][c];
      __syncthreads();                            // every v read: vw_s now takes W
      for (int ii = 0; ii < 32; ++ii) {
        const int i = i0 + ii;
        float acc = (beta_s[i] * expf(gam_s[i])) * k_s[i][c];
#pragma unroll
        for (int j = 0; j < CH; ++j) acc = fmaf(t_s[i][j], bv[j], acc);
        vw_s[i][c] = acc;
      }
    }
    __syncthreads();
    // v_new = U - W S. Each thread sums its 64 state rows; the lower half subtracts its sums from U
    // in place, the upper half hands its sums over through x_s, then the lower half subtracts those.
    for (int i = 0; i < CH; ++i) {
      float acc = 0.f;
#pragma unroll
      for (int r = 0; r < 64; r += 4) {
        const float4 wv = *reinterpret_cast<const float4*>(&vw_s[i][r0 + r]);
        acc = fmaf(wv.x, S[r], acc);
        acc = fmaf(wv.y, S[r + 1], acc);
        acc = fmaf(wv.z, S[r + 2], acc);
        acc = fmaf(wv.w, S[r + 3], acc);
      }
      if (r0) x_s[i][c] = acc;
      else u_s[i][c] = u_s[i][c] - acc;
    }
    __syncthreads();
    if (!r0) {
      for (int i = 0; i < CH; ++i) u_s[i][c] = u_s[i][c] - x_s[i][c];
    }
    __syncthreads();
    // S = S e^{gam_last} + (k e^{gam_last - gam})^T v_new
    {
      const float cd = expf(gam_s[CH - 1]);
      float acc[64];
#pragma unroll
      for (int r = 0; r < 64; ++r) acc[r] = 0.f;
      for (int i = 0; i < CH; ++i) {
        const float vn = u_s[i][c], e = ed_s[i];
#pragma unroll
        for (int r = 0; r < 64; r += 4) {
          const float4 kv = *reinterpret_cast<const float4*>(&k_s[i][r0 + r]);
          acc[r] = fmaf(kv.x * e, vn, acc[r]);
          acc[r + 1] = fmaf(kv.y * e, vn, acc[r + 1]);
          acc[r + 2] = fmaf(kv.z * e, vn, acc[r + 2]);
          acc[r + 3] = fmaf(kv.w * e, vn, acc[r + 3]);
        }
      }
#pragma unroll
      for (int r = 0; r < 64; ++r) S[r] = S[r] * cd + acc[r];
    }
    __syncthreads();
  }
#pragma unroll
  for (int r = 0; r < 64; ++r) st[(r0 + r) * DV + c] = S[r];
  // conv state: the last 3 rows of [conv_in; pre] for this thread's channel, and (one head per key
  // head) the q channels of key head kh
  a.conv_out[0 * a.C + ch] = f2bf(x3);
  a.conv_out[1 * a.C + ch] = f2bf(x2);
  a.conv_out[2 * a.C + ch] = f2bf(x1);
  if (h % rep == 0 && t < DK) {
    const int qc = kh * DK + t;
    for (int j = 0; j < 3; ++j) {
      const int64_t idx = a.P - 3 + j;
      uint16_t v = 0;
      if (idx >= 0) v = a.pre[idx * a.ld + qc];
      else if (a.conv_in) v = a.conv_in[(3 + idx) * a.C + qc];
      a.conv_out[j * a.C + qc] = v;
    }
  }
}

}  // namespace
}  // namespace rf

using namespace rf;

extern "C" int rf_gdn_fill(const uint16_t* pre, int64_t ld, int64_t P, int nk, int nv, int dk, int dv,
                           const uint16_t* conv_w, const uint16_t* conv_in, uint16_t* conv_out, const float* a_log,
                           const float* dt_bias, float* state, hipStream_t stream) {
  if (!pre || !conv_w || !conv_out || !a_log || !dt_bias || !state) return fail(RF_EINVAL_ARG, "rf_gdn_fill: null pointer");
  if (dk != DK || dv != DV) return fail(RF_EUNSUPPORTED, "rf_gdn_fill: key / value head dims %d / %d (128 / 128)", dk, dv);
  if (nk <= 0 || nv <= 0 || nv % nk || nv > 4096) return fail(RF_EINVAL_SHAPE, "rf_gdn_fill: heads nk %d nv %d", nk, nv);
  const int64_t C = 2ll * nk * DK + static_cast<int64_t>(nv) * DV;
  if (P < 0 || ld < C + 2 * nv) return fail(RF_EINVAL_SHAPE, "rf_gdn_fill: P %lld, ld %lld < %lld", (long long)P,
                                            (long long)ld, (long long)(C + 2 * nv));
  if (conv_in == conv_out) return fail(RF_EINVAL_ARG, "rf_gdn_fill: conv_out must not alias conv_in");
  GdnArgs a{pre, ld, P, nk, nv, static_cast<int>(C), conv_w, conv_in, conv_out, a_log, dt_bias, state};
  hipLaunchKernelGGL(k_gdn_fill, dim3(nv), dim3(NT), 0, stream, a);
  return check_launch("rf_gdn_fill");
}
