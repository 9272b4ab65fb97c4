// Gated DeltaNet fill for gfx950: causal conv + SiLU, k l2-norm, gates and the chunked gated delta
// rule's state update over P rows of one layer, continuing a carried state (code/kva/model.py:452-484,
// ops.py:173-262 with need_out = False: the fill keeps only the final state and the conv state).
//
// Per 64-row chunk (gamma = in-chunk cumsum of g, r_i = 1 / |k_i| of the conv output k_i, beta_i):
//   A = tril_{-1}(beta_i r_i r_j (k_i . k_j) e^{gamma_i - gamma_j}),  T = (I + A)^-1
//   X = K S,  Y = beta (V - e^gamma r X),  v_new = T Y              (= U - W S of the reference)
//   S <- e^{gamma_last} S + K^T (r e^{gamma_last - gamma} v_new)
// with K the raw (bf16) conv output, so K K^T, K S and K^T Z multiply exact bf16 values.
//
// Two kernels per pass of up to `chunks` chunks:
//   k_gdn_prep (chunk x value head, 256 threads): conv + SiLU of the key head's k and of the value
//     head's v, row norms, gates, G = K K^T on MFMA, A and T = (I + A)^-1 by forward substitution
//     (fp32). Writes per chunk, in the MFMA operand order the scan reads: K (A operand of K S), K^T (A
//     operand of K^T Z), T split into hi / lo bf16, V (accumulator layout) and the per-row scalars.
//   k_gdn_scan (value head x 16-column block, 4 waves): the sequential chunk recurrence with the fp32
//     state block [128 x 16] in registers, 32 rows per wave. Each product runs on
//     v_mfma_f32_16x16x32_bf16; fp32 operands (S, Y, Z, T) are split into hi + lo bf16 so each product
//     keeps ~2^-16 relative accuracy. The in-lane order of the contraction index is permuted so that an
//     accumulator tile is a B-operand half as it stands: lane group g = lane / 16 holds contraction
//     indices {32s + 4g + e, 32s + 16 + 4g + e : e < 4} of k-step s. The waves split each chunk's
//     products four ways and meet three times per chunk in LDS (X partials, Y, Z); the next chunk's
//     operands load into registers meanwhile.
// k_conv_tail writes the new conv state (the last 3 pre-conv rows of [conv_in; pre]).
//
// With outputs (rf_gdn_forward: the exact layer, ops.py:199-262 with need_out = True), per chunk and value
// head o = Qd S_prev + P v_new with Qd = q_n e^gamma, P = tril(q_n k_n^T e^{gamma_i - gamma_j}) (q_n, k_n
// the l2-normed conv outputs, q_n scaled by dk^-1/2) and v_new = T Y of the state before the chunk. The
// prep also writes Qd, P, T, K and V in plain layouts, the scan stores the state before each chunk, and
// k_gdn_out (chunk x value head) forms the outputs for all chunks in parallel on fp32 MFMA.
#include <algorithm>
#include <mutex>
#include <type_traits>

#include "rf_common.h"

namespace rf {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int DK = 128, DV = 128, CH = 64, TAPS = 4;
constexpr int KST = DK + 8;                        // bf16 row stride of the k / v tiles in LDS
constexpr int FST = CH + 4;                        // fp32 row stride of the 64 x 64 tiles in LDS
// workspace layout per chunk (bytes): every key head's K orders, then every value head's T (hi / lo, its six
// nonzero 16 x 32 blocks), V, scalars
constexpr uint32_t KP_BYTES = 16384, KTP_BYTES = 16384;
constexpr uint32_t TP_BYTES = 12288, VP_BYTES = 16384, SC_BYTES = 1024;
constexpr uint32_t KH_BYTES = KP_BYTES + KTP_BYTES;
constexpr uint32_t VH_BYTES = TP_BYTES + VP_BYTES + SC_BYTES;

// T's 16 x 32 blocks (row tile it, k-step s) that can be nonzero (T is lower triangular: row tiles 0 and 1
// need k-step 0 only), numbered 0 .. 5.
__device__ __forceinline__ int tp_block(int it, int s) { return it < 2 ? it : 2 * it - 2 + s; }
// scalar block: beta [64], q = e^gamma r [64], z = r e^{gamma_last - gamma} [64], decay e^{gamma_last}
constexpr int SC_BETA = 0, SC_Q = 64, SC_Z = 128, SC_DECAY = 192;
// output region per (chunk, value head), after the chunk's scan operands: the state before the chunk
// S [DK][DV] fp32, Qd [CH][DK] fp32, P [CH][CH] fp32, T [CH][CH] fp32, K [CH][DK] bf16, V [CH][DV] bf16
constexpr uint32_t OS_S = 0, OS_QD = 65536, OS_P = 98304, OS_T = 114688, OS_K = 131072, OS_V = 147456;
constexpr uint32_t OUT_HEAD_BYTES = 163840;

__device__ __forceinline__ int kperm(int s, int g, int e) { return 32 * s + 4 * g + (e & 3) + ((e >> 2) << 4); }

__device__ __forceinline__ bf16x8 as_frag(const uint4& u) { return __builtin_bit_cast(bf16x8, u); }

// x = hi + lo: hi = x truncated to bf16, lo = (x - hi) rounded to bf16 (pairs in one v_cvt_pk_bf16_f32).
__device__ __forceinline__ void split8(const float (&x)[8], uint4& hi, uint4& lo) {
  uint32_t h[8];
  float r[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint32_t u = __float_as_uint(x[e]) & 0xffff0000u;
    h[e] = u >> 16;
    r[e] = x[e] - __uint_as_float(u);
  }
  hi = make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16));
  lo = make_uint4(bf16_pair(r[0], r[1]), bf16_pair(r[2], r[3]), bf16_pair(r[4], r[5]), bf16_pair(r[6], r[7]));
}

struct PrepArgs {
  const uint16_t* pre;      // [P, ld] bf16: q | k | v channels, then b [nv], a [nv]
  int64_t ld, P, p_begin;   // this pass's chunks start at row p_begin
  int nk, nv, C;
  const uint16_t* conv_w;   // [C, 4]
  const uint16_t* conv_in;  // [3, C] or null
  const float* a_log;
  const float* dt_bias;
  uint8_t* ws;
  uint32_t chunk_bytes;
  uint32_t out_off;         // the output region's offset in a chunk (prep with outputs)
};

// 8 channels [ch0, ch0 + 8) of input row p (relative to the call's first row); rows before 0 come from
// the carried conv state, rows at or past P are zero.
__device__ __forceinline__ uint4 pre_row(const PrepArgs& a, int64_t p, int ch0) {
  if (p < 0) {
    if (!a.conv_in) return make_uint4(0, 0, 0, 0);
    return *reinterpret_cast<const uint4*>(a.conv_in + (3 + p) * a.C + ch0);
  }
  if (p >= a.P) return make_uint4(0, 0, 0, 0);
  return *reinterpret_cast<const uint4*>(a.pre + p * a.ld + ch0);
}

// Conv + SiLU (bf16) of 8 channels over 4 output rows (thread t: channel group t % 16, rows
// 4 (t / 16) .. + 3) into dst [64][KST]; taps accumulate oldest first, products and sums rounded
// separately as the reference's fp32 tap loop; rows at or past m are zero. conv_load issues the
// thread's loads (weights of its 8 channels, input rows r0 - 3 .. r0 + 3) so that several tiles' loads
// can be in flight together; conv_store computes and writes.
struct ConvIn {
  uint4 w[4];               // channel pairs (ch0 + 2j, ch0 + 2j + 1) x 4 taps
  uint4 x[7];
};

__device__ __forceinline__ void conv_load(const PrepArgs& a, int64_t p0, int ch_base, ConvIn& in) {
  const int t = threadIdx.x, cg = t & 15, r0 = (t >> 4) * 4;
  const int ch0 = ch_base + cg * 8;
#pragma unroll
  for (int j = 0; j < 4; ++j) in.w[j] = *reinterpret_cast<const uint4*>(a.conv_w + (ch0 + 2 * j) * TAPS);
#pragma unroll
  for (int j = 0; j < 7; ++j) in.x[j] = pre_row(a, p0 + r0 - 3 + j, ch0);
}

__device__ __forceinline__ void conv_store(const ConvIn& in, int m, uint16_t* dst) {
  const int t = threadIdx.x, cg = t & 15, r0 = (t >> 4) * 4;
  float w[8][TAPS];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) w[2 * j + e / 4][e % 4] = bf2f(lane_of(in.w[j], e));
  float x[7][8];
#pragma unroll
  for (int j = 0; j < 7; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) x[j][e] = bf2f(lane_of(in.x[j], e));
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    uint16_t o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float acc = __fmul_rn(x[q][e], w[e][0]);
      acc = __fadd_rn(acc, __fmul_rn(x[q + 1][e], w[e][1]));
      acc = __fadd_rn(acc, __fmul_rn(x[q + 2][e], w[e][2]));
      acc = __fadd_rn(acc, __fmul_rn(x[q + 3][e], w[e][3]));
      // SiLU with the hardware exp2 and reciprocal (about 1 ulp each, before the bf16 rounding)
      o[e] = (r0 + q < m) ? f2bf(acc * __builtin_amdgcn_rcpf(1.0f + __expf(-acc))) : 0;
    }
    *reinterpret_cast<uint4*>(dst + (r0 + q) * KST + cg * 8) =
        make_uint4(pack2(o[0], o[1]), pack2(o[2], o[3]), pack2(o[4], o[5]), pack2(o[6], o[7]));
  }
}

// Sum of a value over the 4 lanes of each lane quad (DPP quad permutes, no LDS round trip); every lane
// of the quad gets the same bits ((l0 + l1) + (l2 + l3) in either order of the commutative adds).
__device__ __forceinline__ float quad_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xb1, 0xf, 0xf, false));  // lanes ^ 1
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4e, 0xf, 0xf, false));  // lanes ^ 2
  return v;
}

// Block = (chunk, value head h). The K-side work (conv of the key head's k, norms, G = K K^T) is
// recomputed by each of the key head's value heads; the first of them writes K's operand orders.
// Up to BATCH independent layers' fills per launch (the late GDN layers of a fill do not depend on each
// other): prep blocks take their layer from blockIdx.z, scan blocks from blockIdx.x / (8 nv).
constexpr int BATCH = RF_GDN_BATCH_MAX;
struct PrepBatch {
  PrepArgs a[BATCH];
};

// At most 128 VGPRs and no AGPRs (130 allocated as 136): two prep blocks fit on a CU beside one scan block
// (240 registers per SIMD), so the fill's prep of the next pass runs alongside the scan.
template <bool OUT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_num_vgpr(128))) void k_gdn_prep(PrepBatch pb) {
  const PrepArgs a = pb.a[blockIdx.z];
  __shared__ __align__(16) uint16_t k_s[CH * KST];  // the k tile, then T (fp32)
  __shared__ __align__(16) uint16_t v_s[CH * KST];
  __shared__ __align__(16) float a_s[CH * FST];     // A
  __shared__ float r_s[CH], beta_s[CH], gate_s[CH], gam_s[CH];
  __shared__ __align__(16) uint16_t q_s[OUT ? CH * KST : 8];   // the q tile (outputs only)
  __shared__ float rq_s[OUT ? CH : 1];

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, gi = lane >> 4, ln = lane & 15;
  const int c = blockIdx.x, h = blockIdx.y, rep = a.nv / a.nk, kh = h / rep;
  const int64_t p0 = a.p_begin + static_cast<int64_t>(c) * CH;
  const int m = static_cast<int>(min(static_cast<int64_t>(CH), a.P - p0));
  uint8_t* cbase = a.ws + static_cast<size_t>(c) * a.chunk_bytes;

  // row t's gate inputs first, so their latency overlaps the conv loads
  float braw = 0.f, araw = 0.f;
  if (t < m) {
    const int64_t row = (p0 + t) * a.ld;
    braw = bf2f(a.pre[row + a.C + h]);
    araw = bf2f(a.pre[row + a.C + a.nv + h]);
  }
  {
    ConvIn ik, iv;
    conv_load(a, p0, a.nk * DK + kh * DK, ik);
    conv_load(a, p0, 2 * a.nk * DK + h * DV, iv);
    conv_store(ik, m, k_s);
    conv_store(iv, m, v_s);
  }
  if constexpr (OUT) {
    ConvIn iq;
    conv_load(a, p0, kh * DK, iq);
    conv_store(iq, m, q_s);
  }
  uint8_t* obase = cbase + a.out_off + static_cast<size_t>(h) * OUT_HEAD_BYTES;
  if (t < CH) {
    float beta = 0.f, g = 0.f;
    if (t < m) {
      beta = bf2f(f2bf(1.0f / (1.0f + expf(-braw))));
      const float av = araw + a.dt_bias[h];
      g = -expf(a.a_log[h]) * (av > 20.0f ? av : log1pf(expf(av)));
    }
    beta_s[t] = beta;
    gate_s[t] = g;
  }
  __syncthreads();
  {  // row norms: 4 threads per row
    const int row = t >> 2, q = (t & 3) * 32;
    float s = 0.f;
    for (int e = 0; e < 32; ++e) {
      const float f = bf2f(k_s[row * KST + q + e]);
      s = fmaf(f, f, s);
    }
    s += __shfl_xor(s, 1, 64);
    s += __shfl_xor(s, 2, 64);
    if ((t & 3) == 0) r_s[row] = 1.0f / sqrtf(s + 1e-6f);
    if constexpr (OUT) {
      float sq = 0.f;
      for (int e = 0; e < 32; ++e) {
        const float f = bf2f(q_s[row * KST + q + e]);
        sq = fmaf(f, f, sq);
      }
      sq += __shfl_xor(sq, 1, 64);
      sq += __shfl_xor(sq, 2, 64);
      if ((t & 3) == 0) rq_s[row] = 1.0f / sqrtf(sq + 1e-6f);
    }
  }
  if (t < CH) {  // gamma_t = gate_0 + ... + gate_t, added in row order (the serial cumsum's bits)
    float acc = 0.f;
    for (int i = 0; i <= t; ++i) acc += gate_s[i];
    gam_s[t] = acc;
  }
  // G = K K^T, lower 16 x 16 tiles of tile row `wave`, kept in registers
  f32x4 G[4];
#pragma unroll
  for (int tj = 0; tj < 4; ++tj) {
    G[tj] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (tj > wave) continue;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const uint4 ua = *reinterpret_cast<const uint4*>(k_s + (16 * wave + ln) * KST + 32 * s + 8 * gi);
      const uint4 ub = *reinterpret_cast<const uint4*>(k_s + (16 * tj + ln) * KST + 32 * s + 8 * gi);
      G[tj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_frag(ua), as_frag(ub), G[tj], 0, 0, 0);
    }
  }
  // outputs: QK = Q K^T (raw conv outputs, exact bf16 products), lower tiles of tile row `wave`, and the
  // plain K tile
  f32x4 QK[4];
  if constexpr (OUT) {
#pragma unroll
    for (int tj = 0; tj < 4; ++tj) {
      QK[tj] = f32x4{0.f, 0.f, 0.f, 0.f};
      if (tj > wave) continue;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const uint4 ua = *reinterpret_cast<const uint4*>(q_s + (16 * wave + ln) * KST + 32 * s + 8 * gi);
        const uint4 ub = *reinterpret_cast<const uint4*>(k_s + (16 * tj + ln) * KST + 32 * s + 8 * gi);
        QK[tj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_frag(ua), as_frag(ub), QK[tj], 0, 0, 0);
      }
    }
    uint4* ko = reinterpret_cast<uint4*>(obase + OS_K);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int idx = t + 256 * k, row = idx >> 4, cc = idx & 15;
      ko[idx] = *reinterpret_cast<const uint4*>(k_s + row * KST + cc * 8);
    }
  }
  if (h % rep == 0) {  // K in the scan's operand orders: Kp [it][s][lane][8] = K[16 it + lane % 16][kperm(s, g, e)],
                       // Ktp [t][s][lane][8] = K[kperm(s, g, e)][16 t + lane % 16]
    uint4* kp = reinterpret_cast<uint4*>(cbase + static_cast<size_t>(kh) * KH_BYTES);
    uint4* ktp = reinterpret_cast<uint4*>(cbase + static_cast<size_t>(kh) * KH_BYTES + KP_BYTES);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int idx = t + 256 * k, l = idx & 63, g = l >> 4, n = l & 15;
      {
        const int it = idx >> 8, s = (idx >> 6) & 3;
        const uint16_t* row = k_s + (16 * it + n) * KST + 32 * s + 4 * g;
        const uint2 lo = *reinterpret_cast<const uint2*>(row), hi = *reinterpret_cast<const uint2*>(row + 16);
        kp[idx] = make_uint4(lo.x, lo.y, hi.x, hi.y);
      }
      {
        const int tt = idx >> 7, s = (idx >> 6) & 1;
        uint16_t v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = k_s[kperm(s, g, e) * KST + 16 * tt + n];
        ktp[idx] = make_uint4(pack2(v[0], v[1]), pack2(v[2], v[3]), pack2(v[4], v[5]), pack2(v[6], v[7]));
      }
    }
  }
  __syncthreads();                                  // r_s, gam_s ready; k_s free
  if constexpr (OUT) {
    // Qd[i][e] = q_i[e] rq_i dk^-1/2 e^{gamma_i}; P[i][j] = QK_ij rq_i dk^-1/2 r_j e^{gamma_i - gamma_j}, j <= i
    const float qscale = 0.08838834764831845f;      // 128^-1/2
    float* qd = reinterpret_cast<float*>(obase + OS_QD);
    for (int idx = t; idx < CH * DK; idx += 256) {
      const int i = idx >> 7, e = idx & 127;
      qd[idx] = bf2f(q_s[i * KST + e]) * rq_s[i] * qscale * expf(gam_s[i]);
    }
    float* pm = reinterpret_cast<float*>(obase + OS_P);
#pragma unroll
    for (int tj = 0; tj < 4; ++tj)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * wave + 4 * gi + r, j = 16 * tj + ln;
        pm[i * CH + j] = (tj <= wave && j <= i)
                             ? ((QK[tj][r] * rq_s[i] * qscale) * r_s[j]) * expf(gam_s[i] - gam_s[j])
                             : 0.f;
      }
  }
  // A = tril_{-1}(beta_i (G_ij r_i r_j) e^{gamma_i - gamma_j}); lane (gi, ln) holds G[16 wave + 4 gi + r][16 tj + ln]
#pragma unroll
  for (int tj = 0; tj < 4; ++tj)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = 16 * wave + 4 * gi + r, j = 16 * tj + ln;
      a_s[i * FST + j] = (tj <= wave && j < i)
                             ? (beta_s[i] * (G[tj][r] * r_s[i] * r_s[j])) * expf(gam_s[i] - gam_s[j])
                             : 0.f;
    }
  uint8_t* vbase = cbase + static_cast<size_t>(a.nk) * KH_BYTES + static_cast<size_t>(h) * VH_BYTES;
  {  // V in the scan's accumulator order: Vp [cb][lane][4 it + r] = V[16 it + 4 g + r][16 cb + lane % 16]
    uint4* vp = reinterpret_cast<uint4*>(vbase + TP_BYTES);
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int idx = t + 256 * k, cb = idx >> 6, l = idx & 63, g = l >> 4, n = l & 15;
      uint16_t v[16];
#pragma unroll
      for (int it = 0; it < 4; ++it)
#pragma unroll
        for (int r = 0; r < 4; ++r) v[4 * it + r] = v_s[(16 * it + 4 * g + r) * KST + 16 * cb + n];
      vp[2 * idx] = make_uint4(pack2(v[0], v[1]), pack2(v[2], v[3]), pack2(v[4], v[5]), pack2(v[6], v[7]));
      vp[2 * idx + 1] = make_uint4(pack2(v[8], v[9]), pack2(v[10], v[11]), pack2(v[12], v[13]), pack2(v[14], v[15]));
    }
  }
  if constexpr (OUT) {
    uint4* vo = reinterpret_cast<uint4*>(obase + OS_V);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int idx = t + 256 * k, row = idx >> 4, cc = idx & 15;
      vo[idx] = *reinterpret_cast<const uint4*>(v_s + row * KST + cc * 8);
    }
  }
  if (wave == 1) {
    float* sc = reinterpret_cast<float*>(vbase + TP_BYTES + VP_BYTES);
    const float gl = gam_s[CH - 1];
    sc[SC_BETA + lane] = beta_s[lane];
    sc[SC_Q + lane] = expf(gam_s[lane]) * r_s[lane];
    sc[SC_Z + lane] = r_s[lane] * expf(gl - gam_s[lane]);
    sc[SC_DECAY + lane] = lane == 0 ? expf(gl) : 0.f;
  }
  __syncthreads();                                  // A complete
  float* t_s = reinterpret_cast<float*>(k_s);       // T [64][FST] fp32 in the k tile's space
  float* p_s = reinterpret_cast<float*>(v_s) + wave * 256;   // per-wave 16 x 16 fp32 scratch (V is written out)
  {
    // T = (I + A)^-1 in 16 x 16 blocks (A strictly lower, so T is unit lower triangular). First wave w
    // inverts diagonal block w by forward substitution, T[i][j] = delta_ij - sum_{m < i} A[i][m] T[m][j]
    // within the block, four lanes per column (part p sums the terms m = 4k + p and keeps T[4k + p][j];
    // a quad sum combines the parts; A is zero on and above the diagonal and tk is zero until its row is
    // done, so every term past row i vanishes), and zeroes the blocks right of it.
    const int col = lane >> 2, part = lane & 3, b0 = 16 * wave;
    float tk[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float acc = 0.f;
#pragma unroll
      for (int k = 0; 4 * k < i; ++k) acc = fmaf(-a_s[(b0 + i) * FST + b0 + 4 * k + part], tk[k], acc);
      const float tij = (i == col ? 1.f : 0.f) + quad_sum(acc);
      if (part == (i & 3)) tk[i >> 2] = tij;
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) t_s[(b0 + 4 * k + part) * FST + b0 + col] = tk[k];
    for (int j = wave + 1; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) t_s[(b0 + 4 * e + (lane >> 4)) * FST + 16 * j + (lane & 15)] = 0.f;
  }
  __syncthreads();
  // Then the blocks below the diagonal, one block diagonal at a time (wave j takes block (j + d, j)):
  // T_ij = -T_ii (sum_{m = j .. i-1} A_im T_mj), both products on v_mfma_f32_16x16x4f32 (lane l feeds
  // X[l % 16][l / 16] and Y[l / 16][l % 16] and holds Z[4 (l / 16) + r][l % 16]), fp32 throughout.
  for (int d = 1; d < 4; ++d) {
    if (wave + d < 4) {
      const int bi = wave + d, bj = wave, lr = lane & 15, lk = lane >> 4;
      f32x4 pz = {0.f, 0.f, 0.f, 0.f};
      for (int mb = bj; mb < bi; ++mb)
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
          pz = __builtin_amdgcn_mfma_f32_16x16x4f32(a_s[(16 * bi + lr) * FST + 16 * mb + 4 * ks + lk],
                                                    t_s[(16 * mb + 4 * ks + lk) * FST + 16 * bj + lr], pz, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 4; ++r) p_s[(4 * lk + r) * 16 + lr] = pz[r];
      f32x4 tz = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
        tz = __builtin_amdgcn_mfma_f32_16x16x4f32(t_s[(16 * bi + lr) * FST + 16 * bi + 4 * ks + lk],
                                                  p_s[(4 * ks + lk) * 16 + lr], tz, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 4; ++r) t_s[(16 * bi + 4 * lk + r) * FST + 16 * bj + lr] = -tz[r];
    }
    __syncthreads();
  }
  if constexpr (OUT) {
    float* to = reinterpret_cast<float*>(obase + OS_T);
    for (int idx = t; idx < CH * CH; idx += 256) to[idx] = t_s[(idx >> 6) * FST + (idx & 63)];
  }
  {  // T split hi / lo in the scan's A-operand order: Tp [b][hl][lane][8] = T[16 it + lane % 16][kperm(s, g, e)]
     // for the nonzero blocks b = tp_block(it, s) (the blocks it < 2, s = 1 are zero and not stored)
    uint4* tp = reinterpret_cast<uint4*>(vbase);
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int idx = t + 256 * k, it = idx >> 7, s = (idx >> 6) & 1, l = idx & 63, g = l >> 4, n = l & 15;
      if (it < 2 && s == 1) continue;               // wave-uniform
      float x[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = t_s[(16 * it + n) * FST + kperm(s, g, e)];
      uint4 hi, lo;
      split8(x, hi, lo);
      tp[(tp_block(it, s) * 2 + 0) * 64 + l] = hi;
      tp[(tp_block(it, s) * 2 + 1) * 64 + l] = lo;
    }
  }
}

struct ScanArgs {
  const uint8_t* ws;
  uint32_t chunk_bytes;
  int chunks, nk, nv;
  float* state;             // [nv, DK, DV] fp32, updated in place
  uint8_t* out_ws;          // outputs: the workspace again (written: the state before each chunk)
  uint32_t out_off;
};

// One chunk's operands for wave w of a scan block, straight from the workspace into registers.
struct ScanOps {
  uint4 kp[4];              // K frags (row tile it, k-step w): A operand of X_w = K[:, 32w..] S_w
  uint4 kt[2][2];           // K^T frags (row tile 2w + j, k-step s): A operand of the S update
  uint4 tp[2][2];           // T frags (row tile w, k-step s, hi / lo); k-step 1 used only for w >= 2
  uint2 v;                  // V[16w + 4g + r][16 cb + n], r < 4
  float4 be, qq, zz;        // beta, q, z of rows 16w + 4g + r
  float decay;
};

// Loads of one chunk's operands for wave w, in four groups (the scan spreads them over a step's phases).
struct ScanSrc {
  const uint8_t* kb;        // this wave's lane slot in the key head's K orders
  const uint8_t* vb;        // the value head's block
};

__device__ __forceinline__ ScanSrc scan_src(const uint8_t* chunk, uint32_t kh_off, uint32_t vh_off, int lane) {
  return ScanSrc{chunk + kh_off + lane * 16, chunk + vh_off};
}

__device__ __forceinline__ void load_part(ScanOps& o, const ScanSrc& q, int part, int cb, int w, int lane) {
  if (part == 0) {
#pragma unroll
    for (int it = 0; it < 4; ++it) o.kp[it] = *reinterpret_cast<const uint4*>(q.kb + (it * 4 + w) * 1024);
  } else if (part == 1) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int s = 0; s < 2; ++s)
        o.kt[j][s] = *reinterpret_cast<const uint4*>(q.kb + KP_BYTES + ((2 * w + j) * 2 + s) * 1024);
  } else if (part == 2) {
    // every wave issues the same loads (uniform wait counts); waves 0 and 1 load their k-step 0 block twice
    // (their k-step 1 block is zero and not stored)
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int hl = 0; hl < 2; ++hl)
        o.tp[s][hl] = *reinterpret_cast<const uint4*>(q.vb + (tp_block(w, w < 2 ? 0 : s) * 2 + hl) * 1024 + lane * 16);
  } else {
    o.v = *reinterpret_cast<const uint2*>(q.vb + TP_BYTES + cb * 2048 + lane * 32 + w * 8);
    const float* sc = reinterpret_cast<const float*>(q.vb + TP_BYTES + VP_BYTES);
    const int r0 = 16 * w + 4 * (lane >> 4);
    o.be = *reinterpret_cast<const float4*>(sc + SC_BETA + r0);
    o.qq = *reinterpret_cast<const float4*>(sc + SC_Q + r0);
    o.zz = *reinterpret_cast<const float4*>(sc + SC_Z + r0);
    o.decay = sc[SC_DECAY];
  }
}

// 4 values -> hi (truncated to bf16) and lo (the rest rounded to bf16), as split8.
__device__ __forceinline__ void split4(const float (&x)[4], uint2& hi, uint2& lo) {
  uint32_t h[4];
  float r[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t u = __float_as_uint(x[e]) & 0xffff0000u;
    h[e] = u >> 16;
    r[e] = x[e] - __uint_as_float(u);
  }
  hi = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
  lo = make_uint2(bf16_pair(r[0], r[1]), bf16_pair(r[2], r[3]));
}

// Block = (value head, 16-column block), 4 waves, one per SIMD. Wave w keeps state rows 32w .. 32w + 31
// (row tiles 2w, 2w + 1, accumulator layout) and per chunk:
//   X_w = K[:, 32w .. 32w + 31] S_w (its k-step of X = K S), then the four X_w meet in LDS and X = the
//   sum over w in order; wave w forms row tile w of Y = beta (V - q X) and of v_new = T Y (T lower
//   triangular: tiles 0 and 1 need k-step 0 only), and row tile w of Z = z v_new; Y and Z are shared as
//   hi / lo bf16 B-operand frags through LDS; S_w <- decay S_w + K^T[32w .., :] Z.
// Three barriers per chunk; the operands of the chunk two steps ahead load into registers meanwhile,
// in four groups between the phases so the address unit streams them in the background.
struct ScanBatch {
  ScanArgs a[BATCH];
};

template <bool OUT>
__global__ __launch_bounds__(256) void k_gdn_scan(ScanBatch sbatch) {
  const int per_layer = sbatch.a[0].nv * 8;
  const int layer = blockIdx.x / per_layer;
  const ScanArgs a = sbatch.a[layer];
  __shared__ __align__(16) f32x4 xp[4][4][64];        // X_w partials [wave][row tile][lane]
  __shared__ __align__(16) uint4 yf[2][2][64];        // Y frags [k-step][hi / lo][lane]
  __shared__ __align__(16) uint4 zf[2][2][64];        // Z frags
  const int t = threadIdx.x, lane = t & 63, w = t >> 6, gi = lane >> 4, ln = lane & 15;
  // block b runs on XCD b % 8: XCD x takes (head, column block) pairs [x nv, (x + 1) nv), so the
  // blocks that share a head's (and a key head's) operands share an L2
  const int b = blockIdx.x - layer * per_layer, pair = (b & 7) * a.nv + (b >> 3);
  const int h = pair >> 3, cb = pair & 7, kh = h / (a.nv / a.nk);
  float* st = a.state + static_cast<size_t>(h) * DK * DV + cb * 16 + ln;
  f32x4 S[2];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) S[j][r] = st[(16 * (2 * w + j) + 4 * gi + r) * DV];

  const uint32_t kh_off = static_cast<uint32_t>(kh) * KH_BYTES;
  const uint32_t vh_off = static_cast<uint32_t>(a.nk) * KH_BYTES + static_cast<uint32_t>(h) * VH_BYTES;
  // One chunk step from its operands o; the four load groups of the chunk two steps on go out between
  // the phases into L (the buffer the previous step freed). Past the last chunk (active false) only the
  // loads run, so every path issues the same loads and waits on the same counts.
  auto step = [&](const ScanOps& o, ScanOps& L, const ScanSrc& from, bool active, int cidx) {
    if constexpr (OUT) {
      if (active) {                                 // the state before chunk cidx, for the outputs
        float* sp = reinterpret_cast<float*>(a.out_ws + static_cast<size_t>(cidx) * a.chunk_bytes + a.out_off +
                                             static_cast<size_t>(h) * OUT_HEAD_BYTES + OS_S) + cb * 16 + ln;
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) sp[(16 * (2 * w + j) + 4 * gi + r) * DV] = S[j][r];
      }
    }
    if (active) {
      // X_w = K[:, 32w ..] S_w: S_w's rows in k-step order are (tile 2w, r) then (tile 2w + 1, r)
      {
        float x[8];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          x[r] = S[0][r];
          x[4 + r] = S[1][r];
        }
        uint4 bh, bl;
        split8(x, bh, bl);
#pragma unroll
        for (int it = 0; it < 4; ++it) {
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_frag(o.kp[it]), as_frag(bh), acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_frag(o.kp[it]), as_frag(bl), acc, 0, 0, 0);
          xp[w][it][lane] = acc;
        }
      }
    }
    load_part(L, from, 0, cb, w, lane);
    if (active) {
      __syncthreads();
      // row tile w: X, Y = beta (V - q X), its hi / lo halves into k-step w / 2, slots 4 (w % 2) ..
      {
        f32x4 X = xp[0][w][lane];
#pragma unroll
        for (int q = 1; q < 4; ++q) X += xp[q][w][lane];
        const float bb[4] = {o.be.x, o.be.y, o.be.z, o.be.w}, q4[4] = {o.qq.x, o.qq.y, o.qq.z, o.qq.w};
        const uint32_t vv[2] = {o.v.x, o.v.y};
        float y[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float v = bf2f((vv[r >> 1] >> (16 * (r & 1))) & 0xffffu);
          y[r] = bb[r] * (v - q4[r] * X[r]);
        }
        uint2 hi, lo;
        split4(y, hi, lo);
        reinterpret_cast<uint2*>(&yf[w >> 1][0][lane])[w & 1] = hi;
        reinterpret_cast<uint2*>(&yf[w >> 1][1][lane])[w & 1] = lo;
      }
    }
    load_part(L, from, 1, cb, w, lane);
    if (active) {
      __syncthreads();
      // v_new row tile w = sum over k-steps of T Y; Z = z v_new into the Z frags
      {
        f32x4 vn = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          if (s == 1 && w < 2) continue;
          const bf16x8 th = as_frag(o.tp[s][0]), tl = as_frag(o.tp[s][1]);
          const bf16x8 yh = as_frag(yf[s][0][lane]), yl = as_frag(yf[s][1][lane]);
          vn = __builtin_amdgcn_mfma_f32_16x16x32_bf16(th, yh, vn, 0, 0, 0);
          vn = __builtin_amdgcn_mfma_f32_16x16x32_bf16(th, yl, vn, 0, 0, 0);
          vn = __builtin_amdgcn_mfma_f32_16x16x32_bf16(tl, yh, vn, 0, 0, 0);
        }
        const float z4[4] = {o.zz.x, o.zz.y, o.zz.z, o.zz.w};
        float z[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) z[r] = z4[r] * vn[r];
        uint2 hi, lo;
        split4(z, hi, lo);
        reinterpret_cast<uint2*>(&zf[w >> 1][0][lane])[w & 1] = hi;
        reinterpret_cast<uint2*>(&zf[w >> 1][1][lane])[w & 1] = lo;
      }
    }
    load_part(L, from, 2, cb, w, lane);
    if (active) {
      __syncthreads();
      // S_w <- decay S_w + K^T Z
      {
        bf16x8 zh[2], zl[2];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          zh[s] = as_frag(zf[s][0][lane]);
          zl[s] = as_frag(zf[s][1][lane]);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          f32x4 acc = S[j] * o.decay;
#pragma unroll
          for (int s = 0; s < 2; ++s) {
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_frag(o.kt[j][s]), zh[s], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_frag(o.kt[j][s]), zl[s], acc, 0, 0, 0);
          }
          S[j] = acc;
        }
      }
    }
    load_part(L, from, 3, cb, w, lane);
  };
  auto src = [&](int c) {
    return scan_src(a.ws + static_cast<size_t>(min(c, a.chunks - 1)) * a.chunk_bytes, kh_off, vh_off, lane);
  };
  // three buffers in rotation: chunk c + 2 loads during chunk c's step (indices past the last chunk reload
  // it; those copies are never used)
  ScanOps b0, b1, b2;
  for (int part = 0; part < 4; ++part) {
    load_part(b0, src(0), part, cb, w, lane);
    load_part(b1, src(1), part, cb, w, lane);
  }
  // Wait for the two prologue chunks here, once. The compiler may issue the prologue loads in any order
  // (chunk 0's first operands last), and the wait counts at the loop head merge that entry with the back
  // edge: without this wait every step would start with a wait for all but the newest few loads, which
  // leaves the chunk-ahead loads no time in flight.
  __builtin_amdgcn_s_waitcnt(0x0f70);               // vmcnt(0)
  for (int c = 0; c < a.chunks; c += 3) {
    step(b0, b2, src(c + 2), true, c);
    step(b1, b0, src(c + 3), c + 1 < a.chunks, c + 1);
    step(b2, b1, src(c + 4), c + 2 < a.chunks, c + 2);
  }
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) st[(16 * (2 * w + j) + 4 * gi + r) * DV] = S[j][r];
}

struct OutArgs {
  const uint8_t* ws;
  uint32_t chunk_bytes, out_off;
  int nk;
  int64_t P, p_begin;
  uint16_t* out;            // [P, >= nv DV] bf16
  int64_t ldo;
};

constexpr int SST = DV + 4;                        // fp32 row stride of S and Y in LDS

// Block = (chunk, value head h); wave w forms output rows 16w .. 16w + 15 of the chunk. On
// v_mfma_f32_16x16x4f32 (lane l feeds A[l % 16][l / 16] and B[l / 16][l % 16], holds D[4 (l / 16) + r][l % 16]):
//   X = K S, Y = beta (V - q X) (q = e^gamma r), v_new = T Y, O = Qd S + P v_new
// with S the state before the chunk (LDS), Y then v_new shared through LDS; fp32 throughout, bf16 out.
// T and P are lower triangular, but their products run over all 16 k-steps: two other shapes (a trip
// count taken from the wave index; the k-steps unrolled by 8) gave wrong products. Both compiled to
// accumulators rotated through v_accvgpr moves at the loop head, the first read 6 wait states after an
// 8-pass MFMA. The shape used compiles fully unrolled: 768 MFMAs, no v_accvgpr moves or writes, and at
// least 10 wait states between an MFMA and the first read of its result. The wave index is made
// wave-uniform (an SGPR), which changes only the address arithmetic. Each product loads all its A values
// first and reads the next k-step's B values from LDS before the current step's MFMAs (a scheduling
// barrier keeps that order; left to itself the compiler read each pair of B values just before its two
// MFMAs and waited on LDS before each pair). The code keeps those properties (768 MFMAs, no v_accvgpr
// moves, at least 10 wait states). The outputs are checked against the oracle's chunked rule at the
// hybrid's widths, and any change here must be rechecked on the GPU.
__global__ __launch_bounds__(256) void k_gdn_out(OutArgs a) {
  __shared__ __align__(16) float s_l[DK * SST];
  __shared__ __align__(16) float y_l[CH * SST];
  const int t = threadIdx.x, lane = t & 63, lr = lane & 15, lk = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);
  const int c = blockIdx.x, h = blockIdx.y;
  const uint8_t* chunk = a.ws + static_cast<size_t>(c) * a.chunk_bytes;
  const uint8_t* ob = chunk + a.out_off + static_cast<size_t>(h) * OUT_HEAD_BYTES;
  const float* S = reinterpret_cast<const float*>(ob + OS_S);
  const float* Qd = reinterpret_cast<const float*>(ob + OS_QD);
  const float* Pm = reinterpret_cast<const float*>(ob + OS_P);
  const float* T = reinterpret_cast<const float*>(ob + OS_T);
  const uint16_t* K = reinterpret_cast<const uint16_t*>(ob + OS_K);
  const uint16_t* V = reinterpret_cast<const uint16_t*>(ob + OS_V);
  const float* sc = reinterpret_cast<const float*>(chunk + static_cast<size_t>(a.nk) * KH_BYTES +
                                                   static_cast<size_t>(h) * VH_BYTES + TP_BYTES + VP_BYTES);
  for (int i = t; i < DK * DV / 4; i += 256) {
    const int row = i / (DV / 4), c4 = i % (DV / 4);
    *reinterpret_cast<float4*>(s_l + row * SST + 4 * c4) = reinterpret_cast<const float4*>(S)[i];
  }
  __syncthreads();
  const int r0 = 16 * w;
  f32x4 acc[8];
  // acc += A B over NKS 4-deep k-steps: A from a_of(ks) (this lane's row r0 + lr, k 4 ks + lk), B from the
  // LDS rows bl (row 4 ks + lk, column 16 nt + lr), the next k-step's B values read before this step's MFMAs
  auto product = [&](auto a_of, const float* bl, auto nks_c) {
    constexpr int NKS = decltype(nks_c)::value;
    float avs[NKS];                                 // every A value of the product in flight at once
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) avs[ks] = a_of(ks);
    float bv[2][8];
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) bv[0][nt] = bl[lk * SST + 16 * nt + lr];
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      const float av = avs[ks];
      if (ks + 1 < NKS) {
#pragma unroll
        for (int nt = 0; nt < 8; ++nt) bv[(ks + 1) & 1][nt] = bl[(4 * (ks + 1) + lk) * SST + 16 * nt + lr];
      }
      __builtin_amdgcn_sched_barrier(0);            // (the reads stay ahead of this step's MFMAs)
#pragma unroll
      for (int nt = 0; nt < 8; ++nt)
        acc[nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv[ks & 1][nt], acc[nt], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) acc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
  product([&](int ks) { return bf2f(K[(r0 + lr) * DK + 4 * ks + lk]); }, s_l,     // X = K S
          std::integral_constant<int, DK / 4>{});
#pragma unroll
  for (int r = 0; r < 4; ++r) {                     // Y = beta (V - q X)
    const int i = r0 + 4 * lk + r;
    const float be = sc[SC_BETA + i], qs = sc[SC_Q + i];
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      const int col = 16 * nt + lr;
      y_l[i * SST + col] = be * (bf2f(V[i * DV + col]) - qs * acc[nt][r]);
    }
  }
  __syncthreads();
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) acc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
  product([&](int ks) { return T[(r0 + lr) * CH + 4 * ks + lk]; }, y_l,            // v_new = T Y
          std::integral_constant<int, CH / 4>{});
  __syncthreads();                                  // every wave has read Y
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) y_l[(r0 + 4 * lk + r) * SST + 16 * nt + lr] = acc[nt][r];
  __syncthreads();
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) acc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
  product([&](int ks) { return Qd[(r0 + lr) * DK + 4 * ks + lk]; }, s_l,           // O = Qd S ...
          std::integral_constant<int, DK / 4>{});
  product([&](int ks) { return Pm[(r0 + lr) * CH + 4 * ks + lk]; }, y_l,           // ... + P v_new
          std::integral_constant<int, CH / 4>{});
  const int64_t p0 = a.p_begin + static_cast<int64_t>(c) * CH;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int64_t p = p0 + r0 + 4 * lk + r;
    if (p >= a.P) continue;
    uint16_t* dst = a.out + p * a.ldo + static_cast<int64_t>(h) * DV + lr;
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) dst[16 * nt] = f2bf(acc[nt][r]);
  }
}

// conv_out[j][ch] = row P - 3 + j of [conv_in; pre] (conv_in rows -3..-1; zeros if conv_in is null)
__global__ void k_conv_tail(const uint16_t* pre, int64_t ld, int64_t P, int C, const uint16_t* conv_in,
                            uint16_t* conv_out) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= 3 * C) return;
  const int j = idx / C, ch = idx % C;
  const int64_t p = P - 3 + j;
  uint16_t v = 0;
  if (p >= 0) v = pre[p * ld + ch];
  else if (conv_in) v = conv_in[(3 + p) * C + ch];
  conv_out[idx] = v;
}

inline uint32_t chunk_bytes(int nk, int nv) { return static_cast<uint32_t>(nk) * KH_BYTES + static_cast<uint32_t>(nv) * VH_BYTES; }

int check_heads(const char* fn, int nk, int nv, int dk, int dv) {
  if (dk != DK || dv != DV) return fail(RF_EUNSUPPORTED, "%s: key / value head dims %d / %d (128 / 128)", fn, dk, dv);
  if (nk <= 0 || nv <= 0 || nv % nk || nv > 1024) return fail(RF_EINVAL_SHAPE, "%s: heads nk %d nv %d", fn, nk, nv);
  return RF_OK;
}

}  // namespace
}  // namespace rf

using namespace rf;

extern "C" int rf_gdn_workspace_bytes(int64_t rows, int nk, int nv, int dk, int dv, size_t* bytes) {
  if (const int e = check_heads("rf_gdn_workspace_bytes", nk, nv, dk, dv)) return e;
  if (rows < 0 || !bytes) return fail(RF_EINVAL_ARG, "rf_gdn_workspace_bytes: rows %lld", (long long)rows);
  const int64_t chunks = rows > 0 ? (rows + CH - 1) / CH : 1;
  *bytes = static_cast<size_t>(chunks) * chunk_bytes(nk, nv);
  return RF_OK;
}

extern "C" int rf_gdn_forward_workspace_bytes(int64_t rows, int nk, int nv, int dk, int dv, size_t* bytes) {
  if (const int e = check_heads("rf_gdn_forward_workspace_bytes", nk, nv, dk, dv)) return e;
  if (rows < 0 || !bytes) return fail(RF_EINVAL_ARG, "rf_gdn_forward_workspace_bytes: rows %lld", (long long)rows);
  const int64_t chunks = rows > 0 ? (rows + CH - 1) / CH : 1;
  *bytes = static_cast<size_t>(chunks) * (chunk_bytes(nk, nv) + static_cast<size_t>(nv) * OUT_HEAD_BYTES);
  return RF_OK;
}

namespace {

// One layer's operands of a GDN fill or forward.
struct LayerIO {
  const uint16_t* pre;
  int64_t ld;
  const uint16_t* conv_w;
  const uint16_t* conv_in;
  uint16_t* conv_out;
  const float* a_log;
  const float* dt_bias;
  float* state;
};

constexpr int MAX_DEVICES = 64;

// A second stream per device (default priority) for the fill's prep launches, and the events that order
// them against the scans on the caller's stream; made on first use with that device current and kept.
struct SideQueue {
  bool tried = false;
  hipStream_t stream = nullptr;
  hipEvent_t start = nullptr;
  hipEvent_t prepped[2] = {nullptr, nullptr};       // prep of the pass in buffer b written
  hipEvent_t scanned[2] = {nullptr, nullptr};       // scan of the pass in buffer b done reading
};

std::mutex g_side_mu;
SideQueue g_side[MAX_DEVICES];

// The current device's side queue (g_side_mu held), or null when it cannot be made or the caller's stream
// belongs to another device: the fill then runs both kernels on the caller's stream.
SideQueue* side_queue(hipStream_t stream) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) {
    (void)hipGetLastError();
    return nullptr;
  }
  if (stream) {
    hipDevice_t sdev = -1;
    if (hipStreamGetDevice(stream, &sdev) != hipSuccess || sdev != dev) {
      (void)hipGetLastError();
      return nullptr;
    }
  }
  SideQueue& q = g_side[dev];
  if (!q.tried) {
    q.tried = true;
    bool ok = hipStreamCreateWithFlags(&q.stream, hipStreamNonBlocking) == hipSuccess;
    ok = ok && hipEventCreateWithFlags(&q.start, hipEventDisableTiming) == hipSuccess;
    for (int b = 0; b < 2; ++b) {
      ok = ok && hipEventCreateWithFlags(&q.prepped[b], hipEventDisableTiming) == hipSuccess;
      ok = ok && hipEventCreateWithFlags(&q.scanned[b], hipEventDisableTiming) == hipSuccess;
    }
    if (!ok) {
      (void)hipGetLastError();
      q.stream = nullptr;                           // handles made before the failure are kept, unused
    }
  }
  return q.stream ? &q : nullptr;
}

int conv_tails(const char* fn, const LayerIO* io, int n, int64_t P, int C, hipStream_t stream) {
  for (int l = 0; l < n; ++l) {
    hipLaunchKernelGGL(k_conv_tail, dim3((3 * C + 255) / 256), dim3(256), 0, stream, io[l].pre, io[l].ld, P, C,
                       io[l].conv_in, io[l].conv_out);
    if (const int e = check_launch(fn)) return e;
  }
  return RF_OK;
}

int hip_check(const char* fn, hipError_t e, const char* what) {
  return e == hipSuccess ? RF_OK : fail(RF_EHIP, "%s: %s: %s", fn, what, hipGetErrorString(e));
}

// The fill of n layers as one pipeline of passes (every pass of layer 0, then of layer 1, ...) through two
// workspace buffers: the scan of pass i (the caller's stream) runs while the prep of pass i + 1 (the side
// stream) writes the other buffer. A scan block (one per CU, one wave per SIMD) leaves room on its CU for
// two prep blocks; the two kernels slow each other (the scan's chunk steps wait on memory behind the
// prep's traffic), so the gain over one stream is about a tenth for one layer, and two layers do better
// with their scans side by side in one launch (gdn_run's batched passes). Pass
// i's prep waits for the scan of pass i - 2 (its buffer's last reader); the caller's stream waits for every
// prep through the scans, so work queued after the fill on that stream is ordered after all of it. Every
// chunk runs the same arithmetic as in the one-stream schedule: the results are bit-identical.
int fill_overlapped(const char* fn, SideQueue& q, const LayerIO* io, int n, int64_t P, int nk, int nv, int C,
                    uint8_t* ws, int64_t per_pass, size_t half, uint32_t cbytes, uint32_t sbytes, hipStream_t stream) {
  const int64_t chunks = (P + CH - 1) / CH;
  if (const int e = hip_check(fn, hipEventRecord(q.start, stream), "hipEventRecord")) return e;
  if (const int e = hip_check(fn, hipStreamWaitEvent(q.stream, q.start, 0), "hipStreamWaitEvent")) return e;
  int64_t item = 0;
  for (int l = 0; l < n; ++l) {
    const LayerIO& L = io[l];
    for (int64_t c0 = 0; c0 < chunks; c0 += per_pass, ++item) {
      const int nc = static_cast<int>(std::min<int64_t>(per_pass, chunks - c0));
      const int b = static_cast<int>(item & 1);
      uint8_t* wb = ws + b * half;
      if (item >= 2)
        if (const int e = hip_check(fn, hipStreamWaitEvent(q.stream, q.scanned[b], 0), "hipStreamWaitEvent")) return e;
      PrepBatch pb{};
      pb.a[0] = PrepArgs{L.pre, L.ld, P, c0 * CH, nk, nv, C, L.conv_w, L.conv_in, L.a_log, L.dt_bias, wb, cbytes, sbytes};
      hipLaunchKernelGGL(k_gdn_prep<false>, dim3(nc, nv, 1), dim3(256), 0, q.stream, pb);
      if (const int e = check_launch(fn)) return e;
      if (const int e = hip_check(fn, hipEventRecord(q.prepped[b], q.stream), "hipEventRecord")) return e;
      if (const int e = hip_check(fn, hipStreamWaitEvent(stream, q.prepped[b], 0), "hipStreamWaitEvent")) return e;
      ScanBatch sb{};
      sb.a[0] = ScanArgs{wb, cbytes, nc, nk, nv, L.state, wb, sbytes};
      hipLaunchKernelGGL(k_gdn_scan<false>, dim3(nv * 8), dim3(256), 0, stream, sb);
      if (const int e = check_launch(fn)) return e;
      if (const int e = hip_check(fn, hipEventRecord(q.scanned[b], stream), "hipEventRecord")) return e;
    }
  }
  return RF_OK;
}

// The fill (out null) or the forward (one layer, out given) of n layers over the same P rows. The fill with
// `overlap` runs fill_overlapped when the workspace holds two chunks (and the side queue exists); otherwise,
// per pass of up to what each layer's share of the workspace holds, one prep and one scan launch cover every
// layer on the caller's stream.
int gdn_run(const char* fn, const LayerIO* io, int n, int64_t P, int nk, int nv, int dk, int dv, uint16_t* out,
            int64_t ldo, void* workspace, size_t ws_bytes, hipStream_t stream, bool overlap = false) {
  if (n < 1 || n > BATCH || (out && n != 1)) return fail(RF_EINVAL_ARG, "%s: %d layers (1 .. %d)", fn, n, BATCH);
  if (!workspace) return fail(RF_EINVAL_ARG, "%s: null workspace", fn);
  if (const int e = check_heads(fn, nk, nv, dk, dv)) return e;
  const int64_t C = 2ll * nk * DK + static_cast<int64_t>(nv) * DV;
  for (int l = 0; l < n; ++l) {
    const LayerIO& L = io[l];
    if (!L.pre || !L.conv_w || !L.conv_out || !L.a_log || !L.dt_bias || !L.state)
      return fail(RF_EINVAL_ARG, "%s: null pointer (layer %d)", fn, l);
    if (P < 0 || L.ld < C + 2 * nv || L.ld % 8)
      return fail(RF_EINVAL_SHAPE, "%s: P %lld, ld %lld (need >= %lld and a multiple of 8)", fn, (long long)P,
                  (long long)L.ld, (long long)(C + 2 * nv));
    if (!aligned16(L.pre) || !aligned16(L.conv_w) || (L.conv_in && !aligned16(L.conv_in)))
      return fail(RF_EINVAL_ARG, "%s: pre, conv_w and conv_in must be 16-byte aligned", fn);
    if (L.conv_in == L.conv_out) return fail(RF_EINVAL_ARG, "%s: conv_out must not alias conv_in", fn);
    for (int m = 0; m < l; ++m)
      if (io[m].state == L.state || io[m].conv_out == L.conv_out)
        return fail(RF_EINVAL_ARG, "%s: layers %d and %d share a state or conv_out buffer", fn, m, l);
  }
  if (out && (ldo < static_cast<int64_t>(nv) * DV || ldo % 8))
    return fail(RF_EINVAL_SHAPE, "%s: ldo %lld (>= nv dv = %d, a multiple of 8)", fn, (long long)ldo, nv * DV);
  if (!aligned16(workspace)) return fail(RF_EINVAL_ARG, "%s: workspace must be 16-byte aligned", fn);
  const uint32_t sbytes = chunk_bytes(nk, nv);
  const uint64_t cb64 = sbytes + (out ? static_cast<uint64_t>(nv) * OUT_HEAD_BYTES : 0);
  if (cb64 > 0x7fffffffull) return fail(RF_EINVAL_SHAPE, "%s: %d value heads", fn, nv);
  const uint32_t cbytes = static_cast<uint32_t>(cb64);
  const int64_t chunks = (P + CH - 1) / CH;
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  if (overlap && !out && chunks > 0) {
    // two buffers, each of up to what half the workspace holds (buffer offsets below 2^31)
    const size_t half = ws_bytes / 2 / 16 * 16;
    const int64_t pp = std::min<int64_t>(static_cast<int64_t>(half / cbytes), 0x7fffffffll / cbytes);
    if (pp >= 1) {
      std::lock_guard<std::mutex> lock(g_side_mu);
      if (SideQueue* q = side_queue(stream)) {
        if (const int e = fill_overlapped(fn, *q, io, n, P, nk, nv, static_cast<int>(C), ws, pp, half, cbytes, sbytes,
                                          stream))
          return e;
        return conv_tails(fn, io, n, P, static_cast<int>(C), stream);
      }
    }
  }
  // each layer's share of the workspace (16-byte aligned); chunks per pass: what a share holds, with buffer
  // offsets below 2^31
  const size_t share = ws_bytes / n / 16 * 16;
  const int64_t per_pass = std::min<int64_t>(static_cast<int64_t>(share / cbytes), 0x7fffffffll / cbytes);
  if (per_pass < 1)
    return fail(RF_EINVAL_ARG, "%s: workspace %zu bytes < %d chunks (%u bytes each)", fn, ws_bytes, n, cbytes);
  for (int64_t c0 = 0; c0 < chunks; c0 += per_pass) {
    const int nc = static_cast<int>(std::min<int64_t>(per_pass, chunks - c0));
    PrepBatch pb{};
    ScanBatch sb{};
    for (int l = 0; l < n; ++l) {
      const LayerIO& L = io[l];
      uint8_t* wl = ws + l * share;
      pb.a[l] = PrepArgs{L.pre, L.ld, P, c0 * CH, nk, nv, static_cast<int>(C), L.conv_w, L.conv_in, L.a_log,
                         L.dt_bias, wl, cbytes, sbytes};
      sb.a[l] = ScanArgs{wl, cbytes, nc, nk, nv, L.state, wl, sbytes};
    }
    if (out) {
      hipLaunchKernelGGL(k_gdn_prep<true>, dim3(nc, nv, 1), dim3(256), 0, stream, pb);
      if (const int e = check_launch(fn)) return e;
      hipLaunchKernelGGL(k_gdn_scan<true>, dim3(nv * 8), dim3(256), 0, stream, sb);
      if (const int e = check_launch(fn)) return e;
      OutArgs oa{ws, cbytes, sbytes, nk, P, c0 * CH, out, ldo};
      hipLaunchKernelGGL(k_gdn_out, dim3(nc, nv), dim3(256), 0, stream, oa);
      if (const int e = check_launch(fn)) return e;
    } else {
      hipLaunchKernelGGL(k_gdn_prep<false>, dim3(nc, nv, n), dim3(256), 0, stream, pb);
      if (const int e = check_launch(fn)) return e;
      hipLaunchKernelGGL(k_gdn_scan<false>, dim3(nv * 8 * n), dim3(256), 0, stream, sb);
      if (const int e = check_launch(fn)) return e;
    }
  }
  return conv_tails(fn, io, n, P, static_cast<int>(C), stream);
}

}  // namespace

extern "C" int rf_gdn_fill(const uint16_t* pre, int64_t ld, int64_t P, int nk, int nv, int dk, int dv,
                           const uint16_t* conv_w, const uint16_t* conv_in, uint16_t* conv_out, const float* a_log,
                           const float* dt_bias, float* state, void* workspace, size_t ws_bytes, hipStream_t stream) {
  const LayerIO io{pre, ld, conv_w, conv_in, conv_out, a_log, dt_bias, state};
  return gdn_run("rf_gdn_fill", &io, 1, P, nk, nv, dk, dv, nullptr, 0, workspace, ws_bytes, stream, true);
}

extern "C" int rf_gdn_fill_batch(const rf_gdn_layer* layers, int n_layers, int64_t P, int nk, int nv, int dk, int dv,
                                 void* workspace, size_t ws_bytes, hipStream_t stream) {
  if (!layers) return fail(RF_EINVAL_ARG, "rf_gdn_fill_batch: null layers");
  if (n_layers < 1 || n_layers > RF_GDN_BATCH_MAX)
    return fail(RF_EINVAL_ARG, "rf_gdn_fill_batch: %d layers (1 .. %d)", n_layers, RF_GDN_BATCH_MAX);
  LayerIO io[RF_GDN_BATCH_MAX];
  for (int l = 0; l < n_layers; ++l) {
    const rf_gdn_layer& L = layers[l];
    io[l] = LayerIO{L.pre, L.ld, L.conv_w, L.conv_in, L.conv_out, L.a_log, L.dt_bias, L.state};
  }
  // two layers: their scans side by side in one launch (two blocks per CU) beat one layer's scan beside the
  // next pass's prep
  return gdn_run("rf_gdn_fill_batch", io, n_layers, P, nk, nv, dk, dv, nullptr, 0, workspace, ws_bytes, stream,
                 n_layers == 1);
}

// ---- allocation-free GDN fill: the per-chunk workspace lives in a file-scope device array

namespace {

constexpr size_t GDN_SCRATCH_BYTES = static_cast<size_t>(RF_GDN_SCRATCH_MAX) << 20;

// The workspace of rf_gdn_fill_noalloc: one copy per GPU (at its own address), held until the process ends.
// Its name is a host-side stand-in: host code uses only the per-device addresses taken below.
static __device__ __align__(256) uint8_t scratch[GDN_SCRATCH_BYTES];

std::mutex g_scratch_mu;
void* g_scratch_ptr[MAX_DEVICES] = {};

// The current device's address of `scratch`, taken once per device (with that device current) and kept.
int scratch_address(const char* fn, hipStream_t stream, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(RF_EHIP, "%s: hipGetDevice: %s", fn, hipGetErrorString(e));
  if (dev < 0 || dev >= MAX_DEVICES) return fail(RF_EINVAL_ARG, "%s: device %d (at most %d)", fn, dev, MAX_DEVICES);
  if (stream) {
    hipDevice_t sdev = -1;
    e = hipStreamGetDevice(stream, &sdev);
    if (e != hipSuccess) return fail(RF_EHIP, "%s: hipStreamGetDevice: %s", fn, hipGetErrorString(e));
    if (sdev != dev)
      return fail(RF_EINVAL_ARG, "%s: the stream belongs to device %d, device %d is current", fn, sdev, dev);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return fail(RF_EHIP, "%s: hipGetSymbolAddress of the scratch array: %s", fn, hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return RF_OK;
}

}  // namespace

extern "C" int rf_gdn_fill_noalloc(const uint16_t* pre, int64_t ld, int64_t P, int nk, int nv, int dk, int dv,
                                   const uint16_t* conv_w, const uint16_t* conv_in, uint16_t* conv_out,
                                   const float* a_log, const float* dt_bias, float* state, hipStream_t stream) {
  const char* fn = "rf_gdn_fill_noalloc";
  if (const int e = check_heads(fn, nk, nv, dk, dv)) return e;
  const size_t per_chunk = chunk_bytes(nk, nv);
  if (per_chunk > GDN_SCRATCH_BYTES)
    return fail(RF_EINVAL_SHAPE, "%s: %d key / %d value heads need %zu bytes per 64-row chunk, more than the %zu-byte "
                "scratch array (RF_GDN_SCRATCH_MAX MiB); use rf_gdn_fill with a workspace", fn, nk, nv, per_chunk,
                GDN_SCRATCH_BYTES);
  void* ws = nullptr;
  if (const int e = scratch_address(fn, stream, &ws)) return e;
  const LayerIO io{pre, ld, conv_w, conv_in, conv_out, a_log, dt_bias, state};
  return gdn_run(fn, &io, 1, P, nk, nv, dk, dv, nullptr, 0, ws, GDN_SCRATCH_BYTES, stream);
}

extern "C" int rf_gdn_forward(const uint16_t* pre, int64_t ld, int64_t P, int nk, int nv, int dk, int dv,
                              const uint16_t* conv_w, const uint16_t* conv_in, uint16_t* conv_out, const float* a_log,
                              const float* dt_bias, float* state, uint16_t* out, int64_t ldo, void* workspace,
                              size_t ws_bytes, hipStream_t stream) {
  if (!out) return fail(RF_EINVAL_ARG, "rf_gdn_forward: null out");
  const LayerIO io{pre, ld, conv_w, conv_in, conv_out, a_log, dt_bias, state};
  return gdn_run("rf_gdn_forward", &io, 1, P, nk, nv, dk, dv, out, ldo, workspace, ws_bytes, stream);
}
