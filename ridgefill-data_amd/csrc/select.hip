// Exact-row selection by window attention mass (the "qattn" selector, code/kva/select.py:223-245
// window_mass): for one exact lower attention layer, the attention probability every key row receives
// from the w window query rows at positions pos0 .. pos0 + w - 1, summed over the query rows and all
// query heads, dense causal softmax over every key (key j visible to a query at position p iff j <= p).
// Per K / V head group g the rows are R = rep * w (query head g rep + r / w, window row r % w).
//
//   k_mass_stats (key block of 256 x group): S^T = K Q^T on v_mfma_f32_32x32x16_bf16 (A = the key block
//       from LDS, B = 32 query rows from memory): a lane holds, for one row, the scores of 16 keys of each
//       32-key step, so each row's block maximum and sum of 2^(s c - max) are lane-local plus one
//       exchange between the lane halves; written per (row, key block);
//   k_mass_rows: per row, the maximum M and the sum L over the key blocks (one wave per row, a fixed
//       merge order);
//   k_mass_cols (key block x group): S = Q K^T on the same MFMA with the roles swapped (A = 32 query rows,
//       B = the keys): a lane now holds, for one key, the scores of 16 rows of each 32-row step, so the
//       column sums of P = 2^(s c - M) / L over the rows are lane-local; rows in order, then the two lane
//       halves; one fp32 partial per (group, key);
//   k_mass_fold: mass[j] += the groups' partials as fp64, in group order (the fp64 accumulator the
//       caller keeps over layers, as window_mass's fp64 sum over layers and groups).
// c = scale * log2(e): base-2 softmax, the same probabilities within fp32 rounding.
#include <stdint.h>

#include <algorithm>

#include "rf_common.h"

namespace rf {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int MKB = 256;                    // keys per block

__device__ __forceinline__ bf16x8 as_frag(const uint4& u) { return __builtin_bit_cast(bf16x8, u); }

struct MassArgs {
  const uint16_t* q;        // [w, >= hq * d]: window row i, query head h at q + i * ldq + h * d
  int64_t ldq;
  int w;
  int64_t pos0;             // window row i sits at position pos0 + i
  const uint16_t* kc;       // K cache [hkv, cap, d] (post-RoPE)
  int64_t head_stride, row_stride;
  int64_t n_end;            // keys 0 .. n_end - 1 (n_end = pos0 + w: later keys are never visible)
  int hq, hkv, nkb;
  float c;                  // scale * log2(e)
  float2* part;             // [hkv][nkb][R]: (block max in base 2, block sum)
  float2* stats;            // [hkv][R]: (M, 1 / L)
  float* colsum;            // [hkv][nkb * MKB]
  const uint4* qp;          // the queries in fragment order: [hkv][R / 32][AD / 16][64 lanes] (k_mass_qpack)
};

// The block's keys [kb * 256, +256) of head g into LDS as [256][AD] bf16, 16-byte chunk c of key row r at
// r * CPR + (c ^ (r % CPR)): a fragment read (32 rows, one chunk per lane half) then hits distinct banks.
template <int AD>
__device__ __forceinline__ void load_keys(const MassArgs& a, int g, int kb, uint4* ks) {
  constexpr int CPR = AD / 8, PER = MKB * CPR / 256;
  const uint16_t* kh = a.kc + g * a.head_stride;
  uint4 v[PER];                                   // every load in flight before the first LDS write
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int s = threadIdx.x + 256 * i, r = s / CPR, ch = s % CPR;
    const int64_t key = static_cast<int64_t>(kb) * MKB + r;
    v[i] = make_uint4(0u, 0u, 0u, 0u);
    if (key < a.n_end) v[i] = *reinterpret_cast<const uint4*>(kh + key * a.row_stride + ch * 8);
  }
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int s = threadIdx.x + 256 * i, r = s / CPR, ch = s % CPR;
    ks[r * CPR + (ch ^ (r % CPR))] = v[i];
  }
}

// The window queries in the order the score products read them: fragment (group g, row step rb, d step s)
// is 64 lanes x 16 bytes, lane (n, hh) holding row rb * 32 + n's d values 16 s + 8 hh .. + 7, so that each
// fragment load is one contiguous 1 KB instead of 32 rows' 32-byte pieces.
template <int AD>
__global__ __launch_bounds__(256) void k_mass_qpack(MassArgs a, uint4* __restrict__ qp) {
  constexpr int NS = AD / 16;
  const int rep = a.hq / a.hkv, R = rep * a.w;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= static_cast<int64_t>(a.hkv) * (R / 32) * NS * 64) return;
  const int lane = static_cast<int>(idx & 63), n = lane & 31, hh = lane >> 5;
  const int64_t f = idx >> 6;
  const int s = static_cast<int>(f % NS), rb = static_cast<int>((f / NS) % (R / 32)), g = static_cast<int>(f / NS / (R / 32));
  const int r = rb * 32 + n, qh = r / a.w, qi = r - qh * a.w;
  qp[idx] = *reinterpret_cast<const uint4*>(a.q + static_cast<int64_t>(qi) * a.ldq +
                                            static_cast<int64_t>(g * rep + qh) * AD + 16 * s + 8 * hh);
}

template <int AD>
__global__ __launch_bounds__(256) void k_mass_stats(MassArgs a) {
  constexpr int CPR = AD / 8, NS = AD / 16;
  __shared__ uint4 ks[MKB * CPR];
  const int kb = blockIdx.x, g = blockIdx.y;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, n = lane & 31, hh = lane >> 5;
  const int rep = a.hq / a.hkv, R = rep * a.w;
  auto qload = [&](int rb, uint4 (&qv)[NS]) {     // row step rb's query fragments
    const uint4* f = a.qp + (static_cast<int64_t>(g) * (R / 32) + rb) * NS * 64 + lane;
#pragma unroll
    for (int s = 0; s < NS; ++s) qv[s] = f[s * 64];
  };
  // the first row step's queries load beside the key block, each later one during the step before it
  uint4 qn[NS];
  if (wv < R / 32) qload(wv, qn);
  load_keys<AD>(a, g, kb, ks);
  __syncthreads();
  const bool full = static_cast<int64_t>(kb + 1) * MKB - 1 <= a.pos0;   // every key visible to every row
  for (int rb = wv; rb < R / 32; rb += 4) {
    const int r = rb * 32 + n, qi = r - (r / a.w) * a.w;
    bf16x8 qf[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) qf[s] = as_frag(qn[s]);
    if (rb + 4 < R / 32) qload(rb + 4, qn);
    // the row's last visible key, relative to the block (32-bit): keys 0 .. rel of the block are visible
    const int rel = static_cast<int>(min<int64_t>(a.pos0 + qi - static_cast<int64_t>(kb) * MKB, MKB));
    // online maximum and sum over the 32-key steps: (mx, sum) of the lane's keys so far
    float mx = -INFINITY, sum = 0.f;
#pragma unroll 2
    for (int sb = 0; sb < 8; ++sb) {             // 32-key steps of the block
      f32x16 acc = {};
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const int kr = sb * 32 + n, ch = 2 * s + hh;
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_frag(ks[kr * CPR + (ch ^ (kr % CPR))]), qf[s], acc, 0, 0, 0);
      }
      float sc[16];
      if (full) {
#pragma unroll
        for (int j = 0; j < 16; ++j) sc[j] = acc[j] * a.c;
      } else {
#pragma unroll
        for (int j = 0; j < 16; ++j) sc[j] = sb * 32 + 8 * (j >> 2) + 4 * hh + (j & 3) <= rel ? acc[j] * a.c : -INFINITY;
      }
      float m2 = mx;
#pragma unroll
      for (int j = 0; j < 16; ++j) m2 = fmaxf(m2, sc[j]);
      if (m2 != -INFINITY) {
        float t = 0.f;
#pragma unroll
        for (int j = 0; j < 16; ++j) t += __builtin_amdgcn_exp2f(sc[j] - m2);
        sum = sum * __builtin_amdgcn_exp2f(mx - m2) + t;     // exp2(-inf) = 0 while nothing was visible
        mx = m2;
      }
    }
    // the two lane halves: the row's block maximum and its sum rescaled to it
    const auto mp = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
    const float m0 = __uint_as_float(mp[0]), m1 = __uint_as_float(mp[1]);
    const float mb = fmaxf(m0, m1);
    const auto sp = __builtin_amdgcn_permlane32_swap(__float_as_uint(sum), __float_as_uint(sum), false, false);
    const float s0 = __uint_as_float(sp[0]), s1 = __uint_as_float(sp[1]);
    mx = mb;
    sum = mb == -INFINITY ? 0.f
                          : (m0 == -INFINITY ? 0.f : s0 * __builtin_amdgcn_exp2f(m0 - mb)) +
                                (m1 == -INFINITY ? 0.f : s1 * __builtin_amdgcn_exp2f(m1 - mb));
    if (hh == 0) a.part[(static_cast<int64_t>(g) * a.nkb + kb) * R + r] = make_float2(mx, sum);
  }
}

// Per row (one wave): M = max over key blocks, L = sum_kb l_kb 2^(m_kb - M). Lane l takes blocks l, l + 64,
// ... (an online merge in block order), then the lanes combine by butterflies in a fixed order.
__global__ __launch_bounds__(256) void k_mass_rows(MassArgs a) {
  const int rep = a.hq / a.hkv, R = rep * a.w, lane = threadIdx.x & 63;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (idx >= static_cast<int64_t>(a.hkv) * R) return;
  const int64_t g = idx / R, r = idx - g * R;
  const float2* p = a.part + g * a.nkb * R + r;       // block kb at p[kb * R]
  float M = -INFINITY, L = 0.f;
  for (int kb = lane; kb < a.nkb; kb += 64) {
    const float2 v = p[static_cast<int64_t>(kb) * R];
    if (v.x == -INFINITY) continue;
    const float m2 = fmaxf(M, v.x);
    L = (M == -INFINITY ? 0.f : L * __builtin_amdgcn_exp2f(M - m2)) + v.y * __builtin_amdgcn_exp2f(v.x - m2);
    M = m2;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float Mo = __shfl_xor(M, o, 64), Lo = __shfl_xor(L, o, 64);
    const float m2 = fmaxf(M, Mo);
    if (m2 != -INFINITY) {
      // the lower lane's part first, so both lanes of the pair form the same bits
      const bool low = (lane & o) == 0;
      const float La = low ? L : Lo, Ma = low ? M : Mo, Lb = low ? Lo : L, Mb = low ? Mo : M;
      L = (Ma == -INFINITY ? 0.f : La * __builtin_amdgcn_exp2f(Ma - m2)) +
          (Mb == -INFINITY ? 0.f : Lb * __builtin_amdgcn_exp2f(Mb - m2));
    }
    M = m2;
  }
  if (lane == 0) a.stats[idx] = make_float2(M, 1.0f / L);   // every row sees key 0, so L >= 1
}

template <int AD>
__global__ __launch_bounds__(256) void k_mass_cols(MassArgs a) {
  constexpr int CPR = AD / 8, NS = AD / 16;
  __shared__ uint4 ks[MKB * CPR];
  __shared__ float2 st[1024];
  __shared__ int rp[1024];                        // the rows' positions relative to the block's first key
  const int kb = blockIdx.x, g = blockIdx.y;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, n = lane & 31, hh = lane >> 5;
  const int rep = a.hq / a.hkv, R = rep * a.w;
  auto qload = [&](int rb, uint4 (&qv)[NS]) {     // row step rb's query fragments
    const uint4* f = a.qp + (static_cast<int64_t>(g) * (R / 32) + rb) * NS * 64 + lane;
#pragma unroll
    for (int s = 0; s < NS; ++s) qv[s] = f[s * 64];
  };
  uint4 qn[NS];
  qload(0, qn);                                   // the first row step's queries load beside the key block
  load_keys<AD>(a, g, kb, ks);
  for (int r = threadIdx.x; r < R; r += 256) {
    st[r] = a.stats[static_cast<int64_t>(g) * R + r];
    rp[r] = static_cast<int>(min<int64_t>(a.pos0 + r % a.w - static_cast<int64_t>(kb) * MKB, MKB));
  }
  __syncthreads();
  const bool full = static_cast<int64_t>(kb + 1) * MKB - 1 <= a.pos0;   // every key visible to every row
  // this wave's two 32-key steps: keys 64 wv + 32 sb + n of the block
  bf16x8 kf[2][NS];
#pragma unroll
  for (int sb = 0; sb < 2; ++sb) {
    const int kr = wv * 64 + sb * 32 + n;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int ch = 2 * s + hh;
      kf[sb][s] = as_frag(ks[kr * CPR + (ch ^ (kr % CPR))]);
    }
  }
  const int64_t key0 = static_cast<int64_t>(kb) * MKB + wv * 64 + n;
  float col[2] = {0.f, 0.f};
  for (int rb = 0; rb < R / 32; ++rb) {          // 32-row steps, in order; the next step's queries in flight
    bf16x8 qf[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) qf[s] = as_frag(qn[s]);
    if (rb + 1 < R / 32) qload(rb + 1, qn);
    // the lane's rows rb * 32 + 8 (j / 4) + 4 hh + j % 4: their statistics and positions
    float mneg[16], inv[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const float2 ml = st[rb * 32 + 8 * (j >> 2) + 4 * hh + (j & 3)];
      mneg[j] = -ml.x;
      inv[j] = ml.y;
    }
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      f32x16 acc = {};
#pragma unroll
      for (int s = 0; s < NS; ++s) acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qf[s], kf[sb][s], acc, 0, 0, 0);
      const int kr = wv * 64 + sb * 32 + n;      // the lane's key, relative to the block
      float cs = 0.f;
      if (full) {
#pragma unroll
        for (int j = 0; j < 16; ++j) cs += __builtin_amdgcn_exp2f(fmaf(acc[j], a.c, mneg[j])) * inv[j];
      } else {
#pragma unroll
        for (int j = 0; j < 16; ++j)
          cs += kr <= rp[rb * 32 + 8 * (j >> 2) + 4 * hh + (j & 3)]
                    ? __builtin_amdgcn_exp2f(fmaf(acc[j], a.c, mneg[j])) * inv[j] : 0.f;
      }
      col[sb] += cs;
    }
  }
#pragma unroll
  for (int sb = 0; sb < 2; ++sb) {
    const auto cp = __builtin_amdgcn_permlane32_swap(__float_as_uint(col[sb]), __float_as_uint(col[sb]), false, false);
    const float tot = __uint_as_float(cp[0]) + __uint_as_float(cp[1]);
    if (hh == 0) a.colsum[static_cast<int64_t>(g) * a.nkb * MKB + key0 + sb * 32] = tot;
  }
}

__global__ __launch_bounds__(256) void k_mass_fold(const float* __restrict__ colsum, int hkv, int64_t stride,
                                                   int64_t n_end, double* __restrict__ mass) {
  const int64_t j = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (j >= n_end) return;
  double s = mass[j];
  for (int g = 0; g < hkv; ++g) s += static_cast<double>(colsum[g * stride + j]);
  mass[j] = s;
}

int64_t mass_blocks(int64_t n_end) { return (n_end + MKB - 1) / MKB; }

// workspace: the row blocks' statistics, the rows' statistics, the column partials, the packed queries
size_t mass_bytes(int w, int hq, int hkv, int d, int64_t n_end) {
  const int64_t R = static_cast<int64_t>(hq / hkv) * w, nkb = mass_blocks(n_end);
  const size_t part = static_cast<size_t>(hkv) * R * nkb * 8, stats = static_cast<size_t>(hkv) * R * 8,
               cols = static_cast<size_t>(hkv) * nkb * MKB * 4, qp = static_cast<size_t>(hkv) * R * d * 2;
  return (part + 255) / 256 * 256 + (stats + 255) / 256 * 256 + (cols + 255) / 256 * 256 + qp;
}

int mass_shape(const char* fn, int w, int hq, int hkv, int d) {
  if (d != 64 && d != 128 && d != 256) return fail(RF_EUNSUPPORTED, "%s: head_dim %d (64, 128 or 256)", fn, d);
  if (hq <= 0 || hkv <= 0 || hq % hkv || w <= 0 || (static_cast<int64_t>(hq / hkv) * w) % 32 ||
      static_cast<int64_t>(hq / hkv) * w > 1024)
    return fail(RF_EINVAL_SHAPE, "%s: %d window rows x %d query heads per K / V head must be a multiple of 32, "
                "at most 1024", fn, w, hkv > 0 ? hq / hkv : 0);
  return RF_OK;
}

}  // namespace
}  // namespace rf

using namespace rf;

extern "C" int rf_window_mass_workspace_bytes(int w, int hq, int hkv, int d, int64_t n_end, size_t* bytes) {
  if (!bytes || n_end <= 0) return fail(RF_EINVAL_ARG, "rf_window_mass_workspace_bytes: arguments");
  if (const int e = mass_shape("rf_window_mass_workspace_bytes", w, hq, hkv, d)) return e;
  *bytes = mass_bytes(w, hq, hkv, d, n_end);
  return RF_OK;
}

extern "C" int rf_window_mass(const uint16_t* q, int64_t ldq, int w, int64_t pos0, int hq, int d, const uint16_t* kbuf,
                              int hkv, int64_t head_stride, int64_t row_stride, float scale, double* mass,
                              void* workspace, size_t ws_bytes, hipStream_t stream) {
  if (!q || !kbuf || !mass || !workspace) return fail(RF_EINVAL_ARG, "rf_window_mass: null pointer");
  if (const int e = mass_shape("rf_window_mass", w, hq, hkv, d)) return e;
  const int64_t n_end = pos0 + w;
  if (pos0 < 0 || ldq < static_cast<int64_t>(hq) * d || ldq % 8 || row_stride < d || row_stride % 8 ||
      head_stride % 8)
    return fail(RF_EINVAL_SHAPE, "rf_window_mass: pos0 %lld, strides q %lld, row %lld, head %lld", (long long)pos0,
                (long long)ldq, (long long)row_stride, (long long)head_stride);
  if (!aligned16(q) || !aligned16(kbuf) || !aligned16(workspace) || (reinterpret_cast<uintptr_t>(mass) & 7u))
    return fail(RF_EINVAL_SHAPE, "rf_window_mass: alignment");
  if (!(scale > 0.f) || !(scale < 1e30f))
    return fail(RF_EINVAL_ARG, "rf_window_mass: scale %g (must be positive)", static_cast<double>(scale));
  const size_t need = mass_bytes(w, hq, hkv, d, n_end);
  if (ws_bytes < need) return fail(RF_EINVAL_SHAPE, "rf_window_mass: workspace %zu bytes < %zu", ws_bytes, need);
  const int64_t nkb = mass_blocks(n_end), R = static_cast<int64_t>(hq / hkv) * w;
  if (nkb > (1 << 20)) return fail(RF_EINVAL_SHAPE, "rf_window_mass: %lld keys", (long long)n_end);
  char* ws = static_cast<char*>(workspace);
  const size_t part = static_cast<size_t>(hkv) * R * nkb * 8, stats = static_cast<size_t>(hkv) * R * 8,
               cols = static_cast<size_t>(hkv) * nkb * MKB * 4;
  const size_t o_stats = (part + 255) / 256 * 256, o_cols = o_stats + (stats + 255) / 256 * 256,
               o_qp = o_cols + (cols + 255) / 256 * 256;
  uint4* qp = reinterpret_cast<uint4*>(ws + o_qp);
  MassArgs a{q, ldq, w, pos0, kbuf, head_stride, row_stride, n_end, hq, hkv, static_cast<int>(nkb),
             scale * 1.4426950408889634f, reinterpret_cast<float2*>(ws), reinterpret_cast<float2*>(ws + o_stats),
             reinterpret_cast<float*>(ws + o_cols), qp};
  const int64_t nq4 = static_cast<int64_t>(hkv) * R * d / 8;       // 16-byte pieces of the packed queries
  const dim3 qgrid(static_cast<unsigned>((nq4 + 255) / 256));
  if (d == 256) hipLaunchKernelGGL(k_mass_qpack<256>, qgrid, dim3(256), 0, stream, a, qp);
  else if (d == 128) hipLaunchKernelGGL(k_mass_qpack<128>, qgrid, dim3(256), 0, stream, a, qp);
  else hipLaunchKernelGGL(k_mass_qpack<64>, qgrid, dim3(256), 0, stream, a, qp);
  if (const int e = check_launch("rf_window_mass (queries)")) return e;
  const dim3 grid(static_cast<unsigned>(nkb), static_cast<unsigned>(hkv));
  if (d == 256) hipLaunchKernelGGL(k_mass_stats<256>, grid, dim3(256), 0, stream, a);
  else if (d == 128) hipLaunchKernelGGL(k_mass_stats<128>, grid, dim3(256), 0, stream, a);
  else hipLaunchKernelGGL(k_mass_stats<64>, grid, dim3(256), 0, stream, a);
  if (const int e = check_launch("rf_window_mass (row blocks)")) return e;
  hipLaunchKernelGGL(k_mass_rows, dim3(static_cast<unsigned>((hkv * R + 3) / 4)), dim3(256), 0, stream, a);
  if (const int e = check_launch("rf_window_mass (rows)")) return e;
  if (d == 256) hipLaunchKernelGGL(k_mass_cols<256>, grid, dim3(256), 0, stream, a);
  else if (d == 128) hipLaunchKernelGGL(k_mass_cols<128>, grid, dim3(256), 0, stream, a);
  else hipLaunchKernelGGL(k_mass_cols<64>, grid, dim3(256), 0, stream, a);
  if (const int e = check_launch("rf_window_mass (columns)")) return e;
  hipLaunchKernelGGL(k_mass_fold, dim3(static_cast<unsigned>((n_end + 255) / 256)), dim3(256), 0, stream, a.colsum,
                     hkv, nkb * MKB, n_end, mass);
  return check_launch("rf_window_mass (fold)");
}
