// Exact-row attention for gfx950: causal attention of a few query rows at arbitrary sorted positions
// over the filled K / V cache of one layer (the attention of Model.layer_rows, code/kva/ops.py:131-155
// attend_at / :158-170 attend_rows), head_dim 64, 128 or 256, grouped-query heads.
//
// A block takes one K / V head and 64 query rows: 64 / rep queries x the rep query heads that share the
// K / V head (rep = hq / hkv). Wave w owns query rows 16w .. 16w + 15. The keys 0 .. (last query's
// position) stream through LDS in tiles of 64; per tile:
//   S^T = K Q^T on v_mfma_f32_16x16x32_bf16 (A = the K tile from LDS, B = the wave's query rows held in
//       registers), scaled, with keys past each query's position masked: lane l holds, for query row
//       l % 16, the scores of keys 16 kb + 4 (l / 16) + i (kb, i < 4);
//   online softmax in fp32 (running max and per-lane partial sums);
//   O += P V on the same MFMA with P (rounded to bf16) as the A operand in the lane layout the scores
//       already have: the contraction order over a 32-key step is permuted to keys {4g .. 4g + 3,
//       16 + 4g .. 16 + 4g + 3} for lane group g, and the V operand is read in that order from a
//       transposed V tile (V^T in LDS).
// The next tile's K / V rows load into registers while the current tile computes. The key range of a
// block can be split over several blocks (blockIdx.z): each writes its unnormalised O with its row maxima
// and sums to a workspace, and k_attend_combine merges them in split order. Scores are fp32
// products of the bf16 q and k values, as the reference's fp32 matmul; the probabilities enter the
// second product as bf16, as the reference's cast (here before normalisation, within rounding).
#include <stdint.h>

#include <algorithm>

#include "rf_common.h"

namespace rf {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int KT = 64;           // keys per tile
constexpr int VROW = KT + 4;     // bf16 stride of a V^T row in LDS (136 bytes)

__device__ __forceinline__ bf16x8 as_frag(const uint4& u) { return __builtin_bit_cast(bf16x8, u); }

struct AttnArgs {
  const uint16_t* q;       // [nq, >= hq * d], query j head h at q + j * ldq + h * d
  int64_t ldq;
  const int64_t* qpos;     // [nq] sorted positions; query j sees keys 0 .. qpos[j]
  int nq;
  const uint16_t* kc;      // cache [hkv, cap, d]
  const uint16_t* vc;
  int64_t head_stride, row_stride;
  int hq, hkv;
  float scale;
  uint16_t* out;           // [nq, >= hq * d]
  int64_t ldo;
  float* part;             // nsplit > 1: per (query block, head, split) O [64][d], max [64], sum [64]
};

template <int AD>
__device__ __forceinline__ float* part_block(const AttnArgs& a, int qblock, int hk, int split) {
  return a.part + ((static_cast<int64_t>(qblock) * a.hkv + hk) * gridDim.z + split) * (64 * AD + 128);
}

// AD = head_dim (64, 128 or 256); K tile rows are AD + 8 bf16 apart in LDS (conflict-free fragment reads).
// NT = threads: 256 (64 query rows per block, key-range splits allowed) or 512 (128 rows: for many queries
// at head_dim 256, each K / V tile serves twice the rows; no splits).
template <int AD, int NT>
__global__ __launch_bounds__(NT) void k_attend_rows(AttnArgs a) {
  constexpr int KROW = AD + 8, NS = AD / 32, NB = AD / 16, CPR = AD / 8;   // d steps, d blocks, chunks per row
  constexpr int LOADS = KT * CPR / NT;                                     // 16-byte K (and V) chunks per thread
  constexpr int ROWS = NT / 4;                                             // query rows per block (16 per wave)
  __shared__ uint16_t ks[KT * KROW];
  __shared__ uint16_t vts[AD * VROW];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6, ln = lane & 15, g = lane >> 4;
  const int rep = a.hq / a.hkv, qb = ROWS / rep;
  const int hk = blockIdx.y;
  const int j0 = blockIdx.x * qb;
  const int jlast = min(j0 + qb, a.nq) - 1;
  const int64_t kmax = a.qpos[jlast];                       // the block reads keys 0 .. kmax

  // the lane's query row for the scores (S^T column ln of wave w)
  const int r = 16 * w + ln;
  const int jq = j0 + r % qb;
  const bool live = jq < a.nq;
  const int64_t mypos = live ? a.qpos[jq] : -1;
  bf16x8 qf[NS];
  {
    const uint16_t* qrow = a.q + static_cast<int64_t>(live ? jq : j0) * a.ldq + (hk * rep + r / qb) * AD;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      uint4 u = make_uint4(0u, 0u, 0u, 0u);
      if (live) u = *reinterpret_cast<const uint4*>(qrow + 32 * s + 8 * g);
      qf[s] = as_frag(u);
    }
  }

  const uint16_t* kh = a.kc + hk * a.head_stride;
  const uint16_t* vh = a.vc + hk * a.head_stride;
  // tile loads: K chunk c of thread t = key (t / CPR) + (NT / CPR) c, 16-byte column t % CPR;
  //             V chunk c = key t & 63, column block (t >> 6) + (NT / 64) c
  uint4 kr[LOADS], vr[LOADS];
  auto load = [&](int64_t k0) {
#pragma unroll
    for (int c = 0; c < LOADS; ++c) {
      const int64_t kk = k0 + t / CPR + (NT / CPR) * c, kv = k0 + (t & 63);
      kr[c] = kk <= kmax ? *reinterpret_cast<const uint4*>(kh + kk * a.row_stride + (t % CPR) * 8)
                         : make_uint4(0u, 0u, 0u, 0u);
      vr[c] = kv <= kmax ? *reinterpret_cast<const uint4*>(vh + kv * a.row_stride + ((t >> 6) + (NT / 64) * c) * 8)
                         : make_uint4(0u, 0u, 0u, 0u);
    }
  };
  auto store = [&]() {
#pragma unroll
    for (int c = 0; c < LOADS; ++c) {
      *reinterpret_cast<uint4*>(ks + (t / CPR + (NT / CPR) * c) * KROW + (t % CPR) * 8) = kr[c];
      const int key = t & 63, d0 = ((t >> 6) + (NT / 64) * c) * 8;
#pragma unroll
      for (int e = 0; e < 8; ++e) vts[(d0 + e) * VROW + key] = lane_of(vr[c], e);
    }
  };

  f32x4 o[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) o[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, lpart = 0.f;
  // this block's share of the key tiles
  const int ntiles = static_cast<int>(kmax / KT) + 1;
  const int ns = gridDim.z, sp = blockIdx.z;
  const int it0 = static_cast<int>(static_cast<int64_t>(ntiles) * sp / ns);
  const int it1 = static_cast<int>(static_cast<int64_t>(ntiles) * (sp + 1) / ns);
  if (it0 < it1) load(static_cast<int64_t>(it0) * KT);
  for (int it = it0; it < it1; ++it) {
    const int64_t k0 = static_cast<int64_t>(it) * KT;
    __syncthreads();                                          // the previous tile's reads are done
    store();
    __syncthreads();
    if (it + 1 < it1) load(k0 + KT);

    // scores of the wave's 16 query rows against the tile's 64 keys
    f32x4 sc[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const uint4 kf = *reinterpret_cast<const uint4*>(ks + (16 * kb + ln) * KROW + 32 * s + 8 * g);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_frag(kf), qf[s], acc, 0, 0, 0);
      }
      sc[kb] = acc;
    }
    float tmax = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t key = k0 + 16 * kb + 4 * g + i;
        const float s = key <= mypos ? sc[kb][i] * a.scale : -INFINITY;
        sc[kb][i] = s;
        tmax = fmaxf(tmax, s);
      }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float mnew = fmaxf(m, tmax);
    const float mref = mnew == -INFINITY ? 0.f : mnew;      // a row with every key masked so far
    const float alpha = expf(m - mref);
    m = mnew;
    float psum = 0.f;
    uint32_t pp[4][2];                                        // bf16 pairs: (kb, i = 0,1) and (kb, i = 2,3)
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      float p[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        p[i] = expf(sc[kb][i] - mref);
        psum += p[i];
      }
      pp[kb][0] = bf16_pair(p[0], p[1]);
      pp[kb][1] = bf16_pair(p[2], p[3]);
    }
    lpart = lpart * alpha + psum;
    // the O rows this lane accumulates are query rows 4g + i of the wave: their rescale factors
    float al[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) al[i] = __shfl(alpha, 4 * g + i, 64);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int i = 0; i < 4; ++i) o[nb][i] *= al[i];
    // O += P V over two 32-key steps; lane group g's 8 contraction slots are keys {4g..4g+3, 16+4g..+3}
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      const bf16x8 pa = as_frag(make_uint4(pp[2 * st][0], pp[2 * st][1], pp[2 * st + 1][0], pp[2 * st + 1][1]));
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const uint16_t* vrow = vts + (16 * nb + ln) * VROW + 32 * st + 4 * g;
        const uint2 lo = *reinterpret_cast<const uint2*>(vrow), hi = *reinterpret_cast<const uint2*>(vrow + 16);
        o[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa, as_frag(make_uint4(lo.x, lo.y, hi.x, hi.y)), o[nb], 0, 0, 0);
      }
    }
  }
  // normalise and write: lane holds O[query row 4g + i][d = 16 nb + ln]
  float lsum = lpart;
  lsum += __shfl_xor(lsum, 16, 64);
  lsum += __shfl_xor(lsum, 32, 64);
  if (NT == 256 && ns > 1) {                                  // unnormalised partials for the combine
    float* pb = part_block<AD>(a, blockIdx.x, hk, sp);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int rr = 16 * w + 4 * g + i;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) pb[rr * AD + 16 * nb + ln] = o[nb][i];
    }
    if (g == 0) {
      pb[64 * AD + r] = m;
      pb[64 * AD + 64 + r] = lsum;
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float li = __shfl(lsum, 4 * g + i, 64);
    const int rr = 16 * w + 4 * g + i;
    const int jo = j0 + rr % qb;
    if (jo >= a.nq) continue;
    uint16_t* dst = a.out + static_cast<int64_t>(jo) * a.ldo + (hk * rep + rr / qb) * AD + ln;
    const float inv = 1.0f / li;
#pragma unroll
    for (int nb = 0; nb < NB; nb += 2) {
      const uint32_t pr = bf16_pair(o[nb][i] * inv, o[nb + 1][i] * inv);
      dst[16 * nb] = static_cast<uint16_t>(pr & 0xffffu);
      dst[16 * (nb + 1)] = static_cast<uint16_t>(pr >> 16);
    }
  }
}

// Merges the key-range splits of one (query block, K / V head): M = max_s m_s, L = sum_s l_s e^{m_s - M},
// O = sum_s O_s e^{m_s - M} / L, in split order; thread t takes query row t / 4 and a quarter of d.
template <int AD>
__global__ __launch_bounds__(256) void k_attend_combine(AttnArgs a, int ns) {
  const int t = threadIdx.x, r = t >> 2, q4 = t & 3;
  const int rep = a.hq / a.hkv, qb = 64 / rep;
  const int hk = blockIdx.y, jo = blockIdx.x * qb + r % qb;
  if (jo >= a.nq) return;
  const int64_t stride = 64 * AD + 128;
  const float* base = a.part + (static_cast<int64_t>(blockIdx.x) * a.hkv + hk) * ns * stride;
  float mx = -INFINITY;
  for (int sp = 0; sp < ns; ++sp) mx = fmaxf(mx, base[sp * stride + 64 * AD + r]);
  float l = 0.f;
  float acc[AD / 4];
#pragma unroll
  for (int e = 0; e < AD / 4; ++e) acc[e] = 0.f;
  for (int sp = 0; sp < ns; ++sp) {
    const float* pb = base + sp * stride;
    const float ms = pb[64 * AD + r];
    const float f = ms == -INFINITY ? 0.f : expf(ms - mx);
    l += pb[64 * AD + 64 + r] * f;
#pragma unroll
    for (int e = 0; e < AD / 4; ++e) acc[e] += pb[r * AD + q4 * (AD / 4) + e] * f;
  }
  const float inv = 1.0f / l;
  uint16_t* dst = a.out + static_cast<int64_t>(jo) * a.ldo + (hk * rep + r / qb) * AD + q4 * (AD / 4);
#pragma unroll
  for (int e = 0; e < AD / 4; e += 8)
    *reinterpret_cast<uint4*>(dst + e) =
        make_uint4(bf16_pair(acc[e] * inv, acc[e + 1] * inv), bf16_pair(acc[e + 2] * inv, acc[e + 3] * inv),
                   bf16_pair(acc[e + 4] * inv, acc[e + 5] * inv), bf16_pair(acc[e + 6] * inv, acc[e + 7] * inv));
}

// out[j, :] = bf16(x[j, :] + y[j, :]) for `rows` rows of width H, and out's row sum-of-squares partials
// (the next RMSNorm's statistics, in the order every producer uses). One wave per row.
__global__ __launch_bounds__(256) void k_residual_add(const uint16_t* __restrict__ x, int64_t ldx,
                                                      const uint16_t* __restrict__ y, int64_t ldy,
                                                      uint16_t* __restrict__ out, int64_t ldo,
                                                      float* __restrict__ ssq, int64_t rows, int H) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const uint16_t* xr = x + row * ldx;
  const uint16_t* yr = y + row * ldy;
  uint16_t* orow = out + row * ldo;
  row_partials([&](int64_t o) {
    const uint2 u = *reinterpret_cast<const uint2*>(xr + o), v = *reinterpret_cast<const uint2*>(yr + o);
    const uint2 r = make_uint2(bf16_pair(bf2f(u.x & 0xffffu) + bf2f(v.x & 0xffffu), bf2f(u.x >> 16) + bf2f(v.x >> 16)),
                               bf16_pair(bf2f(u.y & 0xffffu) + bf2f(v.y & 0xffffu), bf2f(u.y >> 16) + bf2f(v.y >> 16)));
    *reinterpret_cast<uint2*>(orow + o) = r;
    return r;
  }, ssq + row * (H / SSQ_COLS), H / SSQ_COLS, lane);
}

// act[j, c] = bf16(bf16(silu(gate[j, c])) * up[j, c]) with gate = gu[:, :I], up = gu[:, I:2I]: SwiGLU
// with the reference's roundings (F.silu on bf16, then the bf16 product).
__global__ __launch_bounds__(256) void k_silu_mul(const uint16_t* __restrict__ gu, int64_t ldg, int64_t rows, int I,
                                                  uint16_t* __restrict__ act, int64_t lda) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int cpr = I / 8;
  if (i >= rows * cpr) return;
  const int64_t row = i / cpr;
  const int c = static_cast<int>(i - row * cpr);
  const uint4 gv = *reinterpret_cast<const uint4*>(gu + row * ldg + c * 8);
  const uint4 uv = *reinterpret_cast<const uint4*>(gu + row * ldg + I + c * 8);
  float r[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float gx = bf2f(lane_of(gv, e));
    r[e] = bf2f(f2bf(gx / (1.0f + expf(-gx)))) * bf2f(lane_of(uv, e));
  }
  *reinterpret_cast<uint4*>(act + row * lda + c * 8) =
      make_uint4(bf16_pair(r[0], r[1]), bf16_pair(r[2], r[3]), bf16_pair(r[4], r[5]), bf16_pair(r[6], r[7]));
}

}  // namespace
}  // namespace rf

using namespace rf;

namespace rf {
namespace {
// Key-range splits for nq queries: enough blocks for about three per CU, at most one split per key tile,
// at most 32, and what the workspace holds.
// Qwen3.5's attention output gate (code/kva/model.py:444-445, o * torch.sigmoid(gate) in bf16): out =
// bf16(o * bf16(sigmoid(g))), 8 values per thread.
__global__ __launch_bounds__(256) void k_sigmoid_mul(const uint16_t* __restrict__ o, int64_t ldo,
                                                     const uint16_t* __restrict__ g, int64_t ldg, int64_t rows, int n,
                                                     uint16_t* __restrict__ out, int64_t ld_out) {
  const int64_t cpr = n / 8, idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= rows * cpr) return;
  const int64_t r = idx / cpr, c = (idx - r * cpr) * 8;
  const uint4 ov = *reinterpret_cast<const uint4*>(o + r * ldo + c);
  const uint4 gv = *reinterpret_cast<const uint4*>(g + r * ldg + c);
  uint16_t res[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float sg = bf2f(f2bf(1.0f / (1.0f + expf(-bf2f(lane_of(gv, e))))));
    res[e] = f2bf(bf2f(lane_of(ov, e)) * sg);
  }
  *reinterpret_cast<uint4*>(out + r * ld_out + c) =
      make_uint4(pack2(res[0], res[1]), pack2(res[2], res[3]), pack2(res[4], res[5]), pack2(res[6], res[7]));
}

// The GDN output norm (ops.rms_norm_gated, code/kva/ops.py:28-33) per (row, head) of dv values:
// y = bf16(w * bf16(x / sqrt(mean(x^2) + eps))), out = bf16(y * silu(z)) with silu(z) = z / (1 + e^-z) in
// fp32. dv / 8 lanes per (row, head), 8 values each; every lane of a group reaches the shuffles.
__global__ __launch_bounds__(256) void k_gated_norm(const uint16_t* __restrict__ x, int64_t ldx,
                                                    const uint16_t* __restrict__ z, int64_t ldz,
                                                    const uint16_t* __restrict__ wt, int64_t rows, int heads, int dv,
                                                    float eps, uint16_t* __restrict__ y, int64_t ldy) {
  const int g = dv / 8, t = threadIdx.x, sub = t % g;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * (256 / g) + t / g;
  const bool ok = item < rows * heads;
  const int64_t r = ok ? item / heads : 0;
  const int64_t col = (ok ? item % heads : 0) * dv + sub * 8;
  const uint4 xv = *reinterpret_cast<const uint4*>(x + r * ldx + col);
  float xf[8], s = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    xf[e] = bf2f(lane_of(xv, e));
    s = fmaf(xf[e], xf[e], s);
  }
  for (int m = g >> 1; m >= 1; m >>= 1) s += __shfl_xor(s, m);
  if (!ok) return;
  const float inv = 1.0f / sqrtf(s / static_cast<float>(dv) + eps);
  const uint4 zv = *reinterpret_cast<const uint4*>(z + r * ldz + col);
  const uint4 wv = *reinterpret_cast<const uint4*>(wt + sub * 8);
  uint16_t res[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float yv = bf2f(f2bf(bf2f(lane_of(wv, e)) * bf2f(f2bf(xf[e] * inv))));
    const float zf = bf2f(lane_of(zv, e));
    res[e] = f2bf(yv * (zf / (1.0f + expf(-zf))));
  }
  *reinterpret_cast<uint4*>(y + r * ldy + col) =
      make_uint4(pack2(res[0], res[1]), pack2(res[2], res[3]), pack2(res[4], res[5]), pack2(res[6], res[7]));
}

int attend_splits(int64_t nq, int hq, int hkv, int d, int64_t cache_rows, size_t ws_bytes) {
  const int64_t qb = 64 / (hq / hkv);
  const int64_t blocks = (nq + qb - 1) / qb * hkv;
  int64_t ns = (768 + blocks - 1) / blocks;
  ns = std::min<int64_t>(ns, std::min<int64_t>(32, (cache_rows + KT - 1) / KT));
  const int64_t per = blocks * (64 * static_cast<int64_t>(d) + 128) * 4;
  ns = std::min<int64_t>(ns, static_cast<int64_t>(ws_bytes / static_cast<size_t>(per)));
  return static_cast<int>(std::max<int64_t>(ns, 1));
}
}  // namespace
}  // namespace rf

extern "C" int rf_attend_rows_workspace_bytes(int64_t nq, int hq, int hkv, int d, int64_t cache_rows, size_t* bytes) {
  if (!bytes || nq < 0 || hq <= 0 || hkv <= 0 || hq % hkv || 64 % (hq / hkv) || (d != 64 && d != 128 && d != 256))
    return fail(RF_EINVAL_ARG, "rf_attend_rows_workspace_bytes: arguments");
  const int ns = attend_splits(nq, hq, hkv, d, cache_rows, SIZE_MAX);
  const int64_t qb = 64 / (hq / hkv);
  *bytes = ns > 1 ? static_cast<size_t>((nq + qb - 1) / qb * hkv * ns * (64 * static_cast<int64_t>(d) + 128) * 4) : 0;
  return RF_OK;
}

extern "C" int rf_attend_rows(const uint16_t* q, int64_t ldq, const int64_t* qpos, int64_t nq, int hq, int d,
                              const uint16_t* kbuf, const uint16_t* vbuf, int hkv, int64_t head_stride,
                              int64_t row_stride, int64_t cache_rows, float scale, uint16_t* out, int64_t ldo,
                              void* workspace, size_t ws_bytes, hipStream_t stream) {
  if (!q || !qpos || !kbuf || !vbuf || !out) return fail(RF_EINVAL_ARG, "rf_attend_rows: null pointer");
  if (d != 64 && d != 128 && d != 256)
    return fail(RF_EUNSUPPORTED, "rf_attend_rows: head_dim %d (the kernel takes 64, 128, 256)", d);
  if (hq <= 0 || hkv <= 0 || hq % hkv || 64 % (hq / hkv))
    return fail(RF_EUNSUPPORTED, "rf_attend_rows: %d query heads over %d K / V heads (need a group of at most 64 "
                "dividing 64)", hq, hkv);
  if (nq < 0 || nq > (1 << 30) || ldq < static_cast<int64_t>(hq) * d || ldo < static_cast<int64_t>(hq) * d ||
      ldq % 8 || ldo % 8 || row_stride < d || row_stride % 8 || head_stride % 8 || cache_rows <= 0)
    return fail(RF_EINVAL_SHAPE, "rf_attend_rows: shapes / strides (nq %lld, ldq %lld, ldo %lld)", (long long)nq,
                (long long)ldq, (long long)ldo);
  if (!aligned16(q) || !aligned16(kbuf) || !aligned16(vbuf)) return fail(RF_EINVAL_SHAPE, "rf_attend_rows: alignment");
  if (nq == 0) return RF_OK;
  if (workspace && (reinterpret_cast<uintptr_t>(workspace) & 15u))
    return fail(RF_EINVAL_SHAPE, "rf_attend_rows: workspace alignment");
  // many queries at head_dim 256 (an exact tail): 128-row blocks, no key-range splits
  const bool wide = d == 256 && nq >= 2048;
  const int ns = (workspace && !wide) ? attend_splits(nq, hq, hkv, d, cache_rows, ws_bytes) : 1;
  AttnArgs a{q, ldq, qpos, static_cast<int>(nq), kbuf, vbuf, head_stride, row_stride, hq, hkv, scale, out, ldo,
             static_cast<float*>(workspace)};
  const int qb = (wide ? 128 : 64) / (hq / hkv);
  const dim3 grid(static_cast<unsigned>((nq + qb - 1) / qb), static_cast<unsigned>(hkv), static_cast<unsigned>(ns));
  if (wide) hipLaunchKernelGGL((k_attend_rows<256, 512>), grid, dim3(512), 0, stream, a);
  else if (d == 256) hipLaunchKernelGGL((k_attend_rows<256, 256>), grid, dim3(256), 0, stream, a);
  else if (d == 128) hipLaunchKernelGGL((k_attend_rows<128, 256>), grid, dim3(256), 0, stream, a);
  else hipLaunchKernelGGL((k_attend_rows<64, 256>), grid, dim3(256), 0, stream, a);
  if (ns > 1) {
    const int st = check_launch("rf_attend_rows");
    if (st != RF_OK) return st;
    const dim3 g2(grid.x, grid.y);
    if (d == 256) hipLaunchKernelGGL(k_attend_combine<256>, g2, dim3(256), 0, stream, a, ns);
    else if (d == 128) hipLaunchKernelGGL(k_attend_combine<128>, g2, dim3(256), 0, stream, a, ns);
    else hipLaunchKernelGGL(k_attend_combine<64>, g2, dim3(256), 0, stream, a, ns);
  }
  return check_launch("rf_attend_rows");
}

extern "C" int rf_residual_add(const uint16_t* x, int64_t ldx, const uint16_t* y, int64_t ldy, uint16_t* out,
                               int64_t ldo, float* ssq, int64_t rows, int64_t H, hipStream_t stream) {
  if (!x || !y || !out || !ssq) return fail(RF_EINVAL_ARG, "rf_residual_add: null pointer");
  if (rows < 0 || H <= 0 || H % SSQ_COLS || ldx < H || ldy < H || ldo < H || ldx % 8 || ldy % 8 || ldo % 8)
    return fail(RF_EINVAL_SHAPE, "rf_residual_add: rows %lld, H %lld (multiple of 256), strides", (long long)rows,
                (long long)H);
  if (!aligned16(x) || !aligned16(y) || !aligned16(out)) return fail(RF_EINVAL_SHAPE, "rf_residual_add: alignment");
  if (rows == 0) return RF_OK;
  hipLaunchKernelGGL(k_residual_add, dim3(static_cast<unsigned>((rows + 3) / 4)), dim3(256), 0, stream, x, ldx, y, ldy,
                     out, ldo, ssq, rows, static_cast<int>(H));
  return check_launch("rf_residual_add");
}

extern "C" int rf_silu_mul(const uint16_t* gu, int64_t ldg, int64_t rows, int64_t I, uint16_t* act, int64_t lda,
                           hipStream_t stream) {
  if (!gu || !act) return fail(RF_EINVAL_ARG, "rf_silu_mul: null pointer");
  if (rows < 0 || I <= 0 || I % 8 || ldg < 2 * I || lda < I || ldg % 8 || lda % 8)
    return fail(RF_EINVAL_SHAPE, "rf_silu_mul: rows %lld, I %lld, strides", (long long)rows, (long long)I);
  if (!aligned16(gu) || !aligned16(act)) return fail(RF_EINVAL_SHAPE, "rf_silu_mul: alignment");
  if (rows == 0) return RF_OK;
  const int64_t n = rows * (I / 8);
  hipLaunchKernelGGL(k_silu_mul, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, stream, gu, ldg, rows,
                     static_cast<int>(I), act, lda);
  return check_launch("rf_silu_mul");
}

extern "C" int rf_sigmoid_mul(const uint16_t* o, int64_t ldo, const uint16_t* g, int64_t ldg, int64_t rows, int64_t n,
                              uint16_t* out, int64_t ld_out, hipStream_t stream) {
  if (!o || !g || !out) return fail(RF_EINVAL_ARG, "rf_sigmoid_mul: null pointer");
  if (rows < 0 || n <= 0 || n % 8 || n > (1 << 30) || ldo < n || ldg < n || ld_out < n || ldo % 8 || ldg % 8 ||
      ld_out % 8)
    return fail(RF_EINVAL_SHAPE, "rf_sigmoid_mul: rows %lld, n %lld (multiple of 8), strides", (long long)rows,
                (long long)n);
  if (!aligned16(o) || !aligned16(g) || !aligned16(out)) return fail(RF_EINVAL_SHAPE, "rf_sigmoid_mul: alignment");
  if (rows == 0) return RF_OK;
  const int64_t total = rows * (n / 8);
  hipLaunchKernelGGL(k_sigmoid_mul, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0, stream, o, ldo, g,
                     ldg, rows, static_cast<int>(n), out, ld_out);
  return check_launch("rf_sigmoid_mul");
}

extern "C" int rf_gated_rms_norm(const uint16_t* x, int64_t ldx, const uint16_t* z, int64_t ldz, const uint16_t* weight,
                                 int64_t rows, int heads, int dv, float eps, uint16_t* y, int64_t ldy,
                                 hipStream_t stream) {
  if (!x || !z || !weight || !y) return fail(RF_EINVAL_ARG, "rf_gated_rms_norm: null pointer");
  if (rows < 0 || heads <= 0 || (dv != 64 && dv != 128 && dv != 256) || ldx < static_cast<int64_t>(heads) * dv ||
      ldz < static_cast<int64_t>(heads) * dv || ldy < static_cast<int64_t>(heads) * dv || ldx % 8 || ldz % 8 ||
      ldy % 8)
    return fail(RF_EINVAL_SHAPE, "rf_gated_rms_norm: rows %lld, heads %d, dv %d (64, 128 or 256), strides",
                (long long)rows, heads, dv);
  if (!aligned16(x) || !aligned16(z) || !aligned16(weight) || !aligned16(y))
    return fail(RF_EINVAL_SHAPE, "rf_gated_rms_norm: alignment");
  if (rows == 0) return RF_OK;
  const int64_t items = rows * heads, per = 256 / (dv / 8);
  hipLaunchKernelGGL(k_gated_norm, dim3(static_cast<unsigned>((items + per - 1) / per)), dim3(256), 0, stream, x, ldx,
                     z, ldz, weight, rows, heads, dv, eps, y, ldy);
  return check_launch("rf_gated_rms_norm");
}
