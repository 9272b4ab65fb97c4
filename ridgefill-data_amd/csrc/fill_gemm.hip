// bf16 MFMA GEMM core for gfx950 and the two fill GEMMs built on it:
//   rf_map_apply      x = b W^T + c, rounded to bf16, plus the rows' sum-of-squares partials;
//   rf_norm_kv_write  [K | V] = rms_norm(x) W_kv^T with the norm gain folded into W_kv, per-head
//                     k_norm, RoPE on K, written straight into the [hkv, cap, d] cache slots.
//
// Tiling. A workgroup of 4 wave64s computes a 256 x 256 output tile over K in 64-deep steps. Both
// operands are K-contiguous (row-major activations, F.linear-layout weights), so each 64-deep K slice
// of a 128-row operand half is 128 rows of one full 128-byte cache line each. The slices go from memory
// straight into LDS (buffer_load_dwordx4 ... lds, no staging registers; the buffer's range check turns
// rows past M into zeros), one instruction per 8 full lines, with the 16-byte chunk index XOR-ed by
// (row >> 1) & 7 so the MFMA fragment reads hit all banks. A ring of ten 16 KiB slots (the whole LDS)
// holds 2.5 steps; one wait and one barrier per step.
//
// Each wave owns a 128 x 128 quarter and issues v_mfma_f32_32x32x16_bf16 on 4 x 4 sub-tiles. The
// weight tile is the MFMA's A operand and the activation tile its B operand, so the accumulator of a
// lane holds, for one activation row (lane % 32), four runs of 4 consecutive output columns: the
// epilogue rounds them to bf16 and writes 8-byte runs into a row-major LDS image of the 256 x 256
// tile, which a row pass then reads as 16-byte chunks (32 threads per 256-column row) to compute
// row statistics, apply k_norm / RoPE and issue coalesced 128-bit stores.
#include <algorithm>
#include <type_traits>

#include "rf_common.h"

namespace rf {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int BM = 256, BN = 256, BK = 64, NTHR = 256;
constexpr int CPR = BK / 8;                    // 16-byte chunks per 128-byte operand row of a slot
constexpr int SLOT_ROWS = 128;                 // a slot: 128 rows of one operand over one 64-deep K step
constexpr int SLOT_U4 = SLOT_ROWS * CPR;       // 16 KiB
constexpr int NSLOT = 10;                      // slots in the ring: 2.5 K steps
constexpr int LDS_U4 = NSLOT * SLOT_U4;        // 160 KiB, the whole LDS of a CU
constexpr int IMAGE_U4 = 256 * 32;             // the epilogue's 256 x 256 bf16 image (128 KiB)
static_assert(LDS_U4 >= IMAGE_U4 + 2048, "the epilogue's image and its 32 KiB of side data must fit");

__device__ __forceinline__ bf16x8 as_frag(const uint4& u) { return __builtin_bit_cast(bf16x8, u); }

// Logical tile -> (tile row, tile column). Tiles go in groups of GROUP_M tile rows walked column by
// column, so the ~32 tiles one XCD runs at a time form a GROUP_M x 8 block: per K step its L2 sees
// GROUP_M activation slices and 8 weight slices instead of 2 and 16.
// The Gram's square products (4096 x 4096 over 65536-deep K) take groups of 8 tile rows, an 8 x 4 block per
// XCD: measured 1777 against 1807 us per launch (same box, alternating builds; 4 x 8 stays best for the
// fill's map and K / V launches, 16 x 2 is slower for both).
constexpr int GROUP_M = 4, GRAM_GROUP_M = 8;
template <int G = GROUP_M>
__device__ __forceinline__ void tile_coords(int tile, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int per_group = G * tiles_n;
  const int g = tile / per_group, in = tile - g * per_group;
  const int rows = min(G, tiles_m - g * G);
  tm = g * G + in % rows;
  tn = in / rows;
}

// Chunk swizzle of a slot: row r's 16-byte chunk c (of 8) lives at r * 8 + (c ^ slot_swz(r)). A fragment
// read takes one chunk of 32 consecutive rows; the LDS serves 16 lanes of 16 bytes per cycle, and rows
// r .. r + 15 then cover all 16 bank groups (row parity picks the half of the 256-byte bank line, the
// swizzle the chunk within it).
__device__ __forceinline__ int slot_swz(int row) { return (row >> 1) & 7; }

typedef __attribute__((address_space(3))) void* lds_ptr;

// Raw buffer resource over [base, base + bytes): loads past the end return zeros (rows >= M).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), static_cast<int>(bytes),
                                           0x00020000);
}

// s_waitcnt with vmcnt <= n and lgkmcnt = 0 (expcnt not waited), gfx9 encoding.
template <int n>
__device__ __forceinline__ void wait_vm_lgkm0() {
  static_assert(n >= 0 && n < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((n & 15) | (7 << 4) | (0 << 8) | ((n >> 4) << 14));
}

// Ring slot of quarter q of K step kt: (4 kt + q) % NSLOT. Quarters 0, 1 are activation rows 0-127 /
// 128-255, quarters 2, 3 weight rows 0-127 / 128-255. The loops carry the step's ring phase ph = (4 kt) %
// NSLOT instead of kt, so that a slot is one conditional subtraction, slot_at(ph, q) (q < 12), rather
// than a division by 10 on the scalar unit before every direct load; next_ph(ph) is the phase of step
// kt + 1.
__device__ __forceinline__ int slot_at(int ph, int q) { return ph + q >= NSLOT ? ph + q - NSLOT : ph + q; }
__device__ __forceinline__ int next_ph(int ph) { return slot_at(ph, 4); }

// Load i (0..3) of this wave into ring slot `slot` for K step kt, straight from memory (buffer_load_dwordx4
// ... lds): 8 rows x 128 bytes, full cache lines. Lane L writes slot chunk (32w + 8i) * 8 + L, i.e. row
// 32w + 8i + L / 8, physical chunk L % 8, and so fetches logical chunk (L % 8) ^ slot_swz(row) of that row;
// `voff` holds the lane's byte offset of that (row, chunk), the step's K offset goes in the scalar offset.
__device__ __forceinline__ void issue_load_at(__amdgpu_buffer_rsrc_t rs, uint32_t voff, int slot, int kt, int i,
                                              char* lds, int w) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr)(lds + slot * (SLOT_U4 * 16) + (32 * w + 8 * i) * (CPR * 16)),
                                           16, voff, kt * BK * 2, 0, 0);
}

// acc[nt][mt] += W[n0 + wn*128 + nt*32 .. +32, :] . X[m0 + wm*128 + mt*32 .. +32, :]^T over all of K
// (K % 64 == 0), from zero (ZERO) or from the accumulators' values on entry. Rows of X at or past M read
// as zeros. Ends with a barrier: LDS is free for the epilogue.
//
// Pipeline. K goes in 64-deep steps. A step's operands are four 16 KiB quarters (activation rows 0-127 and
// 128-255, weight rows 0-127 and 128-255), each 128 rows of full 128-byte lines; the ring holds ten
// quarters (2.5 steps, the whole LDS). Wave (wm, wn) reads activation quarter wm and weight quarter wn. A
// step is four 16-deep slices of 16 MFMAs; the fragments of slice j + 1 are read during slice j, one LDS
// read after each of its first 8 MFMAs. One wait and one barrier per step, between slices 2 and 3: by
// then every wave has read all of the step's fragments (its quarters are free) and step kt + 1 has
// landed. Loads for step kt + 2: its activation quarters during slices 0 and 1 of step kt (into the
// slots step kt - 1's weights left), its weight quarters during slice 3 (into the slots step kt's
// activations just left). So each barrier waits with 8 loads per wave still in flight, and the last
// loads of a step are issued four slices (64 MFMAs) before the barrier that needs them.
template <bool ZERO = true>
__device__ __forceinline__ void mainloop(const uint16_t* __restrict__ X, int64_t ldx,
                                         const uint16_t* __restrict__ W, int64_t ldw, int M, int K,
                                         int m0, int n0, uint4* lds, f32x16 (&acc)[4][4]) {
  const int t = threadIdx.x, lane = t & 63;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);      // wave-uniform: slot arithmetic stays scalar
  const int wm = w >> 1, wn = w & 1;
  const int rows_x = min(M - m0, BM);
  const __amdgpu_buffer_rsrc_t rx = buffer_rsrc(X + static_cast<int64_t>(m0) * ldx,
                                                static_cast<uint32_t>(rows_x * ldx * 2));
  const __amdgpu_buffer_rsrc_t rw = buffer_rsrc(W + static_cast<int64_t>(n0) * ldw, static_cast<uint32_t>(BN * ldw * 2));
  // per-lane byte offsets of load i of half h: row h*128 + 32w + 8i + lane/8, chunk (lane%8) ^ slot_swz(row)
  uint32_t vx[2][4], vw[2][4];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 32 * w + 8 * i + (lane >> 3);
      const int ch = (lane & 7) ^ slot_swz(r);
      vx[h][i] = static_cast<uint32_t>(((h * 128 + r) * ldx + ch * 8) * 2);
      vw[h][i] = static_cast<uint32_t>(((h * 128 + r) * ldw + ch * 8) * 2);
    }

  if (ZERO) {
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.f;
  }

  char* base = reinterpret_cast<char*>(lds);
  const int nk = K / BK;
  const int lr = lane & 31, lk = lane >> 5, swz = slot_swz(lr);
  bf16x8 fx[2][4], fw[2][4];
  // fragment r (0..7) of slice ks of step kt: r < 4 -> weight block r, else activation block r - 4
  // (steps are named by their ring phase ph and, for the loads' K offset, their index kt)
  auto read_one = [&](int ph, int ks, int r, bf16x8 (&ax)[4], bf16x8 (&aw)[4]) {
    const int ch = (ks * 2 + lk) ^ swz;
    if (r < 4) aw[r] = as_frag(lds[slot_at(ph, 2 + wn) * SLOT_U4 + (r * 32 + lr) * CPR + ch]);
    else ax[r - 4] = as_frag(lds[slot_at(ph, wm) * SLOT_U4 + ((r - 4) * 32 + lr) * CPR + ch]);
  };
  // load j (0..7) of step kt's (phase ph) activation (wt = false) or weight (wt = true) quarters
  auto load = [&](int kt, int ph, bool wt, int j) {
    const int h = j >> 2, i = j & 3;
    if (wt) issue_load_at(rw, vw[h][i], slot_at(ph, 2 + h), kt, i, base, w);
    else issue_load_at(rx, vx[h][i], slot_at(ph, h), kt, i, base, w);
  };
  // one slice: 16 MFMAs on (ax, aw); reads of the next slice's fragments after the first 8 (`rd`);
  // `ld` 0: no loads, 1: activation loads lo .. lo + 3 of step lkt after MFMAs 1, 5, 9, 13,
  // 2: all 8 weight loads of step lkt, one after every even MFMA. Spreading the loads keeps the
  // texture units' queues from filling, which would stall the wave's in-order issue of MFMAs.
  auto slice = [&](const bf16x8 (&ax)[4], const bf16x8 (&aw)[4], bool rd, int rph, int rks, bf16x8 (&nx)[4],
                   bf16x8 (&nw)[4], int ld, int lkt, int lph, int lo) {
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int qi = q >> 2, qj = (qi & 1) ? 3 - (q & 3) : (q & 3);   // snake: one operand changes per MFMA
      acc[qi][qj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(aw[qi], ax[qj], acc[qi][qj], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
      if (q < 8 && rd) read_one(rph, rks, q, nx, nw);
      if (ld == 2 && !(q & 1)) load(lkt, lph, true, q >> 1);
      if (ld == 1 && (q & 3) == 1) load(lkt, lph, false, lo + (q >> 2));
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // `steady` (compile-time): step kt + 2 exists, so its loads are issued and the wait is exact
  auto step = [&](int kt, int ph, auto steady) {
    const int ph1 = next_ph(ph), ph2 = next_ph(ph1);
    slice(fx[0], fw[0], true, ph, 1, fx[1], fw[1], steady ? 1 : 0, kt + 2, ph2, 0);
    slice(fx[1], fw[1], true, ph, 2, fx[0], fw[0], steady ? 1 : 0, kt + 2, ph2, 4);
    slice(fx[0], fw[0], true, ph, 3, fx[1], fw[1], 0, 0, 0, 0);
    if (steady) wait_vm_lgkm0<8>();
    else wait_vm_lgkm0<0>();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    slice(fx[1], fw[1], steady || kt + 1 < nk, ph1, 0, fx[0], fw[0], steady ? 2 : 0, kt + 2, ph2, 0);
  };

  // prologue: steps 0 and 1, then step 0's first fragments
  for (int j = 0; j < 8; ++j) load(0, 0, false, j);
  for (int j = 0; j < 8; ++j) load(0, 0, true, j);
  if (nk > 1) {
    for (int j = 0; j < 8; ++j) load(1, 4, false, j);
    for (int j = 0; j < 8; ++j) load(1, 4, true, j);
    wait_vm_lgkm0<16>();
  } else {
    wait_vm_lgkm0<0>();
  }
  __builtin_amdgcn_s_barrier();
  for (int r = 0; r < 8; ++r) read_one(0, 0, r, fx[0], fw[0]);
  int kt = 0, ph = 0;
  for (; kt + 2 < nk; ++kt, ph = next_ph(ph)) step(kt, ph, std::true_type{});
  for (; kt < nk; ++kt, ph = next_ph(ph)) step(kt, ph, std::false_type{});
  wait_vm_lgkm0<0>();
  __syncthreads();
}

// After the main loop the LDS past the image (32 KiB) holds per-tile side data the epilogues read: the
// bias tile, the rows' norm scales, the rows' sum-of-squares halves. What is known before the loop
// (bias, norm scales) waits in registers through it and is written there after it.

// Epilogue stage 1: value(mt, nt, g, e, acc) rounded to bf16 into the row-major LDS image of the tile.
// Lane (lr, lk) holds, for tile row wm*128 + mt*32 + lr, columns wn*128 + nt*32 + 8g + 4lk + e.
// Image layout: row r's 16-byte chunk c lives at slot r * 32 + (c ^ (r & 31)).
// With SSQ, ss[mt] receives the sum of squares of the lane's 64 rounded values of that row, a sequential
// fma chain in (nt, g, e) order (the order rf_row_ssq reproduces).
template <bool SSQ, class F>
__device__ __forceinline__ void stage_tile(uint4* lds, const f32x16 (&acc)[4][4], F value, float (&ss)[4]) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int wm = w >> 1, wn = w & 1, lr = lane & 31, lk = lane >> 5;
  char* base = reinterpret_cast<char*>(lds);
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    const int row = wm * 128 + mt * 32 + lr;
    float sq = 0.f;
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int c0 = wn * 128 + nt * 32 + 8 * g + 4 * lk;
        const uint32_t p0 = bf16_pair(value(mt, nt, g, 0, acc[nt][mt][4 * g + 0]),
                                      value(mt, nt, g, 1, acc[nt][mt][4 * g + 1]));
        const uint32_t p1 = bf16_pair(value(mt, nt, g, 2, acc[nt][mt][4 * g + 2]),
                                      value(mt, nt, g, 3, acc[nt][mt][4 * g + 3]));
        if (SSQ) {
          const float r0 = bf_lo(p0), r1 = bf_hi(p0), r2 = bf_lo(p1), r3 = bf_hi(p1);
          sq = fmaf(r0, r0, sq);
          sq = fmaf(r1, r1, sq);
          sq = fmaf(r2, r2, sq);
          sq = fmaf(r3, r3, sq);
        }
        const int off = row * 512 + (((c0 >> 3) ^ (row & 31)) << 4) + ((c0 & 7) << 1);
        *reinterpret_cast<uint2*>(base + off) = make_uint2(p0, p1);
      }
    ss[mt] = sq;
  }
}

__device__ __forceinline__ uint4 image_chunk(const uint4* lds, int row, int c) {
  return lds[row * 32 + (c ^ (row & 31))];
}

// Input RMSNorm scale 1 / sqrt(mean(x^2) + eps) of tile row threadIdx.x (row m0 + threadIdx.x) from
// its sum-of-squares partials, summed in order. Called before the main loop (its loads overlap the
// first operand loads); the value is published to the other waves through LDS after the loop.
__device__ __forceinline__ float row_scale(const float* __restrict__ ssq, int nparts, float width, float eps, int M,
                                           int m0) {
  const int gm = m0 + static_cast<int>(threadIdx.x);
  float s = 0.f;
  if (gm < M) {
    const float* q = ssq + static_cast<int64_t>(gm) * nparts;
    for (int i = 0; i < nparts; ++i) s += q[i];
  }
  return 1.0f / sqrtf(s / width + eps);
}

// Split K. With fewer output tiles than CUs, the K range of each tile is cut into `splits` ranges,
// each one block of k_gemm_partial, which stores its fp32 sums as row-major planes
// part[split][row][column] (rows < M only). The reduce kernels (k_*_reduce) then run the tile's
// epilogue as a row pass over many small blocks of 8 rows x 256 columns: each thread adds the splits of
// its 8 columns in split order (the same bits every run) and finishes them as the unsplit epilogue
// does. Every epilogue here is row-local, so this needs no tile-wide step.
__device__ __forceinline__ void store_partial(float* __restrict__ part, int64_t ldp, int M, int m0, int n0,
                                              const f32x16 (&acc)[4][4]) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, wm = w >> 1, wn = w & 1, lr = lane & 31, lk = lane >> 5;
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    const int gm = m0 + wm * 128 + mt * 32 + lr;
    if (gm >= M) continue;
    float* row = part + static_cast<int64_t>(gm) * ldp + n0 + wn * 128 + 4 * lk;
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *reinterpret_cast<float4*>(row + nt * 32 + 8 * g) =
            make_float4(acc[nt][mt][4 * g], acc[nt][mt][4 * g + 1], acc[nt][mt][4 * g + 2], acc[nt][mt][4 * g + 3]);
  }
}

// Split sp of every tile: X[rows of the tile, kbeg .. kbeg + klen) . W[columns, same K range]^T into
// part + sp * M * N.
__global__ __launch_bounds__(NTHR) void k_gemm_partial(const uint16_t* __restrict__ X, int64_t ldx,
                                                       const uint16_t* __restrict__ W, int64_t ldw, int M, int N,
                                                       int K, int kper, float* __restrict__ part) {
  __shared__ uint4 lds[LDS_U4];
  const int tiles_n = N / BN, tiles = ((M + BM - 1) / BM) * tiles_n;
  const int tile = blockIdx.x % tiles, sp = blockIdx.x / tiles;
  const int tm = tile / tiles_n, tn = tile - tm * tiles_n;
  const int kbeg = sp * kper, klen = min(K - kbeg, kper);
  f32x16 acc[4][4];
  mainloop(X + kbeg, ldx, W + kbeg, ldw, M, klen, tm * BM, tn * BN, lds, acc);
  store_partial(part + static_cast<int64_t>(sp) * M * N, N, M, tm * BM, tn * BN, acc);
}

// ---- split partials of products with few rows (M <= ROWS_MAX): the exact rows' projections.
//
// A 256 x 256 tile wastes most of its MFMA work and its weight reads on a few hundred rows. Here a block
// takes every row of its row block (RT row tiles of 32, MT = 32 RT <= 160 rows, row blocks of about equal
// size) against RN = 256 weight rows, over its split's K range. Wave w computes output columns
// n0 + 64w .. + 63 for all MT rows (2 x RT accumulators: per 16-deep slice RT + 2 fragment reads feed 2 RT
// MFMAs). Operands stream through an LDS ring of S stages (one 64-deep K step each: MT activation rows,
// then the 256 weight rows, 128-byte rows with the slot swizzle) filled straight from memory by
// buffer_load ... lds, S - 1 steps ahead; one wait and one barrier per step. The products are k_gemm_partial's: the same MFMA, the
// weight fragment as its first operand, K in the same order, so a split's partial sums are bit-identical
// to the 256 x 256 path over the same K range (and with one split, to the unsplit kernels' sums).
constexpr int RN = 256;
constexpr int64_t ROWS_MAX = 512;

template <int RT>
struct RowsCfg {
  static constexpr int MT = 32 * RT;
  static constexpr int ROWS = MT + RN;              // stage rows
  static constexpr int STAGE_U4 = ROWS * CPR;
  static constexpr int S = (LDS_U4 / STAGE_U4) < 6 ? (LDS_U4 / STAGE_U4) : 6;
  static constexpr int L = ROWS / 32;               // loads per wave per stage (8 rows of 128 bytes each)
};

// s_waitcnt vmcnt <= n * L (lgkmcnt 0) for a run-time n in [0, 4]
template <int L>
__device__ __forceinline__ void wait_steps(int n) {
  switch (n) {
    case 0: wait_vm_lgkm0<0>(); break;
    case 1: wait_vm_lgkm0<L>(); break;
    case 2: wait_vm_lgkm0<2 * L>(); break;
    case 3: wait_vm_lgkm0<3 * L>(); break;
    default: wait_vm_lgkm0<4 * L>(); break;
  }
}

template <int RT>
__device__ __forceinline__ void rows_partial(const uint16_t* __restrict__ X, int64_t ldx, const uint16_t* __restrict__ W,
                                             int64_t ldw, int M, int N, int K, int kper, int rblocks,
                                             float* __restrict__ part, uint4* lds) {
  using C = RowsCfg<RT>;
  static_assert(C::S >= 3 && (C::S - 2) * C::L < 64, "ring depth");
  const int t = threadIdx.x, lane = t & 63;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);
  // block -> (row block, column block, split), row blocks fastest over a contiguous run of logical blocks
  // per XCD: the row blocks of one column block run together on one XCD, so its weight rows are read
  // from memory once and meet in that XCD's L2
  const int cblocks = N / RN;
  const int u = xcd_tile(blockIdx.x, gridDim.x);
  const int rbk = u % rblocks, rest = u / rblocks;
  const int cb = rest % cblocks, sp = rest / cblocks;
  // row blocks of about equal size, each a whole number of row tiles
  const int per = (M + rblocks - 1) / rblocks;
  const int m0 = rbk * per, rows_x = max(0, min(M - m0, per));
  const int n0 = cb * RN;
  const int kbeg = sp * kper, klen = max(0, min(K - kbeg, kper));
  const int nk = klen / BK;
  const __amdgpu_buffer_rsrc_t rx = buffer_rsrc(X + static_cast<int64_t>(m0) * ldx + kbeg,
                                                static_cast<uint32_t>(rows_x * ldx * 2));
  const __amdgpu_buffer_rsrc_t rw = buffer_rsrc(W + static_cast<int64_t>(n0) * ldw + kbeg,
                                                static_cast<uint32_t>(RN * ldw * 2));
  // load i of this wave: stage rows 8 (4 i + w) .. + 7 (activation rows below MT, then weight rows);
  // lane L fetches row + L / 8, logical chunk (L % 8) ^ slot_swz(row) into physical chunk L % 8
  uint32_t voff[C::L];
#pragma unroll
  for (int i = 0; i < C::L; ++i) {
    const int r = 8 * (4 * i + w) + (lane >> 3);
    const int ch = (lane & 7) ^ slot_swz(r);
    voff[i] = r < C::MT ? static_cast<uint32_t>((r * ldx + ch * 8) * 2)
                        : static_cast<uint32_t>(((r - C::MT) * ldw + ch * 8) * 2);
  }
  char* base = reinterpret_cast<char*>(lds);
  auto issue_one = [&](int kt, int st, int i) {
    const int j = 4 * i + w;                        // wave-uniform
    lds_ptr dst = (lds_ptr)(base + st * (C::STAGE_U4 * 16) + j * 1024);
    if (8 * j < C::MT) __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, dst, 16, voff[i], kt * BK * 2, 0, 0);
    else __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, dst, 16, voff[i], kt * BK * 2, 0, 0);
  };
  auto issue = [&](int kt, int st) {
#pragma unroll
    for (int i = 0; i < C::L; ++i) issue_one(kt, st, i);
  };

  f32x16 acc[2][RT];
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[c][rt][r] = 0.f;

  const int lr = lane & 31, lk = lane >> 5, swz = slot_swz(lr);
  bf16x8 fa[2][RT], fb[2][2];
  // fragment r of slice ks of the step in stage st into buffer b: activation row tile r (r < RT), else
  // this wave's weight rows 32 (r - RT) .. + 31
  auto read = [&](int st, int ks, int b, int r) {
    const int ch = (ks * 2 + lk) ^ swz;
    const uint4* s = lds + st * C::STAGE_U4;
    if (r < RT) fa[b][r] = as_frag(s[(r * 32 + lr) * CPR + ch]);
    else fb[b][r - RT] = as_frag(s[(C::MT + 64 * w + 32 * (r - RT) + lr) * CPR + ch]);
  };

  for (int kt = 0; kt < C::S - 1; ++kt)
    if (kt < nk) issue(kt, kt);
  int st = 0;                                       // stage of step kt
  for (int kt = 0; kt < nk; ++kt) {
    wait_steps<C::L>(min(C::S - 2, nk - 1 - kt));   // this step's loads (every wave's, after the barrier)
    __builtin_amdgcn_s_barrier();                   // and every wave is done with step kt - 1's stage
    // step kt + S - 1 into the stage step kt - 1 left, one load after every other MFMA below (a burst of
    // loads fills the texture units' queue, and the wave's in-order issue then stalls its MFMAs)
    const bool more = kt + C::S - 1 < nk;
    const int lkt = kt + C::S - 1, lst = st == 0 ? C::S - 1 : st - 1;
#pragma unroll
    for (int r = 0; r < RT + 2; ++r) read(st, 0, 0, r);
    // slice ks: its 2 RT MFMAs, one read of slice ks + 1's fragments after each (the LDS reads run under
    // the MFMAs instead of ahead of them)
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int b = ks & 1;
#pragma unroll
      for (int q = 0; q < 2 * RT; ++q) {
        acc[q / RT][q % RT] =
            __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[b][q / RT], fa[b][q % RT], acc[q / RT][q % RT], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        if (ks < 3 && q < RT + 2) read(st, ks + 1, b ^ 1, q);
        const int g = ks * 2 * RT + q;              // MFMA index in the step
        if (more && !(g & 1) && (g >> 1) < C::L) issue_one(lkt, lst, g >> 1);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int r = 2 * RT; r < RT + 2; ++r)           // RT = 1: the third fragment
        if (ks < 3) read(st, ks + 1, b ^ 1, r);
    }
    // loads left over when the step has fewer than 2 L MFMAs
#pragma unroll
    for (int i = 4 * RT; i < C::L; ++i)
      if (more) issue_one(lkt, lst, i);
    st = st + 1 == C::S ? 0 : st + 1;
  }
  wait_vm_lgkm0<0>();
  // lane (lr, lk) holds row 32 rt + lr, columns 64 w + 32 c + 8 g + 4 lk + e (e < 4) of accumulator (c, rt)
  float* pp = part + static_cast<int64_t>(sp) * M * N;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int r = rt * 32 + lr;
    if (r >= rows_x) continue;
    float* row = pp + static_cast<int64_t>(m0 + r) * N + n0 + 64 * w + 4 * lk;
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *reinterpret_cast<float4*>(row + 32 * c + 8 * g) =
            make_float4(acc[c][rt][4 * g], acc[c][rt][4 * g + 1], acc[c][rt][4 * g + 2], acc[c][rt][4 * g + 3]);
  }
}

template <int RT>
__global__ __launch_bounds__(NTHR) void k_rows_partial(const uint16_t* __restrict__ X, int64_t ldx,
                                                       const uint16_t* __restrict__ W, int64_t ldw, int M, int N,
                                                       int K, int kper, int rblocks, float* __restrict__ part) {
  __shared__ uint4 lds[RowsCfg<RT>::S * RowsCfg<RT>::STAGE_U4];
  rows_partial<RT>(X, ldx, W, ldw, M, N, K, kper, rblocks, part, lds);
}

// The split sums of 8 consecutive columns col .. col + 7 of row gm: 8 fp32 values, splits added in order.
__device__ __forceinline__ void split_sums(const float* __restrict__ part, int splits, int64_t plane, int64_t off,
                                           float (&v)[8]) {
  const float4* p = reinterpret_cast<const float4*>(part + off);
  float4 a = p[0], b = p[1];
  for (int sp = 1; sp < splits; ++sp) {
    const float4* q = reinterpret_cast<const float4*>(part + sp * plane + off);
    const float4 c = q[0], d = q[1];
    a.x += c.x; a.y += c.y; a.z += c.z; a.w += c.w;
    b.x += d.x; b.y += d.y; b.z += d.z; b.w += d.w;
  }
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

__global__ __launch_bounds__(NTHR) void k_map_apply(const uint16_t* __restrict__ B, int64_t ldb,
                                                    const uint16_t* __restrict__ W,
                                                    const uint16_t* __restrict__ bias,
                                                    uint16_t* __restrict__ X, int64_t ldx,
                                                    float* __restrict__ ssq, int M, int N, int K) {
  __shared__ uint4 lds[LDS_U4];
  float* halves = reinterpret_cast<float*>(lds + IMAGE_U4);    // [2][256] row sum-of-squares halves
  const int tiles_n = N / BN;
  int tm, tn;
  tile_coords(xcd_tile(blockIdx.x, gridDim.x), (M + BM - 1) / BM, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int t = threadIdx.x;
  const int lane = t & 63, w = t >> 6, wm = w >> 1, wn = w & 1, lr = lane & 31, lk = lane >> 5;
  // the accumulators start at the bias: lane (lr, lk) holds columns wn*128 + nt*32 + 8g + 4lk + e
  f32x16 acc[4][4];
#pragma unroll
  for (int nt = 0; nt < 4; ++nt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const uint2 bq = bias ? *reinterpret_cast<const uint2*>(bias + n0 + wn * 128 + nt * 32 + 8 * g + 4 * lk)
                            : make_uint2(0u, 0u);
      const float b0 = bf_lo(bq.x), b1 = bf_hi(bq.x), b2 = bf_lo(bq.y), b3 = bf_hi(bq.y);
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        acc[nt][mt][4 * g + 0] = b0;
        acc[nt][mt][4 * g + 1] = b1;
        acc[nt][mt][4 * g + 2] = b2;
        acc[nt][mt][4 * g + 3] = b3;
      }
    }
  mainloop<false>(B, ldb, W, K, M, K, m0, n0, lds, acc);
  float ss[4];
  stage_tile<true>(lds, acc, [&](int, int, int, int, float a) { return a; }, ss);
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    const float tot = ss[mt] + __shfl_xor(ss[mt], 32, 64);     // the row's 128 columns of this wave
    if (lk == 0) halves[wn * 256 + wm * 128 + mt * 32 + lr] = tot;
  }
  __syncthreads();

  const int nparts = N / SSQ_COLS;
  if (m0 + t < M) ssq[static_cast<int64_t>(m0 + t) * nparts + tn] = halves[t] + halves[256 + t];
  const int ch = t & 31;
#pragma unroll 4
  for (int it = 0; it < BM / 8; ++it) {
    const int row = it * 8 + (t >> 5);
    const int gm = m0 + row;
    if (gm < M) *reinterpret_cast<uint4*>(X + static_cast<int64_t>(gm) * ldx + n0 + ch * 8) = image_chunk(lds, row, ch);
  }
}

struct KvArgs {
  const float* ssq;
  int nparts;
  float h;            // norm width (the GEMM's K)
  float eps;
  int hkv, d;
  const uint16_t* knorm;
  int knorm_kind;
  const uint16_t* cs;
  int rot;
  uint16_t* kbuf;
  uint16_t* vbuf;
  int64_t head_stride, row_stride, slot0;
  const int64_t* pos;   // RoPE table row of input row j: pos[j] (null: j)
  const int64_t* slot = nullptr;   // cache slot of input row j: slot[j] (null: slot0 + j; reduce epilogue only)
  int64_t pos_lim = 0;             // > 0: rows with pos[j] outside [0, pos_lim) are skipped (reduce epilogue only)
};

// k_norm of one chunk's 8 values given the head's inverse RMS (code/kva/ops.py:14-25 per head), with
// the reference's roundings: bf16(w * bf16(x r)) (rms_norm) or bf16(x r (1 + w)) (rms_norm_zc).
__device__ __forceinline__ void knorm_chunk(float (&f)[8], float rinv, const uint4& kw, int kind) {
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    const float w0 = bf2f(lane_of(kw, e)), w1 = bf2f(lane_of(kw, e + 1));
    uint32_t p;
    if (kind == 0) {
      const uint32_t n = bf16_pair(f[e] * rinv, f[e + 1] * rinv);
      p = bf16_pair(w0 * bf_lo(n), w1 * bf_hi(n));
    } else {
      p = bf16_pair(f[e] * rinv * (1.0f + w0), f[e + 1] * rinv * (1.0f + w1));
    }
    f[e] = bf_lo(p);
    f[e + 1] = bf_hi(p);
  }
}

// The K / V (or query) epilogue's per-lane constants for the 16-byte chunk ch (columns n0 + 8 ch ..
// n0 + 8 ch + 7) of a 256-column tile column: K or V, head and offset, the k_norm gains of the chunk
// and of its RoPE partner, and the RoPE table offsets (the same for every row).
struct KvLane {
  bool is_k, norm, rope;
  int j0, pj0, fi0, half, group;
  uint16_t* dst0;
  uint4 kn, kn_p;
  __device__ KvLane(const KvArgs& a, int n0, int ch) {
    const int d = a.d, kw = a.hkv * a.d;
    half = a.rot >> 1;
    group = d >> 3;                                 // chunks per head: a power of two <= 32
    const int col = n0 + ch * 8;
    is_k = col < kw;
    const int cc = is_k ? col : col - kw;
    const int head = cc / d;
    j0 = cc - head * d;
    dst0 = (is_k ? a.kbuf : a.vbuf) + head * a.head_stride + j0;
    norm = is_k && a.knorm != nullptr;
    rope = is_k && j0 < a.rot;
    pj0 = j0 < half ? j0 + half : j0 - half;
    fi0 = j0 < half ? j0 : j0 - half;                // table index of the chunk's first element
    kn = make_uint4(0u, 0u, 0u, 0u);
    kn_p = kn;
    if (norm) {
      kn = *reinterpret_cast<const uint4*>(a.knorm + j0);
      if (rope && half >= 8) kn_p = *reinterpret_cast<const uint4*>(a.knorm + pj0);
    }
  }
};

// The RoPE table entries one K chunk of row gm needs: 8 cos and 8 sin values (rot / 2 >= 8), or the
// row's whole 8-entry table (rot == 8). Zeros for chunks without RoPE.
struct RopeEnt {
  uint4 c, s;
};
__device__ __forceinline__ RopeEnt rope_fetch(const KvArgs& a, const KvLane& L, int64_t gm, bool ok) {
  RopeEnt r{make_uint4(0u, 0u, 0u, 0u), make_uint4(0u, 0u, 0u, 0u)};
  if (ok && L.rope) {
    const uint16_t* cs = a.cs + (a.pos ? a.pos[gm] : gm) * a.rot;
    if (L.half >= 8) {
      r.c = *reinterpret_cast<const uint4*>(cs + L.fi0);
      r.s = *reinterpret_cast<const uint4*>(cs + L.half + L.fi0);
    } else {
      r.c = *reinterpret_cast<const uint4*>(cs);
    }
  }
  return r;
}

// The same for rows indexed by slot (no position array), without branches: every lane loads, rows past
// M read row M - 1, chunks without RoPE read entry 0 (their values are not used). Straight-line loads
// keep the compiler's wait counts exact, so loads issued rows ahead overlap the rows before them.
__device__ __forceinline__ RopeEnt rope_fetch_ahead(const KvArgs& a, const KvLane& L, int64_t gm, int M) {
  const int64_t g = gm < M ? gm : M - 1;
  const uint16_t* cs = a.cs + g * a.rot;
  const int fi = L.rope ? L.fi0 : 0;
  RopeEnt r;
  if (L.half >= 8) {                              // uniform (a kernel argument)
    r.c = *reinterpret_cast<const uint4*>(cs + fi);
    r.s = *reinterpret_cast<const uint4*>(cs + L.half + fi);
  } else {
    r.c = *reinterpret_cast<const uint4*>(cs);
    r.s = make_uint4(0u, 0u, 0u, 0u);
  }
  return r;
}

// The K epilogue's configuration: KV_ANY reads it from the arguments at run time; KV_D128 (no k_norm)
// and KV_D128_KNORM (Llama-style k_norm) fix d = 128 and full rotary (rot = d) at compile time, so the
// 8B-class fill's row pass has no branches on uniform values (each costs a pipeline refetch per chunk).
enum KvMode { KV_ANY = 0, KV_D128 = 1, KV_D128_KNORM = 2 };

// k_norm and RoPE of one K chunk v of a row: `ss` the head's sum of squares (for k_norm), pv the chunk
// holding v's rotate_half partners (rot / 2 >= 8), `re` the row's table entries. Lanes without RoPE
// (partial rotary) get the normed chunk unrotated, by select: no divergent branches, so the callers'
// loads and stores keep exact wait counts.
template <int MODE = KV_ANY>
__device__ __forceinline__ uint4 k_chunk(const KvArgs& a, const KvLane& L, const uint4& v, const uint4& pv, float ss,
                                         const RopeEnt& re) {
  const bool knorm = MODE == KV_ANY ? a.knorm != nullptr : MODE == KV_D128_KNORM;
  const int kind = MODE == KV_ANY ? a.knorm_kind : 0;
  const int j0 = L.j0, half = MODE == KV_ANY ? L.half : 64;
  const float dd = MODE == KV_ANY ? static_cast<float>(a.d) : 128.f;
  float f[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) f[e] = bf2f(lane_of(v, e));
  float rinv = 0.f;
  if (knorm) {
    rinv = 1.0f / sqrtf(ss / dd + a.eps);
    knorm_chunk(f, rinv, L.kn, kind);
  }
  // rotate_half partner values of this chunk, negated for the first half of the rotated dims: a chunk
  // lies wholly in one half (rot / 2 is a multiple of 8), so the sign is the chunk's (or, for rot == 8,
  // element e's: e < 4)
  float pf[8];
  if (half >= 8) {
    const uint32_t sg = j0 < half ? 0x80008000u : 0u;   // bf16 sign bits (k_norm is odd in its input)
    const uint4 pn = make_uint4(pv.x ^ sg, pv.y ^ sg, pv.z ^ sg, pv.w ^ sg);
#pragma unroll
    for (int e = 0; e < 8; ++e) pf[e] = bf2f(lane_of(pn, e));
    if (knorm) knorm_chunk(pf, rinv, L.kn_p, kind);
  } else {                                        // half == 4: the partner is in the same chunk
#pragma unroll
    for (int e = 0; e < 8; ++e) pf[e] = e < 4 ? -f[e ^ 4] : f[e ^ 4];
  }
  float c[8], sn[8];
  if (half >= 8) {                                // 8 consecutive table entries of each half
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      c[e] = bf2f(lane_of(re.c, e));
      sn[e] = bf2f(lane_of(re.s, e));
    }
  } else {                                        // rot == 8: entries 0..3 serve both halves of the chunk
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      c[e] = bf2f(lane_of(re.c, e & 3));
      sn[e] = bf2f(lane_of(re.c, 4 + (e & 3)));
    }
  }
  // x cos + rotate_half(x) sin with each product rounded to bf16, then the sum (ops.py:66-77)
  float y[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint32_t pr = bf16_pair(f[e] * c[e], pf[e] * sn[e]);
    y[e] = bf_lo(pr) + bf_hi(pr);
  }
  if (MODE == KV_ANY && a.rot < a.d) {            // partial rotary: chunks past rot unrotated
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = L.rope ? y[e] : f[e];
  }
  return make_uint4(bf16_pair(y[0], y[1]), bf16_pair(y[2], y[3]), bf16_pair(y[4], y[5]), bf16_pair(y[6], y[7]));
}

// The head's sum of squares of a K chunk for k_norm: the chunk's own, summed over the head's chunks
// (the lanes of one 32-lane row group, all of which must call this). 0 without k_norm.
template <int MODE = KV_ANY>
__device__ __forceinline__ float head_ssq(const KvArgs& a, const KvLane& L, const uint4& v) {
  float ss = 0.f;
  if (MODE == KV_ANY ? a.knorm != nullptr : MODE == KV_D128_KNORM) {   // uniform
    ss = chunk_ssq(v);
    const int group = MODE == KV_ANY ? L.group : 16;
#pragma unroll
    for (int o = 1; o < 32; o <<= 1)
      if (o < group) ss += __shfl_xor(ss, o, 64);
  }
  return ss;
}

// One row's chunk of the K / V epilogue: get(c) returns the row's normed bf16 chunk c (of the tile
// column); k_norm and RoPE for K chunks (k_chunk, with the row's table entries `re`, rope_fetch), then
// a streaming store into slot slot0 + gm (slot[gm] if given). All lanes of a 32-lane row group call this, ok or not.
template <class Get>
__device__ __forceinline__ void kv_chunk_row(const KvArgs& a, const KvLane& L, Get get, int ch, int64_t gm, bool ok,
                                             const RopeEnt& re) {
  const uint4 v = get(ch);
  const float ss = head_ssq(a, L, v);
  if (!ok) return;
  uint16_t* dst = L.dst0 + (a.slot ? a.slot[gm] : a.slot0 + gm) * a.row_stride;
  if (!L.is_k || (!L.norm && !L.rope)) {
    st_stream16(dst, v);
    return;
  }
  const uint4 pv = L.half >= 8 ? get(ch + (L.pj0 - L.j0) / 8) : v;
  st_stream16(dst, k_chunk(a, L, v, pv, ss, re));
}

// Row pass of a tile of K columns only (slot-indexed rows): rows it * 8 + t / 32, chunk t % 32, in
// groups of 8 rows per thread, one loop iteration each (the loop is not unrolled: the instruction cache
// holds one group's code, not the pass's). The RoPE table entries of the next group are fetched before
// this group's math, and the group's 8 stores go out after it, so every wait covers only loads issued a
// group earlier.
template <int MODE>
__device__ __forceinline__ void k_rows(const KvArgs& a, const KvLane& L, const uint4* lds, int m0, int M) {
  const int t = threadIdx.x, ch = t & 31;
  RopeEnt cur[8], nxt[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) cur[u] = rope_fetch_ahead(a, L, m0 + u * 8 + (t >> 5), M);
#pragma unroll 1
  for (int g = 0; g < BM / 64; ++g) {
#pragma unroll
    for (int u = 0; u < 8; ++u) nxt[u] = rope_fetch_ahead(a, L, m0 + (((g + 1) & 3) * 8 + u) * 8 + (t >> 5), M);
    uint4 o[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int row = (g * 8 + u) * 8 + (t >> 5);
      const uint4 v = image_chunk(lds, row, ch);
      const bool half8 = MODE == KV_ANY ? L.half >= 8 : true;
      const uint4 pv = half8 ? image_chunk(lds, row, ch + (L.pj0 - L.j0) / 8) : v;
      const float ss = head_ssq<MODE>(a, L, v);
      o[u] = (MODE != KV_ANY || L.norm || L.rope) ? k_chunk<MODE>(a, L, v, pv, ss, cur[u]) : v;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int gm = m0 + (g * 8 + u) * 8 + (t >> 5);
      if (gm < M) st_stream16(L.dst0 + (a.slot0 + gm) * a.row_stride, o[u]);
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) cur[u] = nxt[u];
  }
}

// Row pass of a tile of V columns only: a copy of the image into the cache slots.
__device__ __forceinline__ void v_rows(const KvArgs& a, const KvLane& L, const uint4* lds, int m0, int M) {
  const int t = threadIdx.x, ch = t & 31;
#pragma unroll 8
  for (int it = 0; it < BM / 8; ++it) {
    const int row = it * 8 + (t >> 5);
    const int gm = m0 + row;
    if (gm < M) st_stream16(L.dst0 + (a.slot0 + gm) * a.row_stride, image_chunk(lds, row, ch));
  }
}

__global__ __launch_bounds__(NTHR) void k_norm_kv(const uint16_t* __restrict__ Xin, int64_t ldx,
                                                  const uint16_t* __restrict__ W, int M, int N, int K,
                                                  KvArgs a) {
  __shared__ uint4 lds[LDS_U4];
  float* rsc = reinterpret_cast<float*>(lds + IMAGE_U4);         // [256] row norm scales
  const int tiles_n = N / BN;
  int tm, tn;
  tile_coords(xcd_tile(blockIdx.x, gridDim.x), (M + BM - 1) / BM, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const float my_rs = row_scale(a.ssq, a.nparts, a.h, a.eps, M, m0);
  f32x16 acc[4][4];
  mainloop(Xin, ldx, W, K, M, K, m0, n0, lds, acc);
  rsc[threadIdx.x] = my_rs;
  __syncthreads();

  // Input RMSNorm: the gain is folded into W, so each row is scaled by 1 / sqrt(mean(x^2) + eps).
  const int lane = threadIdx.x & 63, wm = threadIdx.x >> 7;
  float rs[4], unused[4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) rs[mt] = rsc[wm * 128 + mt * 32 + (lane & 31)];
  stage_tile<false>(lds, acc, [&](int mt, int, int, int, float v) { return v * rs[mt]; }, unused);
  __syncthreads();

  // row pass: rows it * 8 + t / 32
  const int t = threadIdx.x, ch = t & 31;
  const KvLane L(a, n0, ch);
  const int kw = a.hkv * a.d;
  const bool d128 = a.d == 128 && a.rot == 128 && !a.pos;
  if (n0 + BN <= kw && d128 && !a.knorm) {
    k_rows<KV_D128>(a, L, lds, m0, M);
  } else if (n0 + BN <= kw && d128 && a.knorm_kind == 0) {
    k_rows<KV_D128_KNORM>(a, L, lds, m0, M);
  } else if (n0 + BN <= kw && !a.pos) {
    k_rows<KV_ANY>(a, L, lds, m0, M);
  } else if (n0 >= kw) {
    v_rows(a, L, lds, m0, M);
  } else {
    for (int it = 0; it < BM / 8; ++it) {
      const int row = it * 8 + (t >> 5);
      const int gm = m0 + row;
      kv_chunk_row(a, L, [&](int c) { return image_chunk(lds, row, c); }, ch, gm, gm < M, rope_fetch(a, L, gm, gm < M));
    }
  }
}

// out = bf16(r_row * (x W^T)) with W's columns carrying the input norm gain (rf_fold_norm) and
// r_row = 1 / sqrt(mean(x^2) + eps) from the row partials: F.linear of the normed input, as the GDN
// in-projections (code/kva/model.py:448-450) compute it.
__global__ __launch_bounds__(NTHR) void k_norm_linear(const uint16_t* __restrict__ Xin, int64_t ldx,
                                                      const uint16_t* __restrict__ W, int M, int N, int K,
                                                      const float* __restrict__ ssq, float eps,
                                                      uint16_t* __restrict__ out, int64_t ldo) {
  __shared__ uint4 lds[LDS_U4];
  float* rsc = reinterpret_cast<float*>(lds + IMAGE_U4);
  const int tiles_n = N / BN;
  int tm, tn;
  tile_coords(xcd_tile(blockIdx.x, gridDim.x), (M + BM - 1) / BM, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const float my_rs = row_scale(ssq, K / SSQ_COLS, static_cast<float>(K), eps, M, m0);
  f32x16 acc[4][4];
  mainloop(Xin, ldx, W, K, M, K, m0, n0, lds, acc);
  rsc[threadIdx.x] = my_rs;
  __syncthreads();
  const int lane = threadIdx.x & 63, wm = threadIdx.x >> 7;
  float rs[4], unused[4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) rs[mt] = rsc[wm * 128 + mt * 32 + (lane & 31)];
  stage_tile<false>(lds, acc, [&](int mt, int, int, int, float v) { return v * rs[mt]; }, unused);
  __syncthreads();
  const int t = threadIdx.x, ch = t & 31;
#pragma unroll 4
  for (int it = 0; it < BM / 8; ++it) {
    const int row = it * 8 + (t >> 5);
    const int gm = m0 + row;
    if (gm < M)
      *reinterpret_cast<uint4*>(out + static_cast<int64_t>(gm) * ldo + n0 + ch * 8) = image_chunk(lds, row, ch);
  }
}

// ---- split-K epilogues: a block takes 8 rows x one 256-column tile column (grid: row groups x
// tile columns); thread t owns row t / 32 of the group and its 16-byte chunk t % 32.

constexpr int RED_ROWS = 8;

// The unsplit map epilogue on split sums: x = bf16(sum + bias) and the rows' sum-of-squares partial of
// this 256-column group, formed in the order every producer uses (one wave per row).
// res (optional): the residual stream, X = bf16(res + bf16(sum + bias)) (rf_residual_add's rounding after
// the product's), the statistics then being X's.
__global__ __launch_bounds__(256) void k_map_apply_reduce(const float* __restrict__ part, int splits,
                                                          const uint16_t* __restrict__ bias, uint16_t* __restrict__ X,
                                                          int64_t ldx, float* __restrict__ ssq, int M, int N,
                                                          const uint16_t* __restrict__ res = nullptr, int64_t ldr = 0) {
  __shared__ uint4 img[RED_ROWS * 32];
  const int t = threadIdx.x, r = t >> 5, ch = t & 31, tn = blockIdx.y, n0 = tn * BN;
  const int m = blockIdx.x * RED_ROWS + r;
  uint4 o = make_uint4(0u, 0u, 0u, 0u);
  if (m < M) {
    float v[8];
    split_sums(part, splits, static_cast<int64_t>(M) * N, static_cast<int64_t>(m) * N + n0 + ch * 8, v);
    if (bias) {
      const uint4 b = *reinterpret_cast<const uint4*>(bias + n0 + ch * 8);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] += bf2f(lane_of(b, e));
    }
    if (res) {
      const uint4 h = *reinterpret_cast<const uint4*>(res + static_cast<int64_t>(m) * ldr + n0 + ch * 8);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = bf2f(lane_of(h, e)) + bf2f(f2bf(v[e]));
    }
    o = make_uint4(bf16_pair(v[0], v[1]), bf16_pair(v[2], v[3]), bf16_pair(v[4], v[5]), bf16_pair(v[6], v[7]));
    *reinterpret_cast<uint4*>(X + static_cast<int64_t>(m) * ldx + n0 + ch * 8) = o;
  }
  img[r * 32 + (ch ^ r)] = o;
  __syncthreads();
  const int lane = t & 63, w = t >> 6;
  for (int rr = 2 * w; rr < 2 * w + 2; ++rr) {
    const int mm = blockIdx.x * RED_ROWS + rr;
    if (mm >= M) break;                             // wave-uniform
    row_partials([&](int64_t c) {
      const uint4 q = img[rr * 32 + ((static_cast<int>(c) >> 3) ^ rr)];
      return (c & 4) ? make_uint2(q.z, q.w) : make_uint2(q.x, q.y);
    }, ssq + static_cast<int64_t>(mm) * (N / SSQ_COLS) + tn, 1, lane);
  }
}

// The unsplit norm + linear epilogue on split sums: out = bf16(sum * r_row).
__global__ __launch_bounds__(256) void k_norm_linear_reduce(const float* __restrict__ part, int splits,
                                                            const float* __restrict__ ssq, int K, float eps,
                                                            uint16_t* __restrict__ out, int64_t ldo, int M, int N) {
  const int t = threadIdx.x, r = t >> 5, ch = t & 31, n0 = blockIdx.y * BN;
  const int m = blockIdx.x * RED_ROWS + r;
  if (m >= M) return;
  const int nparts = K / SSQ_COLS;
  float s2 = 0.f;
  for (int i = 0; i < nparts; ++i) s2 += ssq[static_cast<int64_t>(m) * nparts + i];
  const float rs = 1.0f / sqrtf(s2 / static_cast<float>(K) + eps);
  float v[8];
  split_sums(part, splits, static_cast<int64_t>(M) * N, static_cast<int64_t>(m) * N + n0 + ch * 8, v);
  *reinterpret_cast<uint4*>(out + static_cast<int64_t>(m) * ldo + n0 + ch * 8) =
      make_uint4(bf16_pair(v[0] * rs, v[1] * rs), bf16_pair(v[2] * rs, v[3] * rs), bf16_pair(v[4] * rs, v[5] * rs),
                 bf16_pair(v[6] * rs, v[7] * rs));
}

// SwiGLU on the split sums of a [gate; up] product (gate columns [0, I), up columns [I, 2 I) of the partial
// planes, row stride N): act = bf16(bf16(silu(g)) * u) with g, u = bf16(sum * r_row), the roundings of the
// unsplit norm + linear epilogue followed by rf_silu_mul.
__global__ __launch_bounds__(256) void k_swiglu_reduce(const float* __restrict__ part, int splits,
                                                       const float* __restrict__ ssq, int K, float eps,
                                                       uint16_t* __restrict__ act, int64_t lda, int M, int N, int I) {
  const int t = threadIdx.x, r = t >> 5, ch = t & 31, n0 = blockIdx.y * BN;
  const int m = blockIdx.x * RED_ROWS + r;
  if (m >= M) return;
  const int nparts = K / SSQ_COLS;
  float s2 = 0.f;
  for (int i = 0; i < nparts; ++i) s2 += ssq[static_cast<int64_t>(m) * nparts + i];
  const float rs = 1.0f / sqrtf(s2 / static_cast<float>(K) + eps);
  float g[8], u[8], o[8];
  const int64_t plane = static_cast<int64_t>(M) * N, at = static_cast<int64_t>(m) * N + n0 + ch * 8;
  split_sums(part, splits, plane, at, g);
  split_sums(part, splits, plane, at + I, u);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float gx = bf2f(f2bf(g[e] * rs)), ux = bf2f(f2bf(u[e] * rs));
    o[e] = bf2f(f2bf(gx / (1.0f + expf(-gx)))) * ux;
  }
  *reinterpret_cast<uint4*>(act + static_cast<int64_t>(m) * lda + n0 + ch * 8) =
      make_uint4(bf16_pair(o[0], o[1]), bf16_pair(o[2], o[3]), bf16_pair(o[4], o[5]), bf16_pair(o[6], o[7]));
}

// The unsplit K / V (or query) epilogue on split sums: the normed chunk bf16(sum * r_row), then k_norm,
// RoPE and the cache write of kv_chunk_row.
__global__ __launch_bounds__(256) void k_norm_kv_reduce(const float* __restrict__ part, int splits, int M, int N,
                                                        KvArgs a) {
  __shared__ uint4 img[RED_ROWS * 32];
  const int t = threadIdx.x, r = t >> 5, ch = t & 31, n0 = blockIdx.y * BN;
  const int m = blockIdx.x * RED_ROWS + r;
  uint4 o = make_uint4(0u, 0u, 0u, 0u);
  if (m < M) {
    float s2 = 0.f;
    for (int i = 0; i < a.nparts; ++i) s2 += a.ssq[static_cast<int64_t>(m) * a.nparts + i];
    const float rs = 1.0f / sqrtf(s2 / a.h + a.eps);
    float v[8];
    split_sums(part, splits, static_cast<int64_t>(M) * N, static_cast<int64_t>(m) * N + n0 + ch * 8, v);
    o = make_uint4(bf16_pair(v[0] * rs, v[1] * rs), bf16_pair(v[2] * rs, v[3] * rs), bf16_pair(v[4] * rs, v[5] * rs),
                   bf16_pair(v[6] * rs, v[7] * rs));
  }
  img[r * 32 + (ch ^ r)] = o;
  __syncthreads();
  const KvLane L(a, n0, ch);
  bool ok = m < M;
  if (ok && a.pos_lim > 0) {                        // positions checked on the device: no table read or write
    const int64_t p = a.pos[m];                     // outside the table and the cache
    ok = p >= 0 && p < a.pos_lim;
  }
  kv_chunk_row(a, L, [&](int c) { return image_chunk(img, r, c); }, ch, m, ok, rope_fetch(a, L, m, ok));
}

// Adds a run's fp32 sums (acc) into the fp64 accumulator C for the tile at (m0, n0), rows < M. The sums go
// through LDS, half the tile (128 rows) at a time, as a row-major fp32 image (row r's 16-byte chunk c at
// r * 64 + (c ^ (r & 15)): the accumulator writes and the row reads both hit 16 distinct bank groups per
// 16 lanes), so that each wave instruction of the read-modify-write of C covers 2 KB of one row of C instead
// of 16 bytes in each of 32 rows. Needs the LDS free on entry; leaves it free.
__device__ __forceinline__ void fold_tile(const f32x16 (&acc)[4][4], uint4* lds, double* __restrict__ C,
                                          int64_t ldc, int M, int m0, int n0) {
  const int t = threadIdx.x, lane = t & 63;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wm = w >> 1, wn = w & 1, lr = lane & 31, lk = lane >> 5;
  float4* img = reinterpret_cast<float4*>(lds);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    if (wm == h) {
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < 4; ++nt)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int r = mt * 32 + lr, c = wn * 32 + nt * 8 + 2 * g + lk;
            img[r * 64 + (c ^ (r & 15))] = make_float4(acc[nt][mt][4 * g], acc[nt][mt][4 * g + 1],
                                                       acc[nt][mt][4 * g + 2], acc[nt][mt][4 * g + 3]);
          }
    }
    __syncthreads();
    // wave w: image rows 32w .. 32w + 31 in 4 batches of 8; batch b + 1's rows of C load before batch b's
    // stores, so two batches' loads are in flight (the compiler keeps loads of C behind earlier stores to
    // C, so it would not overlap them by itself). Loads are unconditional (rows past M read row M - 1, not
    // stored): a conditional load would make the stores wait for every load in flight.
    double2 v[2][8][2];
    auto load_batch = [&](int b, double2 (&d)[8][2]) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int gm = min(m0 + h * 128 + w * 32 + b * 8 + i, M - 1);
        const double* p = C + static_cast<int64_t>(gm) * ldc + n0 + 4 * lane;
        d[i][0] = *reinterpret_cast<const double2*>(p);
        d[i][1] = *reinterpret_cast<const double2*>(p + 2);
      }
    };
    load_batch(0, v[0]);
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      if (b + 1 < 4) load_batch(b + 1, v[(b + 1) & 1]);
      double2 (&d)[8][2] = v[b & 1];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int j = w * 32 + b * 8 + i, gm = m0 + h * 128 + j;
        if (gm < M) {
          const float4 a = img[j * 64 + (lane ^ (j & 15))];
          d[i][0].x += a.x;
          d[i][0].y += a.y;
          d[i][1].x += a.z;
          d[i][1].y += a.w;
          double* p = C + static_cast<int64_t>(gm) * ldc + n0 + 4 * lane;
          *reinterpret_cast<double2*>(p) = d[i][0];
          *reinterpret_cast<double2*>(p + 2) = d[i][1];
        }
      }
    }
    __syncthreads();
  }
}

// Writes a run's fp32 sums (acc) of one tile as a row-major [256, 256] fp32 plane, through the LDS image of
// fold_tile (half the tile at a time), so that each wave instruction stores 1 KB of one row. Needs the LDS
// free on entry; leaves it free.
__device__ __forceinline__ void store_tile(const f32x16 (&acc)[4][4], uint4* lds, float* __restrict__ out) {
  const int t = threadIdx.x, lane = t & 63;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wm = w >> 1, wn = w & 1, lr = lane & 31, lk = lane >> 5;
  float4* img = reinterpret_cast<float4*>(lds);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    if (wm == h) {
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < 4; ++nt)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int r = mt * 32 + lr, c = wn * 32 + nt * 8 + 2 * g + lk;
            img[r * 64 + (c ^ (r & 15))] = make_float4(acc[nt][mt][4 * g], acc[nt][mt][4 * g + 1],
                                                       acc[nt][mt][4 * g + 2], acc[nt][mt][4 * g + 3]);
          }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 32; ++i) {                // wave w: image rows 32 w .. 32 w + 31
      const int j = w * 32 + i;
      *reinterpret_cast<float4*>(out + static_cast<int64_t>(h * 128 + j) * BN + 4 * lane) =
          img[j * 64 + (lane ^ (j & 15))];
    }
    __syncthreads();
  }
}

// The schedule of a Gram launch. Logical tiles [0, T - ptiles) run whole, one block each: their runs are
// added into C as they end (fold_tile). The last ptiles logical tiles are cut into their runs, one block
// per (tile, run), each writing its run's fp32 sums to part ([ptiles * runs][256][256], run order within a
// tile); k_gram_fold then adds each tile's runs into C in run order. Same sums, same order: the two
// schedules give the same bits. The run blocks come first in the grid (pieces of them, a multiple of 8, so
// the whole tiles keep their XCD placement), which spreads a launch of slightly more tiles than CUs over
// one round of whole tiles and a short round of runs instead of two rounds of whole tiles.
struct GramPlan {
  int pieces;             // grid blocks before the whole tiles (>= ptiles * runs, a multiple of 8)
  int ptiles, runs;
  float* part;
  int upper;              // the logical tiles are C's block-upper tiles only (gram_coords)
};

// Logical tile -> (tile row, tile column) of a Gram launch: tile_coords over every tile, or with `upper` the
// block-upper tiles (tn >= tm) row by row, for the symmetric X^T X (tiles_m <= tiles_n, tile < the count).
__device__ __forceinline__ void gram_coords(int tile, int tiles_m, int tiles_n, bool upper, int& tm, int& tn) {
  if (!upper) {
    tile_coords<GRAM_GROUP_M>(tile, tiles_m, tiles_n, tm, tn);
    return;
  }
  int r = 0;
  while (r + 1 < tiles_m && tile >= tiles_n - r) {
    tile -= tiles_n - r;
    ++r;
  }
  tm = r;
  tn = r + tile;
}

// C[m, n] += sum_k A[m, k] B[n, k]: bf16 products summed in fp32 over runs of at most `fold` of K, each run's
// sums added into the fp64 accumulator C as it ends (fold_tile), or stored for k_gram_fold (GramPlan). Each
// tile owns its 256 x 256 block of C, so the read-modify-write is race-free and the result does not depend
// on the schedule.
__global__ __launch_bounds__(NTHR) void k_gram(const uint16_t* __restrict__ A, int64_t lda,
                                               const uint16_t* __restrict__ B, int64_t ldb, int M, int N, int K,
                                               int fold, double* __restrict__ C, int64_t ldc, GramPlan pl) {
  __shared__ uint4 lds[LDS_U4];
  const int tiles_m = (M + BM - 1) / BM, tiles_n = N / BN;
  const int whole = static_cast<int>(gridDim.x) - pl.pieces;
  int tm, tn;
  f32x16 acc[4][4];
  if (static_cast<int>(blockIdx.x) < pl.pieces) {
    const int p = blockIdx.x, t = p / pl.runs, run = p - t * pl.runs;
    if (t >= pl.ptiles) return;                     // padding block (block-uniform; no barrier reached)
    gram_coords(whole + t, tiles_m, tiles_n, pl.upper, tm, tn);
    const int k0 = run * fold, k1 = min(k0 + fold, K);
    mainloop(A + k0, lda, B + k0, ldb, M, k1 - k0, tm * BM, tn * BN, lds, acc);
    store_tile(acc, lds, pl.part + static_cast<int64_t>(p) * BM * BN);
    return;
  }
  gram_coords(xcd_tile(blockIdx.x - pl.pieces, whole), tiles_m, tiles_n, pl.upper, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  for (int k0 = 0; k0 < K; k0 += fold) {
    const int k1 = min(k0 + fold, K);
    mainloop(A + k0, lda, B + k0, ldb, M, k1 - k0, m0, n0, lds, acc);
    fold_tile(acc, lds, C, ldc, M, m0, n0);
  }
}

// C += the stored runs of the last ptiles logical tiles (GramPlan), each tile's runs in run order: block =
// 4 rows of one tile, thread = 4 consecutive columns (whole 1 KB rows of the planes, 2 KB rows of C).
__global__ __launch_bounds__(256) void k_gram_fold(const float* __restrict__ part, int ptiles, int runs, int whole,
                                                   int M, int N, double* __restrict__ C, int64_t ldc, int upper) {
  const int t = blockIdx.x >> 6, row = (blockIdx.x & 63) * 4 + (threadIdx.x >> 6), c4 = threadIdx.x & 63;
  if (t >= ptiles) return;
  int tm, tn;
  gram_coords(whole + t, (M + BM - 1) / BM, N / BN, upper, tm, tn);
  const int gm = tm * BM + row;
  if (gm >= M) return;
  double* p = C + static_cast<int64_t>(gm) * ldc + tn * BN + 4 * c4;
  double2 v0 = *reinterpret_cast<const double2*>(p), v1 = *reinterpret_cast<const double2*>(p + 2);
  const float* q = part + (static_cast<int64_t>(t) * runs * BM + row) * BN + 4 * c4;
  for (int r = 0; r < runs; ++r) {
    const float4 a = *reinterpret_cast<const float4*>(q + static_cast<int64_t>(r) * BM * BN);
    v0.x += a.x;
    v0.y += a.y;
    v1.x += a.z;
    v1.y += a.w;
  }
  *reinterpret_cast<double2*>(p) = v0;
  *reinterpret_cast<double2*>(p + 2) = v1;
}

// The MFMA throughput the power budget allows: back-to-back v_mfma_f32_32x32x16_bf16 on register operands,
// four independent accumulators per wave each with its own pair of operands (pseudo-random bf16: random
// sign, mantissa and two low exponent bits, magnitudes 2^-7 .. 2^-3), so the operands change from one
// MFMA to the next as a GEMM's fragments do; no memory traffic but one store per lane at the end. A
// measurement, not part of the fill.
__global__ __launch_bounds__(256) void k_mfma_ceiling(int iters, float* __restrict__ out) {
  const uint32_t id = blockIdx.x * 256u + threadIdx.x;
  uint32_t h = id * 0x9e3779b9u + 0x7f4a7c15u;
  auto next = [&]() {
    h ^= h << 13;
    h ^= h >> 17;
    h ^= h << 5;
    return (h & 0x81ff81ffu) | 0x3c003c00u;
  };
  bf16x8 a[4], b[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t a0 = next(), a1 = next(), a2 = next(), a3 = next();
    const uint32_t b0 = next(), b1 = next(), b2 = next(), b3 = next();
    a[j] = __builtin_bit_cast(bf16x8, make_uint4(a0, a1, a2, a3));
    b[j] = __builtin_bit_cast(bf16x8, make_uint4(b0, b1, b2, b3));
  }
  f32x16 acc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[j][r] = 0.f;
  for (int i = 0; i < iters; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[j], b[j], acc[j], 0, 0, 0);
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) sum += acc[j][r];
  out[id] = sum;
}

// ---- Persistent tiles: one block per CU runs a sequence of output tiles over one continuous ring of K
// steps, so the next tile's first operand steps load while this tile finishes (no pipeline fill and no
// block dispatch per tile), and a launch can hold the tiles of several layers (no tail per layer).
//
// The ring is the one of mainloop, indexed by a global step g that runs on across tiles (slot of quarter
// q: (4 g + q) % 10). In a tile's last step the weight quarters of step g + 2 (the next tile's step 1) are
// not loaded during slice 3: the epilogue of the tile runs first, in the four slots of that last step
// (two activation slots, 32 KiB contiguous, for a 64-row image; a weight slot for per-tile side data),
// which nothing loads into until those deferred loads, issued after the epilogue's closing barrier. They
// still have three slices before the barrier that needs them, as in the steady loop. The MFMA k order
// and the epilogue arithmetic are those of the per-tile kernels, so the results are bit-identical.

// Buffer resources of one tile's operands: activation rows m0 .. (range-checked past the tile's rows) and
// the tile's 256 weight rows.
struct TileOps {
  __amdgpu_buffer_rsrc_t rx, rw;
};


// This block's tiles of T logical tiles: first + stride * i for i < cnt. With 256 blocks (T >= 256) XCD x
// (blocks x, x + 8, ...) takes a contiguous eighth of the logical order and its 32 blocks walk it 32 tiles
// at a time, so the tiles an XCD runs together form GROUP_M x 8 groups as in the per-tile kernels. With
// fewer tiles than 256, one tile per block (xcd_tile order).
struct Share {
  int first, stride, cnt;
};
__device__ __forceinline__ Share block_share(int T) {
  if (static_cast<int>(gridDim.x) < 256) return Share{xcd_tile(blockIdx.x, gridDim.x), 0, 1};
  const int x = blockIdx.x & 7, c = blockIdx.x >> 3;
  const int q = T >> 3, r = T & 7;
  const int lo = x * q + min(x, r), size = q + (x < r ? 1 : 0);
  return Share{lo + c, 32, c < size ? (size - c + 31) / 32 : 0};
}

int persistent_grid(int64_t tiles) { return static_cast<int>(std::min<int64_t>(tiles, 256)); }

// Tile row of row ir (0..63) of epilogue round r's image: image rows 0..31 are tile rows r*32 .. r*32 + 31
// (waves wm = 0), rows 32..63 tile rows 128 + r*32 .. (wm = 1).
__device__ __forceinline__ int round_row(int ir, int r) { return (ir >> 5) * 128 + r * 32 + (ir & 31); }

// threadIdx.x as a value the compiler cannot move: the epilogues derive their lane arithmetic from it, so
// that arithmetic stays in the epilogue instead of being hoisted out of the tile loop and kept live (in
// registers the main loop needs) across every K step.
__device__ __forceinline__ int pinned_tid() {
  int t = static_cast<int>(threadIdx.x);
  asm volatile("" : "+v"(t));
  return t;
}

// One accumulator element read out of its AGPR where it is used (the compiler otherwise copies whole
// accumulator vectors into VGPRs ahead of the epilogue, more registers than the tile loop has spare).
__device__ __forceinline__ float agpr_read(float a) {
  float v;
  asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(v) : "a"(a));
  return v;
}

// Epilogue round r (compile-time MT = r): the wave's rows wm*128 + r*32 + lr, rounded to bf16 by value(nt, g,
// e, acc), into a 64-row image (row wm*32 + lr; row i's chunk c at i * 32 + (c ^ (i & 31))). With SSQ, ss
// receives the sum of squares of the lane's 64 rounded values in (nt, g, e) order, as stage_tile forms it.
template <int MT, bool SSQ, class F>
__device__ __forceinline__ void stage_round(uint4* img, const f32x16 (&acc)[4][4], F value, float& ss, int t) {
  const int lane = t & 63, w = t >> 6;
  const int wm = w >> 1, wn = w & 1, lr = lane & 31, lk = lane >> 5;
  char* base = reinterpret_cast<char*>(img);
  const int row = wm * 32 + lr;
  float sq = 0.f;
#pragma unroll
  for (int nt = 0; nt < 4; ++nt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int c0 = wn * 128 + nt * 32 + 8 * g + 4 * lk;
      const uint32_t p0 = bf16_pair(value(nt, g, 0, agpr_read(acc[nt][MT][4 * g + 0])),
                                    value(nt, g, 1, agpr_read(acc[nt][MT][4 * g + 1])));
      const uint32_t p1 = bf16_pair(value(nt, g, 2, agpr_read(acc[nt][MT][4 * g + 2])),
                                    value(nt, g, 3, agpr_read(acc[nt][MT][4 * g + 3])));
      if (SSQ) {
        const float r0 = bf_lo(p0), r1 = bf_hi(p0), r2 = bf_lo(p1), r3 = bf_hi(p1);
        sq = fmaf(r0, r0, sq);
        sq = fmaf(r1, r1, sq);
        sq = fmaf(r2, r2, sq);
        sq = fmaf(r3, r3, sq);
      }
      const int off = row * 512 + (((c0 >> 3) ^ (row & 31)) << 4) + ((c0 & 7) << 1);
      *reinterpret_cast<uint2*>(base + off) = make_uint2(p0, p1);
    }
  ss = sq;
}

// Runs this block's tiles 0 .. cnt - 1 (cnt >= 1; every tile K = nk * 64 deep, nk >= 2): ops(i) gives tile
// i's operand resources; begin(i, acc) sets its accumulators' starting values; end(i, acc, img, side) is its
// epilogue, with img (32 KiB) and side (32 KiB) of LDS to itself. end must finish with a barrier after
// every wave's last LDS access. pre(i, side) runs in tile i's last K step as soon as side is free (after
// that step's barrier, one slice before the epilogue): loads it issues into side land during that slice.
template <class Ops, class Begin, class Pre, class End>
__device__ __forceinline__ void stream_tiles(int cnt, int nk, int64_t ldx, int64_t ldw, Ops ops, Begin begin, Pre pre,
                                             End end, uint4* lds) {
  const int t = threadIdx.x, lane = t & 63;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wm = w >> 1, wn = w & 1;
  uint32_t vx[2][4], vw[2][4];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 32 * w + 8 * i + (lane >> 3);
      const int ch = (lane & 7) ^ slot_swz(r);
      vx[h][i] = static_cast<uint32_t>(((h * 128 + r) * ldx + ch * 8) * 2);
      vw[h][i] = static_cast<uint32_t>(((h * 128 + r) * ldw + ch * 8) * 2);
    }
  char* base = reinterpret_cast<char*>(lds);
  const int lr = lane & 31, lk = lane >> 5, swz = slot_swz(lr);
  bf16x8 fx[2][4], fw[2][4];
  f32x16 acc[4][4];
  TileOps cur = ops(0);
  TileOps nxt = cnt > 1 ? ops(1) : cur;

  // (global steps are named by their ring phase, slot_at / next_ph)
  // fragment r (0..7) of slice ks of the global step of phase ph: r < 4 -> weight block r, else activation
  // block r - 4
  auto read_one = [&](int ph, int ks, int r, bf16x8 (&ax)[4], bf16x8 (&aw)[4]) {
    const int ch = (ks * 2 + lk) ^ swz;
    if (r < 4) aw[r] = as_frag(lds[slot_at(ph, 2 + wn) * SLOT_U4 + (r * 32 + lr) * CPR + ch]);
    else ax[r - 4] = as_frag(lds[slot_at(ph, wm) * SLOT_U4 + ((r - 4) * 32 + lr) * CPR + ch]);
  };
  // load j (0..7) of the activation (wt = false) or weight quarters of the global step of phase ph:
  // tile-local step k of o
  auto load = [&](const TileOps& o, int ph, int k, bool wt, int j) {
    const int h = j >> 2, i = j & 3;
    if (wt) issue_load_at(o.rw, vw[h][i], slot_at(ph, 2 + h), k, i, base, w);
    else issue_load_at(o.rx, vx[h][i], slot_at(ph, h), k, i, base, w);
  };
  // as mainloop's slice, with the loads' source o, global step phase lph and tile-local step lk2
  auto slice = [&](const bf16x8 (&ax)[4], const bf16x8 (&aw)[4], bool rd, int rph, int rks, bf16x8 (&nx)[4],
                   bf16x8 (&nw)[4], int ld, const TileOps& o, int lph, int lk2, int lo) {
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int qi = q >> 2, qj = (qi & 1) ? 3 - (q & 3) : (q & 3);   // snake: one operand changes per MFMA
      acc[qi][qj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(aw[qi], ax[qj], acc[qi][qj], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
      if (q < 8 && rd) read_one(rph, rks, q, nx, nw);
      if (ld == 2 && !(q & 1)) load(o, lph, lk2, true, q >> 1);
      if (ld == 1 && (q & 3) == 1) load(o, lph, lk2, false, lo + (q >> 2));
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // global step g; the loads of step g + 2 (source o2, tile-local step k2) when `has2`; its weight
  // quarters in slice 3 unless `defer`; `has1`: step g + 1 exists (its first fragments are read)
  // (`defer` marks a tile's last step: its weight slots, free after the barrier, go to pre(i, ...))
  auto step = [&](int ph, const TileOps& o2, int k2, auto has2, auto defer, bool has1, int i) {
    const int ph1 = next_ph(ph), ph2 = next_ph(ph1);
    slice(fx[0], fw[0], true, ph, 1, fx[1], fw[1], has2 ? 1 : 0, o2, ph2, k2, 0);
    slice(fx[1], fw[1], true, ph, 2, fx[0], fw[0], has2 ? 1 : 0, o2, ph2, k2, 4);
    slice(fx[0], fw[0], true, ph, 3, fx[1], fw[1], 0, o2, 0, 0, 0);
    if (has2) wait_vm_lgkm0<8>();
    else wait_vm_lgkm0<0>();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    if (defer) {
      pre(i, lds + slot_at(ph, 2) * SLOT_U4);
      __builtin_amdgcn_sched_barrier(0);
    }
    slice(fx[1], fw[1], has1, ph1, 0, fx[0], fw[0], (has2 && !defer) ? 2 : 0, o2, ph2, k2, 0);
  };

  // prologue: steps 0 and 1 of tile 0 (phases 0 and 4), then the accumulators and step 0's first fragments
  for (int j = 0; j < 8; ++j) load(cur, 0, 0, false, j);
  for (int j = 0; j < 8; ++j) load(cur, 0, 0, true, j);
  for (int j = 0; j < 8; ++j) load(cur, 4, 1, false, j);
  for (int j = 0; j < 8; ++j) load(cur, 4, 1, true, j);
  begin(0, acc);
  wait_vm_lgkm0<16>();
  __builtin_amdgcn_s_barrier();
  for (int r = 0; r < 8; ++r) read_one(0, 0, r, fx[0], fw[0]);
  int ph = 0;                                     // phase of the global step
  for (int i = 0; i < cnt; ++i) {
    const bool more = i + 1 < cnt;
    for (int kt = 0; kt + 2 < nk; ++kt, ph = next_ph(ph))
      step(ph, cur, kt + 2, std::true_type{}, std::false_type{}, true, i);
    // the tile's last two steps: step g + 2 is the next tile's step 0, then its step 1
    step(ph, nxt, 0, more, std::false_type{}, true, i);
    const int ph_last = next_ph(ph);
    step(ph_last, nxt, 1, more, std::true_type{}, false, i);
    ph = next_ph(ph_last);
    // ph is the next tile's first step (landed: the last barrier waited for it); the step before it
    // (phase ph_last) left its four slots free: activation slots (img) and weight slots (side), each pair
    // contiguous. The next tile's first fragments are read after the epilogue, so that they do not hold
    // registers through it.
    end(i, acc, lds + slot_at(ph_last, 0) * SLOT_U4, reinterpret_cast<float*>(lds + slot_at(ph_last, 2) * SLOT_U4));
    if (more) {
      for (int j = 0; j < 8; ++j) load(nxt, next_ph(ph), 1, true, j);   // the deferred weight quarters of its step 1
      cur = nxt;
      if (i + 2 < cnt) nxt = ops(i + 2);
      begin(i + 1, acc);
      for (int r = 0; r < 8; ++r) read_one(ph, 0, r, fx[0], fw[0]);
    }
  }
  wait_vm_lgkm0<0>();
}

// Per-layer operands of a batched launch (one launch for the fill of several late layers: every layer
// reads the same rows b, and has its own map, bias, output rows and statistics).
constexpr int MAXL = 32;
struct MapLayers {
  const uint16_t* w[MAXL];
  const uint16_t* c[MAXL];
  uint16_t* x[MAXL];
  float* ssq[MAXL];
};

// rf_map_apply on persistent tiles, for nl layers at once: x_l = b W_l^T + c_l, the accumulators starting
// at the bias, and the rows' sum-of-squares partials; logical tile u is layer u / (tiles of a layer).
// RES (one layer): x = bf16(res + bf16(b W^T + c)), rf_residual_add's rounding after the product's, the
// statistics then being x's (a lane loads the residual of its 64 values of a round, the next round's
// while the current one is written).
template <bool RES = false>
__global__ __launch_bounds__(NTHR) void k_map_apply_p(const uint16_t* __restrict__ B, int64_t ldb, MapLayers ml, int nl,
                                                      int64_t ldx, int M, int N, int K,
                                                      const uint16_t* __restrict__ res = nullptr, int64_t ldr = 0) {
  __shared__ uint4 lds[LDS_U4];
  const int tiles_n = N / BN, tiles_m = (M + BM - 1) / BM, per = tiles_m * tiles_n;
  const Share sh = block_share(nl * per);
  if (sh.cnt == 0) return;
  const int t = threadIdx.x, lane = t & 63, wn = (t >> 6) & 1, lk = lane >> 5;
  auto coords = [&](int i, int& l, int& tm, int& tn) {
    const int u = sh.first + i * sh.stride;
    l = u / per;
    tile_coords(u - l * per, tiles_m, tiles_n, tm, tn);
  };
  auto ops = [&](int i) {
    int l, tm, tn;
    coords(i, l, tm, tn);
    const int m0 = tm * BM;
    return TileOps{buffer_rsrc(B + static_cast<int64_t>(m0) * ldb, static_cast<uint32_t>(min(M - m0, BM) * ldb * 2)),
                   buffer_rsrc(ml.w[l] + static_cast<int64_t>(tn) * BN * K, static_cast<uint32_t>(BN * K * 2))};
  };
  // bias of the next tile to begin: lane (lr, lk) holds columns wn*128 + nt*32 + 8g + 4lk + e
  uint2 bq[4][4];
  auto load_bias = [&](int i) {
    int l, tm, tn;
    coords(i, l, tm, tn);
    const uint16_t* c = ml.c[l];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        bq[nt][g] = c ? *reinterpret_cast<const uint2*>(c + tn * BN + wn * 128 + nt * 32 + 8 * g + 4 * lk)
                      : make_uint2(0u, 0u);
  };
  auto begin = [&](int, f32x16 (&acc)[4][4]) {
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float b0 = bf_lo(bq[nt][g].x), b1 = bf_hi(bq[nt][g].x), b2 = bf_lo(bq[nt][g].y), b3 = bf_hi(bq[nt][g].y);
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
          acc[nt][mt][4 * g + 0] = b0;
          acc[nt][mt][4 * g + 1] = b1;
          acc[nt][mt][4 * g + 2] = b2;
          acc[nt][mt][4 * g + 3] = b3;
        }
      }
  };
  auto end = [&](int i, const f32x16 (&acc)[4][4], uint4* img, float* side) {
    int l, tm, tn;
    coords(i, l, tm, tn);
    const int t = pinned_tid(), lane = t & 63, w = t >> 6, wm = w >> 1, wn = w & 1, lr = lane & 31, lk = lane >> 5;
    const int m0 = tm * BM, n0 = tn * BN, ch = t & 31;
    uint16_t* X = ml.x[l];
    float* S = ml.ssq[l];
    if (i + 1 < sh.cnt) load_bias(i + 1);
    // the residual of round r's values of this lane: row wm*128 + r*32 + lr, columns wn*128 + nt*32 + 8g +
    // 4lk .. + 3 (rows past M read row M - 1; they are not stored)
    uint2 rq[2][4][4];
    auto load_res = [&](int r, uint2 (&q)[4][4]) {
      const int gm = min(m0 + wm * 128 + r * 32 + lr, M - 1);
      const uint16_t* rr = res + static_cast<int64_t>(gm) * ldr + n0 + wn * 128 + 4 * lk;
#pragma unroll
      for (int nt = 0; nt < 4; ++nt)
#pragma unroll
        for (int g = 0; g < 4; ++g) q[nt][g] = *reinterpret_cast<const uint2*>(rr + nt * 32 + 8 * g);
    };
    if constexpr (RES) load_res(0, rq[0]);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      __builtin_amdgcn_sched_barrier(0);
      float ss = 0.f;
      if constexpr (RES) {
        auto resv = [&](int nt, int g, int e, float a) {
          const uint2 q = rq[r & 1][nt][g];
          const uint32_t u = e < 2 ? q.x : q.y;
          return ((e & 1) ? bf_hi(u) : bf_lo(u)) + bf2f(f2bf(a));
        };
        switch (r) {
          case 0: stage_round<0, true>(img, acc, resv, ss, t); break;
          case 1: stage_round<1, true>(img, acc, resv, ss, t); break;
          case 2: stage_round<2, true>(img, acc, resv, ss, t); break;
          default: stage_round<3, true>(img, acc, resv, ss, t); break;
        }
        if (r < 3) load_res(r + 1, rq[(r + 1) & 1]);
      } else {
        auto ident = [](int, int, int, float a) { return a; };
        switch (r) {
          case 0: stage_round<0, true>(img, acc, ident, ss, t); break;
          case 1: stage_round<1, true>(img, acc, ident, ss, t); break;
          case 2: stage_round<2, true>(img, acc, ident, ss, t); break;
          default: stage_round<3, true>(img, acc, ident, ss, t); break;
        }
      }
      const float tot = ss + __shfl_xor(ss, 32, 64);             // the row's 128 columns of this wave
      if (lk == 0) side[wn * 64 + wm * 32 + lr] = tot;
      __syncthreads();
      if (t < 64) {
        const int gm = m0 + round_row(t, r);
        if (gm < M) S[static_cast<int64_t>(gm) * tiles_n + tn] = side[t] + side[64 + t];
      }
#pragma unroll 4
      for (int it = 0; it < 8; ++it) {
        const int ir = it * 8 + (t >> 5);
        const int gm = m0 + round_row(ir, r);
        if (gm < M) *reinterpret_cast<uint4*>(X + static_cast<int64_t>(gm) * ldx + n0 + ch * 8) = image_chunk(img, ir, ch);
      }
      __syncthreads();
    }
    // (RES: nothing of the residual loads stays in flight into the next tile's K loop, whose registers
    // they share; without this wait the compiler guards that loop's fragment reads with vmcnt waits)
    if constexpr (RES) wait_vm_lgkm0<0>();
  };
  load_bias(0);
  stream_tiles(sh.cnt, K / BK, ldb, K, ops, begin, [](int, uint4*) {}, end, lds);
}

// Per-layer operands of a batched K / V fill.
struct KvLayers {
  const uint16_t* x[MAXL];
  const float* ssq[MAXL];
  const uint16_t* wkv[MAXL];
  const uint16_t* knorm[MAXL];
  uint16_t* kbuf[MAXL];
  uint16_t* vbuf[MAXL];
};

// Input RMSNorm scales 1 / sqrt(mean(x^2) + eps) of a tile's 256 rows from their nparts = 4 q4 partials
// (q4 <= 4), summed in order as row_scale sums them. The tile's partials are one contiguous block, loaded
// 16 bytes a lane: load k holds rows k * 256 / q4 + t / q4, lane t % q4 their partials 4 (t % q4) .. + 3.
// parts_load issues the loads (all before any use); parts_sum adds each row's partials in order along its
// q4 lanes (lane j starts from lane j - 1's running sum), leaving the scale of row k * 256 / q4 + t / q4 in
// sc[k] of the row's last lane (t % q4 == q4 - 1). Both run without branches: all four loads issue (loads
// k >= q4 repeat load 0) and every loaded register is read, so no load is left in flight on any path the
// compiler's wait counting follows (a pending load there would make the next tile's K loop wait for all
// loads at every step).
__device__ __forceinline__ void parts_load(const float* __restrict__ ssq, int q4, int M, int m0, int t, float4 (&v)[4]) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int kk = k < q4 ? k : 0;
    const int row = min(m0 + kk * (256 / q4) + t / q4, M - 1);
    v[k] = *reinterpret_cast<const float4*>(ssq + static_cast<int64_t>(row) * (4 * q4) + 4 * (t % q4));
  }
}
__device__ __forceinline__ void parts_sum(const float4 (&v)[4], int q4, float width, float eps, int t, float (&sc)[4]) {
  const int lane = t & 63, j = t % q4;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float s = 0.f;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {                // steps jj >= q4 change no lane (j < q4)
      const float prev = __shfl(s, lane > 0 ? lane - 1 : 0, 64);
      float a = jj == 0 ? 0.f : prev;
      a += v[k].x;
      a += v[k].y;
      a += v[k].z;
      a += v[k].w;
      s = j == jj ? a : s;
    }
    sc[k] = 1.0f / sqrtf(s / width + eps);
  }
}

// RoPE table rows of epilogue round r (64 image rows) from the table cs (resource rcs, slot-indexed rows < M,
// rb = rot * 2 bytes a row: 16 .. 256, a power of two) straight into LDS at tab (row ir at ir * rb bytes):
// each load instruction fills 1 KiB, 1024 / rb rows of rb / 16 lanes each. Rows past M read row M - 1 (never
// stored). The caller waits (vmcnt) before the barrier after which tab is read.
__device__ __forceinline__ void table_round(__amdgpu_buffer_rsrc_t rcs, int rb, int r, int m0, int M, uint4* tab, int t) {
  const int w = __builtin_amdgcn_readfirstlane(t >> 6), lane = t & 63;
  const int lpr = rb >> 4, rpi = 64 / lpr, nload = (64 * rb) >> 10;
  for (int k = w; k < nload; k += 4) {               // wave-uniform
    const int ir = k * rpi + lane / lpr;
    const int gm = min(m0 + round_row(ir, r), M - 1);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rcs, (lds_ptr)(tab + k * 64), 16,
                                             static_cast<uint32_t>(gm * rb + (lane % lpr) * 16), 0, 0, 0);
  }
}

// Row pass of epilogue round r for a K tile with its RoPE entries in LDS (tab, as table_round lays them out,
// rb bytes a row): image rows u*8 + t/32 (u < 8), chunk t % 32.
template <int MODE>
__device__ __forceinline__ void k_round_tab(const KvArgs& a, const KvLane& L, const uint4* img, const uint4* tab, int rb,
                                            int r, int m0, int M, int t) {
  const int ch = t & 31, upr = MODE == KV_ANY ? rb >> 4 : 16;
  const int half = MODE == KV_ANY ? L.half : 64;
  const int fc = L.rope ? L.fi0 >> 3 : 0;           // chunks past rot read entry 0 (unused)
  constexpr int G = MODE == KV_D128 ? 4 : 2;        // rows in flight (k_norm needs more registers a row)
#pragma unroll
  for (int h = 0; h < 8 / G; ++h) {
    uint4 o[G];
#pragma unroll
    for (int v4 = 0; v4 < G; ++v4) {
      const int ir = (h * G + v4) * 8 + (t >> 5);
      const uint4 v = image_chunk(img, ir, ch);
      const bool half8 = MODE == KV_ANY ? half >= 8 : true;
      const uint4 pv = half8 ? image_chunk(img, ir, ch + (L.pj0 - L.j0) / 8) : v;
      const float ss = head_ssq<MODE>(a, L, v);
      RopeEnt re;
      if (half8) {
        re.c = tab[ir * upr + fc];
        re.s = tab[ir * upr + (half >> 3) + fc];
      } else {                                        // rot == 8: the row's whole table in one chunk
        re.c = tab[ir * upr];
        re.s = make_uint4(0u, 0u, 0u, 0u);
      }
      o[v4] = (MODE != KV_ANY || L.norm || L.rope) ? k_chunk<MODE>(a, L, v, pv, ss, re) : v;
    }
#pragma unroll
    for (int v4 = 0; v4 < G; ++v4) {
      const int gm = m0 + round_row((h * G + v4) * 8 + (t >> 5), r);
      if (gm < M) st_stream16(L.dst0 + (a.slot0 + gm) * a.row_stride, o[v4]);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// rf_norm_kv_write on persistent tiles for nl layers at once (slot-indexed rows, no position array). The
// base arguments `a0` carry what the layers share (norm width, eps, heads, RoPE table, strides, first
// slot); the layer's statistics, weights, k_norm gains and cache buffers come from kl. KMODE is the K
// tiles' epilogue (one per launch: it follows from the configuration). A K tile's RoPE table rows go from
// the table straight into LDS (buffer_load ... lds) one round ahead, double-buffered in the two weight
// slots of its last K step (rounds 0 and 1 from that step on, pre). V tiles copy; tiles holding K and V
// columns (KV_ANY only) go chunk by chunk. Takes H a multiple of 1024 up to 4096 and a power-of-two rot <= 128 (persistent_kv_ok).
template <int KMODE>
__global__ __launch_bounds__(NTHR) void k_norm_kv_p(KvLayers kl, int nl, int64_t ldx, int M, int N, int K, KvArgs a0) {
  __shared__ uint4 lds[LDS_U4];
  const int tiles_n = N / BN, tiles_m = (M + BM - 1) / BM, per = tiles_m * tiles_n;
  const Share sh = block_share(nl * per);
  if (sh.cnt == 0) return;
  const int t = threadIdx.x;
  const int rb = a0.rot * 2;                        // bytes of a RoPE table row
  auto coords = [&](int i, int& l, int& tm, int& tn) {
    const int u = sh.first + i * sh.stride;
    l = u / per;
    tile_coords(u - l * per, tiles_m, tiles_n, tm, tn);
  };
  auto ops = [&](int i) {
    int l, tm, tn;
    coords(i, l, tm, tn);
    const int m0 = tm * BM;
    return TileOps{buffer_rsrc(kl.x[l] + static_cast<int64_t>(m0) * ldx, static_cast<uint32_t>(min(M - m0, BM) * ldx * 2)),
                   buffer_rsrc(kl.wkv[l] + static_cast<int64_t>(tn) * BN * K, static_cast<uint32_t>(BN * K * 2))};
  };
  const int q4 = a0.nparts / 4;
  auto parts_of = [&](int i, float4 (&v)[4], int tt) {
    int l, tm, tn;
    coords(i, l, tm, tn);
    parts_load(kl.ssq[l], q4, M, tm * BM, tt, v);
  };
  float sc[4];                    // the current tile's row scales (parts_sum's layout)
  {
    float4 v[4];
    parts_of(0, v, t);
    parts_sum(v, q4, a0.h, a0.eps, t, sc);
  }
  auto begin = [&](int, f32x16 (&acc)[4][4]) {
#pragma unroll
    for (int p = 0; p < 4; ++p)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[p][q][r] = 0.f;
  };
  const int kw = a0.hkv * a0.d;
  auto pre = [&](int i, uint4* side) {
    int l, tm, tn;
    coords(i, l, tm, tn);
    if (tn * BN + BN <= kw) {
      const int tp = pinned_tid();
      const __amdgpu_buffer_rsrc_t rcs = buffer_rsrc(a0.cs, static_cast<uint32_t>(M) * static_cast<uint32_t>(rb));
      table_round(rcs, rb, 0, tm * BM, M, side, tp);
      table_round(rcs, rb, 1, tm * BM, M, side + SLOT_U4, tp);
    }
  };
  auto end = [&](int i, const f32x16 (&acc)[4][4], uint4* img, float* side_f) {
    int l, tm, tn;
    coords(i, l, tm, tn);
    const int t = pinned_tid(), lane = t & 63, wm = t >> 7;
    const int m0 = tm * BM, n0 = tn * BN, ch = t & 31;
    const bool more = i + 1 < sh.cnt;
    uint4* side = reinterpret_cast<uint4*>(side_f);
    KvArgs a = a0;
    a.ssq = kl.ssq[l];
    a.knorm = kl.knorm[l];
    a.kbuf = kl.kbuf[l];
    a.vbuf = kl.vbuf[l];
    const KvLane L(a, n0, ch);
    // 1: K columns only; 4: V columns only; 5: both
    const int mode = n0 + BN <= kw ? 1 : (n0 >= kw || KMODE != KV_ANY) ? 4 : 5;
    const bool tab = mode == 1;
    // the rows' norm scales, through the image area (free until round 0 is staged)
    float* rsx = reinterpret_cast<float*>(img);
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (k < q4 && t % q4 == q4 - 1) rsx[k * (256 / q4) + t / q4] = sc[k];
    __syncthreads();
    float rs[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) rs[mt] = rsx[wm * 128 + mt * 32 + (lane & 31)];
    __syncthreads();
    const __amdgpu_buffer_rsrc_t rcs = buffer_rsrc(a0.cs, static_cast<uint32_t>(M) * static_cast<uint32_t>(rb));
    float4 pv4[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      __builtin_amdgcn_sched_barrier(0);
      if (r == 3) parts_of(more ? i + 1 : i, pv4, t);   // unconditional (see parts_load)
      float unused;
      switch (r) {
        case 0: stage_round<0, false>(img, acc, [&](int, int, int, float v) { return v * rs[0]; }, unused, t); break;
        case 1: stage_round<1, false>(img, acc, [&](int, int, int, float v) { return v * rs[1]; }, unused, t); break;
        case 2: stage_round<2, false>(img, acc, [&](int, int, int, float v) { return v * rs[2]; }, unused, t); break;
        default: stage_round<3, false>(img, acc, [&](int, int, int, float v) { return v * rs[3]; }, unused, t); break;
      }
      if (tab) __builtin_amdgcn_s_waitcnt(0x0f70);      // vmcnt(0): this round's table rows are in LDS
      __syncthreads();
      if (mode == 1) {
        k_round_tab<KMODE>(a, L, img, side + (r & 1) * SLOT_U4, rb, r, m0, M, t);
      } else if (mode == 4) {
#pragma unroll
        for (int it = 0; it < 8; ++it) {
          const int ir = it * 8 + (t >> 5);
          const int gm = m0 + round_row(ir, r);
          if (gm < M) st_stream16(L.dst0 + (a.slot0 + gm) * a.row_stride, image_chunk(img, ir, ch));
        }
      } else if (KMODE == KV_ANY) {
        for (int it = 0; it < 8; ++it) {
          const int ir = it * 8 + (t >> 5);
          const int gm = m0 + round_row(ir, r);
          kv_chunk_row(a, L, [&](int c) { return image_chunk(img, ir, c); }, ch, gm, gm < M,
                       rope_fetch(a, L, gm, gm < M));
        }
      }
      __syncthreads();
      if (tab && r + 2 < 4) table_round(rcs, rb, r + 2, m0, M, side + (r & 1) * SLOT_U4, t);
    }
    parts_sum(pv4, q4, a0.h, a0.eps, t, sc);
  };
  stream_tiles(sh.cnt, K / BK, ldx, K, ops, begin, pre, end, lds);
}

// Per-layer operands of a batched norm + linear launch.
// Entries of a batched norm + linear: entry l is rows m[l] of x[l] against the n[l] weight rows of w[l]
// (n[l] a multiple of 256) into out[l]; its tiles are the logical tiles [start[l], start[l + 1]).
struct LinLayers {
  const uint16_t* x[MAXL];
  const float* ssq[MAXL];
  const uint16_t* w[MAXL];
  uint16_t* out[MAXL];
  int m[MAXL], n[MAXL];
  int start[MAXL + 1];
};

// rf_norm_linear on persistent tiles for nl entries at once: out_l = bf16(r_row * (x_l W_l^T)), r_row from the
// rows' statistics (parts_load / parts_sum; K a multiple of 1024 up to 4096); one input row stride ldx, one
// output row stride ldo. An entry's tile computes exactly what the per-entry kernel computes for it.
__global__ __launch_bounds__(NTHR) void k_norm_linear_p(LinLayers ll, int nl, int64_t ldx, int64_t ldo, int K,
                                                        float eps) {
  __shared__ uint4 lds[LDS_U4];
  const Share sh = block_share(ll.start[nl]);
  if (sh.cnt == 0) return;
  const int t = threadIdx.x, q4 = K / (4 * SSQ_COLS);
  const float width = static_cast<float>(K);
  auto coords = [&](int i, int& l, int& tm, int& tn) {
    const int u = sh.first + i * sh.stride;
    l = 0;
    while (l + 1 < nl && u >= ll.start[l + 1]) ++l;
    tile_coords(u - ll.start[l], (ll.m[l] + BM - 1) / BM, ll.n[l] / BN, tm, tn);
  };
  auto ops = [&](int i) {
    int l, tm, tn;
    coords(i, l, tm, tn);
    const int m0 = tm * BM;
    return TileOps{buffer_rsrc(ll.x[l] + static_cast<int64_t>(m0) * ldx,
                               static_cast<uint32_t>(min(ll.m[l] - m0, BM) * ldx * 2)),
                   buffer_rsrc(ll.w[l] + static_cast<int64_t>(tn) * BN * K, static_cast<uint32_t>(BN * K * 2))};
  };
  auto parts_of = [&](int i, float4 (&v)[4], int tt) {
    int l, tm, tn;
    coords(i, l, tm, tn);
    parts_load(ll.ssq[l], q4, ll.m[l], tm * BM, tt, v);
  };
  float sc[4];
  {
    float4 v[4];
    parts_of(0, v, t);
    parts_sum(v, q4, width, eps, t, sc);
  }
  auto begin = [&](int, f32x16 (&acc)[4][4]) {
#pragma unroll
    for (int p = 0; p < 4; ++p)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[p][q][r] = 0.f;
  };
  auto end = [&](int i, const f32x16 (&acc)[4][4], uint4* img, float*) {
    int l, tm, tn;
    coords(i, l, tm, tn);
    const int t = pinned_tid(), lane = t & 63, wm = t >> 7;
    const int m0 = tm * BM, n0 = tn * BN, ch = t & 31, M = ll.m[l];
    uint16_t* out = ll.out[l];
    float* rsx = reinterpret_cast<float*>(img);     // the rows' norm scales, through the image area
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (k < q4 && t % q4 == q4 - 1) rsx[k * (256 / q4) + t / q4] = sc[k];
    __syncthreads();
    float rs[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) rs[mt] = rsx[wm * 128 + mt * 32 + (lane & 31)];
    __syncthreads();
    float4 pv4[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      __builtin_amdgcn_sched_barrier(0);
      if (r == 3) parts_of(i + 1 < sh.cnt ? i + 1 : i, pv4, t);   // unconditional (see parts_load)
      float unused;
      switch (r) {
        case 0: stage_round<0, false>(img, acc, [&](int, int, int, float v) { return v * rs[0]; }, unused, t); break;
        case 1: stage_round<1, false>(img, acc, [&](int, int, int, float v) { return v * rs[1]; }, unused, t); break;
        case 2: stage_round<2, false>(img, acc, [&](int, int, int, float v) { return v * rs[2]; }, unused, t); break;
        default: stage_round<3, false>(img, acc, [&](int, int, int, float v) { return v * rs[3]; }, unused, t); break;
      }
      __syncthreads();
#pragma unroll
      for (int it = 0; it < 8; ++it) {
        const int ir = it * 8 + (t >> 5);
        const int gm = m0 + round_row(ir, r);
        if (gm < M) *reinterpret_cast<uint4*>(out + static_cast<int64_t>(gm) * ldo + n0 + ch * 8) = image_chunk(img, ir, ch);
      }
      __syncthreads();
    }
    parts_sum(pv4, q4, width, eps, t, sc);
  };
  stream_tiles(sh.cnt, K / BK, ldx, K, ops, begin, [](int, uint4*) {}, end, lds);
}

int grid_of(int64_t M, int64_t N) { return static_cast<int>(((M + BM - 1) / BM) * (N / BN)); }

// The persistent K / V kernel takes H a multiple of 1024 up to 4096 (its row statistics: 4 .. 16 partials,
// 16 bytes a lane) and a power-of-two rot <= 128 (a RoPE table row fills whole 16-byte lanes of a 1 KiB
// load, and a round's 64 rows fit one 16 KiB slot).
// The persistent norm + linear kernel: H a multiple of 1024 up to 4096 (as persistent_kv_ok).
bool persistent_lin_ok(int64_t H) { return H % 1024 == 0 && H / SSQ_COLS <= 16; }

bool persistent_kv_ok(int64_t H, int rot, int64_t M) {
  return H % 1024 == 0 && H / SSQ_COLS <= 16 && rot <= 128 && (rot & (rot - 1)) == 0 && M * rot * 2 < (1ll << 32);
}

// The persistent K / V kernel for nl layers of M rows; the K epilogue's compile-time mode from the
// configuration in a (d 128 with full rotary: without k_norm, or with Llama-style k_norm; anything else).
void launch_norm_kv_p(const KvLayers& kl, int nl, int64_t ldx, int64_t M, int64_t N, int64_t K, const KvArgs& a,
                      hipStream_t stream) {
  const dim3 grid(persistent_grid(nl * static_cast<int64_t>(grid_of(M, N)))), block(NTHR);
  const bool d128 = a.d == 128 && a.rot == 128;
  if (d128 && !a.knorm)
    hipLaunchKernelGGL(k_norm_kv_p<KV_D128>, grid, block, 0, stream, kl, nl, ldx, static_cast<int>(M),
                       static_cast<int>(N), static_cast<int>(K), a);
  else if (d128 && a.knorm_kind == 0)
    hipLaunchKernelGGL(k_norm_kv_p<KV_D128_KNORM>, grid, block, 0, stream, kl, nl, ldx, static_cast<int>(M),
                       static_cast<int>(N), static_cast<int>(K), a);
  else
    hipLaunchKernelGGL(k_norm_kv_p<KV_ANY>, grid, block, 0, stream, kl, nl, ldx, static_cast<int>(M),
                       static_cast<int>(N), static_cast<int>(K), a);
}

// K splits for an M x N x K product: enough blocks to give every CU one (256), at least 512 of K per
// split, at most 16 splits; 1 when the tiles alone fill the GPU.
int split_count(int64_t M, int64_t N, int64_t K) {
  const int64_t tiles = std::max<int64_t>(grid_of(M, N), 1);
  int64_t s = std::min<int64_t>(std::min<int64_t>(256 / tiles, K / 512), 16);
  return static_cast<int>(std::max<int64_t>(s, 1));
}

// How an M x N x K product runs: rows [0, m_fused) through the fused kernel, rows [m_fused, M) with K split
// `splits` ways (k_gemm_partial + a reduce kernel) when splits > 1. Too few tiles for the GPU: all rows
// split. Otherwise, when whole tile rows fill the waves (N / 256 divides 256) and the last wave is at
// most half full, its tile rows are split, so that wave takes a fraction of a tile's time.
// Products of at most ROWS_MAX rows take k_rows_partial (rt row tiles per row block, rblocks row blocks)
// for every row, split so that about one block runs per CU, then the reduce epilogue.
struct Plan {
  int64_t m_fused;
  int splits;
  int rt = 0;
  int rblocks = 0;
  bool split() const { return splits > 1 || rt > 0; }
};

Plan plan(int64_t M, int64_t N, int64_t K) {
  if (M <= ROWS_MAX && N % RN == 0) {
    const int64_t rb = (M + 159) / 160, per = (M + rb - 1) / rb;
    const int64_t blocks = rb * (N / RN);
    const int64_t s = std::max<int64_t>(1, std::min<int64_t>(std::min<int64_t>(256 / blocks, K / 512), 16));
    return Plan{0, static_cast<int>(s), static_cast<int>((per + 31) / 32), static_cast<int>(rb)};
  }
  const int64_t tiles_n = N / BN, trows = (M + BM - 1) / BM;
  if (trows * tiles_n < 256) {
    const int s = split_count(M, N, K);
    return s > 1 ? Plan{0, s} : Plan{M, 1};
  }
  if (256 % tiles_n == 0) {
    const int64_t rem = trows % (256 / tiles_n);
    if (rem && 2 * rem * tiles_n <= 256) {
      const int64_t s = std::min<int64_t>(std::min<int64_t>(256 / (rem * tiles_n), K / 512), 16);
      if (s > 1) return Plan{(trows - rem) * BM, static_cast<int>(s)};
    }
  }
  return Plan{M, 1};
}

size_t split_bytes(int64_t M, int64_t N, int64_t K) {
  const Plan p = plan(M, N, K);
  return p.split() ? static_cast<size_t>(p.splits) * (M - p.m_fused) * N * 4 : 0;
}

// Workspace of a product over `rows` scattered rows run in chunks of ROWS_MAX rows, each chunk planned on
// its own: the largest of a full chunk's and the last (shorter) chunk's split bytes. A shorter chunk can
// need more than a full one, since fewer row blocks leave room for more K splits.
size_t rows_split_bytes(int64_t rows, int64_t N, int64_t K) {
  size_t b = 0;
  if (rows >= ROWS_MAX) b = split_bytes(ROWS_MAX, N, K);
  if (rows % ROWS_MAX) b = std::max(b, split_bytes(rows % ROWS_MAX, N, K));
  return b;
}

// The plan an entry point follows with this workspace: the split part only if the workspace holds it.
Plan plan_with(int64_t M, int64_t N, int64_t K, const void* ws, size_t ws_bytes) {
  const Plan p = plan(M, N, K);
  if (!p.split() || !ws || ws_bytes < split_bytes(M, N, K)) return Plan{M, 1};
  return p;
}

// The split partials of rows [m0, M) of an M x N x K product into ws.
void launch_partials(const uint16_t* X, int64_t ldx, const uint16_t* W, int64_t ldw, int64_t M, int64_t N, int64_t K,
                     const Plan& p, void* ws, hipStream_t stream) {
  const int64_t rows = M - p.m_fused;
  const int kper = static_cast<int>((K / p.splits + BK - 1) / BK * BK);
  if (p.rt > 0) {
    const dim3 grid(static_cast<unsigned>(N / RN * p.rblocks * p.splits));
    const int m = static_cast<int>(rows), n = static_cast<int>(N), k = static_cast<int>(K);
    float* out = static_cast<float*>(ws);
    switch (p.rt) {
      case 1: hipLaunchKernelGGL(k_rows_partial<1>, grid, dim3(NTHR), 0, stream, X, ldx, W, ldw, m, n, k, kper, p.rblocks, out); break;
      case 2: hipLaunchKernelGGL(k_rows_partial<2>, grid, dim3(NTHR), 0, stream, X, ldx, W, ldw, m, n, k, kper, p.rblocks, out); break;
      case 3: hipLaunchKernelGGL(k_rows_partial<3>, grid, dim3(NTHR), 0, stream, X, ldx, W, ldw, m, n, k, kper, p.rblocks, out); break;
      case 4: hipLaunchKernelGGL(k_rows_partial<4>, grid, dim3(NTHR), 0, stream, X, ldx, W, ldw, m, n, k, kper, p.rblocks, out); break;
      default: hipLaunchKernelGGL(k_rows_partial<5>, grid, dim3(NTHR), 0, stream, X, ldx, W, ldw, m, n, k, kper, p.rblocks, out); break;
    }
    return;
  }
  hipLaunchKernelGGL(k_gemm_partial, dim3(grid_of(rows, N) * p.splits), dim3(NTHR), 0, stream, X + p.m_fused * ldx,
                     ldx, W, ldw, static_cast<int>(rows), static_cast<int>(N), static_cast<int>(K), kper,
                     static_cast<float*>(ws));
}

dim3 reduce_grid(int64_t M, int64_t N) {
  return dim3(static_cast<unsigned>((M + RED_ROWS - 1) / RED_ROWS), static_cast<unsigned>(N / BN));
}

}  // namespace
}  // namespace rf

using namespace rf;

extern "C" int rf_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, size_t* bytes) {
  if (!bytes || M < 0 || N <= 0 || N % BN || K <= 0 || K % BK)
    return fail(RF_EINVAL_ARG, "rf_gemm_workspace_bytes: M %lld, N %lld (multiple of 256), K %lld (multiple of 64)",
                (long long)M, (long long)N, (long long)K);
  *bytes = M ? split_bytes(M, N, K) : 0;
  return RF_OK;
}

extern "C" int rf_rows_workspace_bytes(int64_t rows, int64_t N, int64_t K, size_t* bytes) {
  if (!bytes || rows < 0 || N <= 0 || N % BN || K <= 0 || K % BK)
    return fail(RF_EINVAL_ARG, "rf_rows_workspace_bytes: rows %lld, N %lld (multiple of 256), K %lld (multiple of 64)",
                (long long)rows, (long long)N, (long long)K);
  *bytes = rows_split_bytes(rows, N, K);
  return RF_OK;
}

extern "C" int rf_map_apply(const uint16_t* b, int64_t ldb, const uint16_t* w, const uint16_t* c, uint16_t* x,
                            int64_t ldx, float* ssq, int64_t P, int64_t h_in, int64_t h_out, void* workspace,
                            size_t ws_bytes, hipStream_t stream) {
  if (!b || !w || !x || !ssq) return fail(RF_EINVAL_ARG, "rf_map_apply: null pointer");
  if (P < 0 || P > (1ll << 30)) return fail(RF_EINVAL_SHAPE, "rf_map_apply: P = %lld out of range", (long long)P);
  if (h_in <= 0 || h_in % BK || h_out <= 0 || h_out % BN)
    return fail(RF_EINVAL_SHAPE, "rf_map_apply: h_in %lld must be a multiple of 64 and h_out %lld of 256",
                (long long)h_in, (long long)h_out);
  if (ldb < h_in || ldx < h_out || ldb % 8 || ldx % 8 || ldb > (1 << 21) || h_in > (1 << 21))
    return fail(RF_EINVAL_SHAPE, "rf_map_apply: row strides ldb %lld / ldx %lld", (long long)ldb, (long long)ldx);
  if (!aligned16(b) || !aligned16(w) || !aligned16(x) || (c && !aligned16(c)))
    return fail(RF_EINVAL_SHAPE, "rf_map_apply: pointers must be 16-byte aligned");
  if (workspace && !aligned16(workspace)) return fail(RF_EINVAL_SHAPE, "rf_map_apply: workspace alignment");
  if (P == 0) return RF_OK;
  const Plan pl = plan_with(P, h_out, h_in, workspace, ws_bytes);
  const int64_t mf = pl.m_fused, rows = P - mf;
  if (mf > 0 && h_in / BK >= 2) {
    MapLayers ml{};
    ml.w[0] = w;
    ml.c[0] = c;
    ml.x[0] = x;
    ml.ssq[0] = ssq;
    hipLaunchKernelGGL(k_map_apply_p<false>, dim3(persistent_grid(grid_of(mf, h_out))), dim3(NTHR), 0, stream, b, ldb,
                       ml, 1, ldx, static_cast<int>(mf), static_cast<int>(h_out), static_cast<int>(h_in),
                       static_cast<const uint16_t*>(nullptr), static_cast<int64_t>(0));
  } else if (mf > 0) {
    hipLaunchKernelGGL(k_map_apply, dim3(grid_of(mf, h_out)), dim3(NTHR), 0, stream, b, ldb, w, c, x, ldx, ssq,
                       static_cast<int>(mf), static_cast<int>(h_out), static_cast<int>(h_in));
  }
  if (pl.split()) {
    launch_partials(b, ldb, w, h_in, P, h_out, h_in, pl, workspace, stream);
    hipLaunchKernelGGL(k_map_apply_reduce, reduce_grid(rows, h_out), dim3(256), 0, stream,
                       static_cast<const float*>(workspace), pl.splits, c, x + mf * ldx, ldx,
                       ssq + mf * (h_out / SSQ_COLS), static_cast<int>(rows), static_cast<int>(h_out));
  }
  return check_launch("rf_map_apply");
}

extern "C" int rf_map_apply_residual(const uint16_t* x, int64_t ldx, const uint16_t* w, const uint16_t* res,
                                     int64_t ldr, uint16_t* out, int64_t ldo, float* ssq, int64_t M, int64_t K,
                                     int64_t N, void* workspace, size_t ws_bytes, hipStream_t stream) {
  const char* fn = "rf_map_apply_residual";
  if (!x || !w || !res || !out || !ssq) return fail(RF_EINVAL_ARG, "%s: null pointer", fn);
  if (M < 0 || M > (1ll << 30)) return fail(RF_EINVAL_SHAPE, "%s: M = %lld out of range", fn, (long long)M);
  if (K <= 0 || K % BK || N <= 0 || N % BN)
    return fail(RF_EINVAL_SHAPE, "%s: K %lld must be a multiple of 64 and N %lld of 256", fn, (long long)K, (long long)N);
  if (ldx < K || ldo < N || ldr < N || ldx % 8 || ldo % 8 || ldr % 8 || ldx > (1 << 21) || K > (1 << 21))
    return fail(RF_EINVAL_SHAPE, "%s: row strides ldx %lld / ldr %lld / ldo %lld", fn, (long long)ldx, (long long)ldr,
                (long long)ldo);
  if (!aligned16(x) || !aligned16(w) || !aligned16(res) || !aligned16(out) || (workspace && !aligned16(workspace)))
    return fail(RF_EINVAL_SHAPE, "%s: pointers must be 16-byte aligned", fn);
  if (M == 0) return RF_OK;
  const Plan pl = plan_with(M, N, K, workspace, ws_bytes);
  if (pl.split() && pl.m_fused == 0) {             // every row through the split sums: the residual in the reduce
    launch_partials(x, ldx, w, K, M, N, K, pl, workspace, stream);
    hipLaunchKernelGGL(k_map_apply_reduce, reduce_grid(M, N), dim3(256), 0, stream,
                       static_cast<const float*>(workspace), pl.splits, nullptr, out, ldo, ssq, static_cast<int>(M),
                       static_cast<int>(N), res, ldr);
    return check_launch(fn);
  }
  const int64_t mf = pl.m_fused, rows = M - mf;
  if (mf == 0 || K / BK < 2) {                     // no persistent tiles (K = 64): the product, then the residual
    const int rc = rf_map_apply(x, ldx, w, nullptr, out, ldo, ssq, M, K, N, workspace, ws_bytes, stream);
    if (rc != RF_OK) return rc;
    return rf_residual_add(res, ldr, out, ldo, out, ldo, ssq, M, N, stream);
  }
  // the residual in the tiles' epilogue for rows [0, mf), in the split sums' epilogue for the rest
  MapLayers ml{};
  ml.w[0] = w;
  ml.x[0] = out;
  ml.ssq[0] = ssq;
  hipLaunchKernelGGL(k_map_apply_p<true>, dim3(persistent_grid(grid_of(mf, N))), dim3(NTHR), 0, stream, x, ldx, ml, 1,
                     ldo, static_cast<int>(mf), static_cast<int>(N), static_cast<int>(K), res, ldr);
  if (pl.split()) {
    launch_partials(x, ldx, w, K, M, N, K, pl, workspace, stream);
    hipLaunchKernelGGL(k_map_apply_reduce, reduce_grid(rows, N), dim3(256), 0, stream,
                       static_cast<const float*>(workspace), pl.splits, nullptr, out + mf * ldo, ldo,
                       ssq + mf * (N / SSQ_COLS), static_cast<int>(rows), static_cast<int>(N), res + mf * ldr, ldr);
  }
  return check_launch(fn);
}

extern "C" int rf_norm_linear_swiglu(const uint16_t* x, int64_t ldx, const float* ssq, int64_t P, int64_t H, float eps,
                                     const uint16_t* w, int64_t I, uint16_t* act, int64_t lda, uint16_t* gu,
                                     int64_t ldg, void* workspace, size_t ws_bytes, hipStream_t stream) {
  const char* fn = "rf_norm_linear_swiglu";
  if (!x || !ssq || !w || !act) return fail(RF_EINVAL_ARG, "%s: null pointer", fn);
  if (P < 0 || P > (1ll << 30) || H <= 0 || H % SSQ_COLS || I <= 0 || I % BN)
    return fail(RF_EINVAL_SHAPE, "%s: P %lld, H %lld (multiple of 256), I %lld (multiple of 256)", fn, (long long)P,
                (long long)H, (long long)I);
  if (ldx < H || ldx % 8 || ldx > (1 << 21) || lda < I || lda % 8)
    return fail(RF_EINVAL_SHAPE, "%s: strides ldx %lld, lda %lld", fn, (long long)ldx, (long long)lda);
  if (!aligned16(x) || !aligned16(w) || !aligned16(act) || (workspace && !aligned16(workspace)))
    return fail(RF_EINVAL_SHAPE, "%s: pointers must be 16-byte aligned", fn);
  if (!(eps >= 0.f)) return fail(RF_EINVAL_ARG, "%s: eps %g", fn, static_cast<double>(eps));
  if (P == 0) return RF_OK;
  const int64_t N = 2 * I;
  const Plan pl = plan_with(P, N, H, workspace, ws_bytes);
  if (pl.split() && pl.m_fused == 0) {             // every row through the split sums: SwiGLU in the reduce
    launch_partials(x, ldx, w, H, P, N, H, pl, workspace, stream);
    hipLaunchKernelGGL(k_swiglu_reduce, reduce_grid(P, I), dim3(256), 0, stream, static_cast<const float*>(workspace),
                       pl.splits, ssq, static_cast<int>(H), eps, act, lda, static_cast<int>(P), static_cast<int>(N),
                       static_cast<int>(I));
    return check_launch(fn);
  }
  if (!gu || ldg < N || ldg % 8 || !aligned16(gu))
    return fail(RF_EINVAL_ARG, "%s: this shape runs unsplit and needs the [P, 2 I] gate / up buffer gu", fn);
  const int rc = rf_norm_linear(x, ldx, ssq, P, H, eps, w, N, gu, ldg, workspace, ws_bytes, stream);
  if (rc != RF_OK) return rc;
  return rf_silu_mul(gu, ldg, P, I, act, lda, stream);
}

extern "C" int rf_norm_kv_write(const uint16_t* x, int64_t ldx, const float* ssq, int64_t P, int64_t H, float eps,
                                const uint16_t* wkv, int hkv, int d, const uint16_t* knorm, int knorm_kind,
                                const uint16_t* cs, int rot, uint16_t* kbuf, uint16_t* vbuf,
                                int64_t head_stride, int64_t row_stride, int64_t slot_begin, int64_t cap,
                                void* workspace, size_t ws_bytes, hipStream_t stream) {
  if (!x || !ssq || !wkv || !cs || !kbuf || !vbuf) return fail(RF_EINVAL_ARG, "rf_norm_kv_write: null pointer");
  if (P < 0 || P > (1ll << 30)) return fail(RF_EINVAL_SHAPE, "rf_norm_kv_write: P = %lld out of range", (long long)P);
  if (H <= 0 || H % BK || H % SSQ_COLS)
    return fail(RF_EINVAL_SHAPE, "rf_norm_kv_write: H = %lld must be a multiple of 256", (long long)H);
  if (d <= 0 || d % 8 || 256 % d || hkv <= 0 || (2ll * hkv * d) % BN)
    return fail(RF_EUNSUPPORTED, "rf_norm_kv_write: head_dim %d / kv heads %d (need 256 %% d == 0, d %% 8 == 0, "
                "2 hkv d %% 256 == 0)", d, hkv);
  if (rot <= 0 || rot > d || rot % 2 || ((rot / 2) % 8 && rot / 2 != 4))
    return fail(RF_EUNSUPPORTED, "rf_norm_kv_write: rotary dims %d of head_dim %d", rot, d);
  if (knorm && knorm_kind != 0 && knorm_kind != 1)
    return fail(RF_EINVAL_ARG, "rf_norm_kv_write: knorm_kind %d", knorm_kind);
  if (ldx < H || ldx % 8 || ldx > (1 << 21) || head_stride % 8 || row_stride % 8 || row_stride < d)
    return fail(RF_EINVAL_SHAPE, "rf_norm_kv_write: strides (ldx %lld, head %lld, row %lld)", (long long)ldx,
                (long long)head_stride, (long long)row_stride);
  if (slot_begin < 0 || slot_begin + P > cap)
    return fail(RF_EINVAL_SHAPE, "rf_norm_kv_write: rows [%lld, %lld) exceed cache capacity %lld",
                (long long)slot_begin, (long long)(slot_begin + P), (long long)cap);
  if (!aligned16(x) || !aligned16(wkv) || !aligned16(kbuf) || !aligned16(vbuf) || !aligned16(cs) ||
      (knorm && !aligned16(knorm)))
    return fail(RF_EINVAL_SHAPE, "rf_norm_kv_write: pointers must be 16-byte aligned");
  if (!(eps >= 0.f)) return fail(RF_EINVAL_ARG, "rf_norm_kv_write: eps %g", static_cast<double>(eps));
  if (P == 0) return RF_OK;
  KvArgs a{ssq, static_cast<int>(H / SSQ_COLS), static_cast<float>(H), eps, hkv, d, knorm, knorm_kind, cs, rot,
           kbuf, vbuf, head_stride, row_stride, slot_begin, nullptr};
  const int64_t N = 2ll * hkv * d;
  if (workspace && !aligned16(workspace)) return fail(RF_EINVAL_SHAPE, "rf_norm_kv_write: workspace alignment");
  const Plan pl = plan_with(P, N, H, workspace, ws_bytes);
  const int64_t mf = pl.m_fused, rows = P - mf;
  if (mf > 0 && persistent_kv_ok(H, rot, mf)) {
    KvLayers kl{};
    kl.x[0] = x;
    kl.ssq[0] = ssq;
    kl.wkv[0] = wkv;
    kl.knorm[0] = knorm;
    kl.kbuf[0] = kbuf;
    kl.vbuf[0] = vbuf;
    launch_norm_kv_p(kl, 1, ldx, mf, N, H, a, stream);
  } else if (mf > 0) {
    hipLaunchKernelGGL(k_norm_kv, dim3(grid_of(mf, N)), dim3(NTHR), 0, stream, x, ldx, wkv, static_cast<int>(mf),
                       static_cast<int>(N), static_cast<int>(H), a);
  }
  if (pl.split()) {
    launch_partials(x, ldx, wkv, H, P, N, H, pl, workspace, stream);
    KvArgs ar = a;                                  // the split rows: statistics, slots and table rows from mf
    ar.ssq += mf * ar.nparts;
    ar.slot0 += mf;
    ar.cs += mf * rot;
    hipLaunchKernelGGL(k_norm_kv_reduce, reduce_grid(rows, N), dim3(256), 0, stream,
                       static_cast<const float*>(workspace), pl.splits, static_cast<int>(rows), static_cast<int>(N), ar);
  }
  return check_launch("rf_norm_kv_write");
}

extern "C" int rf_norm_kv_rows(const uint16_t* x, int64_t ldx, const float* ssq, int64_t rows, int64_t H,
                               float eps, const uint16_t* wkv, int hkv, int d, const uint16_t* knorm, int knorm_kind,
                               const uint16_t* cs, int rot, const int64_t* pos, int64_t pos_limit, uint16_t* kbuf,
                               uint16_t* vbuf, int64_t head_stride, int64_t row_stride, void* workspace,
                               size_t ws_bytes, hipStream_t stream) {
  const char* fn = "rf_norm_kv_rows";
  if (!x || !ssq || !wkv || !cs || !pos || !kbuf || !vbuf || !workspace)
    return fail(RF_EINVAL_ARG, "%s: null pointer", fn);
  if (rows < 0 || rows > (1ll << 30)) return fail(RF_EINVAL_SHAPE, "%s: rows = %lld out of range", fn, (long long)rows);
  if (H <= 0 || H % BK || H % SSQ_COLS)
    return fail(RF_EINVAL_SHAPE, "%s: H = %lld must be a multiple of 256", fn, (long long)H);
  if (d <= 0 || d % 8 || 256 % d || hkv <= 0 || (2ll * hkv * d) % BN)
    return fail(RF_EUNSUPPORTED, "%s: head_dim %d / kv heads %d (need 256 %% d == 0, d %% 8 == 0, 2 hkv d %% 256 == 0)",
                fn, d, hkv);
  if (rot <= 0 || rot > d || rot % 2 || ((rot / 2) % 8 && rot / 2 != 4))
    return fail(RF_EUNSUPPORTED, "%s: rotary dims %d of head_dim %d", fn, rot, d);
  if (knorm && knorm_kind != 0 && knorm_kind != 1) return fail(RF_EINVAL_ARG, "%s: knorm_kind %d", fn, knorm_kind);
  if (ldx < H || ldx % 8 || ldx > (1 << 21) || head_stride % 8 || row_stride % 8 || row_stride < d)
    return fail(RF_EINVAL_SHAPE, "%s: strides (ldx %lld, head %lld, row %lld)", fn, (long long)ldx,
                (long long)head_stride, (long long)row_stride);
  if (!aligned16(x) || !aligned16(wkv) || !aligned16(kbuf) || !aligned16(vbuf) || !aligned16(cs) ||
      !aligned16(workspace) || (knorm && !aligned16(knorm)))
    return fail(RF_EINVAL_SHAPE, "%s: pointers must be 16-byte aligned", fn);
  if (!(eps >= 0.f)) return fail(RF_EINVAL_ARG, "%s: eps %g", fn, static_cast<double>(eps));
  const int64_t N = 2ll * hkv * d;
  // chunks of at most ROWS_MAX rows, each through the few-rows partials and the reduce epilogue (the only
  // epilogue that writes to per-row slots)
  if (pos_limit <= 0) return fail(RF_EINVAL_ARG, "%s: pos_limit %lld", fn, (long long)pos_limit);
  const size_t need = rows_split_bytes(rows, N, H);
  if (ws_bytes < need)
    return fail(RF_EINVAL_ARG, "%s: workspace %zu bytes, needs %zu (rf_rows_workspace_bytes of %lld x %lld x %lld)",
                fn, ws_bytes, need, (long long)rows, (long long)N, (long long)H);
  for (int64_t r0 = 0; r0 < rows; r0 += ROWS_MAX) {
    const int64_t m = std::min<int64_t>(ROWS_MAX, rows - r0);
    const Plan pl = plan(m, N, H);
    KvArgs a{ssq + r0 * (H / SSQ_COLS), static_cast<int>(H / SSQ_COLS), static_cast<float>(H), eps, hkv, d, knorm,
             knorm_kind, cs, rot, kbuf, vbuf, head_stride, row_stride, 0, pos + r0};
    a.slot = pos + r0;
    a.pos_lim = pos_limit;
    launch_partials(x + r0 * ldx, ldx, wkv, H, m, N, H, pl, workspace, stream);
    hipLaunchKernelGGL(k_norm_kv_reduce, reduce_grid(m, N), dim3(256), 0, stream, static_cast<const float*>(workspace),
                       pl.splits, static_cast<int>(m), static_cast<int>(N), a);
  }
  return check_launch(fn);
}

extern "C" int rf_norm_qkv_rows(const uint16_t* x, int64_t ldx, const float* ssq, int64_t rows, int64_t H,
                                float eps, const uint16_t* wqkv, int hq, int hkv, int d, const uint16_t* qnorm,
                                const uint16_t* knorm, int norm_kind, const uint16_t* cs, int rot, const int64_t* pos,
                                int64_t pos_limit, uint16_t* q, int64_t ldq, uint16_t* kbuf, uint16_t* vbuf,
                                int64_t head_stride, int64_t row_stride, void* workspace, size_t ws_bytes,
                                hipStream_t stream) {
  const char* fn = "rf_norm_qkv_rows";
  if (!x || !ssq || !wqkv || !cs || !pos || !q || !kbuf || !vbuf || !workspace)
    return fail(RF_EINVAL_ARG, "%s: null pointer", fn);
  if (rows < 0 || rows > (1ll << 30)) return fail(RF_EINVAL_SHAPE, "%s: rows = %lld out of range", fn, (long long)rows);
  if (H <= 0 || H % BK || H % SSQ_COLS)
    return fail(RF_EINVAL_SHAPE, "%s: H = %lld must be a multiple of 256", fn, (long long)H);
  if (d <= 0 || d % 8 || 256 % d || hq <= 0 || hkv <= 0 || (static_cast<int64_t>(hq) * d) % BN ||
      (2ll * hkv * d) % BN)
    return fail(RF_EUNSUPPORTED, "%s: head_dim %d, %d query / %d kv heads (need 256 %% d == 0, d %% 8 == 0, hq d and "
                "2 hkv d multiples of 256)", fn, d, hq, hkv);
  if (rot <= 0 || rot > d || rot % 2 || ((rot / 2) % 8 && rot / 2 != 4))
    return fail(RF_EUNSUPPORTED, "%s: rotary dims %d of head_dim %d", fn, rot, d);
  if ((qnorm || knorm) && norm_kind != 0 && norm_kind != 1) return fail(RF_EINVAL_ARG, "%s: norm_kind %d", fn, norm_kind);
  if (ldx < H || ldx % 8 || ldx > (1 << 21) || ldq < static_cast<int64_t>(hq) * d || ldq % 8 || head_stride % 8 ||
      row_stride % 8 || row_stride < d)
    return fail(RF_EINVAL_SHAPE, "%s: strides (ldx %lld, ldq %lld, head %lld, row %lld)", fn, (long long)ldx,
                (long long)ldq, (long long)head_stride, (long long)row_stride);
  if (!aligned16(x) || !aligned16(wqkv) || !aligned16(q) || !aligned16(kbuf) || !aligned16(vbuf) || !aligned16(cs) ||
      !aligned16(workspace) || (qnorm && !aligned16(qnorm)) || (knorm && !aligned16(knorm)))
    return fail(RF_EINVAL_SHAPE, "%s: pointers must be 16-byte aligned", fn);
  if (!(eps >= 0.f)) return fail(RF_EINVAL_ARG, "%s: eps %g", fn, static_cast<double>(eps));
  const int64_t NQ = static_cast<int64_t>(hq) * d, NKV = 2ll * hkv * d, N = NQ + NKV;
  if (pos_limit <= 0) return fail(RF_EINVAL_ARG, "%s: pos_limit %lld", fn, (long long)pos_limit);
  const size_t need = rows_split_bytes(rows, N, H);
  if (ws_bytes < need)
    return fail(RF_EINVAL_ARG, "%s: workspace %zu bytes, needs %zu (rf_rows_workspace_bytes of %lld x %lld x %lld)",
                fn, ws_bytes, need, (long long)rows, (long long)N, (long long)H);
  const float* part = static_cast<const float*>(workspace);
  for (int64_t r0 = 0; r0 < rows; r0 += ROWS_MAX) {
    const int64_t m = std::min<int64_t>(ROWS_MAX, rows - r0);
    const Plan pl = plan(m, N, H);
    launch_partials(x + r0 * ldx, ldx, wqkv, H, m, N, H, pl, workspace, stream);
    const int nparts = static_cast<int>(H / SSQ_COLS);
    const float* s0 = ssq + r0 * nparts;
    // the query columns [0, NQ): every column a "K" column of hq heads, row j to q row r0 + j
    KvArgs aq{s0, nparts, static_cast<float>(H), eps, hq, d, qnorm, norm_kind, cs, rot, q + r0 * ldq,
              q + r0 * ldq, static_cast<int64_t>(d), ldq, 0, pos + r0};
    aq.pos_lim = pos_limit;
    const dim3 gq = reduce_grid(m, NQ), gkv = reduce_grid(m, NKV);
    hipLaunchKernelGGL(k_norm_kv_reduce, gq, dim3(256), 0, stream, part, pl.splits, static_cast<int>(m),
                       static_cast<int>(N), aq);
    // the K / V columns [NQ, N): the partial planes' rows keep their stride N, the cache slot is the position
    KvArgs akv{s0, nparts, static_cast<float>(H), eps, hkv, d, knorm, norm_kind, cs, rot, kbuf, vbuf, head_stride,
               row_stride, 0, pos + r0};
    akv.slot = pos + r0;
    akv.pos_lim = pos_limit;
    hipLaunchKernelGGL(k_norm_kv_reduce, gkv, dim3(256), 0, stream, part + NQ, pl.splits, static_cast<int>(m),
                       static_cast<int>(N), akv);
  }
  return check_launch(fn);
}

extern "C" int rf_norm_q(const uint16_t* x, int64_t ldx, const float* ssq, int64_t rows, int64_t H, float eps,
                         const uint16_t* wq, int hq, int d, const uint16_t* qnorm, int qnorm_kind, const uint16_t* cs,
                         int rot, const int64_t* pos, uint16_t* q, int64_t ldq, void* workspace, size_t ws_bytes,
                         hipStream_t stream) {
  if (!x || !ssq || !wq || !cs || !pos || !q) return fail(RF_EINVAL_ARG, "rf_norm_q: null pointer");
  if (rows < 0 || rows > (1ll << 30)) return fail(RF_EINVAL_SHAPE, "rf_norm_q: rows = %lld out of range", (long long)rows);
  if (H <= 0 || H % BK || H % SSQ_COLS) return fail(RF_EINVAL_SHAPE, "rf_norm_q: H = %lld must be a multiple of 256",
                                                   (long long)H);
  if (d <= 0 || d % 8 || 256 % d || hq <= 0 || (static_cast<int64_t>(hq) * d) % BN)
    return fail(RF_EUNSUPPORTED, "rf_norm_q: head_dim %d / heads %d (need 256 %% d == 0, d %% 8 == 0, hq d %% 256 == 0)",
                d, hq);
  if (rot <= 0 || rot > d || rot % 2 || ((rot / 2) % 8 && rot / 2 != 4))
    return fail(RF_EUNSUPPORTED, "rf_norm_q: rotary dims %d of head_dim %d", rot, d);
  if (qnorm && qnorm_kind != 0 && qnorm_kind != 1) return fail(RF_EINVAL_ARG, "rf_norm_q: qnorm_kind %d", qnorm_kind);
  if (ldx < H || ldx % 8 || ldx > (1 << 21) || ldq < static_cast<int64_t>(hq) * d || ldq % 8)
    return fail(RF_EINVAL_SHAPE, "rf_norm_q: strides (ldx %lld, ldq %lld)", (long long)ldx, (long long)ldq);
  if (!aligned16(x) || !aligned16(wq) || !aligned16(q) || !aligned16(cs) || (qnorm && !aligned16(qnorm)))
    return fail(RF_EINVAL_SHAPE, "rf_norm_q: pointers must be 16-byte aligned");
  if (!(eps >= 0.f)) return fail(RF_EINVAL_ARG, "rf_norm_q: eps %g", static_cast<double>(eps));
  if (rows == 0) return RF_OK;
  // every output column is a "K" column: hkv = hq heads, row j at q + j ldq, head h at + h d
  KvArgs a{ssq, static_cast<int>(H / SSQ_COLS), static_cast<float>(H), eps, hq, d, qnorm, qnorm_kind, cs, rot,
           q, q, static_cast<int64_t>(d), ldq, 0, pos};
  const int64_t N = static_cast<int64_t>(hq) * d;
  if (workspace && !aligned16(workspace)) return fail(RF_EINVAL_SHAPE, "rf_norm_q: workspace alignment");
  const Plan pl = plan_with(rows, N, H, workspace, ws_bytes);
  const int64_t mf = pl.m_fused, rs = rows - mf;
  if (mf > 0)
    hipLaunchKernelGGL(k_norm_kv, dim3(grid_of(mf, N)), dim3(NTHR), 0, stream, x, ldx, wq, static_cast<int>(mf),
                       static_cast<int>(N), static_cast<int>(H), a);
  if (pl.split()) {
    launch_partials(x, ldx, wq, H, rows, N, H, pl, workspace, stream);
    KvArgs ar = a;                                  // the split rows: statistics, outputs and positions from mf
    ar.ssq += mf * ar.nparts;
    ar.slot0 += mf;
    ar.pos += mf;
    hipLaunchKernelGGL(k_norm_kv_reduce, reduce_grid(rs, N), dim3(256), 0, stream,
                       static_cast<const float*>(workspace), pl.splits, static_cast<int>(rs), static_cast<int>(N), ar);
  }
  return check_launch("rf_norm_q");
}

extern "C" int rf_mfma_ceiling(int blocks, int iters, float* out, hipStream_t stream) {
  if (!out || blocks <= 0 || blocks > (1 << 20) || iters <= 0)
    return fail(RF_EINVAL_ARG, "rf_mfma_ceiling: blocks %d, iters %d", blocks, iters);
  hipLaunchKernelGGL(k_mfma_ceiling, dim3(blocks), dim3(256), 0, stream, iters, out);
  return check_launch("rf_mfma_ceiling");
}

// The run-split schedule of a Gram launch (GramPlan). Every tile: used when the tiles take more than one
// round of CUs but at most two, and their split-off runs fit in two rounds; ptiles = 0 otherwise. Block-upper
// tiles (the symmetric X^T X, at most one round of them): all of them split into their runs, which spreads
// the half-size product over every CU; past one round, as for every tile.
struct GramShape {
  int64_t tiles, runs, ptiles;
};
static GramShape gram_shape(int64_t M, int64_t N, int64_t K, int64_t fold_rows, bool upper) {
  const int64_t fold = (fold_rows == 0 || fold_rows > K) ? K : fold_rows;
  const int64_t tm = (M + BM - 1) / BM, tn = N / BN;
  GramShape g{upper ? tm * tn - tm * (tm - 1) / 2 : tm * tn, (K + fold - 1) / fold, 0};
  const int64_t ncu = 256;
  if (upper && g.tiles <= ncu && g.runs >= 2)
    g.ptiles = g.tiles;
  else if (g.tiles > ncu && g.tiles < 2 * ncu && g.runs >= 2 && (g.tiles - ncu) * g.runs <= 2 * ncu)
    g.ptiles = g.tiles - ncu;
  return g;
}

static int gram_workspace(const char* who, int64_t M, int64_t N, int64_t K, int64_t fold_rows, bool upper,
                          size_t* bytes) {
  if (!bytes || M < 0 || M > (1 << 30) || N <= 0 || N % BN || K <= 0 || K % 64 || fold_rows < 0 || fold_rows % 64 ||
      (upper && M > N))
    return fail(RF_EINVAL_ARG, "%s: M %lld, N %lld (multiple of 256%s), K %lld, fold_rows %lld", who, (long long)M,
                (long long)N, upper ? ", at least M" : "", (long long)K, (long long)fold_rows);
  const GramShape g = gram_shape(M, N, K, fold_rows, upper);
  *bytes = static_cast<size_t>(g.ptiles * g.runs) * BM * BN * sizeof(float);
  return RF_OK;
}

static int gram_launch(const char* who, const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb, int64_t M,
                       int64_t N, int64_t K, int64_t fold_rows, double* c, int64_t ldc, void* workspace,
                       size_t workspace_bytes, bool upper, hipStream_t stream) {
  if (!a || !b || !c) return fail(RF_EINVAL_ARG, "%s: null pointer", who);
  if (M < 0 || M > (1 << 30) || N <= 0 || N % BN || K <= 0 || K % 64 || (upper && M > N))
    return fail(RF_EINVAL_SHAPE, "%s: M %lld, N %lld (multiple of 256%s), K %lld (multiple of 64)", who,
                (long long)M, (long long)N, upper ? ", at least M" : "", (long long)K);
  if (lda < K || ldb < K || lda % 8 || ldb % 8 || lda > (1 << 21) || ldb > (1 << 21) || ldc < N || ldc % 2)
    return fail(RF_EINVAL_SHAPE, "%s: strides lda %lld, ldb %lld, ldc %lld", who, (long long)lda, (long long)ldb,
                (long long)ldc);
  if (!aligned16(a) || !aligned16(b) || !aligned16(c))
    return fail(RF_EINVAL_SHAPE, "%s: pointers must be 16-byte aligned", who);
  if (fold_rows < 0 || fold_rows % 64)
    return fail(RF_EINVAL_ARG, "%s: fold_rows %lld (0 or a multiple of 64)", who, (long long)fold_rows);
  if (M == 0) return RF_OK;
  const int64_t fold = (fold_rows == 0 || fold_rows > K) ? K : fold_rows;
  const GramShape g = gram_shape(M, N, K, fold_rows, upper);
  const size_t need = static_cast<size_t>(g.ptiles * g.runs) * BM * BN * sizeof(float);
  GramPlan pl{0, 0, 1, nullptr, upper ? 1 : 0};
  if (g.ptiles > 0 && workspace && workspace_bytes >= need) {     // else every tile whole (same bits)
    if (!aligned16(workspace)) return fail(RF_EINVAL_ARG, "%s: workspace must be 16-byte aligned", who);
    pl = GramPlan{static_cast<int>((g.ptiles * g.runs + 7) / 8 * 8), static_cast<int>(g.ptiles),
                  static_cast<int>(g.runs), static_cast<float*>(workspace), upper ? 1 : 0};
  }
  const int grid = static_cast<int>(g.tiles - pl.ptiles) + pl.pieces;
  hipLaunchKernelGGL(k_gram, dim3(grid), dim3(NTHR), 0, stream, a, lda, b, ldb, static_cast<int>(M),
                     static_cast<int>(N), static_cast<int>(K), static_cast<int>(fold), c, ldc, pl);
  if (pl.ptiles > 0) {
    const int rc = check_launch(who);
    if (rc != RF_OK) return rc;
    hipLaunchKernelGGL(k_gram_fold, dim3(pl.ptiles * 64), dim3(256), 0, stream, pl.part, pl.ptiles, pl.runs,
                       static_cast<int>(g.tiles - pl.ptiles), static_cast<int>(M), static_cast<int>(N), c, ldc,
                       pl.upper);
  }
  return check_launch(who);
}

extern "C" int rf_gram_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t fold_rows, size_t* bytes) {
  return gram_workspace("rf_gram_workspace_bytes", M, N, K, fold_rows, false, bytes);
}

extern "C" int rf_gram_accumulate(const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb, int64_t M,
                                  int64_t N, int64_t K, int64_t fold_rows, double* c, int64_t ldc, void* workspace,
                                  size_t workspace_bytes, hipStream_t stream) {
  return gram_launch("rf_gram_accumulate", a, lda, b, ldb, M, N, K, fold_rows, c, ldc, workspace, workspace_bytes,
                     false, stream);
}

extern "C" int rf_gram_upper_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t fold_rows, size_t* bytes) {
  return gram_workspace("rf_gram_upper_workspace_bytes", M, N, K, fold_rows, true, bytes);
}

extern "C" int rf_gram_accumulate_upper(const uint16_t* a, int64_t lda, int64_t M, int64_t N, int64_t K,
                                        int64_t fold_rows, double* c, int64_t ldc, void* workspace,
                                        size_t workspace_bytes, hipStream_t stream) {
  return gram_launch("rf_gram_accumulate_upper", a, lda, a, lda, M, N, K, fold_rows, c, ldc, workspace,
                     workspace_bytes, true, stream);
}

extern "C" int rf_norm_linear(const uint16_t* x, int64_t ldx, const float* ssq, int64_t P, int64_t H, float eps,
                              const uint16_t* w, int64_t N, uint16_t* out, int64_t ldo, void* workspace,
                              size_t ws_bytes, hipStream_t stream) {
  if (!x || !ssq || !w || !out) return fail(RF_EINVAL_ARG, "rf_norm_linear: null pointer");
  if (P < 0 || P > (1ll << 30) || H <= 0 || H % SSQ_COLS || N <= 0 || N % BN)
    return fail(RF_EINVAL_SHAPE, "rf_norm_linear: P %lld, H %lld (multiple of 256), N %lld (multiple of 256)",
                (long long)P, (long long)H, (long long)N);
  if (ldx < H || ldx % 8 || ldx > (1 << 21) || ldo < N || ldo % 8)
    return fail(RF_EINVAL_SHAPE, "rf_norm_linear: strides ldx %lld, ldo %lld", (long long)ldx, (long long)ldo);
  if (!aligned16(x) || !aligned16(w) || !aligned16(out)) return fail(RF_EINVAL_SHAPE, "rf_norm_linear: alignment");
  if (!(eps >= 0.f)) return fail(RF_EINVAL_ARG, "rf_norm_linear: eps");
  if (workspace && !aligned16(workspace)) return fail(RF_EINVAL_SHAPE, "rf_norm_linear: workspace alignment");
  if (P == 0) return RF_OK;
  const Plan pl = plan_with(P, N, H, workspace, ws_bytes);
  const int64_t mf = pl.m_fused, rows = P - mf;
  if (mf > 0 && persistent_lin_ok(H)) {
    LinLayers ll{};
    ll.x[0] = x;
    ll.ssq[0] = ssq;
    ll.w[0] = w;
    ll.out[0] = out;
    ll.m[0] = static_cast<int>(mf);
    ll.n[0] = static_cast<int>(N);
    ll.start[0] = 0;
    ll.start[1] = grid_of(mf, N);
    hipLaunchKernelGGL(k_norm_linear_p, dim3(persistent_grid(grid_of(mf, N))), dim3(NTHR), 0, stream, ll, 1, ldx, ldo,
                       static_cast<int>(H), eps);
  } else if (mf > 0) {
    hipLaunchKernelGGL(k_norm_linear, dim3(grid_of(mf, N)), dim3(NTHR), 0, stream, x, ldx, w, static_cast<int>(mf),
                       static_cast<int>(N), static_cast<int>(H), ssq, eps, out, ldo);
  }
  if (pl.split()) {
    launch_partials(x, ldx, w, H, P, N, H, pl, workspace, stream);
    hipLaunchKernelGGL(k_norm_linear_reduce, reduce_grid(rows, N), dim3(256), 0, stream,
                       static_cast<const float*>(workspace), pl.splits, ssq + mf * (H / SSQ_COLS), static_cast<int>(H),
                       eps, out + mf * ldo, ldo, static_cast<int>(rows), static_cast<int>(N));
  }
  return check_launch("rf_norm_linear");
}

extern "C" int rf_map_apply_batch(int nl, const uint16_t* b, int64_t ldb, const uint16_t* const* w,
                                  const uint16_t* const* c, uint16_t* const* x, int64_t ldx, float* const* ssq, int64_t P,
                                  int64_t h_in, int64_t h_out, hipStream_t stream) {
  if (nl < 1 || nl > MAXL) return fail(RF_EINVAL_ARG, "rf_map_apply_batch: %d layers (1 .. %d)", nl, MAXL);
  if (!b || !w || !x || !ssq) return fail(RF_EINVAL_ARG, "rf_map_apply_batch: null pointer");
  if (P < 0 || P > (1ll << 30)) return fail(RF_EINVAL_SHAPE, "rf_map_apply_batch: P = %lld out of range", (long long)P);
  if (h_in <= 0 || h_in % BK || h_in < 2 * BK || h_out <= 0 || h_out % BN)
    return fail(RF_EINVAL_SHAPE, "rf_map_apply_batch: h_in %lld must be a multiple of 64 (>= 128) and h_out %lld of 256",
                (long long)h_in, (long long)h_out);
  if (ldb < h_in || ldx < h_out || ldb % 8 || ldx % 8 || ldb > (1 << 21) || h_in > (1 << 21))
    return fail(RF_EINVAL_SHAPE, "rf_map_apply_batch: row strides ldb %lld / ldx %lld", (long long)ldb, (long long)ldx);
  if (static_cast<int64_t>(nl) * grid_of(P, h_out) > (1ll << 30))
    return fail(RF_EINVAL_SHAPE, "rf_map_apply_batch: too many tiles");
  MapLayers ml{};
  for (int l = 0; l < nl; ++l) {
    if (!w[l] || !x[l] || !ssq[l]) return fail(RF_EINVAL_ARG, "rf_map_apply_batch: null pointer for layer %d", l);
    if (!aligned16(w[l]) || !aligned16(x[l]) || (c && c[l] && !aligned16(c[l])))
      return fail(RF_EINVAL_SHAPE, "rf_map_apply_batch: layer %d pointers must be 16-byte aligned", l);
    ml.w[l] = w[l];
    ml.c[l] = c ? c[l] : nullptr;
    ml.x[l] = x[l];
    ml.ssq[l] = ssq[l];
  }
  if (!aligned16(b)) return fail(RF_EINVAL_SHAPE, "rf_map_apply_batch: b must be 16-byte aligned");
  if (P == 0) return RF_OK;
  hipLaunchKernelGGL(k_map_apply_p<false>, dim3(persistent_grid(nl * static_cast<int64_t>(grid_of(P, h_out)))),
                     dim3(NTHR), 0, stream, b, ldb, ml, nl, ldx, static_cast<int>(P), static_cast<int>(h_out),
                     static_cast<int>(h_in), static_cast<const uint16_t*>(nullptr), static_cast<int64_t>(0));
  return check_launch("rf_map_apply_batch");
}

extern "C" int rf_norm_kv_write_batch(int nl, const uint16_t* const* x, int64_t ldx, const float* const* ssq, int64_t P,
                                      int64_t H, float eps, const uint16_t* const* wkv, int hkv, int d,
                                      const uint16_t* const* knorm, int knorm_kind, const uint16_t* cs, int rot,
                                      uint16_t* const* kbuf, uint16_t* const* vbuf, int64_t head_stride,
                                      int64_t row_stride, int64_t slot_begin, int64_t cap, hipStream_t stream) {
  if (nl < 1 || nl > MAXL) return fail(RF_EINVAL_ARG, "rf_norm_kv_write_batch: %d layers (1 .. %d)", nl, MAXL);
  if (!x || !ssq || !wkv || !cs || !kbuf || !vbuf) return fail(RF_EINVAL_ARG, "rf_norm_kv_write_batch: null pointer");
  if (P < 0 || P > (1ll << 30))
    return fail(RF_EINVAL_SHAPE, "rf_norm_kv_write_batch: P = %lld out of range", (long long)P);
  if (H <= 0 || H % SSQ_COLS)
    return fail(RF_EINVAL_SHAPE, "rf_norm_kv_write_batch: H = %lld must be a multiple of 256", (long long)H);
  if (d <= 0 || d % 8 || 256 % d || hkv <= 0 || (2ll * hkv * d) % BN)
    return fail(RF_EUNSUPPORTED, "rf_norm_kv_write_batch: head_dim %d / kv heads %d (need 256 %% d == 0, d %% 8 == 0, "
                "2 hkv d %% 256 == 0)", d, hkv);
  if (rot <= 0 || rot > d || rot % 2 || ((rot / 2) % 8 && rot / 2 != 4))
    return fail(RF_EUNSUPPORTED, "rf_norm_kv_write_batch: rotary dims %d of head_dim %d", rot, d);
  if (knorm && knorm_kind != 0 && knorm_kind != 1)
    return fail(RF_EINVAL_ARG, "rf_norm_kv_write_batch: knorm_kind %d", knorm_kind);
  if (ldx < H || ldx % 8 || ldx > (1 << 21) || head_stride % 8 || row_stride % 8 || row_stride < d)
    return fail(RF_EINVAL_SHAPE, "rf_norm_kv_write_batch: strides (ldx %lld, head %lld, row %lld)", (long long)ldx,
                (long long)head_stride, (long long)row_stride);
  if (slot_begin < 0 || slot_begin + P > cap)
    return fail(RF_EINVAL_SHAPE, "rf_norm_kv_write_batch: rows [%lld, %lld) exceed cache capacity %lld",
                (long long)slot_begin, (long long)(slot_begin + P), (long long)cap);
  if (!aligned16(cs)) return fail(RF_EINVAL_SHAPE, "rf_norm_kv_write_batch: cs must be 16-byte aligned");
  if (!(eps >= 0.f)) return fail(RF_EINVAL_ARG, "rf_norm_kv_write_batch: eps %g", static_cast<double>(eps));
  const int64_t N = 2ll * hkv * d;
  if (static_cast<int64_t>(nl) * grid_of(P, N) > (1ll << 30))
    return fail(RF_EINVAL_SHAPE, "rf_norm_kv_write_batch: too many tiles");
  KvLayers kl{};
  for (int l = 0; l < nl; ++l) {
    if (!x[l] || !ssq[l] || !wkv[l] || !kbuf[l] || !vbuf[l] || (knorm && !knorm[l]))
      return fail(RF_EINVAL_ARG, "rf_norm_kv_write_batch: null pointer for layer %d", l);
    if (!aligned16(x[l]) || !aligned16(wkv[l]) || !aligned16(kbuf[l]) || !aligned16(vbuf[l]) ||
        (knorm && !aligned16(knorm[l])))
      return fail(RF_EINVAL_SHAPE, "rf_norm_kv_write_batch: layer %d pointers must be 16-byte aligned", l);
    kl.x[l] = x[l];
    kl.ssq[l] = ssq[l];
    kl.wkv[l] = wkv[l];
    kl.knorm[l] = knorm ? knorm[l] : nullptr;
    kl.kbuf[l] = kbuf[l];
    kl.vbuf[l] = vbuf[l];
  }
  if (P == 0) return RF_OK;
  KvArgs a{nullptr, static_cast<int>(H / SSQ_COLS), static_cast<float>(H), eps, hkv, d, nullptr, knorm_kind, cs, rot,
           nullptr, nullptr, head_stride, row_stride, slot_begin, nullptr};
  a.knorm = knorm ? knorm[0] : nullptr;            // the K epilogue's mode follows the (shared) configuration
  if (persistent_kv_ok(H, rot, P)) {
    launch_norm_kv_p(kl, nl, ldx, P, N, H, a, stream);
  } else {                                          // other widths: the per-tile kernel, one launch per layer
    for (int l = 0; l < nl; ++l) {
      KvArgs al = a;
      al.ssq = kl.ssq[l];
      al.knorm = kl.knorm[l];
      al.kbuf = kl.kbuf[l];
      al.vbuf = kl.vbuf[l];
      hipLaunchKernelGGL(k_norm_kv, dim3(grid_of(P, N)), dim3(NTHR), 0, stream, kl.x[l], ldx, kl.wkv[l],
                         static_cast<int>(P), static_cast<int>(N), static_cast<int>(H), al);
    }
  }
  return check_launch("rf_norm_kv_write_batch");
}

extern "C" int rf_norm_linear_batch(int nl, const uint16_t* const* x, int64_t ldx, const float* const* ssq,
                                    const int64_t* rows, int64_t H, float eps, const uint16_t* const* w,
                                    const int64_t* n, uint16_t* const* out, int64_t ldo, hipStream_t stream) {
  const char* fn = "rf_norm_linear_batch";
  if (nl < 1 || nl > MAXL) return fail(RF_EINVAL_ARG, "%s: %d entries (1 .. %d)", fn, nl, MAXL);
  if (!x || !ssq || !w || !out || !rows || !n) return fail(RF_EINVAL_ARG, "%s: null pointer", fn);
  if (H <= 0 || H % SSQ_COLS) return fail(RF_EINVAL_SHAPE, "%s: H %lld (multiple of 256)", fn, (long long)H);
  if (ldx < H || ldx % 8 || ldx > (1 << 21) || ldo % 8)
    return fail(RF_EINVAL_SHAPE, "%s: strides ldx %lld, ldo %lld", fn, (long long)ldx, (long long)ldo);
  if (!(eps >= 0.f)) return fail(RF_EINVAL_ARG, "%s: eps", fn);
  LinLayers ll{};
  int64_t tiles = 0;
  int live = 0;
  for (int l = 0; l < nl; ++l) {
    if (rows[l] < 0 || rows[l] > (1ll << 30) || n[l] <= 0 || n[l] % BN || ldo < n[l])
      return fail(RF_EINVAL_SHAPE, "%s: entry %d: rows %lld, N %lld (multiple of 256, <= ldo %lld)", fn, l,
                  (long long)rows[l], (long long)n[l], (long long)ldo);
    if (!x[l] || !ssq[l] || !w[l] || !out[l]) return fail(RF_EINVAL_ARG, "%s: null pointer in entry %d", fn, l);
    if (!aligned16(x[l]) || !aligned16(w[l]) || !aligned16(out[l]))
      return fail(RF_EINVAL_SHAPE, "%s: entry %d pointers must be 16-byte aligned", fn, l);
    if (rows[l] == 0) continue;                     // nothing to compute: left out of the launch
    ll.x[live] = x[l];
    ll.ssq[live] = ssq[l];
    ll.w[live] = w[l];
    ll.out[live] = out[l];
    ll.m[live] = static_cast<int>(rows[l]);
    ll.n[live] = static_cast<int>(n[l]);
    ll.start[live] = static_cast<int>(tiles);
    tiles += grid_of(rows[l], n[l]);
    if (tiles > (1ll << 30)) return fail(RF_EINVAL_SHAPE, "%s: too many tiles", fn);
    ++live;
  }
  ll.start[live] = static_cast<int>(tiles);
  if (live == 0) return RF_OK;
  if (persistent_lin_ok(H)) {
    hipLaunchKernelGGL(k_norm_linear_p, dim3(persistent_grid(tiles)), dim3(NTHR), 0, stream, ll, live, ldx, ldo,
                       static_cast<int>(H), eps);
  } else {                                          // other widths: the per-tile kernel, one launch per entry
    for (int l = 0; l < live; ++l)
      hipLaunchKernelGGL(k_norm_linear, dim3(grid_of(ll.m[l], ll.n[l])), dim3(NTHR), 0, stream, ll.x[l], ldx, ll.w[l],
                         ll.m[l], ll.n[l], static_cast<int>(H), ll.ssq[l], eps, ll.out[l], ldo);
  }
  return check_launch(fn);
}
