// Causal attention of many consecutive queries over one layer's K / V cache: the exact tail's
// attention in Model.layer (code/kva/ops.py:107-128 attend, queries bottom-right aligned with the keys),
// head_dim 64 or 128 with grouped-query heads in groups of 1, 2, 4 or 8, and head_dim 256 (Qwen3.5's gated
// attention, code/kva/model.py:436-446) in groups of up to 16 (runs of eight heads per block, the group's
// other heads in further blocks). The layout below is the d 64 / 128 one; at d 256 the key tiles are 32
// keys and each wave holds its 32 queries' 256-wide rows.
//
// K and V tiles stream from the caches into LDS as full 128-byte lines with direct loads
// (buffer_load_dwordx4 ... lds), both row-major ([key, d]); the V^T operand of the second product is read
// out of the row-major V tile with LDS transpose reads (ds_read_b64_tr_b16). A block takes one K / V head
// and 256 query rows (256 / rep
// consecutive queries x the rep query heads sharing the K / V head); 8 waves, each owning 32 query rows
// of one head. The keys 0 .. (the block's last query position) go through LDS in tiles of 64, three
// tiles in flight and four stages. Per tile and wave:
//   S^T = K Q^T on v_mfma_f32_32x32x16_bf16 (A = the K tile, B = the wave's queries held in registers):
//       lane l holds, for query l % 32, the scores of keys 8 (j / 4) + 4 (l / 32) + j % 4 of each
//       32-key half (j < 16);
//   online softmax in fp32 in the base-2 domain, keys past the query's position masked; every value a
//       lane holds belongs to its own query, so the maximum, the rescale and the row sum need no lane
//       exchange except the one between the lane halves. The reference maximum is raised lazily (only
//       when a score exceeds it by more than 2^8), so the O rescale runs on few tiles;
//   O^T += V^T P^T on the same MFMA: P (rounded to bf16) is the B operand straight from the score
//       registers, the contraction order over each 16-key step being keys {0..3, 8..11} + 4 (l / 32)
//       of the step, and the V^T fragment is read in that order: two transpose reads, each giving a lane
//       4 consecutive keys of its d column.
// Each SIMD holds two waves, so one wave's softmax (VALU) can issue beside the other's MFMAs, and the
// next tile's score MFMAs run in the same instruction block as this tile's exponentials. (Waves of 64
// query rows, one per SIMD, read half as much LDS per tile but measured 11 % slower: the second wave's
// overlap matters more here than the LDS reads.) With few query blocks the key range is split over
// blocks whose partials k_causal_combine merges in a fixed order: split sp takes the W key tiles
// [sp W, (sp + 1) W) (the last split of a query block may be shorter), and splits past the block's last
// query exit at once. The splits start at key 0 for every query block, so the query blocks of one K / V
// head and split read the same tiles; they are placed side by side on one XCD, whose L2 then serves the
// tiles to all of them from one read of memory.
// The probabilities enter the second product as bf16 before normalisation (the reference casts after
// it; the difference is within rounding), scores are fp32 products of the bf16 q and k values as the
// reference's fp32 matmul, and the output is O / (row sum) rounded to bf16.
#include <stdint.h>

#include <algorithm>

#include "rf_common.h"

namespace rf {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// Per head_dim: keys per tile KT; 8 waves per block (two per SIMD), 32 query rows each. d 64 / 128:
// 64-key tiles. d 256: 32-key tiles keep four 32 KB stages in LDS; a wave's queries take 64 registers and
// its O^T 128 of the 256 two waves per SIMD leave it, so the tile loads' per-lane offsets are recomputed
// at each issue instead of held, and a few values still spill (outside the key loop but for one query
// fragment and the edge tiles' lane offset).
template <int AD>
struct Cfg {
  static constexpr int KT = AD == 256 ? 32 : 64;
  static constexpr int NW = 8;
  static constexpr int NTHR = 64 * NW;
  static constexpr int QROWS = 32 * NW;  // query rows (query, head) per block: 32 per wave
  static constexpr int KB = KT / 32;     // 32-key halves of a tile
};
constexpr int NSTAGE = 4;              // LDS stages: three tiles in flight, one still read

__device__ __forceinline__ bf16x8 as_frag(const uint4& u) { return __builtin_bit_cast(bf16x8, u); }

typedef __attribute__((address_space(3))) void* lds_ptr;

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

// LDS layout of one stage: the K tile then the V tile, each 64 keys x AD row-major in 16-byte chunks. K row
// r's chunk c sits at r * KCPR + (c ^ (r % KCPR)): the score fragment reads (32 rows, one chunk per lane)
// hit distinct banks. V row r's chunk c sits at K_U4 + r * KCPR + (c ^ (4 vsw(r))): a transpose read takes
// 8 bytes in each of 4 consecutive rows over 4 chunks per row per 32 lanes, and the swizzle moves the four
// rows onto four different 64-byte bank ranges.
template <int AD>
struct Layout {
  static constexpr int KT = Cfg<AD>::KT, NW = Cfg<AD>::NW;
  static constexpr int KCPR = AD / 8;
  static constexpr int K_U4 = KT * KCPR;
  static constexpr int V_U4 = KT * KCPR;
  static constexpr int STAGE_U4 = K_U4 + V_U4;
  static constexpr int KLOADS = K_U4 / 64 / NW;     // direct-load instructions per wave per tile
  static constexpr int VLOADS = V_U4 / 64 / NW;
  static constexpr int LOADS = KLOADS + VLOADS;
  static_assert(KLOADS * 64 * NW == K_U4 && VLOADS * 64 * NW == V_U4, "tile loads must split evenly");
  static_assert(NSTAGE * STAGE_U4 * 16 <= 160 * 1024, "stages fit the LDS");
  __device__ static int kslot(int row, int c) { return row * KCPR + (c ^ (row & (KCPR - 1))); }
  // d 128 / 256: a row is 256 / 512 bytes, rows r .. r + 3 shift by 0, 64, 128, 192 bytes; d 64: rows are
  // 128 bytes, row parity already picks the half of a 256-byte bank line, and rows r, r + 2 shift by 0 and 64
  __device__ static int vsw(int row) { return AD >= 128 ? (row & 3) : ((row >> 1) & 1); }
  __device__ static int vslot(int row, int c) { return K_U4 + row * KCPR + (c ^ (4 * vsw(row))); }
};

struct CausalArgs {
  const uint16_t* q;       // [nq, >= hq * d]: query j head h at q + j * ldq + h * d
  int64_t ldq;
  int nq;
  const int64_t* qpos;     // sorted query positions (query j sees keys 0 .. qpos[j]), or null:
  int64_t slot0;           // query j at slot0 + j
  const uint16_t* kc;      // K cache [hkv, cap, d]
  int64_t head_stride, row_stride;
  int64_t n_keys;
  const uint16_t* vc;      // V cache, as kc
  int hq, hkv;
  float scale_log2;        // scale * log2(e)
  uint16_t* out;           // [nq, >= hq * d]
  int64_t ldo;
  float* part;             // splits > 1: per (query block, head block, split) O [QROWS][d], max, sum [QROWS]
  int split_tiles;         // W: key tiles per split
  int hpb;                 // query heads per block (all rep of a K / V head, or a run of NW of them)
};

__device__ __forceinline__ int64_t query_pos(const CausalArgs& a, int j) { return a.qpos ? a.qpos[j] : a.slot0 + j; }

// partials of (query block qb, head block hb, split sp); head blocks are gridDim.y = hkv (rep / hpb)
template <int AD>
__device__ __forceinline__ float* part_block(const CausalArgs& a, int qb, int hb, int sp) {
  constexpr int QROWS = Cfg<AD>::QROWS;
  return a.part + ((static_cast<int64_t>(qb) * gridDim.y + hb) * gridDim.z + sp) * (QROWS * (AD + 2));
}

// The direct loads of one tile into stage st: instruction i of wave w fills 64 consecutive 16-byte slots
// (lane L slot (w * n + i) * 64 + L) from the per-lane offsets koff / voff plus the tile's byte offset.
template <int AD>
__device__ __forceinline__ void issue_tile(__amdgpu_buffer_rsrc_t rk, __amdgpu_buffer_rsrc_t rv,
                                           const uint32_t (&koff)[Layout<AD>::KLOADS],
                                           const uint32_t (&voff)[Layout<AD>::VLOADS], char* st, uint32_t kbyte,
                                           uint32_t vbyte, int w) {
  using L = Layout<AD>;
#pragma unroll
  for (int i = 0; i < L::KLOADS; ++i)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_ptr)(st + (w * L::KLOADS + i) * 1024), 16, koff[i], kbyte, 0, 0);
#pragma unroll
  for (int i = 0; i < L::VLOADS; ++i)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lds_ptr)(st + (L::K_U4 + (w * L::VLOADS + i) * 64) * 16), 16,
                                             voff[i], vbyte, 0, 0);
}

// Headroom of the lazy softmax rescale: the running reference maximum is raised only when a score
// exceeds it by more than this (in base 2), so probabilities stay below 2^8 and the O rescale runs
// only on the tiles that raise it.
constexpr float RESCALE_LOG2 = 8.0f;

// Per-lane LDS byte offsets of the fragments within a stage, the same for every tile. K fragment (key
// half kb, d step s): row 32 kb + n, chunk 2 s + hh, at k(s) + kb * 32 KCPR 16 (row 32 kb + n has the
// swizzle of row n). V^T fragment (d block b, 16-key step stp): lane l = 16 g + t takes, in each of two
// transpose reads, row 16 stp + 8 i + 4 (g / 2) + t / 4 (i = 0, 1) at d 32 b + 16 (g % 2) + 4 (t % 4)
// (8 bytes), and receives keys 16 stp + 8 i + 4 (g / 2) + 0 .. 3 of d 32 b + 16 (g % 2) + t: the fragment
// order {0..3, 8..11} + 4 hh. Its byte offset is v(b) + (16 stp + 8 i) KCPR 16 (rows 16 stp + 8 i + r have
// the swizzle of row r).
// Both are one XOR per read: the K chunk 2 s + hh = 2 s ^ hh, so its swizzled byte offset within row n is
// 32 s ^ 16 (hh ^ (n % KCPR)), and the row's base n KCPR 16 has no bits in common with it; the V^T block
// offset 64 (b ^ vsw) = 64 b ^ 64 vsw sits in bits 6 .. 8, which the rest of the V offset leaves clear.
template <int AD>
struct FragOffsets {
  uint32_t kz, vz;
  __device__ FragOffsets(int lane) {
    using L = Layout<AD>;
    const int n = lane & 31, hh = lane >> 5, g = lane >> 4, t = lane & 15;
    kz = static_cast<uint32_t>(n * L::KCPR * 16) | static_cast<uint32_t>(16 * (hh ^ (n & (L::KCPR - 1))));
    const int r0 = 4 * (g >> 1) + (t >> 2), cl = 2 * (g & 1) + ((t & 3) >> 1);
    vz = static_cast<uint32_t>((L::K_U4 + r0 * L::KCPR + cl) * 16 + 8 * (t & 1)) |
         static_cast<uint32_t>(64 * L::vsw(r0));
  }
  __device__ uint32_t k(int s) const { return kz ^ static_cast<uint32_t>(32 * s); }
  __device__ uint32_t v(int b) const { return vz ^ static_cast<uint32_t>(64 * b); }
};

typedef short s16x4 __attribute__((ext_vector_type(4)));

// Four keys of one d column per lane out of the row-major V tile (ds_read_b64_tr_b16).
__device__ __forceinline__ uint2 read_tr(const char* p) {
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(p));
  return __builtin_bit_cast(uint2, v);
}

// The two lane halves' values of a lane pair (l, l ^ 32), the same in both lanes: v of the lower lane
// and v of the upper lane (one v_permlane32_swap).
__device__ __forceinline__ void lane_pair(float v, float& lo, float& hi) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  lo = __uint_as_float(r[0]);
  hi = __uint_as_float(r[1]);
}

// S^T = K Q^T for one key tile (KB halves of 32 keys) and the wave's 32 queries: sc[kb][j] = the raw
// score of key 32 kb + 8 (j / 4) + 4 hh + j % 4 of the tile for query n. (The stage pointers are
// __restrict__: the LDS reads then carry alias information, and the compiler does not make them wait for
// the direct loads in flight into the other stages; the kernel's own waits order them.)
template <int AD>
__device__ __forceinline__ void tile_scores(const char* __restrict__ st, const bf16x8 (&qf)[AD / 16],
                                            f32x16 (&sc)[Cfg<AD>::KB], const FragOffsets<AD>& fo) {
  using L = Layout<AD>;
  constexpr int NS = AD / 16, KB = Cfg<AD>::KB;
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
    for (int r = 0; r < 16; ++r) sc[kb][r] = 0.f;
#pragma unroll
    for (int s = 0; s < NS; ++s)
      sc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
          as_frag(*reinterpret_cast<const uint4*>(st + fo.k(s) + kb * 32 * L::KCPR * 16)), qf[s], sc[kb], 0, 0, 0);
  }
}

// One tile's softmax and products, with the next tile's scores interleaved: mask the scores sc of the
// tile at key k0 when some key lies past some query of the wave (edge), raise the lane's reference
// maximum mref (raw-score units, -inf until a key is visible) lazily, then in one block the base-2
// probabilities exp2(fma(s, c, -mref c)) of sc (c = scale * log2(e) > 0) beside the MFMAs of the next
// tile's scores sn (from stage sn_st), and O^T += V^T P^T from this tile's stage st.
template <int AD>
__device__ __forceinline__ void tile_step(const char* __restrict__ st, const char* __restrict__ sn_st,
                                          const bf16x8 (&qf)[AD / 16], f32x16 (&sc)[Cfg<AD>::KB],
                                          f32x16 (&sn)[Cfg<AD>::KB], f32x16 (&o)[AD / 32], float& mref, float& lsum,
                                          int k0, bool edge, int mypos, int hh, float c,
                                          const FragOffsets<AD>& fo) {
  using L = Layout<AD>;
  constexpr int NB = AD / 32, NS = AD / 16, KB = Cfg<AD>::KB, KT = Cfg<AD>::KT;
  constexpr int NP = 8 * KB;                            // probability pairs per lane
  if (edge) {
    // key 32 kb + 8 (j / 4) + 4 hh + j % 4 of the tile is past the query when its offset exceeds rel
    const int rel = min(max(mypos - k0, -1), KT) - 4 * hh;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int j = 0; j < 16; ++j)
        if (32 * kb + 8 * (j >> 2) + (j & 3) > rel) sc[kb][j] = -INFINITY;
  }
  float tmax = -INFINITY;
#pragma unroll
  for (int kb = 0; kb < KB; ++kb)
#pragma unroll
    for (int j = 0; j < 16; ++j) tmax = fmaxf(tmax, sc[kb][j]);
  float lo, hi;
  lane_pair(tmax, lo, hi);
  tmax = fmaxf(lo, hi);
  if (tmax > mref + RESCALE_LOG2 / c) {                 // raise the reference (always on the first visible key)
    const float alpha = __builtin_amdgcn_exp2f((mref - tmax) * c);    // 0 while mref is -inf
    mref = tmax;
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[b][r] *= alpha;
    lsum *= alpha;
  }
  const float mc = mref == -INFINITY ? 0.f : mref * c;  // every key so far masked (a split past the query)
  // the next tile's KB NS score MFMAs, the NP probability pairs spread between them
  float psum = 0.f;
  uint32_t pk[NP];
#pragma unroll
  for (int kb = 0; kb < KB; ++kb)
#pragma unroll
    for (int r = 0; r < 16; ++r) sn[kb][r] = 0.f;
#pragma unroll
  for (int q = 0; q < KB * NS; ++q) {
    const int kb = q / NS, s = q % NS;
    sn[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
        as_frag(*reinterpret_cast<const uint4*>(sn_st + fo.k(s) + kb * 32 * L::KCPR * 16)), qf[s], sn[kb], 0, 0, 0);
#pragma unroll
    for (int e = q * NP / (KB * NS); e < (q + 1) * NP / (KB * NS); ++e) {
      const int pkb = e / 8, pj = 2 * (e % 8);
      const float p0 = __builtin_amdgcn_exp2f(fmaf(sc[pkb][pj], c, -mc));
      const float p1 = __builtin_amdgcn_exp2f(fmaf(sc[pkb][pj + 1], c, -mc));
      psum += p0 + p1;
      pk[e] = bf16_pair(p0, p1);
    }
  }
  lsum += psum;
  // O^T[d, query] += V^T[d, keys] P^T[keys, query] over the tile's 16-key steps (keys 16 stp ..: chunks
  // 2 stp and 2 stp + 1; P^T step stp = the lane's probabilities 8 stp .. 8 stp + 7)
#pragma unroll
  for (int stp = 0; stp < KT / 16; ++stp) {
    const bf16x8 pf = __builtin_bit_cast(bf16x8, make_uint4(pk[4 * stp], pk[4 * stp + 1], pk[4 * stp + 2],
                                                             pk[4 * stp + 3]));
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const char* vp = st + fo.v(b) + 16 * stp * L::KCPR * 16;
      const uint2 vl = read_tr(vp), vh = read_tr(vp + 8 * L::KCPR * 16);
      o[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_frag(make_uint4(vl.x, vl.y, vh.x, vh.y)), pf, o[b], 0, 0, 0);
    }
  }
}

template <int AD>
__global__ __launch_bounds__(Cfg<AD>::NTHR, 1) void k_attend_causal(CausalArgs a) {
  using L = Layout<AD>;
  constexpr int NS = AD / 16;      // 16-deep d steps of S^T
  constexpr int NB = AD / 32;      // 32-row d blocks of O^T
  constexpr int KT = Cfg<AD>::KT, QROWS = Cfg<AD>::QROWS, KB = Cfg<AD>::KB;
  __shared__ uint4 lds[NSTAGE * L::STAGE_U4];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6, n = lane & 31, hh = lane >> 5;
  const int rep = a.hq / a.hkv, qp = QROWS / a.hpb;        // consecutive queries per block
  // block -> (query block, split, head block), query blocks fastest: each XCD takes a contiguous run, so
  // the query blocks of one (head block, split) run side by side on one XCD and read the same key tiles
  // through its L2. Head block hb: K / V head hb / (rep / hpb), its query heads from (hb % (rep / hpb)) hpb.
  const int qbs = gridDim.x, ns = gridDim.z;
  const int u = xcd_tile(blockIdx.x + qbs * (blockIdx.y + gridDim.y * blockIdx.z), qbs * gridDim.y * ns);
  const int qb = u % qbs, sp = (u / qbs) % ns, hb = u / (qbs * ns);
  const int hk = hb / (rep / a.hpb), hoff = (hb % (rep / a.hpb)) * a.hpb;
  const int j0 = qb * qp;
  const int jlast = min(j0 + qp, a.nq) - 1;
  const int64_t kmax = min(query_pos(a, jlast), a.n_keys - 1);     // the block reads keys 0 .. kmax
  const int ntiles = static_cast<int>(kmax / KT) + 1;
  // this block's share of the key tiles: split sp, tiles [sp W, (sp + 1) W) from key 0, the same key
  // tiles for every query block
  const int it0 = sp * a.split_tiles;
  if (it0 >= ntiles) return;                              // past the last query (block-uniform, before any barrier)
  const int it1 = min(ntiles, it0 + a.split_tiles);

  // the wave's head and queries; lanes past the last query repeat it and write nothing
  const int hg = (32 * w) / qp, po0 = (32 * w) % qp;
  const int jw0 = j0 + po0;
  const int jq = min(jw0 + n, jlast);
  const bool live = jw0 + n <= jlast;
  // positions as int, clamped to -1 .. n_keys - 1 (n_keys < 2^31: the caches' byte range is checked below
  // 2^32): a query past the last key sees every key, one before key 0 none
  auto clamp_pos = [&](int64_t p) { return static_cast<int>(min<int64_t>(max<int64_t>(p, -1), a.n_keys - 1)); };
  const int mypos = clamp_pos(query_pos(a, jq));
  const int wave_first = clamp_pos(query_pos(a, min(jw0, jlast)));
  // a wave whose queries all lie past the block's last one (a partial last query block) skips every tile
  const int wave_last = jw0 <= jlast ? clamp_pos(query_pos(a, min(jw0 + 31, jlast))) : -1;
  const int head = hk * rep + hoff + hg;
  bf16x8 qf[NS];
  {
    const uint16_t* qrow = a.q + static_cast<int64_t>(jq) * a.ldq + head * AD + 8 * hh;
#pragma unroll
    for (int s = 0; s < NS; ++s) qf[s] = as_frag(*reinterpret_cast<const uint4*>(qrow + 16 * s));
  }
  wait_vm_lgkm0<0>();        // the queries are in registers before any tile load is in flight

  const uint16_t* kh = a.kc + hk * a.head_stride;
  const __amdgpu_buffer_rsrc_t rk = buffer_rsrc(kh, static_cast<uint32_t>(a.n_keys * a.row_stride * 2));
  const __amdgpu_buffer_rsrc_t rv = buffer_rsrc(a.vc + hk * a.head_stride, static_cast<uint32_t>(a.n_keys * a.row_stride * 2));
  char* base = reinterpret_cast<char*>(lds);
  const uint32_t rs2 = static_cast<uint32_t>(a.row_stride * 2);     // row bytes (the caches span < 2^32 bytes)
  // lane ln's source offsets for the tile loads (instruction i of wave w fills 64 consecutive slots; the
  // lane's slot gives the row and logical chunk it fetches)
  auto offsets = [&](int ln, uint32_t (&koff)[L::KLOADS], uint32_t (&voff)[L::VLOADS]) {
#pragma unroll
    for (int i = 0; i < L::KLOADS; ++i) {
      const int sl = (w * L::KLOADS + i) * 64 + ln;
      const int row = sl / L::KCPR, pc = sl % L::KCPR, c = pc ^ (row & (L::KCPR - 1));
      koff[i] = static_cast<uint32_t>(row) * rs2 + static_cast<uint32_t>(c * 16);
    }
#pragma unroll
    for (int i = 0; i < L::VLOADS; ++i) {
      const int sl = (w * L::VLOADS + i) * 64 + ln;
      const int row = sl / L::KCPR, pc = sl % L::KCPR, c = pc ^ (4 * L::vsw(row));
      voff[i] = static_cast<uint32_t>(row) * rs2 + static_cast<uint32_t>(c * 16);
    }
  };
  // d 256 recomputes them at each issue rather than holding them across the loop (registers are the limit
  // there): the lane index then comes from v_mbcnt in a volatile asm, which the compiler neither hoists
  // nor keeps in a register
  constexpr bool RECOMPUTE = AD == 256;
  uint32_t koff0[L::KLOADS], voff0[L::VLOADS];
  if constexpr (!RECOMPUTE) offsets(lane, koff0, voff0);
  auto issue = [&](int it) {
    const uint32_t tb = static_cast<uint32_t>(it) * static_cast<uint32_t>(KT) * rs2;
    char* st = base + ((it - it0) % NSTAGE) * L::STAGE_U4 * 16;
    if constexpr (RECOMPUTE) {
      int ln;
      asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(ln));
      uint32_t koff[L::KLOADS], voff[L::VLOADS];
      offsets(ln, koff, voff);
      issue_tile<AD>(rk, rv, koff, voff, st, tb, tb, w);
    } else {
      issue_tile<AD>(rk, rv, koff0, voff0, st, tb, tb, w);
    }
  };

  f32x16 o[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[b][r] = 0.f;
  float m = -INFINITY, lsum = 0.f;                        // reference maximum (raw scores), row sum
  const float c = a.scale_log2;

  // Tile it is processed in iteration it: its softmax and products, with the scores of tile it + 1
  // computed in the same block (the MFMAs run beside the softmax's VALU work). Loads run three tiles
  // ahead into four stages: tile it + 3 goes into the stage of tile it - 1, whose last reads (its V^T)
  // ended before this iteration's barrier.
  const FragOffsets<AD> fo(lane);
  f32x16 sc[KB], sn[KB];
  auto stage = [&](int it) { return base + ((it - it0) % NSTAGE) * L::STAGE_U4 * 16; };
  for (int i = 0; i < 3; ++i)
    if (it0 + i < it1) issue(it0 + i);
  if (it0 + 2 < it1) wait_vm_lgkm0<2 * L::LOADS>();        // tile it0 landed
  else if (it0 + 1 < it1) wait_vm_lgkm0<L::LOADS>();
  else wait_vm_lgkm0<0>();
  __builtin_amdgcn_s_barrier();
  if (it0 < it1) tile_scores<AD>(stage(it0), qf, sc, fo);
  // iteration it: the scores of tile it are in cur, those of tile it + 1 go to nxt. At d 64 / 128 the loop
  // runs two iterations per trip with the buffers' roles swapped, so no scores are copied (8B tail shape:
  // 2041 -> 1924 us); at d 256 that version spills more and measured slower (2086 -> 2217 us), so there
  // the next scores are copied back each iteration.
  auto iteration = [&](int it, f32x16 (&cur)[KB], f32x16 (&nxt)[KB]) {
    if (it + 2 < it1) wait_vm_lgkm0<L::LOADS>();          // tile it + 1 landed, tile it + 2 may fly
    else wait_vm_lgkm0<0>();
    __builtin_amdgcn_s_barrier();                         // every wave's share of it has landed and every
    if (it + 3 < it1) issue(it + 3);                      // wave is done with the stage reloaded here
    const int k0 = it * KT;
    if (k0 > wave_last) return;                           // this and every later tile lie past the wave's queries
    tile_step<AD>(stage(it), stage(it + 1), qf, cur, nxt, o, m, lsum, k0, k0 + KT - 1 > wave_first, mypos, hh, c, fo);
  };
  if constexpr (AD == 256) {
    for (int it = it0; it < it1; ++it) {
      if (it + 2 < it1) wait_vm_lgkm0<L::LOADS>();
      else wait_vm_lgkm0<0>();
      __builtin_amdgcn_s_barrier();
      if (it + 3 < it1) issue(it + 3);
      const int k0 = it * KT;
      if (k0 > wave_last) continue;
      tile_step<AD>(stage(it), stage(it + 1), qf, sc, sn, o, m, lsum, k0, k0 + KT - 1 > wave_first, mypos, hh, c, fo);
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) sc[kb] = sn[kb];
    }
  } else {
    for (int it = it0; it < it1; it += 2) {
      iteration(it, sc, sn);
      if (it + 1 < it1) iteration(it + 1, sn, sc);
    }
  }
  wait_vm_lgkm0<0>();

  // lane holds O[query n][d = 32 b + 8 (j / 4) + 4 hh + j % 4]
  float llo, lhi;
  lane_pair(lsum, llo, lhi);
  const float ltot = llo + lhi;
  if (ns > 1) {                                           // unnormalised partials for k_causal_combine
    float* pb = part_block<AD>(a, qb, hb, sp);
    const int r = 32 * w + n;
    float* orow = pb + r * AD + 4 * hh;
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *reinterpret_cast<float4*>(orow + 32 * b + 8 * g) = make_float4(o[b][4 * g], o[b][4 * g + 1], o[b][4 * g + 2],
                                                                        o[b][4 * g + 3]);
    if (hh == 0) {
      pb[QROWS * AD + r] = m == -INFINITY ? m : m * c;    // base-2 maximum of the reference
      pb[QROWS * AD + QROWS + r] = ltot;
    }
    return;
  }
  if (!live) return;
  const float inv = 1.0f / ltot;
  uint16_t* dst = a.out + static_cast<int64_t>(jq) * a.ldo + head * AD + 4 * hh;
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int g = 0; g < 4; ++g)
      *reinterpret_cast<uint2*>(dst + 32 * b + 8 * g) =
          make_uint2(bf16_pair(o[b][4 * g] * inv, o[b][4 * g + 1] * inv),
                     bf16_pair(o[b][4 * g + 2] * inv, o[b][4 * g + 3] * inv));
}

// Merges the key-range splits of one (query block, head block): M = max_s m_s, L = sum_s l_s 2^(m_s - M),
// O = sum_s O_s 2^(m_s - M) / L (base-2 maxima), splits in order. A thread takes 4 consecutive d of one query
// row (AD / 4 threads per row, blockIdx.z picks 256 of the block's QROWS * AD / 4 such pieces), so the
// partials are read as whole rows and the outputs written as 8-byte runs.
template <int AD>
__global__ __launch_bounds__(256) void k_causal_combine(CausalArgs a, int ns) {
  constexpr int TPR = AD / 4, KT = Cfg<AD>::KT, QROWS = Cfg<AD>::QROWS;
  const int idx = blockIdx.z * 256 + threadIdx.x;
  const int r = idx / TPR, e = 4 * (idx % TPR), w = r / 32, n = r % 32;
  const int rep = a.hq / a.hkv, qp = QROWS / a.hpb;
  const int hb = blockIdx.y, j0 = blockIdx.x * qp;
  const int hk = hb / (rep / a.hpb), hoff = (hb % (rep / a.hpb)) * a.hpb;
  const int hg = (32 * w) / qp, po0 = (32 * w) % qp;
  const int jq = j0 + po0 + n;
  if (jq >= a.nq) return;
  const int64_t stride = QROWS * (AD + 2);
  const float* base = a.part + (static_cast<int64_t>(blockIdx.x) * gridDim.y + hb) * ns * stride;
  // the live splits of this query block (those k_attend_causal ran): ceil(ntiles / W)
  const int jlast = min(j0 + qp, a.nq) - 1;
  const int ntiles = static_cast<int>(min(query_pos(a, jlast), a.n_keys - 1) / KT) + 1;
  const int live = min(ns, (ntiles + a.split_tiles - 1) / a.split_tiles);
  float mx = -INFINITY;
  for (int sp = 0; sp < live; ++sp) mx = fmaxf(mx, base[sp * stride + QROWS * AD + r]);
  float l = 0.f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int sp = 0; sp < live; ++sp) {
    const float* pb = base + sp * stride;
    const float ms = pb[QROWS * AD + r];
    const float f = ms == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ms - mx);
    l += pb[QROWS * AD + QROWS + r] * f;
    const float4 v = *reinterpret_cast<const float4*>(pb + r * AD + e);
    acc.x += v.x * f;
    acc.y += v.y * f;
    acc.z += v.z * f;
    acc.w += v.w * f;
  }
  const float inv = 1.0f / l;
  uint16_t* dst = a.out + static_cast<int64_t>(jq) * a.ldo + (hk * rep + hoff + hg) * AD + e;
  *reinterpret_cast<uint2*>(dst) = make_uint2(bf16_pair(acc.x * inv, acc.y * inv), bf16_pair(acc.z * inv, acc.w * inv));
}

int kt_of(int d) { return d == 256 ? Cfg<256>::KT : Cfg<128>::KT; }
int qrows_of(int d) { return d == 256 ? Cfg<256>::QROWS : Cfg<128>::QROWS; }
// query heads per block: the whole group of a K / V head when its 32-query waves fit the block, else a
// run of as many heads as the block has waves
int hpb_of(int hq, int hkv, int d) { return std::min(hq / hkv, qrows_of(d) / 32); }
// head blocks: hkv K / V heads x (rep / hpb) runs of query heads
int head_blocks(int hq, int hkv, int d) { return hkv * ((hq / hkv) / hpb_of(hq, hkv, d)); }

int64_t key_tiles(int64_t n_keys, int d) { return (n_keys + kt_of(d) - 1) / kt_of(d); }

int64_t queries_per_block(int hq, int hkv, int d) { return qrows_of(d) / hpb_of(hq, hkv, d); }

int64_t query_blocks(int64_t nq, int hq, int hkv, int d) {
  const int64_t qp = queries_per_block(hq, hkv, d);
  return (nq + qp - 1) / qp;
}

size_t part_bytes(int64_t nq, int hq, int hkv, int d, int splits) {
  return splits > 1 ? static_cast<size_t>(query_blocks(nq, hq, hkv, d)) * head_blocks(hq, hkv, d) * splits *
                          qrows_of(d) * (d + 2) * 4
                    : 0;
}

// Key-range splits {ns, W}: W key tiles per split block, ns = ceil(key tiles / W) splits at most. With
// enough query blocks to fill the CUs (blocks per CU: one at d 128, two at d 64, by LDS), none. Else W
// minimises (rounds of live blocks) x (W + 2), the live blocks of query block qb being ceil(ntiles_qb / W)
// per K / V head: ntiles_qb exact for consecutive queries (qpos null), else from query positions spread
// evenly over the keys (the exact rows). A round is about 0.8 of the CUs' block slots: measured at 287
// scattered queries over 28672 keys (32 / 8 heads, d 128), 208 live blocks of 56 tiles take 152 us and
// 240 of 45 tiles 176 us (the blocks slow each other down through the shared K / V reads). Only the time
// depends on these estimates, not the results.
struct Splits {
  int ns, W;
};

Splits causal_plan(int64_t nq, int hq, int hkv, int d, int64_t n_keys, bool scattered, int64_t slot0) {
  const int64_t T = key_tiles(n_keys, d), QB = query_blocks(nq, hq, hkv, d), qp = queries_per_block(hq, hkv, d);
  const int64_t HB = head_blocks(hq, hkv, d), KT = kt_of(d);
  if (QB * HB >= 256 * (d == 64 ? 2 : 1) || T <= 1) return Splits{1, static_cast<int>(std::max<int64_t>(T, 1))};
  const int64_t slots = 208 * (d == 64 ? 2 : 1);
  auto tiles_of = [&](int64_t qb) {
    if (scattered) return std::max<int64_t>(1, (T * (qb + 1) + QB - 1) / QB);
    const int64_t last = slot0 + std::min<int64_t>((qb + 1) * qp, nq) - 1;
    return std::min<int64_t>(T, last / KT + 1);
  };
  int64_t best_w = T, best_cost = INT64_MAX;
  for (int64_t W = std::max<int64_t>(2, (T + 63) / 64); W <= T; ++W) {   // at most 64 splits
    int64_t live = 0;
    for (int64_t qb = 0; qb < QB; ++qb) live += (tiles_of(qb) + W - 1) / W;
    const int64_t cost = ((live * HB + slots - 1) / slots) * (W + 2);
    if (cost < best_cost || (cost == best_cost && W > best_w)) {
      best_cost = cost;
      best_w = W;
    }
  }
  return Splits{static_cast<int>((T + best_w - 1) / best_w), static_cast<int>(best_w)};
}

// head_dim 64 / 128: groups of 1 .. 8 (a block holds every head of a group); 256: groups of 1 .. 16 (runs of
// up to eight heads per block)
bool causal_shape_ok(int hq, int hkv, int d) {
  if ((d != 64 && d != 128 && d != 256) || hq <= 0 || hkv <= 0 || hq % hkv) return false;
  const int rep = hq / hkv;
  return (rep & (rep - 1)) == 0 && rep <= (d == 256 ? 16 : 8);
}

}  // namespace
}  // namespace rf

using namespace rf;

extern "C" int rf_attend_causal_workspace_bytes(int64_t nq, int hq, int hkv, int d, int64_t n_keys, size_t* bytes) {
  if (!bytes || nq < 0 || n_keys < 0) return fail(RF_EINVAL_ARG, "rf_attend_causal_workspace_bytes: arguments");
  if (!causal_shape_ok(hq, hkv, d))
    return fail(RF_EUNSUPPORTED, "rf_attend_causal_workspace_bytes: head_dim %d, %d query heads over %d K / V heads "
                "(d 64, 128 or 256; a group of 1, 2, 4 or 8, or up to 16 at d 256)", d, hq, hkv);
  *bytes = part_bytes(nq, hq, hkv, d, causal_plan(nq, hq, hkv, d, n_keys, true, 0).ns);
  return RF_OK;
}

extern "C" int rf_attend_causal(const uint16_t* q, int64_t ldq, int64_t nq, const int64_t* qpos, int64_t slot0, int hq,
                                int d, const uint16_t* kbuf, const uint16_t* vbuf, int hkv, int64_t head_stride,
                                int64_t row_stride, int64_t n_keys, float scale, uint16_t* out, int64_t ldo,
                                void* workspace, size_t ws_bytes, hipStream_t stream) {
  if (!q || !kbuf || !vbuf || !out) return fail(RF_EINVAL_ARG, "rf_attend_causal: null pointer");
  if (d != 64 && d != 128 && d != 256)
    return fail(RF_EUNSUPPORTED, "rf_attend_causal: head_dim %d (the kernel takes 64, 128, 256)", d);
  if (!causal_shape_ok(hq, hkv, d))
    return fail(RF_EUNSUPPORTED, "rf_attend_causal: %d query heads over %d K / V heads (group of 1, 2, 4 or 8, or up "
                "to 16 at head_dim 256)", hq, hkv);
  if (nq < 0 || nq > (1 << 30) || n_keys <= 0 || (!qpos && (slot0 < 0 || slot0 + nq > n_keys)))
    return fail(RF_EINVAL_SHAPE, "rf_attend_causal: queries at slots [%lld, %lld) past the %lld keys", (long long)slot0,
                (long long)(slot0 + nq), (long long)n_keys);
  if (ldq < static_cast<int64_t>(hq) * d || ldo < static_cast<int64_t>(hq) * d || ldq % 8 || ldo % 4 ||
      row_stride < d || row_stride % 8 || head_stride % 8 || n_keys * row_stride * 2 >= (1ll << 32))
    return fail(RF_EINVAL_SHAPE, "rf_attend_causal: strides (ldq %lld, ldo %lld, row %lld) or %lld keys",
                (long long)ldq, (long long)ldo, (long long)row_stride, (long long)n_keys);
  if (!aligned16(q) || !aligned16(kbuf) || !aligned16(vbuf) || (workspace && !aligned16(workspace)) ||
      (reinterpret_cast<uintptr_t>(out) & 7u))
    return fail(RF_EINVAL_SHAPE, "rf_attend_causal: alignment");
  if (!(scale > 0.f) || !(scale < 1e30f)) return fail(RF_EINVAL_ARG, "rf_attend_causal: scale %g (must be positive)",
                                                      static_cast<double>(scale));
  if (nq == 0) return RF_OK;
  const int64_t T = key_tiles(n_keys, d);
  Splits sp = workspace ? causal_plan(nq, hq, hkv, d, n_keys, qpos != nullptr, slot0) : Splits{1, static_cast<int>(T)};
  while (sp.ns > 1 && ws_bytes < part_bytes(nq, hq, hkv, d, sp.ns)) {     // what the workspace holds
    --sp.ns;
    sp.W = static_cast<int>((T + sp.ns - 1) / sp.ns);
  }
  if (sp.ns == 1) sp.W = static_cast<int>(T);
  const int ns = sp.ns;
  CausalArgs a{q, ldq, static_cast<int>(nq), qpos, slot0, kbuf, head_stride, row_stride, n_keys, vbuf, hq, hkv,
               scale * 1.4426950408889634f, out, ldo, static_cast<float*>(workspace), sp.W, hpb_of(hq, hkv, d)};
  const dim3 grid(static_cast<unsigned>(query_blocks(nq, hq, hkv, d)), static_cast<unsigned>(head_blocks(hq, hkv, d)),
                  static_cast<unsigned>(ns));
  if (d == 256) hipLaunchKernelGGL(k_attend_causal<256>, grid, dim3(Cfg<256>::NTHR), 0, stream, a);
  else if (d == 128) hipLaunchKernelGGL(k_attend_causal<128>, grid, dim3(Cfg<128>::NTHR), 0, stream, a);
  else hipLaunchKernelGGL(k_attend_causal<64>, grid, dim3(Cfg<64>::NTHR), 0, stream, a);
  if (ns > 1) {
    const int st = check_launch("rf_attend_causal");
    if (st != RF_OK) return st;
    const dim3 g2(grid.x, grid.y, static_cast<unsigned>(qrows_of(d) * d / 4 / 256));
    if (d == 256) hipLaunchKernelGGL(k_causal_combine<256>, g2, dim3(256), 0, stream, a, ns);
    else if (d == 128) hipLaunchKernelGGL(k_causal_combine<128>, g2, dim3(256), 0, stream, a, ns);
    else hipLaunchKernelGGL(k_causal_combine<64>, g2, dim3(256), 0, stream, a, ns);
  }
  return check_launch("rf_attend_causal");
}
