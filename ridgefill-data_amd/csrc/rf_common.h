// Shared helpers of librfill: status codes, the thread-local error text, bf16 conversions and the
// per-row sum-of-squares partial used by the fused RMSNorm.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/rfill.h"

namespace rf {

// Error text of the last failing call on this host thread (rf_last_error()).
int fail(int code, const char* fmt, ...);
int check_launch(const char* what);

// Columns covered by one row sum-of-squares partial (the RMSNorm statistics are kept as
// [rows, H / SSQ_COLS] fp32 partials so that producers write them without atomics).
constexpr int SSQ_COLS = 256;

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Logical tile of a hardware block. Blocks are dealt round-robin over the 8 XCDs (block b runs on
// XCD b % 8); this gives every XCD a contiguous run of logical tiles.
__device__ __forceinline__ int xcd_tile(int bid, int nb) {
  const int q = nb >> 3, r = nb & 7, x = bid & 7, i = bid >> 3;
  return (x < r) ? x * (q + 1) + i : r * (q + 1) + (x - r) * q + i;
}

__device__ __forceinline__ float bf2f(uint16_t h) { return __uint_as_float(static_cast<uint32_t>(h) << 16); }

// fp32 -> bf16, round to nearest even (the rounding torch's .to(torch.bfloat16) performs).
__device__ __forceinline__ uint16_t f2bf(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t rounded = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  const uint32_t quiet_nan = (u >> 16) | 0x40u;
  return static_cast<uint16_t>((u & 0x7fffffffu) > 0x7f800000u ? quiet_nan : rounded);   // a select, no branch
}

typedef float rf_f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 rf_bf16x2 __attribute__((ext_vector_type(2)));

// Two floats rounded to bf16 (nearest even, as f2bf for every finite value) in one hardware conversion
// (v_cvt_pk_bf16_f32), lo in bits 0-15, hi in bits 16-31. Both halves must carry values: with a half
// the caller discards, the compiler feeds that operand an undefined register and then drops the masking
// of the unused half, so single values go through f2bf.
__device__ __forceinline__ uint32_t bf16_pair(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(rf_f32x2{lo, hi}, rf_bf16x2));
}

__device__ __forceinline__ float bf_lo(uint32_t p) { return __uint_as_float(p << 16); }
__device__ __forceinline__ float bf_hi(uint32_t p) { return __uint_as_float(p & 0xffff0000u); }

typedef uint32_t rf_u32x4 __attribute__((ext_vector_type(4)));

// A 16-byte streaming store (nontemporal: data written once and not re-read by this kernel).
__device__ __forceinline__ void st_stream16(void* p, const uint4& v) {
  __builtin_nontemporal_store(rf_u32x4{v.x, v.y, v.z, v.w}, reinterpret_cast<rf_u32x4*>(p));
}

__device__ __forceinline__ uint32_t pack2(uint16_t lo, uint16_t hi) {
  return static_cast<uint32_t>(lo) | (static_cast<uint32_t>(hi) << 16);
}

__device__ __forceinline__ uint16_t lane_of(const uint4& v, int e) {
  const uint32_t w = (e < 2) ? v.x : (e < 4) ? v.y : (e < 6) ? v.z : v.w;
  return static_cast<uint16_t>((e & 1) ? (w >> 16) : (w & 0xffffu));
}

// Sum of squares of the 8 bf16 values of one 16-byte chunk, in element order.
__device__ __forceinline__ float chunk_ssq(const uint4& v) {
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float f = bf2f(lane_of(v, e));
    s = fmaf(f, f, s);
  }
  return s;
}

// Butterfly sum over the 32 lanes of each half-wave (lane bits 0..4): a fixed order, so every
// producer of a row partial (GEMM epilogue, row_ssq, row_scatter) gives the same bits.
__device__ __forceinline__ float halfwave_sum(float s) {
#pragma unroll
  for (int o = 16; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
  return s;
}

// One wave per row. The sum of squares of each 256-column group is formed in the order the GEMM
// epilogue forms it, so every producer of a row partial gives the same bits: four partials, one per
// (w, h) in {0, 1}^2, each a sequential fma chain over the 64 columns w*128 + n*32 + 8g + 4h + e
// (n, g, e = 0..3 in that order); then the two h partials of each w are added, then the two w sums.
// Lane L takes group L / 4 (16 groups per pass) and partial q = L % 4 (w = q / 2, h = q % 2).
// piece(o) returns the row's 4 bf16 values at column offset o (8 bytes); it may also store them
// (the scatter's copy, the residual add's sum).
template <class F>
__device__ __forceinline__ void row_partials(F piece, float* ssq_row, int nparts, int lane) {
  const int q = lane & 3, off_q = (q >> 1) * 128 + (q & 1) * 4;
  for (int p0 = 0; p0 < nparts; p0 += 16) {
    const int part = p0 + (lane >> 2);
    const bool ok = part < nparts;
    float s = 0.f;
    if (ok) {
      const int64_t base = static_cast<int64_t>(part) * SSQ_COLS + off_q;
#pragma unroll
      for (int n = 0; n < 4; ++n)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const uint2 v = piece(base + n * 32 + 8 * g);
          const float f0 = bf2f(v.x & 0xffffu), f1 = bf2f(v.x >> 16), f2 = bf2f(v.y & 0xffffu), f3 = bf2f(v.y >> 16);
          s = fmaf(f0, f0, s);
          s = fmaf(f1, f1, s);
          s = fmaf(f2, f2, s);
          s = fmaf(f3, f3, s);
        }
    }
    s += __shfl_xor(s, 1, 64);
    s += __shfl_xor(s, 2, 64);
    if (ok && q == 0) ssq_row[part] = s;
  }
}

}  // namespace rf
