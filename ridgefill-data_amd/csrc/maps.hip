// Map formats: the int8 map layout with per-row group scales of the public RidgeFill release
// ("i8_row128": code/c5/convert.py:4-23, dequant :91-97), expanded to the bf16 maps the fill GEMM reads.
// out[i][j] = bf16(float(codes[i][j]) * float(scale[i][j / group])): the product of an 8-bit integer and
// a bf16 (8-bit mantissa) is exact in fp32, so the cast to bf16 (round to nearest even) is the only
// rounding, as in the reference's codes.to(float32) * scale.to(float32) followed by .to(bfloat16).
// HBM-bound: one pass, 16 codes per thread and iteration (one 16-byte load, two 16-byte stores).
#include <algorithm>

#include "rf_common.h"

namespace rf {
namespace {

__global__ __launch_bounds__(256) void k_dequant_i8(const int8_t* __restrict__ codes, int64_t ldc,
                                                    const uint16_t* __restrict__ scale, int64_t lds, int64_t rows,
                                                    int64_t width, int group, uint16_t* __restrict__ out,
                                                    int64_t ldo) {
  const int64_t cpr = width / 16, total = rows * cpr;
  for (int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t row = idx / cpr, c = idx - row * cpr;
    const uint4 q = *reinterpret_cast<const uint4*>(codes + row * ldc + c * 16);
    const float s = bf2f(scale[row * lds + (c * 16) / group]);   // one group: group % 16 == 0
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
    uint32_t o[8];
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      const uint32_t word = w[p >> 1];
      const int sh = 16 * (p & 1);
      const float a = static_cast<float>(static_cast<int8_t>((word >> sh) & 0xffu)) * s;
      const float b = static_cast<float>(static_cast<int8_t>((word >> (sh + 8)) & 0xffu)) * s;
      o[p] = bf16_pair(a, b);
    }
    uint4* dst = reinterpret_cast<uint4*>(out + row * ldo + c * 16);
    dst[0] = make_uint4(o[0], o[1], o[2], o[3]);
    dst[1] = make_uint4(o[4], o[5], o[6], o[7]);
  }
}

// llama.cpp GGUF map tensors (ggml types) expanded to bf16 rows: F32 (0), F16 (1), Q8_0 (8: blocks of 32
// values, an fp16 scale then 32 int8 codes, 34 bytes) and BF16 (30, copied). F16 and Q8_0 values are
// exact in fp32 (an fp16 scale times an 8-bit integer needs at most 19 significant bits), so the cast to
// bf16 (round to nearest even) is the only rounding, as for ggml's own fp32 dequantisation followed by a
// bf16 cast. Q8_0: one thread per 34-byte block (2-byte loads: blocks are only 2-byte aligned), four
// 16-byte stores; the others: 8 values per thread, 16-byte stores.
__device__ __forceinline__ float half_to_float(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

__global__ __launch_bounds__(256) void k_dequant_q8_0(const uint8_t* __restrict__ src, int64_t lds, int64_t rows,
                                                      int64_t width, uint16_t* __restrict__ out, int64_t ldo) {
  const int64_t bpr = width / 32, total = rows * bpr;
  for (int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t row = idx / bpr, b = idx - row * bpr;
    const uint16_t* blk = reinterpret_cast<const uint16_t*>(src + row * lds + b * 34);
    const float d = half_to_float(blk[0]);
    uint32_t o[16];
#pragma unroll
    for (int p = 0; p < 16; ++p) {
      const uint16_t two = blk[1 + p];
      o[p] = bf16_pair(static_cast<float>(static_cast<int8_t>(two & 0xffu)) * d,
                       static_cast<float>(static_cast<int8_t>(two >> 8)) * d);
    }
    uint4* dst = reinterpret_cast<uint4*>(out + row * ldo + b * 32);
#pragma unroll
    for (int q = 0; q < 4; ++q) dst[q] = make_uint4(o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3]);
  }
}

template <int TYPE>
__global__ __launch_bounds__(256) void k_convert_rows(const uint8_t* __restrict__ src, int64_t lds, int64_t rows,
                                                      int64_t width, uint16_t* __restrict__ out, int64_t ldo) {
  const int64_t cpr = width / 8, total = rows * cpr;
  for (int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t row = idx / cpr, c = idx - row * cpr;
    uint4 o;
    if constexpr (TYPE == 0) {                          // F32
      const uint4* s = reinterpret_cast<const uint4*>(src + row * lds + c * 32);
      const uint4 a = s[0], b = s[1];
      o = make_uint4(bf16_pair(__uint_as_float(a.x), __uint_as_float(a.y)),
                     bf16_pair(__uint_as_float(a.z), __uint_as_float(a.w)),
                     bf16_pair(__uint_as_float(b.x), __uint_as_float(b.y)),
                     bf16_pair(__uint_as_float(b.z), __uint_as_float(b.w)));
    } else if constexpr (TYPE == 1) {                   // F16
      const uint4 a = *reinterpret_cast<const uint4*>(src + row * lds + c * 16);
      const uint32_t w[4] = {a.x, a.y, a.z, a.w};
      uint32_t r[4];
#pragma unroll
      for (int p = 0; p < 4; ++p)
        r[p] = bf16_pair(half_to_float(static_cast<uint16_t>(w[p] & 0xffffu)),
                         half_to_float(static_cast<uint16_t>(w[p] >> 16)));
      o = make_uint4(r[0], r[1], r[2], r[3]);
    } else {                                            // BF16
      o = *reinterpret_cast<const uint4*>(src + row * lds + c * 16);
    }
    *reinterpret_cast<uint4*>(out + row * ldo + c * 8) = o;
  }
}

}  // namespace
}  // namespace rf

using namespace rf;

extern "C" int rf_dequant_i8_rows(const int8_t* codes, int64_t ld_codes, const uint16_t* scale, int64_t ld_scale,
                                  int64_t rows, int64_t width, int group, uint16_t* out, int64_t ld_out,
                                  hipStream_t stream) {
  if (!codes || !scale || !out) return fail(RF_EINVAL_ARG, "rf_dequant_i8_rows: null pointer");
  if (rows < 0 || width <= 0 || group <= 0 || group % 16 || width % group || ld_codes < width || ld_codes % 16 ||
      ld_out < width || ld_out % 8 || ld_scale < width / group)
    return fail(RF_EINVAL_SHAPE,
                "rf_dequant_i8_rows: rows %lld, width %lld, group %d (a multiple of 16 dividing width), strides "
                "codes %lld (>= width, multiple of 16), scale %lld, out %lld (>= width, multiple of 8)",
                (long long)rows, (long long)width, group, (long long)ld_codes, (long long)ld_scale, (long long)ld_out);
  if (!aligned16(codes) || !aligned16(out) || (reinterpret_cast<uintptr_t>(scale) & 1u))
    return fail(RF_EINVAL_SHAPE, "rf_dequant_i8_rows: codes and out must be 16-byte aligned, scale 2-byte");
  if (rows == 0) return RF_OK;
  const int64_t chunks = rows * (width / 16);
  const unsigned blocks = static_cast<unsigned>(std::min<int64_t>((chunks + 255) / 256, 8192));
  hipLaunchKernelGGL(k_dequant_i8, dim3(blocks), dim3(256), 0, stream, codes, ld_codes, scale, ld_scale, rows, width,
                     group, out, ld_out);
  return check_launch("rf_dequant_i8_rows");
}

extern "C" int rf_dequant_gguf_rows(int ggml_type, const void* src, int64_t ld_src, int64_t rows, int64_t width,
                                    uint16_t* out, int64_t ld_out, hipStream_t stream) {
  if (!src || !out) return fail(RF_EINVAL_ARG, "rf_dequant_gguf_rows: null pointer");
  if (ggml_type != 0 && ggml_type != 1 && ggml_type != 8 && ggml_type != 30)
    return fail(RF_EUNSUPPORTED, "rf_dequant_gguf_rows: ggml type %d (F32 = 0, F16 = 1, Q8_0 = 8, BF16 = 30)",
                ggml_type);
  const bool q8 = ggml_type == 8;
  const int64_t unit = q8 ? 32 : 8;
  const int64_t row_bytes = q8 ? width / 32 * 34 : width * (ggml_type == 0 ? 4 : 2);
  if (rows < 0 || width <= 0 || width % unit || ld_src < row_bytes || ld_src % (q8 ? 2 : 16) || ld_out < width ||
      ld_out % 8)
    return fail(RF_EINVAL_SHAPE, "rf_dequant_gguf_rows: rows %lld, width %lld (multiple of %lld), row bytes %lld "
                "(>= %lld, multiple of %d), ld_out %lld (>= width, multiple of 8)", (long long)rows, (long long)width,
                (long long)unit, (long long)ld_src, (long long)row_bytes, q8 ? 2 : 16, (long long)ld_out);
  if ((reinterpret_cast<uintptr_t>(src) & (q8 ? 1u : 15u)) || !aligned16(out))
    return fail(RF_EINVAL_SHAPE, "rf_dequant_gguf_rows: src must be %d-byte aligned, out 16-byte", q8 ? 2 : 16);
  if (rows == 0) return RF_OK;
  const uint8_t* s = static_cast<const uint8_t*>(src);
  const unsigned blocks = static_cast<unsigned>(std::min<int64_t>((rows * (width / unit) + 255) / 256, 8192));
  switch (ggml_type) {
    case 8: hipLaunchKernelGGL(k_dequant_q8_0, dim3(blocks), dim3(256), 0, stream, s, ld_src, rows, width, out, ld_out);
      break;
    case 0: hipLaunchKernelGGL(k_convert_rows<0>, dim3(blocks), dim3(256), 0, stream, s, ld_src, rows, width, out,
                               ld_out);
      break;
    case 1: hipLaunchKernelGGL(k_convert_rows<1>, dim3(blocks), dim3(256), 0, stream, s, ld_src, rows, width, out,
                               ld_out);
      break;
    default: hipLaunchKernelGGL(k_convert_rows<30>, dim3(blocks), dim3(256), 0, stream, s, ld_src, rows, width, out,
                                ld_out);
  }
  return check_launch("rf_dequant_gguf_rows");
}
