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
