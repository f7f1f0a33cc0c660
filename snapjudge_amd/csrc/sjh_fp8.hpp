// sjh_fp8.hpp -- OCP e4m3fn rounding shared by the host quantizer and the
// device quantizer (convert.hip), so both produce the same codes bit for bit.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sjh {

// OCP e4m3fn (1 sign, 4 exponent bits with bias 7, 3 mantissa bits; no
// infinity, S.1111.111 is NaN, largest finite 448), round to nearest with
// ties to even; magnitudes of 448 and above (and infinities) saturate to 448.
__host__ __device__ inline uint8_t fp8_e4m3_rne_bits(uint32_t u) {
  const uint8_t sign = static_cast<uint8_t>((u >> 24) & 0x80u);
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return sign | 0x7f;   // NaN
  if (a >= 0x43e00000u) return sign | 0x7e;  // >= 448
  if (a < 0x3c800000u) {
    // below 2^-6: subnormal steps of 2^-9.  |x| * 512 < 8 is exact in
    // float; round it to an integer, ties to even (8 is the smallest normal,
    // code 0x08)
    const float f = __builtin_bit_cast(float, a) * 512.0f;
    uint32_t m = static_cast<uint32_t>(f);
    const float frac = f - static_cast<float>(m);
    if (frac > 0.5f || (frac == 0.5f && (m & 1u))) ++m;
    return sign | static_cast<uint8_t>(m);
  }
  // normal: round the 23-bit mantissa to 3 bits (ties to even); a carry
  // moves into the exponent
  const uint32_t r = a + 0x7ffffu + ((a >> 20) & 1u);
  const uint32_t code = ((((r >> 23) - 120u) << 3) | ((r >> 20) & 7u));
  return sign | static_cast<uint8_t>(code > 0x7eu ? 0x7eu : code);
}

// Scale of one row: max |w| / 448, or 1 for a row that is all zeros (or whose
// maximum is not finite).  NaN entries never raise the maximum.
__host__ __device__ inline float fp8_row_scale(float amax) {
  return (amax > 0.f && amax <= 3.4028234663852886e38f) ? amax / 448.0f : 1.0f;
}

}  // namespace sjh
