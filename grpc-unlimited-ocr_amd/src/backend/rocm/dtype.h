#pragma once

// bf16 on the host: the top half of an IEEE-754 binary32 in a uint16_t.
// The conversion from fp32 rounds to nearest even and keeps NaN quiet, the
// rule the reference fixes for every bf16 value it stores
// (src/tensor/dtype.h:32-46) and that the gfx950 kernels apply on store.

#include <bit>
#include <cstdint>

namespace uocr::rocm {

inline float bf16_to_f32(std::uint16_t bits) { return std::bit_cast<float>(static_cast<std::uint32_t>(bits) << 16); }

inline std::uint16_t f32_to_bf16(float value) {
  const auto u = std::bit_cast<std::uint32_t>(value);
  const bool is_nan = (u & 0x7fffffffU) > 0x7f800000U;
  if (is_nan) return static_cast<std::uint16_t>((u >> 16) | 0x0040U);  // quiet bit set
  const std::uint32_t lsb = (u >> 16) & 1U;                             // ties go to the even neighbour
  return static_cast<std::uint16_t>((u + 0x7fffU + lsb) >> 16);
}

}  // namespace uocr::rocm
