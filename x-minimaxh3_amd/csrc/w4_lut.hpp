// Grouped int4 -> int8-grid decode helpers shared by the standalone decode
// kernels and the W4A8 GEMM's in-LDS decode.
//
// Rule (CK/backends/eager/w4a8_int8.py:344-363, CK = backends/turbo/vendor/
// comfy_kitchen): byte b holds code[2j] = b & 0xF and code[2j+1] = b >> 4;
// level = code - 8 (or codebook[code]); w8 = clamp(rint(level * s_rel[n, k/G]),
// -127, 127) with s_rel read as fp32 (bf16 s_rel widened exactly).
#pragma once

#include "common.hpp"

namespace xmh3 {

__device__ __forceinline__ int w4_level_code(float level, float srel) {
  float r = rintf(level * srel);
  r = fminf(fmaxf(r, -127.0f), 127.0f);
  return (int)r;
}

template <bool BF16_SREL>
__device__ __forceinline__ float load_srel(const void* p, int64_t i) {
  if constexpr (BF16_SREL) return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
  else return static_cast<const float*>(p)[i];
}

// The 16-entry level table of one (row, group) is four words of int8 (byte
// c % 4 of word c / 4 = the value of code c), each entry clamp(level * s_rel)
// rounded to an integer by the 1.5 * 2^23 addition (clamping first changes
// nothing: the bounds are integers). Four codes are looked up at once: the
// nibbles of two packed bytes are spread to four bytes, v_perm picks each
// byte from the words of codes 0-7 and of codes 8-15, and bit 3 of each code
// selects between them.
__device__ __forceinline__ uint32_t w4_entry4(float l0, float l1, float l2, float l3, float s) {
  const float m = 12582912.0f;   // 1.5 * 2^23
  const uint32_t y0 = __float_as_uint(fminf(fmaxf(l0 * s, -127.0f), 127.0f) + m);
  const uint32_t y1 = __float_as_uint(fminf(fmaxf(l1 * s, -127.0f), 127.0f) + m);
  const uint32_t y2 = __float_as_uint(fminf(fmaxf(l2 * s, -127.0f), 127.0f) + m);
  const uint32_t y3 = __float_as_uint(fminf(fmaxf(l3 * s, -127.0f), 127.0f) + m);
  const uint32_t lo = __builtin_amdgcn_perm(y1, y0, 0x0c0c0400u);
  const uint32_t hi = __builtin_amdgcn_perm(y3, y2, 0x0c0c0400u);
  return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

// 4 int8 outputs from the 4 codes of bytes (sel0, sel1) of w: selector
// 0x01010000 spreads bytes 0-1, 0x03030202 bytes 2-3
template <uint32_t SPREAD>
__device__ __forceinline__ uint32_t w4_lookup4(uint32_t w, const uint32_t (&lut)[4]) {
  const uint32_t t = __builtin_amdgcn_perm(0u, w, SPREAD);            // b0 b0 b1 b1
  const uint32_t codes = (t & 0x000f000fu) | ((t >> 4) & 0x0f000f00u);  // lo hi lo hi nibbles
  const uint32_t sel = codes & 0x07070707u;
  const uint32_t a = __builtin_amdgcn_perm(lut[1], lut[0], sel);       // codes 0-7
  const uint32_t b = __builtin_amdgcn_perm(lut[3], lut[2], sel);       // codes 8-15
  const uint32_t hib = (codes >> 3) & 0x01010101u;
  const uint32_t mask = (hib << 8) - hib;                              // 0xff where code >= 8
  return (b & mask) | (a & ~mask);
}

}  // namespace xmh3
