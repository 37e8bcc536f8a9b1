// Shared device/host helpers for the gfx950 kernels of the quantized
// DiT-block path. Everything here is written for CDNA4 (wave64, MFMA, LDS);
// there is no CUDA or multi-target code.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

namespace xmh3 {

// dtype codes of the reference's op boundary
// (CK/backends/eager/quantization.py:34-42): 0 fp32, 1 fp16, 2 bf16.
enum DtypeCode : int { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2 };
// input-activation codes (CK/backends/_activations.py:19-24).
enum ActCode : int { ACT_NONE = 0, ACT_GELU_TANH = 1, ACT_SWIGLU = 2 };

// status codes returned by every extern "C" entry point
enum Status : int { XMH3_OK = 0, XMH3_EINVAL = 1, XMH3_EHIP = 2, XMH3_EUNSUPPORTED = 3 };

// ---------------------------------------------------------------------------
// scalar conversions (bit exact; fp32 -> bf16 rounds to nearest even)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// fp32 -> bf16, round to nearest even, on gfx950's v_cvt_pk_bf16_f32 (NaN stays
// NaN; finite values round exactly as the integer formula
// (u + 0x7fff + ((u >> 16) & 1)) >> 16 does).
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const bf16x2_t v = __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t);
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ uint32_t f32_to_bf16(float f) { return pack_bf16x2(f, 0.0f) & 0xffffu; }

__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// fp16 <-> fp32 in integer/fp32 arithmetic only, so subnormal fp16 values are
// rounded (nearest even) and widened exactly whatever the wave's f16 denormal
// mode is. Subnormal results come from one fp32 add: |f| + 0.5 places the fp16
// subnormal ulp (2^-24) at the last fp32 mantissa bit.
__device__ __forceinline__ float f16_to_f32(uint32_t h) {
  // branch-free (selects only), usable inside fully unrolled element loops
  const uint32_t s = (h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  const float sub = __uint_as_float(s | __float_as_uint((float)m * 5.9604644775390625e-08f));  // m * 2^-24
  const uint32_t infnan = s | 0x7f800000u | (m << 13);
  const uint32_t nrm = s | ((e + 112u) << 23) | (m << 13);
  return e == 0 ? sub : __uint_as_float(e == 31 ? infnan : nrm);
}
__device__ __forceinline__ uint32_t f32_to_f16(float ff) {
  // branch-free: all three cases are computed and selected, so the function
  // can sit inside fully unrolled epilogue loops
  uint32_t f = __float_as_uint(ff);
  const uint32_t sign = f & 0x80000000u;
  f ^= sign;
  const uint32_t big = (f > (255u << 23)) ? 0x7e00u : 0x7c00u;                // >= 65536, inf, nan
  const uint32_t sub = __float_as_uint(__uint_as_float(f) + 0.5f) - 0x3f000000u;  // < 2^-14
  const uint32_t nrm = (f + 0xc8000fffu + ((f >> 13) & 1u)) >> 13;             // rebias + RNE
  const uint32_t o = (f >= (143u << 23)) ? big : ((f < (113u << 23)) ? sub : nrm);
  return o | (sign >> 16);
}

// Element-type traits: storage type, fp32 view and rounding back to T.
struct BF16T {
  using storage = uint16_t;
  static constexpr int code = DT_BF16;
  __device__ static float load(uint32_t b) { return bf16_to_f32(b); }
  __device__ static uint32_t store(float f) { return f32_to_bf16(f); }
  // bf16(f) in the high half over a zero low half is the rounded value as an
  // fp32 bit pattern: one v_cvt_pk_bf16_f32 with a zero first operand
  __device__ static float round(float f) { return __uint_as_float(pack_bf16x2(0.0f, f)); }
  __device__ static void round2(float& a, float& b) {
    a = round(a);
    b = round(b);
  }
  __device__ static uint32_t store2(float a, float b) { return pack_bf16x2(a, b); }
  __device__ static float tiny() { return 1.17549435e-38f; }
};
struct F16T {
  using storage = uint16_t;
  static constexpr int code = DT_F16;
  __device__ static float load(uint32_t b) { return f16_to_f32(b); }
  __device__ static uint32_t store(float f) { return f32_to_f16(f); }
  __device__ static float round(float f) { return f16_to_f32(f32_to_f16(f)); }
  __device__ static void round2(float& a, float& b) { a = round(a); b = round(b); }
  __device__ static uint32_t store2(float a, float b) { return f32_to_f16(a) | (f32_to_f16(b) << 16); }
  __device__ static float tiny() { return 6.103515625e-05f; }
};
struct F32T {
  using storage = float;
  static constexpr int code = DT_F32;
  __device__ static float load(float f) { return f; }
  __device__ static float store(float f) { return f; }
  __device__ static float round(float f) { return f; }
  __device__ static void round2(float&, float&) {}
  __device__ static float tiny() { return 1.17549435e-38f; }
};

// ---------------------------------------------------------------------------
// wave64 reductions
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// GELU with the tanh approximation, 0.5*h*(1+tanh(u)),
// u = sqrt(2/pi)*(h + 0.044715*h^3), evaluated as h / (1 + exp(-2u)) (the
// same function; no cancellation as tanh(u) -> -1). The exponent
// -2u*log2(e) is h * (c1 + c2*h^2) with c1 = -2*log2(e)*sqrt(2/pi) and
// c2 = 0.044715*c1 (constants from the published formula, products formed in
// double): three VALU operations before the exp.
__device__ __forceinline__ float gelu_tanh_f32(float h) {
  const float c1 = -2.3022082f;    // -2 * log2(e) * sqrt(2/pi)
  const float c2 = -0.10294324f;   // 0.044715 * c1
  const float a = h * __builtin_fmaf(c2, h * h, c1);
  const float e = __builtin_amdgcn_exp2f(a);
  return h * __builtin_amdgcn_rcpf(1.0f + e);
}

// Stochastic rounding noise of the reference's CUDA quantizers
// (CK/backends/cuda/ops/int8_linear.cu:79-91): element idx (row * K + col)
// and seed give u = (h >> 8) * 2^-24 in [0, 1), h the 32-bit PCG-RXS-M-XS
// output hash of lo32(idx + seed) ^ hi32(idx + seed), rounded to T. A code
// is then floor(T(v + u)) for the scaled value v.
__device__ __forceinline__ uint32_t pcg_output_hash(uint32_t x) {
  const uint32_t state = x * 747796405u + 2891336453u;
  const uint32_t word = ((state >> ((state >> 28u) + 4u)) ^ state) * 277803737u;
  return (word >> 22u) ^ word;
}

template <typename T>
__device__ __forceinline__ float sr_noise(uint64_t idx, uint64_t seed) {
  const uint64_t key = idx + seed;
  const uint32_t h = pcg_output_hash((uint32_t)key ^ (uint32_t)(key >> 32));
  return T::round((float)(h >> 8) * 0x1.0p-24f);
}

// ---------------------------------------------------------------------------
// host-side error plumbing (no C++ exception crosses the C ABI)
// ---------------------------------------------------------------------------
void set_last_error(const std::string& msg);
int fail(int code, const std::string& msg);
int check_launch(const char* what);

}  // namespace xmh3

#define XMH3_REQUIRE(cond, msg)                                    \
  do {                                                             \
    if (!(cond)) return ::xmh3::fail(::xmh3::XMH3_EINVAL, (msg));  \
  } while (0)
