// Per-token int8 quantisation with an input activation and the ConvRot
// online rotation (gfx950): the quantizer at the boundary of the reference's
// rotated linears.
//
// Semantics follow the reference's eager path (CK = backends/turbo/vendor/
// comfy_kitchen):
//   a = act(x)        CK/backends/_activations.py:40-53, in x's dtype:
//                     gelu_tanh -> T(gelu(x)); swiglu on [gate | up] rows ->
//                     T(T(silu(gate)) * up), the row halving in width
//   r = T(a_g @ H)    per group g of 256 columns, H the normalised regular
//                     Hadamard matrix H4 (x) H4 (x) H4 (x) H4 / 16
//                     (CK/tensor/int8_utils.py:11-74,
//                     CK/backends/eager/quantization.py:1012-1017)
//   (q, s) = quantize_int8_rowwise(r)   as in quant.hip
// The rotation is evaluated in fp32 as four radix-4 stages (one per base-4
// digit of the column inside its group; H4 is symmetric and
// H4[i][j] = -1 exactly when i + j == 3, so a stage output is
// sum(a_0..a_3) - 2 * a_(3-j)), then rounded to T once: the reference's fp32
// accumulation order inside its bf16 matmul is a library detail, so the last
// bit of r may differ (the parity bar for this op is the tolerance).
//
// Layout: one wave per row. 16 lanes per 256-column group, lane l holding the
// 16 consecutive columns 16*(l%16) .. +15 of group 4*it + l/16 in iteration it
// (digits 0 and 1 of the column inside the lane, digit 2 across the lanes of a
// quad, digit 3 across the four quads of a 16-lane row). The rotated row stays
// in registers (packed 16-bit) until its |max| is known. With group size 0
// the same kernel quantizes the swiglu activation without a rotation.
#include "common.hpp"

#include <type_traits>

namespace xmh3 {

// the sum of the four values held by the lanes that differ in bits m1 and m2
// (m1 | m2) of the lane index, and the value of the lane with both bits
// flipped
__device__ __forceinline__ void quad_terms(float a, int m1, int m2, float& sum, float& mirror) {
  const float t = a + __shfl_xor(a, m1, 64);
  sum = t + __shfl_xor(t, m2, 64);
  mirror = __shfl_xor(a, m1 | m2, 64);
}

// in-lane radix-4 stage over 4 values: b_j = (a0 + a1 + a2 + a3) - 2 a_(3-j)
__device__ __forceinline__ void h4_inlane(float& a0, float& a1, float& a2, float& a3) {
  const float s = (a0 + a1) + (a2 + a3);
  const float b0 = s - 2.0f * a3, b1 = s - 2.0f * a2, b2 = s - 2.0f * a1, b3 = s - 2.0f * a0;
  a0 = b0; a1 = b1; a2 = b2; a3 = b3;
}

template <typename T>
__device__ __forceinline__ float cr_act_gelu(float x) {
  return T::round(gelu_tanh_f32(x));
}

// silu(g) = g / (1 + exp(-g)), rounded to T, times up, rounded to T
template <typename T>
__device__ __forceinline__ float cr_act_swiglu(float g, float u) {
  const float e = __builtin_amdgcn_exp2f(g * -1.4426950408889634f);
  const float s = T::round(g * __builtin_amdgcn_rcpf(1.0f + e));
  return T::round(s * u);
}

template <typename T, int ACT, bool ROT, int NIT>
__global__ __launch_bounds__(256) void convrot_quant_rows_kernel(
    const typename T::storage* __restrict__ x, int64_t ldx, int64_t M, int K,
    int8_t* __restrict__ q, int64_t ldq, float* __restrict__ scale) {
  using S = typename T::storage;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  const S* xr = x + row * ldx;
  const int groups = K >> 8;
  const int g16 = lane & 15;
  uint32_t keep[NIT][8];                  // rotated values, T bits packed in pairs
  float amax = 0.0f;
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const int group = it * 4 + (lane >> 4);
    const bool live = group < groups;
    const int c = (live ? group : 0) * 256 + g16 * 16;
    // 16 values = two 16-byte loads (and two more for the up half)
    uint32_t raw[8], up[8];
    {
      const uint4 r0 = *reinterpret_cast<const uint4*>(xr + c), r1 = *reinterpret_cast<const uint4*>(xr + c + 8);
      raw[0] = r0.x; raw[1] = r0.y; raw[2] = r0.z; raw[3] = r0.w;
      raw[4] = r1.x; raw[5] = r1.y; raw[6] = r1.z; raw[7] = r1.w;
      if constexpr (ACT == ACT_SWIGLU) {
        const uint4 u0 = *reinterpret_cast<const uint4*>(xr + K + c);
        const uint4 u1 = *reinterpret_cast<const uint4*>(xr + K + c + 8);
        up[0] = u0.x; up[1] = u0.y; up[2] = u0.z; up[3] = u0.w;
        up[4] = u1.x; up[5] = u1.y; up[6] = u1.z; up[7] = u1.w;
      }
    }
    float v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float xi = T::load((raw[i >> 1] >> (16 * (i & 1))) & 0xffffu);
      if constexpr (ACT == ACT_SWIGLU) v[i] = cr_act_swiglu<T>(xi, T::load((up[i >> 1] >> (16 * (i & 1))) & 0xffffu));
      else if constexpr (ACT == ACT_GELU_TANH) v[i] = cr_act_gelu<T>(xi);
      else v[i] = xi;
    }
    if constexpr (ROT) {
      // digit 0 (i & 3) and digit 1 (i >> 2), inside the lane
#pragma unroll
      for (int d1 = 0; d1 < 4; ++d1) h4_inlane(v[4 * d1], v[4 * d1 + 1], v[4 * d1 + 2], v[4 * d1 + 3]);
#pragma unroll
      for (int d0 = 0; d0 < 4; ++d0) h4_inlane(v[d0], v[4 + d0], v[8 + d0], v[12 + d0]);
      // digit 2 (lane bits 0-1) and digit 3 (lane bits 2-3), across lanes
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float s, m;
        quad_terms(v[i], 1, 2, s, m);
        v[i] = s - 2.0f * m;
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float s, m;
        quad_terms(v[i], 4, 8, s, m);
        v[i] = T::round((s - 2.0f * m) * 0.0625f);   // H / 16, then the matmul's output dtype
      }
    }
#pragma unroll
    for (int i = 0; i < 16; i += 2) {
      if (live) amax = fmaxf(amax, fmaxf(fabsf(v[i]), fabsf(v[i + 1])));
      keep[it][i >> 1] = (T::store(v[i]) & 0xffffu) | (T::store(v[i + 1]) << 16);
    }
  }
  amax = wave_max(amax);
  const float s = fmaxf(amax / 127.0f, 1e-30f);
  float sT = T::round(s);
  if (sT == 0.0f) sT = T::tiny();
  const float inv = 1.0f / sT;
  int8_t* qr = q + row * ldq;
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const int group = it * 4 + (lane >> 4);
    if (group >= groups) continue;
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      uint32_t word = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int i = 4 * k + b;
        const uint32_t bits = (keep[it][i >> 1] >> (16 * (i & 1))) & 0xffffu;
        const float r = T::load(bits);
        float code;
        if constexpr (std::is_same<T, BF16T>::value) code = rintf(T::round(r * inv));   // see quant.hip
        else code = rintf(T::round(r / sT));
        code = fminf(fmaxf(code, -128.0f), 127.0f);
        word |= (uint32_t)((int)code & 0xff) << (8 * b);
      }
      w[k] = word;
    }
    *reinterpret_cast<uint4*>(qr + group * 256 + g16 * 16) = make_uint4(w[0], w[1], w[2], w[3]);
  }
  if (lane == 0) scale[row] = s;
}

template <typename T, int ACT, bool ROT>
static int launch_convrot_T(const void* x, int64_t ldx, int64_t M, int K, int8_t* q, int64_t ldq, float* scale,
                            hipStream_t st) {
  using S = typename T::storage;
  const int nit = (K / 256 + 3) / 4;
  dim3 grid((unsigned)((M + 3) / 4));
#define XMH3_CR(N)                                                                                   \
  if (nit <= N) {                                                                                    \
    hipLaunchKernelGGL((convrot_quant_rows_kernel<T, ACT, ROT, N>), grid, dim3(256), 0, st,          \
                       static_cast<const S*>(x), ldx, M, K, q, ldq, scale);                          \
    return check_launch("convrot_quant_rows_kernel");                                                \
  }
  XMH3_CR(1) XMH3_CR(2) XMH3_CR(4) XMH3_CR(8) XMH3_CR(12) XMH3_CR(16)
#undef XMH3_CR
  return fail(XMH3_EUNSUPPORTED, "quantize_int8_rowwise_convrot: activated row wider than 16384");
}

int quantize_rows_convrot(const void* x, int x_dtype, int input_act, int64_t M, int64_t K, int64_t ldx,
                          int group_size, int8_t* q, int64_t ldq, float* scale, hipStream_t st) {
  XMH3_REQUIRE(M >= 0 && K >= 0, "quantize_int8_rowwise_convrot: negative size");
  XMH3_REQUIRE(group_size == 256 || group_size == 0,
               "quantize_int8_rowwise_convrot: convrot_groupsize must be 256 (or 0: no rotation)");
  XMH3_REQUIRE(input_act == ACT_NONE || input_act == ACT_GELU_TANH || input_act == ACT_SWIGLU,
               "quantize_int8_rowwise_convrot: unsupported input activation");
  if (M == 0 || K == 0) return XMH3_OK;
  XMH3_REQUIRE(x && q && scale, "quantize_int8_rowwise_convrot: null pointer");
  XMH3_REQUIRE(K % 256 == 0 && K <= 16384, "quantize_int8_rowwise_convrot: K must be a multiple of 256, <= 16384");
  const int64_t in_width = input_act == ACT_SWIGLU ? 2 * K : K;
  XMH3_REQUIRE(ldx >= in_width && ldx % 8 == 0 && (uintptr_t)x % 16 == 0 && ldq >= K && ldq % 16 == 0 &&
                   (uintptr_t)q % 16 == 0,
               "quantize_int8_rowwise_convrot: rows must be 16-byte aligned");
  const int k = (int)K;
#define XMH3_CRA(TT)                                                                                    \
  {                                                                                                     \
    if (group_size == 0) {                                                                              \
      if (input_act == ACT_SWIGLU) return launch_convrot_T<TT, ACT_SWIGLU, false>(x, ldx, M, k, q, ldq, scale, st); \
      return fail(XMH3_EUNSUPPORTED, "quantize_int8_rowwise_convrot: without rotation only swiglu is routed here"); \
    }                                                                                                   \
    if (input_act == ACT_SWIGLU) return launch_convrot_T<TT, ACT_SWIGLU, true>(x, ldx, M, k, q, ldq, scale, st); \
    if (input_act == ACT_GELU_TANH)                                                                     \
      return launch_convrot_T<TT, ACT_GELU_TANH, true>(x, ldx, M, k, q, ldq, scale, st);                \
    return launch_convrot_T<TT, ACT_NONE, true>(x, ldx, M, k, q, ldq, scale, st);                       \
  }
  if (x_dtype == DT_BF16) XMH3_CRA(BF16T)
  if (x_dtype == DT_F16) XMH3_CRA(F16T)
#undef XMH3_CRA
  return fail(XMH3_EUNSUPPORTED, "quantize_int8_rowwise_convrot: dtype must be bf16 or fp16");
}

}  // namespace xmh3

extern "C" int xmh3_quantize_int8_rowwise_convrot(const void* x, int x_dtype, int input_act, int64_t M,
                                                  int64_t K, int64_t ldx, int group_size, int8_t* q,
                                                  float* scale, hipStream_t stream) {
  return xmh3::quantize_rows_convrot(x, x_dtype, input_act, M, K, ldx, group_size, q, K, scale, stream);
}
