// Per-token int8 quantisation with an input activation and the ConvRot
// online rotation (gfx950): the quantizer at the boundary of the reference's
// rotated linears.
//
// Semantics follow the reference's eager path (CK = backends/turbo/vendor/
// comfy_kitchen):
//   a = act(x)        CK/backends/_activations.py:40-53, in x's dtype:
//                     gelu_tanh -> T(gelu(x)); swiglu on [gate | up] rows ->
//                     T(T(silu(gate)) * up), the row halving in width
//   r = T(a_g @ H)    per group g of G = 4^n columns (n = 1..5), H the
//                     normalised regular Hadamard matrix H4 (x) ... (x) H4
//                     (n factors) / 2^n (CK/tensor/int8_utils.py:11-74,
//                     CK/backends/eager/quantization.py:1012-1017)
//   (q, s) = quantize_int8_rowwise(r)   as in quant.hip
// The rotation is evaluated in fp32 as n radix-4 stages (one per base-4
// digit of the column inside its group; H4 is symmetric and
// H4[i][j] = -1 exactly when i + j == 3, so a stage output is
// sum(a_0..a_3) - 2 * a_(3-j)), then rounded to T once. The reference's fp32
// accumulation order inside its bf16 matmul is a library detail; every order
// gives the same fp32 sums when they are exact (a group whose values span at
// most about 8 binades), otherwise the last bit of r may differ. The stages
// sum without the 1/2^n (up to G |a|), so activations beyond 2^117 in
// magnitude overflow here where the normalised matmul would still be finite.
//
// Layout: one block per row, W waves (W * NIT * 4 >= K / 256). In iteration
// it, wave w takes the four 256-column chunks 4 * (it * W + w) .. +3, one
// per 16-lane row of the wave; lane l of a row holds the 16 consecutive
// columns 16 * l .. +15 of its chunk. Base-4 digits 0 and 1 of a column are
// inside the lane, digit 2 in lane bits 0-1, digit 3 in lane bits 2-3,
// digit 4 in lane bits 4-5 (the row): a group of G columns is the run of
// those digits below n. The quad and half-row stages use DPP (quad permutes
// and 16-lane row rotations) and leave each lane with the outputs of the
// lane whose digit is mirrored (3 - d), so lane l stores its codes at slot
// l ^ 3 (n = 3) or l ^ 15 (n >= 4); the row stage (G = 1024) goes through
// lane shuffles and is not mirrored. The rotated row stays in registers
// (fp32 for bf16, packed 16-bit for fp16) until the block knows its |max|.
// With group size 0 the same kernel quantizes the swiglu activation
// without a rotation.
#include "common.hpp"

#include <type_traits>

namespace xmh3 {

// DPP controls (quad_perm and row_ror encodings of the gfx9 DPP word)
constexpr int DPP_QUAD_XOR1 = 0xb1;   // quad_perm:[1,0,3,2]
constexpr int DPP_QUAD_XOR2 = 0x4e;   // quad_perm:[2,3,0,1]
constexpr int DPP_ROW_ROR4 = 0x124;   // row_ror:4
constexpr int DPP_ROW_ROR8 = 0x128;   // row_ror:8

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, true));
}

// radix-4 stage across the four lanes that differ in one base-4 digit of the
// lane index (C1 pairs digit values d and d ^ 2, C2 pairs d and d +- 1).
// With a_d at lane d, H4's row 3 - d is (sum - 2 a_d): lane d returns the
// output of lane 3 - d.
template <int C1, int C2>
__device__ __forceinline__ float h4_lanes_mirrored(float a) {
  const float t = a + dpp_f<C1>(a);
  const float s = t + dpp_f<C2>(t);
  return __builtin_fmaf(a, -2.0f, s);
}

// radix-4 stage across the four 16-lane rows of the wave (digit 4, lane bits
// 4-5): row j gets (sum of the four) - 2 * (row 3 - j) = lane ^ 48
__device__ __forceinline__ float h4_rows(float a) {
  const float t = a + __shfl_xor(a, 16, 64);
  const float s = t + __shfl_xor(t, 32, 64);
  return __builtin_fmaf(__shfl_xor(a, 48, 64), -2.0f, s);
}

// in-lane radix-4 stage over 4 values: b_j = (a0 + a1 + a2 + a3) - 2 a_(3-j)
__device__ __forceinline__ void h4_inlane(float& a0, float& a1, float& a2, float& a3) {
  const float s = (a0 + a1) + (a2 + a3);
  const float b0 = __builtin_fmaf(a3, -2.0f, s), b1 = __builtin_fmaf(a2, -2.0f, s);
  const float b2 = __builtin_fmaf(a1, -2.0f, s), b3 = __builtin_fmaf(a0, -2.0f, s);
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

typedef uint32_t cr_u32x4 __attribute__((ext_vector_type(4)));

// LOGG: radix-4 stages n (group 4^n), 0 = no rotation
template <typename T, int ACT, int LOGG, int NIT>
__global__ __launch_bounds__(512) void convrot_quant_rows_kernel(
    const typename T::storage* __restrict__ x, int64_t ldx, int K, int8_t* __restrict__ q, int64_t ldq,
    float* __restrict__ scale, uint64_t seed) {
  using S = typename T::storage;
  __shared__ float wave_amax[8];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
  const int64_t row = blockIdx.x;
  const S* xr = x + row * ldx;
  const int groups = K >> 8;
  const int g16 = lane & 15;
  // loads of every iteration first: 2 (4 with the up half) x 16 bytes each
  cr_u32x4 raw[NIT][2], up[NIT][2];
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const int group = (it * nwaves + wave) * 4 + (lane >> 4);
    if (group < groups) {
      const int c = group * 256 + g16 * 16;
      raw[it][0] = __builtin_nontemporal_load(reinterpret_cast<const cr_u32x4*>(xr + c));
      raw[it][1] = __builtin_nontemporal_load(reinterpret_cast<const cr_u32x4*>(xr + c + 8));
      if constexpr (ACT == ACT_SWIGLU) {
        up[it][0] = __builtin_nontemporal_load(reinterpret_cast<const cr_u32x4*>(xr + K + c));
        up[it][1] = __builtin_nontemporal_load(reinterpret_cast<const cr_u32x4*>(xr + K + c + 8));
      }
    } else {
      raw[it][0] = raw[it][1] = up[it][0] = up[it][1] = cr_u32x4{0u, 0u, 0u, 0u};
    }
  }
  // bf16: the rotated values stay in fp32 without the final 1/16 (T(16 r) is
  // 16 T(r) exactly, and every code and the scale are taken from products
  // with exact powers of two; a subnormal r has code 0 either way). fp16's
  // narrower exponent range does not allow that: it keeps T(r) packed.
  constexpr bool FOLD = std::is_same<T, BF16T>::value;
  float keepf[FOLD ? NIT : 1][16];
  uint32_t keep[FOLD ? 1 : NIT][8];
  float amax = 0.0f;
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    float v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint32_t w = raw[it][i >> 3][(i >> 1) & 3];
      const float xi = T::load((w >> (16 * (i & 1))) & 0xffffu);
      if constexpr (ACT == ACT_SWIGLU) {
        const uint32_t wu = up[it][i >> 3][(i >> 1) & 3];
        v[i] = cr_act_swiglu<T>(xi, T::load((wu >> (16 * (i & 1))) & 0xffffu));
      } else if constexpr (ACT == ACT_GELU_TANH) {
        v[i] = cr_act_gelu<T>(xi);
      } else {
        v[i] = xi;
      }
    }
    if constexpr (LOGG >= 1) {
      // digit 0 (i & 3) and digit 1 (i >> 2), inside the lane
#pragma unroll
      for (int d1 = 0; d1 < 4; ++d1) h4_inlane(v[4 * d1], v[4 * d1 + 1], v[4 * d1 + 2], v[4 * d1 + 3]);
      if constexpr (LOGG >= 2) {
#pragma unroll
        for (int d0 = 0; d0 < 4; ++d0) h4_inlane(v[d0], v[4 + d0], v[8 + d0], v[12 + d0]);
      }
      // digit 2 (lane bits 0-1), digit 3 (lane bits 2-3), digit 4 (the row)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        if constexpr (LOGG >= 3) v[i] = h4_lanes_mirrored<DPP_QUAD_XOR1, DPP_QUAD_XOR2>(v[i]);
        if constexpr (LOGG >= 4) v[i] = h4_lanes_mirrored<DPP_ROW_ROR8, DPP_ROW_ROR4>(v[i]);
        if constexpr (LOGG >= 5) v[i] = h4_rows(v[i]);
        if constexpr (!FOLD) v[i] *= 1.0f / (float)(1 << LOGG);   // H / 2^n (exact)
      }
    }
    // |max| of the unrounded values (lanes past the last group hold zeros):
    // rounding is monotone, so T(max) is the max of the rounded row
#pragma unroll
    for (int i = 0; i < 16; i += 2) {
      amax = fmaxf(amax, fmaxf(fabsf(v[i]), fabsf(v[i + 1])));
      if constexpr (FOLD) {
        keepf[it][i] = v[i];
        keepf[it][i + 1] = v[i + 1];
      } else {
        keep[it][i >> 1] = T::store2(v[i], v[i + 1]);
      }
    }
  }
  amax = T::round(wave_max(amax));
  if (nwaves > 1) {
    if (lane == 0) wave_amax[wave] = amax;
    __syncthreads();
    amax = wave_amax[0];
    for (int w = 1; w < nwaves; ++w) amax = fmaxf(amax, wave_amax[w]);
  }
  constexpr float unfold = FOLD ? 1.0f / (float)(1 << LOGG) : 1.0f;
  const float s = fmaxf(amax * unfold / 127.0f, 1e-30f);
  float sT = T::round(s);
  if (sT == 0.0f) sT = T::tiny();
  const float inv = 1.0f / sT;
  const float inv_v = inv * unfold;       // applied to the kept values
  int8_t* qr = q + row * ldq;
  constexpr int mirror = (LOGG >= 3 ? 3 : 0) | (LOGG >= 4 ? 12 : 0);
  const int slot = g16 ^ mirror;
  // stochastic rounding (seed != 0): code = floor(T(v + noise)) with the
  // noise of element row * K + col of the [M, K] codes, v the value the
  // nearest path rounds
  const bool sr = seed != 0;
  const uint64_t rbase = (uint64_t)row * (uint64_t)K;
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const int group = (it * nwaves + wave) * 4 + (lane >> 4);
    if (group >= groups) continue;
    const uint64_t cbase = rbase + (uint64_t)(group * 256 + slot * 16);
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if constexpr (FOLD) {
        // rint(T(T(v) * inv)) clamped, as the low byte of c + 1.5 * 2^23 (the
        // fp32 add rounds to the nearest even integer); four bytes by v_perm
        uint32_t y[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          float c = T::round(T::round(keepf[it][4 * k + b]) * inv_v);
          if (sr) c = floorf(T::round(c + sr_noise<T>(cbase + 4 * k + b, seed)));
          y[b] = __float_as_uint(__builtin_amdgcn_fmed3f(c, -128.0f, 127.0f) + 12582912.0f);
        }
        const uint32_t lo = __builtin_amdgcn_perm(y[1], y[0], 0x0c0c0400u);
        const uint32_t hi = __builtin_amdgcn_perm(y[3], y[2], 0x0c0c0400u);
        w[k] = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
      } else {
        uint32_t word = 0;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const int i = 4 * k + b;
          const float r = T::load((keep[it][i >> 1] >> (16 * (i & 1))) & 0xffffu);
          const float v = T::round(r / sT);
          float code = sr ? floorf(T::round(v + sr_noise<T>(cbase + i, seed))) : rintf(v);
          code = fminf(fmaxf(code, -128.0f), 127.0f);
          word |= (uint32_t)((int)code & 0xff) << (8 * b);
        }
        w[k] = word;
      }
    }
    *reinterpret_cast<uint4*>(qr + group * 256 + slot * 16) = make_uint4(w[0], w[1], w[2], w[3]);
  }
  if (threadIdx.x == 0) scale[row] = s;
}

template <typename T, int ACT, int LOGG>
static int launch_convrot_T(const void* x, int64_t ldx, int64_t M, int K, int8_t* q, int64_t ldq, float* scale,
                            uint64_t seed, hipStream_t st) {
  using S = typename T::storage;
  // wave-iterations of four groups each; at most 16 (K <= 16384)
  const int quads = (K / 256 + 3) / 4;
  const int nit = (quads + 7) / 8;
  const int waves = (quads + nit - 1) / nit;
  if (M > 0x7fffffff) return fail(XMH3_EUNSUPPORTED, "quantize_int8_rowwise_convrot: more than 2^31-1 rows");
  const dim3 grid((unsigned)M), block((unsigned)(64 * waves));
  if (nit == 1)
    hipLaunchKernelGGL((convrot_quant_rows_kernel<T, ACT, LOGG, 1>), grid, block, 0, st, static_cast<const S*>(x),
                       ldx, K, q, ldq, scale, seed);
  else
    hipLaunchKernelGGL((convrot_quant_rows_kernel<T, ACT, LOGG, 2>), grid, block, 0, st, static_cast<const S*>(x),
                       ldx, K, q, ldq, scale, seed);
  return check_launch("convrot_quant_rows_kernel");
}

template <typename T, int ACT>
static int launch_convrot_g(const void* x, int64_t ldx, int64_t M, int K, int8_t* q, int64_t ldq, float* scale,
                            int logg, uint64_t seed, hipStream_t st) {
  switch (logg) {
    case 1: return launch_convrot_T<T, ACT, 1>(x, ldx, M, K, q, ldq, scale, seed, st);
    case 2: return launch_convrot_T<T, ACT, 2>(x, ldx, M, K, q, ldq, scale, seed, st);
    case 3: return launch_convrot_T<T, ACT, 3>(x, ldx, M, K, q, ldq, scale, seed, st);
    case 4: return launch_convrot_T<T, ACT, 4>(x, ldx, M, K, q, ldq, scale, seed, st);
    case 5: return launch_convrot_T<T, ACT, 5>(x, ldx, M, K, q, ldq, scale, seed, st);
    default: return fail(XMH3_EINVAL, "quantize_int8_rowwise_convrot: bad group size");
  }
}

template <typename T>
static int launch_convrot_act(const void* x, int64_t ldx, int64_t M, int K, int8_t* q, int64_t ldq, float* scale,
                              int input_act, int logg, uint64_t seed, hipStream_t st) {
  if (logg == 0) return launch_convrot_T<T, ACT_SWIGLU, 0>(x, ldx, M, K, q, ldq, scale, seed, st);
  if (input_act == ACT_SWIGLU)
    return launch_convrot_g<T, ACT_SWIGLU>(x, ldx, M, K, q, ldq, scale, logg, seed, st);
  if (input_act == ACT_GELU_TANH)
    return launch_convrot_g<T, ACT_GELU_TANH>(x, ldx, M, K, q, ldq, scale, logg, seed, st);
  return launch_convrot_g<T, ACT_NONE>(x, ldx, M, K, q, ldq, scale, logg, seed, st);
}

int quantize_rows_convrot(const void* x, int x_dtype, int input_act, int64_t M, int64_t K, int64_t ldx,
                          int group_size, int8_t* q, int64_t ldq, float* scale, uint64_t seed, hipStream_t st) {
  XMH3_REQUIRE(M >= 0 && K >= 0, "quantize_int8_rowwise_convrot: negative size");
  int logg = 0;
  while (logg < 6 && (1 << (2 * logg)) < group_size) ++logg;
  XMH3_REQUIRE(group_size == 0 || (logg >= 1 && logg <= 5 && (1 << (2 * logg)) == group_size),
               "quantize_int8_rowwise_convrot: convrot_groupsize must be 4, 16, 64, 256 or 1024 (or 0: no rotation)");
  XMH3_REQUIRE(input_act == ACT_NONE || input_act == ACT_GELU_TANH || input_act == ACT_SWIGLU,
               "quantize_int8_rowwise_convrot: unsupported input activation");
  if (M == 0 || K == 0) return XMH3_OK;
  XMH3_REQUIRE(x && q && scale, "quantize_int8_rowwise_convrot: null pointer");
  XMH3_REQUIRE(K % 256 == 0 && K <= 16384, "quantize_int8_rowwise_convrot: K must be a multiple of 256, <= 16384");
  XMH3_REQUIRE(group_size == 0 || K % group_size == 0,
               "quantize_int8_rowwise_convrot: K must be a multiple of convrot_groupsize");
  const int64_t in_width = input_act == ACT_SWIGLU ? 2 * K : K;
  XMH3_REQUIRE(ldx >= in_width && ldx % 8 == 0 && (uintptr_t)x % 16 == 0 && ldq >= K && ldq % 16 == 0 &&
                   (uintptr_t)q % 16 == 0,
               "quantize_int8_rowwise_convrot: rows must be 16-byte aligned");
  const int k = (int)K;
  if (group_size == 0 && input_act != ACT_SWIGLU)
    return fail(XMH3_EUNSUPPORTED, "quantize_int8_rowwise_convrot: without rotation only swiglu is routed here");
  if (x_dtype == DT_BF16) return launch_convrot_act<BF16T>(x, ldx, M, k, q, ldq, scale, input_act, logg, seed, st);
  if (x_dtype == DT_F16) return launch_convrot_act<F16T>(x, ldx, M, k, q, ldq, scale, input_act, logg, seed, st);
  return fail(XMH3_EUNSUPPORTED, "quantize_int8_rowwise_convrot: dtype must be bf16 or fp16");
}

}  // namespace xmh3

extern "C" int xmh3_quantize_int8_rowwise_convrot(const void* x, int x_dtype, int input_act, int64_t M,
                                                  int64_t K, int64_t ldx, int group_size, int8_t* q,
                                                  float* scale, hipStream_t stream) {
  return xmh3::quantize_rows_convrot(x, x_dtype, input_act, M, K, ldx, group_size, q, K, scale, 0, stream);
}

extern "C" int xmh3_quantize_int8_rowwise_convrot_sr(const void* x, int x_dtype, int input_act, int64_t M,
                                                     int64_t K, int64_t ldx, int group_size, int8_t* q,
                                                     float* scale, int stochastic, uint64_t seed,
                                                     hipStream_t stream) {
  if (stochastic && seed == 0)
    return xmh3::fail(xmh3::XMH3_EINVAL, "quantize_int8_rowwise_convrot: a stochastic seed must be nonzero");
  return xmh3::quantize_rows_convrot(x, x_dtype, input_act, M, K, ldx, group_size, q, K, scale,
                                     stochastic ? seed : 0, stream);
}
