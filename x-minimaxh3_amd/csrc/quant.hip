// Per-token dynamic int8 quantisation for gfx950.
//
// Semantics (bit exact) follow the reference's eager quantizer,
// CK/backends/eager/quantization.py:815-826,857-875
// (CK = backends/turbo/vendor/comfy_kitchen):
//   amax  = max |x| over the row (in x's dtype, exact)
//   scale = max(amax / 127, 1e-30)          fp32, true division
//   s_T   = T(scale) (0 -> smallest normal of T)
//   v     = T(float(x) / float(s_T))        correctly rounded fp32 divide
//   q     = clamp(rint(v), -128, 127)       ties to even
// and returns the unrounded fp32 scale. An optional input activation
// (GELU-tanh, CK/backends/_activations.py:40-53) is applied first and
// rounded to T, as the reference materialises it.
//
// Layout: one wave64 per row, the whole row held in VGPRs (16-byte loads,
// 8 elements per lane per step), so the row is read from HBM exactly once.
// A block-per-row two-pass kernel covers rows wider than the register path.
#include "common.hpp"

#include <type_traits>

namespace xmh3 {

// 8 elements of T as raw storage
template <typename T> struct Pack8;
template <> struct Pack8<BF16T> { uint4 v; };
template <> struct Pack8<F16T> { uint4 v; };
template <> struct Pack8<F32T> { uint4 v[2]; };

template <typename T>
__device__ __forceinline__ void load8(const typename T::storage* p, Pack8<T>& d) {
  if constexpr (sizeof(typename T::storage) == 2) {
    d.v = *reinterpret_cast<const uint4*>(p);
  } else {
    d.v[0] = *reinterpret_cast<const uint4*>(p);
    d.v[1] = *reinterpret_cast<const uint4*>(p + 4);
  }
}

template <typename T>
__device__ __forceinline__ float get8(const Pack8<T>& d, int j) {
  if constexpr (sizeof(typename T::storage) == 2) {
    uint32_t w = (&d.v.x)[j >> 1];
    return T::load((j & 1) ? (w >> 16) : (w & 0xffffu));
  } else {
    return __uint_as_float((&d.v[j >> 2].x)[j & 3]);
  }
}

template <typename T>
__device__ __forceinline__ void set8(Pack8<T>& d, int j, float f) {
  if constexpr (sizeof(typename T::storage) == 2) {
    uint32_t& w = (&d.v.x)[j >> 1];
    uint32_t b = T::store(f);
    w = (j & 1) ? ((w & 0xffffu) | (b << 16)) : ((w & 0xffff0000u) | b);
  } else {
    (&d.v[j >> 2].x)[j & 3] = __float_as_uint(f);
  }
}

template <typename T>
__device__ __forceinline__ int quant_code_T(float x, float sT) {
  float v = T::round(x / sT);
  float r = rintf(v);
  r = fminf(fmaxf(r, -128.0f), 127.0f);
  return (int)r;
}

// The same code from a reciprocal, for bf16: r = x * fl(1/sT). With x and sT
// both bf16 (8 significant bits), x/sT is never within 2^-17 (relative) of a
// bf16 rounding midpoint: a midpoint has an odd 9-bit significand, so
// x = midpoint * sT would need at least 9 significant bits, and a quotient
// that is not a midpoint differs from one by at least 1/(256 * 2^9) of it. r is
// within 2^-23 (relative) of x/sT (two roundings of 2^-24; 1/sT stays normal
// since sT <= 2^121 for finite bf16 rows), so bf16(r) == bf16(fl(x/sT)) and
// the codes are identical. fp16 and fp32 keep the correctly rounded division.
template <typename T>
__device__ __forceinline__ int quant_code_rcp(float x, float sT, float inv) {
  if constexpr (std::is_same<T, BF16T>::value) {
    float v = T::round(x * inv);
    float q = rintf(v);
    q = fminf(fmaxf(q, -128.0f), 127.0f);
    return (int)q;
  } else {
    return quant_code_T<T>(x, sT);
  }
}

// Four codes packed into one word (byte j = code of x_j). The clamp comes
// before the rounding to an integer (the bounds are integers, so the order
// does not change the result), and c + 1.5 * 2^23 rounds c to the nearest
// even integer in the low bits of its fp32 pattern: its low byte is the
// two's-complement code. Bytes are gathered with v_perm.
template <typename T>
__device__ __forceinline__ float quant_value(float x, float sT, float inv) {
  if constexpr (std::is_same<T, BF16T>::value) return T::round(x * inv);   // see quant_code_rcp
  else return T::round(x / sT);
}
template <typename T>
__device__ __forceinline__ uint32_t quant_word4(float x0, float x1, float x2, float x3, float sT, float inv) {
  const float m = 12582912.0f;   // 1.5 * 2^23
  const uint32_t y0 = __float_as_uint(__builtin_amdgcn_fmed3f(quant_value<T>(x0, sT, inv), -128.0f, 127.0f) + m);
  const uint32_t y1 = __float_as_uint(__builtin_amdgcn_fmed3f(quant_value<T>(x1, sT, inv), -128.0f, 127.0f) + m);
  const uint32_t y2 = __float_as_uint(__builtin_amdgcn_fmed3f(quant_value<T>(x2, sT, inv), -128.0f, 127.0f) + m);
  const uint32_t y3 = __float_as_uint(__builtin_amdgcn_fmed3f(quant_value<T>(x3, sT, inv), -128.0f, 127.0f) + m);
  const uint32_t lo = __builtin_amdgcn_perm(y1, y0, 0x0c0c0400u);
  const uint32_t hi = __builtin_amdgcn_perm(y3, y2, 0x0c0c0400u);
  return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

template <typename T>
__device__ __forceinline__ float scale_for_math(float scale) {
  float sT = T::round(scale);
  return sT == 0.0f ? T::tiny() : sT;
}

__device__ __forceinline__ float row_scale(float amax) {
  float s = amax / 127.0f;
  return s < 1e-30f ? 1e-30f : s;
}

// ---------------------------------------------------------------------------
// register-resident path: NL steps of 512 elements per row
// ---------------------------------------------------------------------------
template <typename T, int ACT, int NL>
__global__ __launch_bounds__(256) void quant_rows_reg_kernel(
    const typename T::storage* __restrict__ x, int64_t ldx, int64_t M, int64_t K,
    int8_t* __restrict__ q, int64_t ldq, float* __restrict__ scale,
    uint32_t* __restrict__ zero_rows) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  const typename T::storage* xr = x + row * ldx;
  Pack8<T> buf[NL];
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    const int64_t col = ((int64_t)i * 64 + lane) * 8;
    if (col < K) {
      load8<T>(xr + col, buf[i]);
      if constexpr (ACT == ACT_GELU_TANH && sizeof(typename T::storage) == 2) {
        // T(gelu) of a pair packed by one conversion; |max| of the unrounded
        // values, rounded once below (rounding is monotone)
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
          const float g0 = gelu_tanh_f32(get8<T>(buf[i], j)), g1 = gelu_tanh_f32(get8<T>(buf[i], j + 1));
          amax = fmaxf(amax, fmaxf(fabsf(g0), fabsf(g1)));
          (&buf[i].v.x)[j >> 1] = T::store2(g0, g1);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          float f = get8<T>(buf[i], j);
          if constexpr (ACT == ACT_GELU_TANH) {
            f = T::round(gelu_tanh_f32(f));
            set8<T>(buf[i], j, f);
          }
          amax = fmaxf(amax, fabsf(f));
        }
      }
    }
  }
  amax = T::round(wave_max(amax));
  const float s = row_scale(amax);
  const float sT = scale_for_math<T>(s);
  const float inv = 1.0f / sT;
  int8_t* qr = q + row * ldq;
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    const int64_t col = ((int64_t)i * 64 + lane) * 8;
    if (col < K) {
      const Pack8<T>& b = buf[i];
      const uint32_t lo = quant_word4<T>(get8<T>(b, 0), get8<T>(b, 1), get8<T>(b, 2), get8<T>(b, 3), sT, inv);
      const uint32_t hi = quant_word4<T>(get8<T>(b, 4), get8<T>(b, 5), get8<T>(b, 6), get8<T>(b, 7), sT, inv);
      *reinterpret_cast<uint2*>(qr + col) = make_uint2(lo, hi);
    }
  }
  if (lane == 0) {
    scale[row] = s;
    if (zero_rows) zero_rows[row] = 0u;
  }
}

// ---------------------------------------------------------------------------
// register-resident path for wide rows: a block of WPR = 4 waves per row
// (one row per block), wave w taking the 512-element steps w, w + 4,
// w + 8, ... (NL each), so a quarter of the row's registers per wave and more
// waves per SIMD to hide the loads; the partial maxima meet in LDS. Same
// per-element operations as the one-wave path, and max is order-free, so the
// codes and scale are identical.
// ---------------------------------------------------------------------------
template <typename T, int ACT, int NL, int WPR>
__global__ __launch_bounds__(256) void quant_rows_reg2_kernel(
    const typename T::storage* __restrict__ x, int64_t ldx, int64_t M, int64_t K,
    int8_t* __restrict__ q, int64_t ldq, float* __restrict__ scale,
    uint32_t* __restrict__ zero_rows) {
  static_assert(WPR == 4, "a block of 4 waves per row");
  __shared__ float part_max[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, half = wave;
  const int64_t row = blockIdx.x;   // the grid has M blocks
  const typename T::storage* xr = x + row * ldx;
  Pack8<T> buf[NL];
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    const int64_t col = ((int64_t)(WPR * i + half) * 64 + lane) * 8;
    if (col < K) {
      load8<T>(xr + col, buf[i]);
      if constexpr (ACT == ACT_GELU_TANH && sizeof(typename T::storage) == 2) {
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
          const float g0 = gelu_tanh_f32(get8<T>(buf[i], j)), g1 = gelu_tanh_f32(get8<T>(buf[i], j + 1));
          amax = fmaxf(amax, fmaxf(fabsf(g0), fabsf(g1)));
          (&buf[i].v.x)[j >> 1] = T::store2(g0, g1);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          float f = get8<T>(buf[i], j);
          if constexpr (ACT == ACT_GELU_TANH) {
            f = T::round(gelu_tanh_f32(f));
            set8<T>(buf[i], j, f);
          }
          amax = fmaxf(amax, fabsf(f));
        }
      }
    }
  }
  amax = wave_max(amax);
  if (lane == 0) part_max[wave] = amax;
  __syncthreads();
  {
    float m = part_max[0];
#pragma unroll
    for (int w = 1; w < WPR; ++w) m = fmaxf(m, part_max[w]);
    amax = T::round(m);
  }
  const float s = row_scale(amax);
  const float sT = scale_for_math<T>(s);
  const float inv = 1.0f / sT;
  int8_t* qr = q + row * ldq;
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    const int64_t col = ((int64_t)(WPR * i + half) * 64 + lane) * 8;
    if (col < K) {
      const Pack8<T>& b = buf[i];
      const uint32_t lo = quant_word4<T>(get8<T>(b, 0), get8<T>(b, 1), get8<T>(b, 2), get8<T>(b, 3), sT, inv);
      const uint32_t hi = quant_word4<T>(get8<T>(b, 4), get8<T>(b, 5), get8<T>(b, 6), get8<T>(b, 7), sT, inv);
      *reinterpret_cast<uint2*>(qr + col) = make_uint2(lo, hi);
    }
  }
  if (lane == 0 && half == 0) {
    scale[row] = s;
    if (zero_rows) zero_rows[row] = 0u;
  }
}

// ---------------------------------------------------------------------------
// generic path: one 256-thread block per row, two passes over the row
// (any K; the second pass re-reads the row, mostly from L2)
// ---------------------------------------------------------------------------
template <typename T, int ACT>
__global__ __launch_bounds__(256) void quant_rows_generic_kernel(
    const typename T::storage* __restrict__ x, int64_t ldx, int64_t M, int64_t K,
    int8_t* __restrict__ q, int64_t ldq, float* __restrict__ scale,
    uint32_t* __restrict__ zero_rows) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const typename T::storage* xr = x + row * ldx;
  float amax = 0.0f;
  for (int64_t k = threadIdx.x; k < K; k += 256) {
    float f = T::load(xr[k]);
    if constexpr (ACT == ACT_GELU_TANH) f = T::round(gelu_tanh_f32(f));
    amax = fmaxf(amax, fabsf(f));
  }
  amax = wave_max(amax);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float s = row_scale(amax);
  const float sT = scale_for_math<T>(s);
  int8_t* qr = q + row * ldq;
  for (int64_t k = threadIdx.x; k < K; k += 256) {
    float f = T::load(xr[k]);
    if constexpr (ACT == ACT_GELU_TANH) f = T::round(gelu_tanh_f32(f));
    qr[k] = (int8_t)quant_code_T<T>(f, sT);
  }
  if (threadIdx.x == 0) {
    scale[row] = s;
    if (zero_rows) zero_rows[row] = 0u;
  }
}

// ---------------------------------------------------------------------------
// requant with a precomputed row amax (bit pattern of the bf16 |g| maximum,
// produced by the fused fc1 epilogue): a pure streaming pass, one wave per
// row (the scale is computed once), 16-byte non-temporal loads of 8 values
// and 8-byte stores of their codes, UNR chunks in flight per lane.
// ---------------------------------------------------------------------------
template <typename T, int UNR>
__global__ __launch_bounds__(256) void requant_rows_kernel(
    const typename T::storage* __restrict__ g, int64_t ldg, int64_t M, int64_t K,
    const uint32_t* __restrict__ row_amax, int8_t* __restrict__ q, int64_t ldq,
    float* __restrict__ scale) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  const float s = row_scale(__uint_as_float(row_amax[row]));
  const float sT = scale_for_math<T>(s);
  const float inv = 1.0f / sT;
  const typename T::storage* gr = g + row * ldg;
  int8_t* qr = q + row * ldq;
  const int chunks = (int)(K >> 3);
  for (int c0 = 0; c0 < chunks; c0 += 64 * UNR) {
    Pack8<T> b[UNR];
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int c = min(c0 + u * 64 + lane, chunks - 1);
      const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(gr + (int64_t)c * 8));
      b[u].v = make_uint4(v.x, v.y, v.z, v.w);
    }
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int c = c0 + u * 64 + lane;
      const Pack8<T>& bb = b[u];
      const uint32_t lo = quant_word4<T>(get8<T>(bb, 0), get8<T>(bb, 1), get8<T>(bb, 2), get8<T>(bb, 3), sT, inv);
      const uint32_t hi = quant_word4<T>(get8<T>(bb, 4), get8<T>(bb, 5), get8<T>(bb, 6), get8<T>(bb, 7), sT, inv);
      if (c < chunks) *reinterpret_cast<uint2*>(qr + (int64_t)c * 8) = make_uint2(lo, hi);
    }
  }
  if (lane == 0) scale[row] = s;
}

// ---------------------------------------------------------------------------
// stochastic rounding (the reference CUDA quantizer's rule,
// CK/backends/cuda/ops/int8_linear.cu:79-91,186-195): element idx = row*K +
// col of the logical [M, K] matrix draws u = (h >> 8) * 2^-24 in [0, 1) with
// h = PCG-RXS-M-XS(lo32(idx + seed) ^ hi32(idx + seed)), rounded to T; its
// code is floor(T(v + T(u))) with v = T(x / T(s)) as in the nearest path.
// The sum is added in fp32 and rounded once to T, which equals T's single
// rounding of the exact sum: when the exact sum of two T values does not fit
// fp32's 24 bits, the smaller one lies below 2^-15 (bf16; 2^-12 for fp16) of
// the larger and cannot reach T's half-step, while every T tie is an exact
// fp32 sum (pcg_output_hash / sr_noise in common.hpp). One block per row;
// the second pass re-reads the row (mostly from L2).
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void quant_rows_sr_kernel(
    const typename T::storage* __restrict__ x, int64_t ldx, int64_t M, int64_t K,
    int8_t* __restrict__ q, int64_t ldq, float* __restrict__ scale, uint64_t seed) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const typename T::storage* xr = x + row * ldx;
  float amax = 0.0f;
  for (int64_t k = threadIdx.x; k < K; k += 256) amax = fmaxf(amax, fabsf(T::load(xr[k])));
  amax = wave_max(amax);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float s = row_scale(amax);
  const float sT = scale_for_math<T>(s);
  int8_t* qr = q + row * ldq;
  const uint64_t base = (uint64_t)row * (uint64_t)K;
  for (int64_t k = threadIdx.x; k < K; k += 256) {
    const float v = T::round(T::load(xr[k]) / sT);
    const float c = floorf(T::round(v + sr_noise<T>(base + (uint64_t)k, seed)));
    qr[k] = (int8_t)fminf(fmaxf(c, -128.0f), 127.0f);
  }
  if (threadIdx.x == 0) scale[row] = s;
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
template <typename T, int ACT>
static int launch_quant_T(const void* x, int64_t ldx, int64_t M, int64_t K, int8_t* q,
                          int64_t ldq, float* scale, uint32_t* zero_rows, hipStream_t st) {
  using S = typename T::storage;
  const S* xs = static_cast<const S*>(x);
  const bool vec_ok = (K % 8 == 0) && (ldx % 8 == 0) && (ldq % 8 == 0) &&
                      ((uintptr_t)x % 16 == 0) && ((uintptr_t)q % 8 == 0);
  const int64_t steps = (K + 511) / 512;
  if (vec_ok && steps > 4 && steps <= 32 && M <= (1LL << 24)) {
    constexpr int W = 4;   // waves per row, one row per block
    dim3 grid((unsigned)M);
#define XMH3_Q2(NLV)                                                                                    \
  if ((steps + W - 1) / W <= NLV) {                                                                     \
    hipLaunchKernelGGL((quant_rows_reg2_kernel<T, ACT, NLV, W>), grid, dim3(256), 0, st, xs, ldx, M, K, \
                       q, ldq, scale, zero_rows);                                                       \
    return check_launch("quant_rows_reg2_kernel");                                                      \
  }
    XMH3_Q2(2) XMH3_Q2(3) XMH3_Q2(4) XMH3_Q2(5) XMH3_Q2(6) XMH3_Q2(8)
#undef XMH3_Q2
  }
  if (vec_ok && steps <= 32) {
    dim3 grid((unsigned)((M + 3) / 4));
#define XMH3_Q(NLV)                                                                                \
  if (steps <= NLV) {                                                                              \
    hipLaunchKernelGGL((quant_rows_reg_kernel<T, ACT, NLV>), grid, dim3(256), 0, st, xs, ldx, M, K, \
                       q, ldq, scale, zero_rows);                                                  \
    return check_launch("quant_rows_reg_kernel");                                                  \
  }
    XMH3_Q(1) XMH3_Q(2) XMH3_Q(3) XMH3_Q(4) XMH3_Q(6) XMH3_Q(8) XMH3_Q(10) XMH3_Q(12) XMH3_Q(16)
    XMH3_Q(20) XMH3_Q(24) XMH3_Q(28) XMH3_Q(32)
#undef XMH3_Q
  }
  hipLaunchKernelGGL((quant_rows_generic_kernel<T, ACT>), dim3((unsigned)M), dim3(256), 0, st, xs,
                     ldx, M, K, q, ldq, scale, zero_rows);
  return check_launch("quant_rows_generic_kernel");
}

int quantize_rows(const void* x, int x_dtype, int input_act, int64_t M, int64_t K, int64_t ldx,
                  int8_t* q, int64_t ldq, float* scale, uint32_t* zero_rows, hipStream_t st) {
  XMH3_REQUIRE(M >= 0 && K >= 0, "quantize_int8_rowwise: negative size");
  XMH3_REQUIRE(input_act == ACT_NONE || input_act == ACT_GELU_TANH,
               "quantize_int8_rowwise: input_act must be none or gelu_tanh");
  XMH3_REQUIRE(M <= 0x7fffffffLL * 4, "quantize_int8_rowwise: too many rows");
  if (M == 0) return XMH3_OK;
  XMH3_REQUIRE(x && q && scale, "quantize_int8_rowwise: null pointer");
  XMH3_REQUIRE(ldx >= K && ldq >= K, "quantize_int8_rowwise: leading dimension < K");
  switch (x_dtype) {
    case DT_BF16:
      return input_act ? launch_quant_T<BF16T, ACT_GELU_TANH>(x, ldx, M, K, q, ldq, scale, zero_rows, st)
                       : launch_quant_T<BF16T, ACT_NONE>(x, ldx, M, K, q, ldq, scale, zero_rows, st);
    case DT_F16:
      return input_act ? launch_quant_T<F16T, ACT_GELU_TANH>(x, ldx, M, K, q, ldq, scale, zero_rows, st)
                       : launch_quant_T<F16T, ACT_NONE>(x, ldx, M, K, q, ldq, scale, zero_rows, st);
    case DT_F32:
      return input_act ? launch_quant_T<F32T, ACT_GELU_TANH>(x, ldx, M, K, q, ldq, scale, zero_rows, st)
                       : launch_quant_T<F32T, ACT_NONE>(x, ldx, M, K, q, ldq, scale, zero_rows, st);
    default:
      return fail(XMH3_EUNSUPPORTED, "quantize_int8_rowwise: dtype must be fp32, fp16 or bf16");
  }
}

int quantize_rows_sr(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, int8_t* q, int64_t ldq,
                     float* scale, uint64_t seed, hipStream_t st) {
  XMH3_REQUIRE(M >= 0 && K >= 0, "quantize_int8_rowwise: negative size");
  XMH3_REQUIRE(M < (1LL << 31), "quantize_int8_rowwise: too many rows for stochastic rounding");
  if (M == 0) return XMH3_OK;
  XMH3_REQUIRE(x && q && scale, "quantize_int8_rowwise: null pointer");
  XMH3_REQUIRE(ldx >= K && ldq >= K, "quantize_int8_rowwise: leading dimension < K");
  const dim3 grid((unsigned)M), block(256);
  switch (x_dtype) {
    case DT_BF16:
      hipLaunchKernelGGL((quant_rows_sr_kernel<BF16T>), grid, block, 0, st, static_cast<const uint16_t*>(x), ldx,
                         M, K, q, ldq, scale, seed);
      break;
    case DT_F16:
      hipLaunchKernelGGL((quant_rows_sr_kernel<F16T>), grid, block, 0, st, static_cast<const uint16_t*>(x), ldx,
                         M, K, q, ldq, scale, seed);
      break;
    case DT_F32:
      hipLaunchKernelGGL((quant_rows_sr_kernel<F32T>), grid, block, 0, st, static_cast<const float*>(x), ldx, M,
                         K, q, ldq, scale, seed);
      break;
    default:
      return fail(XMH3_EUNSUPPORTED, "quantize_int8_rowwise: dtype must be fp32, fp16 or bf16");
  }
  return check_launch("quant_rows_sr_kernel");
}

int requant_rows(const void* g, int g_dtype, int64_t M, int64_t K, int64_t ldg,
                 const uint32_t* row_amax, int8_t* q, int64_t ldq, float* scale, hipStream_t st) {
  XMH3_REQUIRE(M >= 0 && K >= 0, "requant: negative size");
  if (M == 0 || K == 0) return XMH3_OK;
  XMH3_REQUIRE(K % 8 == 0 && ldg % 8 == 0 && ldq % 8 == 0, "requant: K and strides must be multiples of 8");
  XMH3_REQUIRE(g_dtype == DT_BF16 || g_dtype == DT_F16, "requant: dtype must be bf16 or fp16");
  XMH3_REQUIRE(K / 8 < (1LL << 30), "requant: rows too wide");
  XMH3_REQUIRE((uintptr_t)g % 16 == 0 && (uintptr_t)q % 8 == 0, "requant: misaligned pointers");
  dim3 grid((unsigned)((M + 3) / 4));
  if (g_dtype == DT_BF16)
    hipLaunchKernelGGL((requant_rows_kernel<BF16T, 4>), grid, dim3(256), 0, st,
                       static_cast<const uint16_t*>(g), ldg, M, K, row_amax, q, ldq, scale);
  else
    hipLaunchKernelGGL((requant_rows_kernel<F16T, 4>), grid, dim3(256), 0, st,
                       static_cast<const uint16_t*>(g), ldg, M, K, row_amax, q, ldq, scale);
  return check_launch("requant_rows_kernel");
}

}  // namespace xmh3

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
extern "C" int xmh3_quantize_int8_rowwise(const void* x, int x_dtype, int input_act, int64_t M,
                                          int64_t K, int64_t ldx, int8_t* q, float* scale,
                                          hipStream_t stream) {
  return xmh3::quantize_rows(x, x_dtype, input_act, M, K, ldx, q, K, scale, nullptr, stream);
}

extern "C" int xmh3_quantize_int8_rowwise_ex(const void* x, int x_dtype, int input_act, int64_t M,
                                             int64_t K, int64_t ldx, int8_t* q, float* scale,
                                             uint32_t* clear_rows, hipStream_t stream) {
  return xmh3::quantize_rows(x, x_dtype, input_act, M, K, ldx, q, K, scale, clear_rows, stream);
}

extern "C" int xmh3_quantize_int8_rowwise_sr(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx,
                                             int8_t* q, float* scale, int stochastic, uint64_t seed,
                                             hipStream_t stream) {
  if (!stochastic) return xmh3::quantize_rows(x, x_dtype, 0, M, K, ldx, q, K, scale, nullptr, stream);
  return xmh3::quantize_rows_sr(x, x_dtype, M, K, ldx, q, K, scale, seed, stream);
}

extern "C" int xmh3_requant_int8_rows(const void* g, int g_dtype, int64_t M, int64_t K, int64_t ldg,
                                      const uint32_t* row_absmax_bits, int8_t* q, float* scale,
                                      hipStream_t stream) {
  return xmh3::requant_rows(g, g_dtype, M, K, ldg, row_absmax_bits, q, K, scale, stream);
}
