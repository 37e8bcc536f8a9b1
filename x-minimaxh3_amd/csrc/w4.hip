// Grouped int4 weights -> the int8 grid consumed by the int8 GEMM (gfx950).
//
// Rule (CK/backends/eager/w4a8_int8.py:344-363, CK = backends/turbo/vendor/
// comfy_kitchen): byte b holds code[2j] = b & 0xF and code[2j+1] = b >> 4;
// level = code - 8 (or codebook[code]); w8 = clamp(rint(level * s_rel[n, k/G]),
// -127, 127) with s_rel read as fp32 (bf16 s_rel widened exactly).
//
// Each thread turns 8 packed bytes into 16 int8 through a 16-entry level table
// built once per (row, group) in registers: every code of a group maps through
// the same s_rel, so the per-element multiply + rint becomes a lookup.
#include "w4_lut.hpp"

namespace xmh3 {

// G % 16 == 0: the 16 outputs of a thread share one group
template <bool BF16_SREL>
__global__ __launch_bounds__(256) void w4_decode_kernel(const uint8_t* __restrict__ packed,
                                                        const void* __restrict__ s_rel,
                                                        const float* __restrict__ codebook,
                                                        int64_t N, int64_t K, int64_t G,
                                                        int8_t* __restrict__ out) {
  const int64_t per_row = K / 16;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= N * per_row) return;
  const int64_t n = idx / per_row;
  const int64_t k0 = (idx - n * per_row) * 16;
  const float s = load_srel<BF16_SREL>(s_rel, n * (K / G) + k0 / G);
  // 16-entry table: byte c of lut[c/4] is the int8 for code c
  uint32_t lut[4];
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    uint32_t word = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int c = w * 4 + b;
      const float level = codebook ? codebook[c] : (float)(c - 8);
      word |= (uint32_t)(w4_level_code(level, s) & 0xff) << (8 * b);
    }
    lut[w] = word;
  }
  const uint2 p = *reinterpret_cast<const uint2*>(packed + n * (K / 2) + k0 / 2);
  uint32_t o[4];
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const uint32_t src = (w < 2) ? p.x : p.y;
    const uint32_t two = (src >> (16 * (w & 1))) & 0xffffu;  // 2 bytes -> 4 codes
    uint32_t word = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const uint32_t byte = (two >> (8 * (b >> 1))) & 0xffu;
      const uint32_t code = (b & 1) ? (byte >> 4) : (byte & 0xf);
      const uint32_t val = (lut[code >> 2] >> (8 * (code & 3))) & 0xffu;
      word |= val << (8 * b);
    }
    o[w] = word;
  }
  *reinterpret_cast<uint4*>(out + n * K + k0) = make_uint4(o[0], o[1], o[2], o[3]);
}

// G % 32 == 0: 32 outputs (16 packed bytes) per thread, one group, through
// the level table of w4_lut.hpp. Threads are numbered across rows: thread t
// decodes chunk t % (K / 32) of row t / (K / 32) (32-bit, checked on the host).
template <bool BF16_SREL>
__global__ __launch_bounds__(256) void w4_decode32_kernel(const uint8_t* __restrict__ packed,
                                                          const void* __restrict__ s_rel,
                                                          const float* __restrict__ codebook,
                                                          uint32_t total, uint32_t per_row, int64_t K,
                                                          int64_t G, int8_t* __restrict__ out) {
  const uint32_t t = blockIdx.x * 256u + threadIdx.x;
  if (t >= total) return;
  const uint32_t n = t / per_row;
  const int64_t k0 = (int64_t)(t - n * per_row) * 32;
  const float s = load_srel<BF16_SREL>(s_rel, (int64_t)n * (K / G) + k0 / G);
  uint32_t lut[4];
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    float l[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) l[b] = codebook ? codebook[w * 4 + b] : (float)(w * 4 + b - 8);
    lut[w] = w4_entry4(l[0], l[1], l[2], l[3], s);
  }
  const uint4 p = *reinterpret_cast<const uint4*>(packed + (int64_t)n * (K / 2) + k0 / 2);
  const uint32_t pw[4] = {p.x, p.y, p.z, p.w};
  uint32_t o[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o[2 * i] = w4_lookup4<0x01010000u>(pw[i], lut);
    o[2 * i + 1] = w4_lookup4<0x03030202u>(pw[i], lut);
  }
  int8_t* dst = out + (int64_t)n * K + k0;
  *reinterpret_cast<uint4*>(dst) = make_uint4(o[0], o[1], o[2], o[3]);
  *reinterpret_cast<uint4*>(dst + 16) = make_uint4(o[4], o[5], o[6], o[7]);
}

// any G (>= 2, dividing K): one byte (two outputs) per thread
template <bool BF16_SREL>
__global__ __launch_bounds__(256) void w4_decode_generic_kernel(const uint8_t* __restrict__ packed,
                                                                const void* __restrict__ s_rel,
                                                                const float* __restrict__ codebook,
                                                                int64_t N, int64_t K, int64_t G,
                                                                int8_t* __restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= N * (K / 2)) return;
  const int64_t n = idx / (K / 2);
  const int64_t k = (idx - n * (K / 2)) * 2;
  const uint32_t byte = packed[idx];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int c = h ? (int)(byte >> 4) : (int)(byte & 0xf);
    const float s = load_srel<BF16_SREL>(s_rel, n * (K / G) + (k + h) / G);
    const float level = codebook ? codebook[c] : (float)(c - 8);
    out[n * K + k + h] = (int8_t)w4_level_code(level, s);
  }
}

int w4_decode(const uint8_t* packed, const void* s_rel, int s_rel_dtype, const float* codebook,
              int64_t N, int64_t K, int64_t G, int8_t* out, hipStream_t st) {
  XMH3_REQUIRE(N >= 0 && K >= 0 && G > 0, "w4_decode: bad sizes");
  if (N == 0 || K == 0) return XMH3_OK;
  XMH3_REQUIRE(K % 2 == 0 && K % G == 0, "w4_decode: K must be even and a multiple of group_size");
  XMH3_REQUIRE(packed && s_rel && out, "w4_decode: null pointer");
  XMH3_REQUIRE(s_rel_dtype == DT_F32 || s_rel_dtype == DT_BF16, "w4_decode: s_rel must be fp32 or bf16");
  const bool bf = s_rel_dtype == DT_BF16;
  const bool fast32 = (G % 32 == 0) && ((uintptr_t)packed % 16 == 0) && ((uintptr_t)out % 16 == 0) &&
                      N * (K / 32) < (1LL << 31);
  if (fast32) {
    const uint32_t per_row = (uint32_t)(K / 32), total = (uint32_t)(N * (K / 32));
    dim3 grid((total + 255) / 256);
    if (bf)
      hipLaunchKernelGGL(w4_decode32_kernel<true>, grid, dim3(256), 0, st, packed, s_rel, codebook, total, per_row, K, G, out);
    else
      hipLaunchKernelGGL(w4_decode32_kernel<false>, grid, dim3(256), 0, st, packed, s_rel, codebook, total, per_row, K, G, out);
    return check_launch("w4_decode32_kernel");
  }
  const bool fast = (G % 16 == 0) && ((uintptr_t)packed % 8 == 0) && ((uintptr_t)out % 16 == 0);
  if (fast) {
    const int64_t threads = N * (K / 16);
    dim3 grid((unsigned)((threads + 255) / 256));
    if (bf) hipLaunchKernelGGL(w4_decode_kernel<true>, grid, dim3(256), 0, st, packed, s_rel, codebook, N, K, G, out);
    else hipLaunchKernelGGL(w4_decode_kernel<false>, grid, dim3(256), 0, st, packed, s_rel, codebook, N, K, G, out);
    return check_launch("w4_decode_kernel");
  }
  const int64_t threads = N * (K / 2);
  dim3 grid((unsigned)((threads + 255) / 256));
  if (bf) hipLaunchKernelGGL(w4_decode_generic_kernel<true>, grid, dim3(256), 0, st, packed, s_rel, codebook, N, K, G, out);
  else hipLaunchKernelGGL(w4_decode_generic_kernel<false>, grid, dim3(256), 0, st, packed, s_rel, codebook, N, K, G, out);
  return check_launch("w4_decode_generic_kernel");
}

// Operand of the asymmetric W4A8 correction (the weight's per-group offset
// correction[g, n] times the group sums of the activation codes):
//   s[m, g] = T(T(sum_{k in group g} q[m, k]) * T(xs[m]))
// as CK/backends/cuda/__init__.py:2294-2297 forms it before its
// out.addmm_(s, T(correction)). One thread per (row, group).
__device__ __forceinline__ int sum_bytes(uint32_t w) {
  return (int)(int8_t)(w & 0xffu) + (int)(int8_t)((w >> 8) & 0xffu) + (int)(int8_t)((w >> 16) & 0xffu) +
         (int)(int8_t)(w >> 24);
}

template <typename T>
__global__ __launch_bounds__(256) void int8_group_sums_kernel(const int8_t* __restrict__ q, int64_t ldq,
                                                              const float* __restrict__ xs, int64_t M, int G,
                                                              int gs, typename T::storage* __restrict__ out,
                                                              int64_t ldo) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= M * G) return;
  const int64_t m = t / G;
  const int g = (int)(t - m * G);
  const int8_t* p = q + m * ldq + (int64_t)g * gs;
  int sum = 0;
  if (gs % 16 == 0) {
    for (int c = 0; c < gs; c += 16) {
      const uint4 v = *reinterpret_cast<const uint4*>(p + c);
      sum += sum_bytes(v.x) + sum_bytes(v.y) + sum_bytes(v.z) + sum_bytes(v.w);
    }
  } else {
    for (int c = 0; c < gs; ++c) sum += p[c];
  }
  const float v = T::round(T::round((float)sum) * T::round(xs[m]));
  out[m * ldo + g] = (typename T::storage)T::store(v);
}

int int8_group_sums(const int8_t* q, int64_t ldq, const float* xs, int64_t M, int64_t K, int64_t gs, void* out,
                    int out_dtype, int64_t ldo, hipStream_t st) {
  XMH3_REQUIRE(M >= 0 && K >= 0 && gs > 0, "int8_group_sums: bad sizes");
  if (M == 0 || K == 0) return XMH3_OK;
  XMH3_REQUIRE(q && xs && out, "int8_group_sums: null pointer");
  XMH3_REQUIRE(K % gs == 0 && gs <= 4096, "int8_group_sums: K must be a multiple of group_size (<= 4096)");
  const int64_t G = K / gs;
  XMH3_REQUIRE(ldq >= K && ldo >= G && G < (1LL << 31), "int8_group_sums: bad strides");
  if (gs % 16 == 0)
    XMH3_REQUIRE(ldq % 16 == 0 && (uintptr_t)q % 16 == 0, "int8_group_sums: rows must be 16-byte aligned");
  const int64_t threads = M * G;
  XMH3_REQUIRE((threads + 255) / 256 < (1LL << 31), "int8_group_sums: too many groups");
  dim3 grid((unsigned)((threads + 255) / 256));
  if (out_dtype == DT_BF16)
    hipLaunchKernelGGL(int8_group_sums_kernel<BF16T>, grid, dim3(256), 0, st, q, ldq, xs, M, (int)G, (int)gs,
                       static_cast<uint16_t*>(out), ldo);
  else if (out_dtype == DT_F16)
    hipLaunchKernelGGL(int8_group_sums_kernel<F16T>, grid, dim3(256), 0, st, q, ldq, xs, M, (int)G, (int)gs,
                       static_cast<uint16_t*>(out), ldo);
  else if (out_dtype == DT_F32)
    hipLaunchKernelGGL(int8_group_sums_kernel<F32T>, grid, dim3(256), 0, st, q, ldq, xs, M, (int)G, (int)gs,
                       static_cast<float*>(out), ldo);
  else
    return fail(XMH3_EUNSUPPORTED, "int8_group_sums: out dtype must be fp32, fp16 or bf16");
  return check_launch("int8_group_sums_kernel");
}

}  // namespace xmh3

extern "C" int xmh3_int8_group_sums(const int8_t* q, int64_t ldq, const float* xs, int64_t M, int64_t K,
                                    int64_t group_size, void* out, int out_dtype, int64_t ldo,
                                    hipStream_t stream) {
  return xmh3::int8_group_sums(q, ldq, xs, M, K, group_size, out, out_dtype, ldo, stream);
}

extern "C" int xmh3_w4_decode_int8(const uint8_t* packed, const void* s_rel, int s_rel_dtype,
                                   const float* codebook, int64_t N, int64_t K, int64_t group_size,
                                   int8_t* out, hipStream_t stream) {
  return xmh3::w4_decode(packed, s_rel, s_rel_dtype, codebook, N, K, group_size, out, stream);
}
