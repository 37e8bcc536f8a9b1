// W4A8 GEMM: int8 activations x grouped int4 weights (group 128), the int4
// codes unpacked to the int8 grid in LDS inside the ping-pong GEMM
// (gemm_i8_kernels.hpp), with the per-token x per-channel dequant epilogue.
#include "gemm_i8_kernels.hpp"

namespace xmh3 {

int w4a8_gemm(const int8_t* A, int64_t lda, const uint8_t* Bp, int64_t ldbp, const void* s_rel, int srel_dtype,
              int64_t srel_ld, int64_t M, int64_t N, int64_t K, int64_t group_size, const float* sx,
              const float* s_channel, const void* bias, void* out, int out_dtype, int64_t ldo, hipStream_t st) {
  XMH3_REQUIRE(M >= 0 && N >= 0 && K >= 0, "w4a8_gemm: negative size");
  XMH3_REQUIRE(M < (1LL << 31) && N < (1LL << 31) && K <= 131072, "w4a8_gemm: size too large");
  if (M == 0 || N == 0) return XMH3_OK;
  XMH3_REQUIRE(A && Bp && s_rel && sx && s_channel && out, "w4a8_gemm: null operand");
  XMH3_REQUIRE(group_size == 128, "w4a8_gemm: the fused decode takes group size 128");
  XMH3_REQUIRE(K % 256 == 0, "w4a8_gemm: K must be a multiple of 256");
  XMH3_REQUIRE(lda % 16 == 0 && lda >= K && ldbp % 16 == 0 && ldbp >= K / 2 && srel_ld >= K / 128,
               "w4a8_gemm: bad row strides");
  XMH3_REQUIRE((uintptr_t)A % 16 == 0 && (uintptr_t)Bp % 16 == 0, "w4a8_gemm: operands must be 16-byte aligned");
  XMH3_REQUIRE(M * lda < (1LL << 31) && N * ldbp < (1LL << 31), "w4a8_gemm: operand spans must be < 2^31 bytes");
  XMH3_REQUIRE(srel_dtype == DT_BF16 || srel_dtype == DT_F32, "w4a8_gemm: s_rel must be bf16 or fp32");
  XMH3_REQUIRE((uintptr_t)s_rel % 4 == 0, "w4a8_gemm: s_rel must be 4-byte aligned");
  XMH3_REQUIRE(N * srel_ld * (srel_dtype == DT_BF16 ? 2 : 4) < (1LL << 31), "w4a8_gemm: s_rel span must be < 2^31 bytes");
  XMH3_REQUIRE(out_dtype == DT_BF16, "w4a8_gemm: the fused decode writes bf16");
  XMH3_REQUIRE(ldo >= N, "w4a8_gemm: output stride < N");
  GemmArgs a{};
  a.A = A; a.B = reinterpret_cast<const int8_t*>(Bp); a.lda = lda; a.ldb = ldbp;
  a.M = (int)M; a.N = (int)N; a.K = (int)K;
  a.sx = sx; a.sw = s_channel; a.sw_per_channel = 1;
  a.bias = bias; a.out = out; a.ldo = ldo; a.row_amax = nullptr;
  a.tiles_m = (int)((M + BM - 1) / BM);
  a.tiles_n = (int)((N + BN - 1) / BN);
  XMH3_REQUIRE((int64_t)a.tiles_m * a.tiles_n < (1LL << 31), "w4a8_gemm: grid too large");
  a.row_stores = N % 8 == 0 && ldo % 8 == 0 && (uintptr_t)out % 16 == 0;
  a.srel = s_rel; a.srel_ld = srel_ld; a.srel_bf16 = srel_dtype == DT_BF16;
  XMH3_REQUIRE(a.row_stores || (ldo % 4 == 0 && (uintptr_t)out % 8 == 0),
               "w4a8_gemm: output rows must be 8-byte aligned");
  return launch_gemm_w4_T<EPI_DEQUANT, BF16T>(a, st);
}

}  // namespace xmh3

extern "C" int xmh3_w4a8_gemm(const int8_t* A, int64_t lda, const uint8_t* packed, int64_t ldp, const void* s_rel,
                              int s_rel_dtype, int64_t s_rel_ld, int64_t M, int64_t N, int64_t K,
                              int64_t group_size, const float* sx, const float* s_channel, const void* bias,
                              void* out, int out_dtype, int64_t ldo, hipStream_t stream) {
  return xmh3::w4a8_gemm(A, lda, packed, ldp, s_rel, s_rel_dtype, s_rel_ld, M, N, K, group_size, sx, s_channel, bias,
                         out, out_dtype, ldo, stream);
}
