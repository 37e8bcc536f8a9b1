// Host entry points of the int8 GEMM (kernels in gemm_i8_kernels.hpp, one
// translation unit per epilogue / output type: gemm_i8_*.hip).
#include "gemm_i8_kernels.hpp"

namespace xmh3 {

int int8_gemm(const int8_t* A, int64_t lda, const int8_t* B, int64_t ldb, int64_t M, int64_t N,
              int64_t K, const float* sx, const float* sw, int sw_per_channel, const void* bias,
              void* out, int out_dtype, int64_t ldo, int epilogue, uint32_t* row_amax,
              hipStream_t st) {
  XMH3_REQUIRE(M >= 0 && N >= 0 && K >= 0, "int8_gemm: negative size");
  XMH3_REQUIRE(M < (1LL << 31) && N < (1LL << 31) && K < (1LL << 31), "int8_gemm: size too large");
  if (M == 0 || N == 0) return XMH3_OK;
  XMH3_REQUIRE(A && B && out, "int8_gemm: null operand");
  XMH3_REQUIRE(K % 16 == 0, "int8_gemm: K must be a multiple of 16");
  XMH3_REQUIRE(lda % 16 == 0 && ldb % 16 == 0 && lda >= K && ldb >= K,
               "int8_gemm: row strides must be multiples of 16 bytes and >= K");
  XMH3_REQUIRE((uintptr_t)A % 16 == 0 && (uintptr_t)B % 16 == 0, "int8_gemm: operands must be 16-byte aligned");
  XMH3_REQUIRE(ldo >= N, "int8_gemm: output stride < N");
  XMH3_REQUIRE(K <= 131072, "int8_gemm: K > 131072 could overflow int32 accumulators");
  if (epilogue != EPI_INT32) XMH3_REQUIRE(sx && sw, "int8_gemm: scales required");
  if (epilogue == EPI_GELU) {
    XMH3_REQUIRE(row_amax, "int8_gemm: gelu epilogue needs row_amax");
    XMH3_REQUIRE(out_dtype == DT_BF16, "int8_gemm: gelu epilogue writes bf16");
  }
  GemmArgs a;
  a.A = A; a.B = B; a.lda = lda; a.ldb = ldb;
  a.M = (int)M; a.N = (int)N; a.K = (int)K;
  a.sx = sx; a.sw = sw; a.sw_per_channel = sw_per_channel;
  a.bias = bias; a.out = out; a.ldo = ldo; a.row_amax = row_amax;
  a.gate = nullptr; a.ldg = 0; a.gate_f32 = 0; a.gate_rows = nullptr; a.gate_nrows = 0;
  a.tiles_m = (int)((M + BM - 1) / BM);
  a.tiles_n = (int)((N + BN - 1) / BN);
  XMH3_REQUIRE((int64_t)a.tiles_m * a.tiles_n < (1LL << 31), "int8_gemm: grid too large");
  const int esize = (epilogue == EPI_INT32 || out_dtype == DT_F32) ? 4 : 2;
  const bool vec = (ldo % 4 == 0) && ((uintptr_t)out % (4 * esize) == 0);
  a.row_stores = esize == 2 && N % 8 == 0 && ldo % 8 == 0 && (uintptr_t)out % 16 == 0;
  switch (epilogue) {
    case EPI_INT32:
      return launch_gemm<EPI_INT32, F32T>(a, vec, st);
    case EPI_GELU:
      return launch_gemm<EPI_GELU, BF16T>(a, vec, st);
    case EPI_DEQUANT:
      if (out_dtype == DT_BF16) return launch_gemm<EPI_DEQUANT, BF16T>(a, vec, st);
      if (out_dtype == DT_F16) return launch_gemm<EPI_DEQUANT, F16T>(a, vec, st);
      if (out_dtype == DT_F32) return launch_gemm<EPI_DEQUANT, F32T>(a, vec, st);
      return fail(XMH3_EUNSUPPORTED, "int8_gemm: out dtype must be fp32, fp16 or bf16");
    default:
      return fail(XMH3_EINVAL, "int8_gemm: unknown epilogue");
  }
}

int int8_gemm_gated(const int8_t* A, int64_t lda, const int8_t* B, int64_t ldb, int64_t M, int64_t N,
                    int64_t K, const float* sx, const float* sw, int sw_per_channel, const void* bias,
                    void* residual, int res_dtype, int64_t ldr, const void* gate, int gate_dtype, int64_t ldg,
                    int64_t gate_nrows, const int32_t* gate_rows, hipStream_t st) {
  XMH3_REQUIRE(M >= 0 && N >= 0 && K >= 0, "int8_gemm_gated_residual: negative size");
  XMH3_REQUIRE(M < (1LL << 31) && N < (1LL << 31) && K < (1LL << 31), "int8_gemm_gated_residual: size too large");
  if (M == 0 || N == 0) return XMH3_OK;
  XMH3_REQUIRE(A && B && residual && sx && sw && gate && gate_rows, "int8_gemm_gated_residual: null operand");
  XMH3_REQUIRE(gate_nrows >= 1 && gate_nrows < (1LL << 31), "int8_gemm_gated_residual: gate table needs >= 1 row");
  XMH3_REQUIRE(K % 16 == 0, "int8_gemm_gated_residual: K must be a multiple of 16");
  XMH3_REQUIRE(lda % 16 == 0 && ldb % 16 == 0 && lda >= K && ldb >= K,
               "int8_gemm_gated_residual: row strides must be multiples of 16 bytes and >= K");
  XMH3_REQUIRE((uintptr_t)A % 16 == 0 && (uintptr_t)B % 16 == 0,
               "int8_gemm_gated_residual: operands must be 16-byte aligned");
  XMH3_REQUIRE(K <= 131072, "int8_gemm_gated_residual: K > 131072 could overflow int32 accumulators");
  XMH3_REQUIRE(res_dtype == DT_BF16 || res_dtype == DT_F16, "int8_gemm_gated_residual: residual must be bf16 or fp16");
  XMH3_REQUIRE(gate_dtype == DT_F32 || gate_dtype == res_dtype,
               "int8_gemm_gated_residual: gate must be fp32 or the residual's dtype");
  XMH3_REQUIRE(N % 4 == 0 && ldr % 4 == 0 && ldr >= N && ldg % 4 == 0 && ldg >= N,
               "int8_gemm_gated_residual: N and the residual / gate row strides must be multiples of 4");
  XMH3_REQUIRE((uintptr_t)residual % 8 == 0 && (uintptr_t)gate % (gate_dtype == DT_F32 ? 16 : 8) == 0,
               "int8_gemm_gated_residual: residual / gate rows must be 8-byte (fp32 gate: 16-byte) aligned");
  GemmArgs a;
  a.A = A; a.B = B; a.lda = lda; a.ldb = ldb;
  a.M = (int)M; a.N = (int)N; a.K = (int)K;
  a.sx = sx; a.sw = sw; a.sw_per_channel = sw_per_channel;
  a.bias = bias; a.out = residual; a.ldo = ldr; a.row_amax = nullptr;
  a.gate = gate; a.ldg = ldg; a.gate_f32 = gate_dtype == DT_F32; a.gate_rows = gate_rows;
  a.gate_nrows = (int)gate_nrows;
  a.row_stores = 0;
  a.tiles_m = (int)((M + BM - 1) / BM);
  a.tiles_n = (int)((N + BN - 1) / BN);
  XMH3_REQUIRE((int64_t)a.tiles_m * a.tiles_n < (1LL << 31), "int8_gemm_gated_residual: grid too large");
  if (res_dtype == DT_BF16) return launch_gemm<EPI_GATED, BF16T>(a, true, st);
  return launch_gemm<EPI_GATED, F16T>(a, true, st);
}

}  // namespace xmh3

extern "C" int xmh3_int8_gemm(const int8_t* A, int64_t lda, const int8_t* B, int64_t ldb, int64_t M,
                              int64_t N, int64_t K, const float* sx, const float* sw,
                              int sw_per_channel, const void* bias, void* out, int out_dtype,
                              int64_t ldo, int epilogue, uint32_t* row_absmax_bits,
                              hipStream_t stream) {
  return xmh3::int8_gemm(A, lda, B, ldb, M, N, K, sx, sw, sw_per_channel, bias, out, out_dtype, ldo,
                         epilogue, row_absmax_bits, stream);
}

extern "C" int xmh3_int8_gemm_gated_residual(const int8_t* A, int64_t lda, const int8_t* B, int64_t ldb,
                                             int64_t M, int64_t N, int64_t K, const float* sx, const float* sw,
                                             int sw_per_channel, const void* bias, void* residual, int res_dtype,
                                             int64_t ldr, const void* gate, int gate_dtype, int64_t ldg,
                                             int64_t gate_nrows, const int32_t* gate_rows, hipStream_t stream) {
  return xmh3::int8_gemm_gated(A, lda, B, ldb, M, N, K, sx, sw, sw_per_channel, bias, residual, res_dtype, ldr,
                               gate, gate_dtype, ldg, gate_nrows, gate_rows, stream);
}
