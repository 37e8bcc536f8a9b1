// The W8A8 / W4A8 MLP block  y = fc2(gelu_tanh(fc1(x)))  on one stream.
//
// Reference op chain (CK = backends/turbo/vendor/comfy_kitchen):
//   h = int8_linear(x, W1, s1)                      CK/backends/eager/quantization.py:971-1056
//   y = int8_linear(h, W2, s2, input_act="gelu_tanh")
// Kernel chain here (four launches, all on the caller's stream):
//   1. per-token quant of x -> q1, sx
//   2. int8 GEMM q1 x W1^T, epilogue: dequant -> bf16 h
//   3. per-token quant with the GELU input act, one wave per row held in
//      registers: g = bf16(gelu(h)), max|g|, codes -> q2, sg
//   4. int8 GEMM q2 x W2^T, epilogue: dequant -> y
// GELU sits in step 3 rather than in the fc1 epilogue (the GEMM's epilogue
// cannot overlap its MFMAs, while the row quantizer has VALU time to spare
// under its memory traffic; measured 1.81 ms against 1.88 ms for steps 2-3 at
// the 720p shape, identical codes). The W4A8 variant first turns each packed
// int4 weight into the int8 grid, in a workspace region that is idle while
// that weight is live: W1 (before step 2) into q2's region, which step 3
// overwrites only after fc1 has read W1; W2 (after step 3) into h's region,
// which fc2 does not touch. A region too small for its weight (M < D for W1,
// 2M < D for W2) gets a segment of its own at the end.
// Workspace (caller-owned, 256-byte aligned segments):
//   q1 [M,D] i8 | sx [M] f32 | h [M,F] bf16 | (unused) [M] u32 | q2 [M,F] i8 | sg [M] f32
//   (+ W1 [F,D] i8 if M < D, + W2 [D,F] i8 if 2M < D, W4A8 only)
#include "common.hpp"

#include <mutex>

namespace xmh3 {

int quantize_rows(const void* x, int x_dtype, int input_act, int64_t M, int64_t K, int64_t ldx,
                  int8_t* q, int64_t ldq, float* scale, uint32_t* zero_rows, hipStream_t st);
int requant_rows(const void* g, int g_dtype, int64_t M, int64_t K, int64_t ldg,
                 const uint32_t* row_amax, int8_t* q, int64_t ldq, float* scale, hipStream_t st);
int int8_gemm(const int8_t* A, int64_t lda, const int8_t* B, int64_t ldb, int64_t M, int64_t N,
              int64_t K, const float* sx, const float* sw, int sw_per_channel, const void* bias,
              void* out, int out_dtype, int64_t ldo, int epilogue, uint32_t* row_amax,
              hipStream_t st);
int w4_decode(const uint8_t* packed, const void* s_rel, int s_rel_dtype, const float* codebook,
              int64_t N, int64_t K, int64_t G, int8_t* out, hipStream_t st);

// The W4A8 MLP decodes each weight once per call to the int8 grid (21 us per
// 720p weight, HBM-bound) and runs the int8 GEMMs. Decoding inside the GEMM
// (w4a8_gemm, the codes unpacked in LDS) decodes every weight tile once per
// row tile of the activations -- 99 times at 25,200 tokens -- and measured
// slower at every token count from 256 up, so the MLP does not use it.

static inline size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

struct MlpWs {
  int8_t* q1; float* sx; uint16_t* g; uint32_t* amax; int8_t* q2; float* sg;
  int8_t* w1; int8_t* w2;
  size_t bytes;
};

static MlpWs carve(void* base, int64_t M, int64_t D, int64_t F, bool w4) {
  MlpWs w{};
  size_t off = 0;
  auto take = [&](size_t n) { size_t o = off; off = align256(off + n); return o; };
  const size_t o_q1 = take((size_t)M * D), o_sx = take((size_t)M * 4), o_g = take((size_t)M * F * 2),
               o_am = take((size_t)M * 4), o_q2 = take((size_t)M * F), o_sg = take((size_t)M * 4);
  size_t o_w1 = o_q2, o_w2 = o_g;
  if (w4 && M < D) o_w1 = take((size_t)F * D);
  if (w4 && 2 * M < D) o_w2 = take((size_t)D * F);
  w.bytes = off;
  char* b = static_cast<char*>(base);
  if (b) {
    w.q1 = reinterpret_cast<int8_t*>(b + o_q1);
    w.sx = reinterpret_cast<float*>(b + o_sx);
    w.g = reinterpret_cast<uint16_t*>(b + o_g);
    w.amax = reinterpret_cast<uint32_t*>(b + o_am);
    w.q2 = reinterpret_cast<int8_t*>(b + o_q2);
    w.sg = reinterpret_cast<float*>(b + o_sg);
    w.w1 = reinterpret_cast<int8_t*>(b + o_w1);
    w.w2 = reinterpret_cast<int8_t*>(b + o_w2);
  }
  return w;
}

// Steps 1-3: q1, sx <- x; h <- fc1; q2, sg <- gelu(h).
static int mlp_to_q2(const void* x, int x_dtype, int64_t M, int64_t D, int64_t F, int64_t ldx,
                     const int8_t* w1, const float* s1, int s1_pc, const MlpWs& ws, hipStream_t st) {
  int rc = quantize_rows(x, x_dtype, ACT_NONE, M, D, ldx, ws.q1, D, ws.sx, nullptr, st);
  if (rc) return rc;
  rc = int8_gemm(ws.q1, D, w1, D, M, F, D, ws.sx, s1, s1_pc, nullptr, ws.g, DT_BF16, F, 0 /*dequant*/,
                 nullptr, st);
  if (rc) return rc;
  return quantize_rows(ws.g, DT_BF16, ACT_GELU_TANH, M, F, F, ws.q2, F, ws.sg, nullptr, st);
}

// Step 4: y <- fc2(q2).
static int mlp_fc2(int64_t M, int64_t D, int64_t F, const int8_t* w2, const float* s2, int s2_pc, void* y,
                   int64_t ldy, const MlpWs& ws, hipStream_t st) {
  return int8_gemm(ws.q2, F, w2, F, M, D, F, ws.sg, s2, s2_pc, nullptr, y, DT_BF16, ldy, 0 /*dequant*/, nullptr,
                   st);
}

static int mlp_core(const void* x, int x_dtype, int64_t M, int64_t D, int64_t F, int64_t ldx,
                    const int8_t* w1, const float* s1, int s1_pc, const int8_t* w2, const float* s2,
                    int s2_pc, void* y, int64_t ldy, const MlpWs& ws, hipStream_t st) {
  int rc = mlp_to_q2(x, x_dtype, M, D, F, ldx, w1, s1, s1_pc, ws, st);
  if (rc) return rc;
  return mlp_fc2(M, D, F, w2, s2, s2_pc, y, ldy, ws, st);
}

static int check_mlp_shapes(int64_t M, int64_t D, int64_t F, int64_t ldx, int64_t ldy) {
  XMH3_REQUIRE(M >= 0 && D > 0 && F > 0, "mlp: bad sizes");
  XMH3_REQUIRE(D % 16 == 0 && F % 16 == 0, "mlp: d_model and ffn must be multiples of 16");
  XMH3_REQUIRE(ldx >= D && ldy >= D && ldx % 8 == 0, "mlp: bad strides");
  return XMH3_OK;
}

}  // namespace xmh3

using namespace xmh3;

extern "C" size_t xmh3_w8a8_mlp_workspace_bytes(int64_t M, int64_t D, int64_t F) {
  return carve(nullptr, M, D, F, false).bytes;
}

extern "C" size_t xmh3_w4a8_mlp_workspace_bytes(int64_t M, int64_t D, int64_t F, int64_t group_size) {
  (void)group_size;   // every group size decodes to the same int8 grid
  return carve(nullptr, M, D, F, true).bytes;
}

extern "C" int xmh3_w8a8_mlp(const void* x, int x_dtype, int64_t M, int64_t D, int64_t F, int64_t ldx,
                             const int8_t* w1, const float* s1, int s1_per_channel, const int8_t* w2,
                             const float* s2, int s2_per_channel, void* y, int64_t ldy,
                             void* workspace, size_t workspace_bytes, hipStream_t stream) {
  int rc = check_mlp_shapes(M, D, F, ldx, ldy);
  if (rc) return rc;
  if (M == 0) return XMH3_OK;
  MlpWs ws = carve(workspace, M, D, F, false);
  XMH3_REQUIRE(workspace && workspace_bytes >= ws.bytes, "w8a8_mlp: workspace too small");
  XMH3_REQUIRE(x && w1 && s1 && w2 && s2 && y, "w8a8_mlp: null pointer");
  return mlp_core(x, x_dtype, M, D, F, ldx, w1, s1, s1_per_channel, w2, s2, s2_per_channel, y, ldy, ws,
                  stream);
}

extern "C" int xmh3_w4a8_mlp(const void* x, int x_dtype, int64_t M, int64_t D, int64_t F, int64_t ldx,
                             const uint8_t* w1_packed, const void* w1_srel, const float* w1_schannel,
                             const uint8_t* w2_packed, const void* w2_srel, const float* w2_schannel,
                             int srel_dtype, int64_t group_size, void* y, int64_t ldy,
                             void* workspace, size_t workspace_bytes, hipStream_t stream) {
  int rc = check_mlp_shapes(M, D, F, ldx, ldy);
  if (rc) return rc;
  if (M == 0) return XMH3_OK;
  MlpWs ws = carve(workspace, M, D, F, true);
  XMH3_REQUIRE(workspace && workspace_bytes >= ws.bytes, "w4a8_mlp: workspace too small");
  XMH3_REQUIRE(x && w1_packed && w1_srel && w1_schannel && w2_packed && w2_srel && w2_schannel && y,
               "w4a8_mlp: null pointer");
  // W1 may share q2's region and W2 h's region: the order below keeps each
  // decoded weight intact until its GEMM has run (one stream)
  rc = w4_decode(w1_packed, w1_srel, srel_dtype, nullptr, F, D, group_size, ws.w1, stream);
  if (rc) return rc;
  rc = mlp_to_q2(x, x_dtype, M, D, F, ldx, ws.w1, w1_schannel, 1, ws, stream);
  if (rc) return rc;
  rc = w4_decode(w2_packed, w2_srel, srel_dtype, nullptr, D, F, group_size, ws.w2, stream);
  if (rc) return rc;
  return mlp_fc2(M, D, F, ws.w2, w2_schannel, 1, y, ldy, ws, stream);
}

// ---------------------------------------------------------------------------
// Allocation-free variant: the workspace lives in a file-scope device array
// instead of a caller buffer, for callers that cannot allocate (code under
// HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
// Every GPU the library runs on holds its own copy of the array until the
// process ends; all calls on one GPU share it and it keeps the last call's
// contents (nothing in it needs to start at zero: each call writes every
// byte it reads before reading it). Calls that overlap on one GPU race.
// ---------------------------------------------------------------------------
namespace xmh3 {

constexpr size_t kMlpScratchBytes = size_t(64) << 20;   // 64 MiB per GPU
static __device__ __align__(256) uint8_t scratch[kMlpScratchBytes];

constexpr int kMaxDevices = 64;
static void* g_scratch_dev[kMaxDevices];
static std::mutex g_scratch_mu;

// Device address of this GPU's copy of `scratch` (resolved once per device,
// with that device current). The array's name is a host-side stand-in, never
// a device address, so it is only ever used through this pointer.
static int scratch_ptr(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(XMH3_EHIP, "w8a8_mlp_noalloc: no current HIP device");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(XMH3_EHIP, std::string("w8a8_mlp_noalloc: hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return XMH3_OK;
}

}  // namespace xmh3

extern "C" int xmh3_w8a8_mlp_noalloc(const void* x, int x_dtype, int64_t M, int64_t D, int64_t F, int64_t ldx,
                                     const int8_t* w1, const float* s1, int s1_per_channel, const int8_t* w2,
                                     const float* s2, int s2_per_channel, void* y, int64_t ldy,
                                     hipStream_t stream) {
  int rc = check_mlp_shapes(M, D, F, ldx, ldy);
  if (rc) return rc;
  if (M == 0) return XMH3_OK;
  const size_t need = carve(nullptr, M, D, F, false).bytes;
  if (need > kMlpScratchBytes)
    return fail(XMH3_EINVAL, "w8a8_mlp_noalloc: " + std::to_string(M) + " tokens at d_model " + std::to_string(D) +
                                 ", ffn " + std::to_string(F) + " need " + std::to_string(need) +
                                 " bytes of workspace; the static scratch holds " +
                                 std::to_string(kMlpScratchBytes) + " (use xmh3_w8a8_mlp with a workspace)");
  XMH3_REQUIRE(x && w1 && s1 && w2 && s2 && y, "w8a8_mlp_noalloc: null pointer");
  void* base = nullptr;
  rc = scratch_ptr(&base);
  if (rc) return rc;
  const MlpWs ws = carve(base, M, D, F, false);
  return mlp_core(x, x_dtype, M, D, F, ldx, w1, s1, s1_per_channel, w2, s2, s2_per_channel, y, ldy, ws, stream);
}
