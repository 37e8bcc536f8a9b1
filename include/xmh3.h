/*
 * xmh3.h -- C ABI of the MI355X (gfx950) quantized DiT-block hot path.
 *
 * Library: x-minimaxh3_amd/libxmh3_hip.so (hipcc, gfx950 only).
 *
 * Conventions
 *   - Plain pointers to device memory, int64 sizes/strides (in elements unless
 *     stated), int dtype codes, and the caller's HIP stream. Nothing here
 *     allocates; outputs and workspaces are owned by the caller.
 *   - dtype codes follow the reference's op boundary
 *     (CK/backends/eager/quantization.py:34-42): 0 fp32, 1 fp16, 2 bf16.
 *   - input-activation codes follow CK/backends/_activations.py:19-24:
 *     0 none, 1 gelu_tanh, 2 swiglu (swiglu only through the ConvRot quantizer).
 *   - Every entry point returns 0 on success, 1 invalid argument, 2 HIP
 *     launch error, 3 unsupported combination; the message is available from
 *     xmh3_last_error() on the calling thread. No C++ exception crosses the
 *     ABI. All work is stream-ordered; no entry point synchronises the host.
 *
 * Reference paths are relative to the reference root; CK abbreviates
 * backends/turbo/vendor/comfy_kitchen.
 */
#ifndef XMH3_H
#define XMH3_H

#include <stddef.h>
#include <stdint.h>
#ifndef __cplusplus
#include <stdbool.h>
#endif

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* xmh3_stream_t; /* == hipStream_t */

/* Message of the last failing call on this thread. */
const char* xmh3_last_error(void);
int xmh3_abi_version(void);

/*
 * Per-token dynamic int8 quantisation, optionally after GELU-tanh.
 * Replaces: CK/backends/cuda/ops/int8_linear.cu:1035
 *   launch_quantize_int8_rowwise_kernel(in, out, scales, M, K, dtype, ...)
 * (semantics of CK/backends/eager/quantization.py:857-875, the public op
 * CK/__init__.py:702-709 quantize_int8_rowwise; the activation of
 * CK/backends/_activations.py:40-53).
 * x: [M, ldx] of x_dtype; q: int8 [M, K] contiguous; scale: fp32 [M].
 */
int xmh3_quantize_int8_rowwise(const void* x, int x_dtype, int input_act, int64_t M, int64_t K,
                               int64_t ldx, int8_t* q, float* scale, xmh3_stream_t stream);

/*
 * quantize_int8_rowwise with the stochastic_rounding seed: stochastic == 0 is
 * xmh3_quantize_int8_rowwise (no input act); otherwise each code is
 * floor(T(v + T(u))) with v = T(x / T(s)) as in the nearest path and
 * u = (pcg(lo32(k) ^ hi32(k)) >> 8) * 2^-24, k = row * K + col + seed
 * (uint64), pcg the 32-bit PCG-RXS-M-XS output hash: the reference CUDA
 * quantizer's deterministic noise. Scales as xmh3_quantize_int8_rowwise.
 * Replaces: the rowwise quantizer launcher with stochastic = true, seed
 * (CK/backends/cuda/ops/int8_linear.cu:1035-1075, kernel :158-197).
 */
int xmh3_quantize_int8_rowwise_sr(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, int8_t* q,
                                  float* scale, int stochastic, uint64_t seed, xmh3_stream_t stream);

/*
 * As xmh3_quantize_int8_rowwise, and also writes 0 to clear_rows[0..M) (the
 * row-|max| slots the fused MLP's fc1 epilogue accumulates into; NULL = none):
 * the first kernel of the MLP chain. Same reference interface as above.
 */
int xmh3_quantize_int8_rowwise_ex(const void* x, int x_dtype, int input_act, int64_t M, int64_t K,
                                  int64_t ldx, int8_t* q, float* scale, uint32_t* clear_rows,
                                  xmh3_stream_t stream);

/*
 * Per-token int8 quantisation of a rotated linear's input:
 *   a = act(x)  (input_act 0 none, 1 gelu_tanh, 2 swiglu: x rows are
 *               [gate | up], 2*K wide, a = T(T(silu(gate)) * up))
 *   r = T(a_g @ H) per group of G = 4^n columns (H = H4 (x) ... (x) H4 / 2^n)
 *   (q, scale) = quantize_int8_rowwise(r)
 * group_size G in {4, 16, 64, 256, 1024} (the reference's fused kernel takes
 * 256, its eager path any power of 4) or 0 (no rotation; then input_act must
 * be 2). K (the activated width) % 256 == 0 and % G == 0, K <= 16384; x rows
 * 16-byte aligned (ldx % 8 == 0); x bf16 or fp16.
 * q: int8 [M, K] contiguous; scale: fp32 [M].
 * Replaces: CK/backends/cuda/ops/int8_linear.cu:1295
 *   launch_quantize_int8_rowwise_convrot64_kernel(input, output, scales, rows,
 *   cols, group_size, dtype, stochastic, act_code, block_threads, seed, stream)
 * (semantics of CK/backends/eager/quantization.py:998-1023 with convrot=True,
 * CK/tensor/int8_utils.py:11-74, CK/backends/_activations.py:40-53).
 */
int xmh3_quantize_int8_rowwise_convrot(const void* x, int x_dtype, int input_act, int64_t M, int64_t K,
                                       int64_t ldx, int group_size, int8_t* q, float* scale,
                                       xmh3_stream_t stream);

/*
 * xmh3_quantize_int8_rowwise_convrot with the launcher's stochastic, seed
 * pair: stochastic != 0 (seed nonzero) rounds each code as
 * xmh3_quantize_int8_rowwise_sr does, the noise keyed by the code's index
 * row * K + col in the [M, K] output. Replaces the same launcher
 * (CK/backends/cuda/ops/int8_linear.cu:1295, kernel :943-1031, stochastic).
 */
int xmh3_quantize_int8_rowwise_convrot_sr(const void* x, int x_dtype, int input_act, int64_t M, int64_t K,
                                          int64_t ldx, int group_size, int8_t* q, float* scale, int stochastic,
                                          uint64_t seed, xmh3_stream_t stream);

/*
 * Requantise rows whose |max| is already known (bit pattern of the fp32
 * value), the second half of the fused MLP's per-token requant.
 * Replaces the quantizer call inside the fc2 int8_linear with
 * input_act="gelu_tanh" (CK/backends/eager/quantization.py:998,1023).
 * g: bf16/fp16 [M, ldg]; q: int8 [M, K]; scale: fp32 [M].
 */
int xmh3_requant_int8_rows(const void* g, int g_dtype, int64_t M, int64_t K, int64_t ldg,
                           const uint32_t* row_absmax_bits, int8_t* q, float* scale,
                           xmh3_stream_t stream);

/*
 * int8 x int8 -> int32 GEMM on MFMA with a fused epilogue:
 *   epilogue 0: out = T(float(acc) * (sx[m] * sw[n])) (+ bias[n] in T)
 *   epilogue 1: as 0 in bf16, then g = bf16(gelu_tanh(.)) stored, and max|g|
 *               per row folded into row_absmax_bits (must start at 0)
 *   epilogue 2: raw int32 accumulators into out (int32 [M, ldo])
 * A: int8 [M, lda] (activations), B: int8 [N, ldb] (weights, row = output
 * channel), K % 16 == 0, lda/ldb multiples of 16 bytes.
 * Replaces: CK/backends/cuda/ops/cutlass_gemm_int8.cu:612-683
 *   bool launch_cutlass_int8_dequant(a, b, xs, ws, bias, d, M, N, K, out_code, stream)
 * and the dequant kernel CK/backends/cuda/ops/int8_linear.cu:343-409
 * (eager order CK/backends/eager/quantization.py:1028-1054).
 */
int xmh3_int8_gemm(const int8_t* A, int64_t lda, const int8_t* B, int64_t ldb, int64_t M,
                   int64_t N, int64_t K, const float* sx, const float* sw, int sw_per_channel,
                   const void* bias, void* out, int out_dtype, int64_t ldo, int epilogue,
                   uint32_t* row_absmax_bits, xmh3_stream_t stream);

/*
 * fc2 of the H3 block with its gated residual update, in place:
 *   y = T(float(acc) * (sx[m] * sw[n])) (+ bias[n] in T)
 *   residual[m, n] = T(residual[m, n] + y * T(gate[gate_rows[m], n]))
 * T = the residual's dtype (bf16 or fp16); gate fp32 or T, [rows, ldg];
 * gate_rows int32 [M] (the modulation segment row of each token, clamped into
 * [0, gate_nrows) so a bad index cannot read past the table).
 * N, ldr and ldg multiples of 4; residual 8-byte aligned (fp32 gate: 16).
 * Replaces: h3serve/native_engine/model/fused_mlp.py:157-222
 *   _fused_down_gated_residual(hidden, residual, gate, gate_rows, qweight,
 *   weight_scale, bias) with its Triton kernel (fused_mlp.py:58-145), and the
 *   default route it stands for, int8_linear then addcmul_ per segment
 *   (fused_mlp.py:396-426, layers.py:937-953).
 */
int xmh3_int8_gemm_gated_residual(const int8_t* A, int64_t lda, const int8_t* B, int64_t ldb, int64_t M,
                                  int64_t N, int64_t K, const float* sx, const float* sw, int sw_per_channel,
                                  const void* bias, void* residual, int res_dtype, int64_t ldr,
                                  const void* gate, int gate_dtype, int64_t ldg, int64_t gate_nrows,
                                  const int32_t* gate_rows, xmh3_stream_t stream);

/*
 * Operand of the asymmetric W4A8 correction:
 *   out[m, g] = T(T(sum of q[m, g*gs .. g*gs+gs-1]) * T(xs[m]))
 * (T = out_dtype: 0 fp32, 1 fp16, 2 bf16); the caller then adds
 * out @ T(correction) [groups, N] to the int8 linear's output.
 * q: int8 [M, ldq] (16-byte aligned rows when gs % 16 == 0); xs: fp32 [M];
 * out: [M, ldo], ldo >= K / gs.
 * Replaces: the group-sum step of CK/backends/cuda/__init__.py:2294-2297
 *   sx = xq.view(m, groups, group_size).sum(-1, dtype=int32).to(out_dtype)
 *   sx = sx * xs.to(out_dtype)
 */
int xmh3_int8_group_sums(const int8_t* q, int64_t ldq, const float* xs, int64_t M, int64_t K,
                         int64_t group_size, void* out, int out_dtype, int64_t ldo, xmh3_stream_t stream);

/*
 * Grouped int4 -> int8 grid decode (low nibble = even k).
 * Replaces: CK/backends/cuda/ops/w4a8_gemm.cu:94
 *   launch_dequant_int4_grouped_to_int8(qw, s_rel, codebook, out, N, K, G, stream)
 * (eager CK/backends/eager/w4a8_int8.py:344-363).
 * packed: uint8 [N, K/2]; s_rel: fp32 or bf16 [N, K/G]; codebook: fp32 [16]
 * or NULL (levels code-8); out: int8 [N, K].
 */
int xmh3_w4_decode_int8(const uint8_t* packed, const void* s_rel, int s_rel_dtype,
                        const float* codebook, int64_t N, int64_t K, int64_t group_size,
                        int8_t* out, xmh3_stream_t stream);

/*
 * The W8A8 MLP block y = fc2(gelu_tanh(fc1(x))), bf16 output.
 * Replaces the MLP driver's two int8_linear calls
 * (h3serve/native_engine/model/fused_mlp.py:343-405, the op chain
 * CK/__init__.py:722-764 with input_act="gelu_tanh" on fc2).
 * x: [M, ldx] of x_dtype; w1: int8 [F, D]; s1: fp32 [F] or [1];
 * w2: int8 [D, F]; s2: fp32 [D] or [1]; y: bf16 [M, ldy].
 * workspace: xmh3_w8a8_mlp_workspace_bytes(M, D, F) bytes of device memory.
 */
size_t xmh3_w8a8_mlp_workspace_bytes(int64_t M, int64_t D, int64_t F);
int xmh3_w8a8_mlp(const void* x, int x_dtype, int64_t M, int64_t D, int64_t F, int64_t ldx,
                  const int8_t* w1, const float* s1, int s1_per_channel, const int8_t* w2,
                  const float* s2, int s2_per_channel, void* y, int64_t ldy, void* workspace,
                  size_t workspace_bytes, xmh3_stream_t stream);

/*
 * xmh3_w8a8_mlp without a caller workspace: the workspace is a file-scope
 * device array of 64 MiB per GPU (held until the process ends), so the call
 * allocates nothing -- for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). No
 * counterpart in the reference. Same arguments and results as
 * xmh3_w8a8_mlp; returns 1 (invalid argument) when
 * xmh3_w8a8_mlp_workspace_bytes(M, D, F) exceeds 64 MiB (more than 1,439
 * tokens at d_model 5120, ffn 13824; 3,358 at 1536, 6144). All calls on one GPU share the array:
 * calls that overlap on one GPU race.
 */
int xmh3_w8a8_mlp_noalloc(const void* x, int x_dtype, int64_t M, int64_t D, int64_t F, int64_t ldx,
                          const int8_t* w1, const float* s1, int s1_per_channel, const int8_t* w2,
                          const float* s2, int s2_per_channel, void* y, int64_t ldy, xmh3_stream_t stream);

/*
 * W4A8 GEMM with the int4 weights unpacked in LDS: out = T(float(acc) *
 * (sx[m] * s_channel[n])) (+ bias), acc[m, n] = sum_k A[m, k] * w8[n, k],
 * w8 = clamp(rint((code - 8) * s_rel[n, k/128]), +-127) decoded tile by tile
 * inside the GEMM (no decoded weight in memory). A: int8 [M, lda];
 * packed: [N, ldp] bytes (low nibble = even k); s_rel: bf16 or fp32 [N, s_rel_ld]
 * (s_rel_dtype 2 or 0); group_size 128; K % 256 == 0; bf16 output. Every
 * weight tile is decoded once per 256-row tile of A, so this form pays off
 * only where decoding once to memory does not (measured slower than
 * xmh3_w4_decode_int8 + xmh3_int8_gemm at every M from 256 to 25,200).
 * Replaces: CK/backends/cuda/ops/w4a8_gemm.cu:123-165 (column-chunked decode
 * into a scratch buffer feeding the int8 GEMM) and the decode + int8_linear
 * of CK/backends/eager/w4a8_int8.py:457-508.
 */
int xmh3_w4a8_gemm(const int8_t* A, int64_t lda, const uint8_t* packed, int64_t ldp, const void* s_rel,
                   int s_rel_dtype, int64_t s_rel_ld, int64_t M, int64_t N, int64_t K, int64_t group_size,
                   const float* sx, const float* s_channel, const void* bias, void* out, int out_dtype,
                   int64_t ldo, xmh3_stream_t stream);

/*
 * The W4A8 MLP block: grouped int4 weights (uniform levels, no rotation),
 * s_rel fp32 or bf16 [N, K/G], per-channel fp32 s_channel. Each weight is
 * decoded once per call to the int8 grid (HBM-bound) into a workspace region
 * that is idle while it is live, then the W8A8 chain runs: the workspace is
 * the W8A8 one when M >= D (plus F*D bytes when M < D, plus another F*D when
 * 2M < D). group_size is the weights' group (the workspace does not depend
 * on it).
 * Replaces: the chunked W4A8 MLP (h3serve/native_engine/model/fused_mlp.py:222-266)
 * over w4a8_int8_linear (CK/tensor/w4a8_int8.py:89-115, eager
 * CK/backends/eager/w4a8_int8.py:457-508 decomposed as decode + int8_linear).
 */
size_t xmh3_w4a8_mlp_workspace_bytes(int64_t M, int64_t D, int64_t F, int64_t group_size);
int xmh3_w4a8_mlp(const void* x, int x_dtype, int64_t M, int64_t D, int64_t F, int64_t ldx,
                  const uint8_t* w1_packed, const void* w1_srel, const float* w1_schannel,
                  const uint8_t* w2_packed, const void* w2_srel, const float* w2_schannel,
                  int srel_dtype, int64_t group_size, void* y, int64_t ldy, void* workspace,
                  size_t workspace_bytes, xmh3_stream_t stream);

/*
 * Fused AdaLN-modulated RMSNorm + split-half RoPE for Q and K of the same
 * tokens (k_in/k_out may be NULL): RMS over the full row of `width`, rotation
 * per head of head_dim (128) with a table [tokens or 1,
 * head_dim/2, 2, 2] of freqs_dtype (fp32 or x's dtype); scale/shift rows
 * [R, mod_ld] of x's dtype, token t uses row t / mod_group (NULL: no AdaLN).
 * In-place is allowed (q_out == q_in).
 * Replaces: rms_adaln (CK/__init__.py:130-150, eager CK/backends/eager/adaln.py:17-20)
 * followed by apply_rope_split_half (CK/__init__.py:629-650, eager
 * CK/backends/eager/rope.py:39-48).
 */
int xmh3_norm_rope(const void* q_in, void* q_out, const void* k_in, void* k_out, int dtype,
                   int64_t tokens, int64_t width, int64_t ld_in, int64_t ld_out, const void* scale,
                   const void* shift, int mod_dtype, int64_t mod_ld, int64_t mod_group,
                   const void* freqs, int freqs_dtype, int64_t freqs_token_stride, int head_dim,
                   float eps, xmh3_stream_t stream);

/*
 * rms_norm(x [* norm_weight]) * (1 + scale[r]) + shift[r], r = row_map[t]
 * (if non-NULL) else t / mod_group; output in torch's promoted dtype of
 * (x, scale). With a row map, mod_group is the number of rows of the scale /
 * shift tables and map entries are clamped into [0, mod_group), so a bad map
 * never reads outside the tables.
 * Replaces: CK/backends/cuda/ops/adaln.cu:256-313 (launcher of the
 * (RMS-)AdaLN kernels), eager CK/backends/eager/adaln.py:17-20; with
 * norm_weight and row_map the H3 segmented form
 * h3serve/native_engine/model/kernels.py:7586-7634.
 */
int xmh3_rms_adaln(const void* x, void* out, int dtype, int64_t rows, int64_t width, int64_t ld_in,
                   int64_t ld_out, const void* norm_weight, const void* scale, const void* shift,
                   int mod_dtype, int64_t mod_ld, const int32_t* row_map, int64_t mod_group,
                   float eps, xmh3_stream_t stream);

/*
 * Split-half RoPE on strided [B, S, H, head_dim] (last dim contiguous), with
 * (norm=1) or without (norm=0) the per-head RMSNorm with weight; rotates the
 * first rot_dim dims (0 = all), the tail is norm-only. out may alias x.
 * freqs: [*, *, *, rot_dim/2, 2, 2] with element strides freqs_strides[0..2]
 * over (B, S, H) (0 = broadcast).
 * Replaces: CK/backends/cuda/ops/rms_rope.cu:353-384
 *   launch_rms_rope_kernel(...) (split-half mode), eager
 *   CK/backends/eager/rope.py:67-92,178-189 and 39-48.
 */
int xmh3_rope_split_half(void* x, void* out, int dtype, int64_t B, int64_t S, int64_t H,
                         int64_t head_dim, const int64_t* x_strides, const int64_t* out_strides,
                         const void* norm_weight, int weight_dtype, const void* freqs,
                         int freqs_dtype, const int64_t* freqs_strides, int rot_dim, float eps,
                         int norm, xmh3_stream_t stream);

/*
 * xmh3_rope_split_half with the pair layout chosen: split_half = 1 pairs
 * (i, i + rot_dim/2), split_half = 0 the interleaved pairs (2i, 2i + 1) of
 * CK/backends/eager/rope.py:10-16 (rotation f[.,0]*x0 then addcmul_ of
 * f[.,1]*x1, one fused multiply-add in the table dtype), rot_dim and
 * head_dim multiples of 8. Same operands otherwise.
 * Replaces: CK/backends/cuda/ops/rms_rope.cu:353-384 launch_rms_rope_kernel
 *   (both modes), eager CK/backends/eager/rope.py:10-36 (apply_rope*) and
 *   67-118,146-167 (rms_rope*).
 */
int xmh3_rope_heads(void* x, void* out, int dtype, int64_t B, int64_t S, int64_t H, int64_t head_dim,
                    const int64_t* x_strides, const int64_t* out_strides, const void* norm_weight,
                    int weight_dtype, const void* freqs, int freqs_dtype, const int64_t* freqs_strides,
                    int rot_dim, float eps, int norm, int split_half, xmh3_stream_t stream);

/*
 * xmh3_rope_heads of Q and K [B, S, H, head_dim] with one table, each with
 * its own strides, output and norm weight (both of weight_dtype). When the
 * two tensors share strides (and outputs share strides), the per-head norm
 * and full split-half rotation (norm = 1, split_half = 1, rot_dim 0 or
 * head_dim, head_dim 64, 96 or 128, 16-bit values, the table shared by a
 * token's heads) run in one launch over the rows of Q then K; otherwise one
 * xmh3_rope_heads call per tensor. Outputs may alias their inputs.
 * Replaces: CK/backends/cuda/ops/rms_rope.cu:353-384 launch_rms_rope_kernel
 *   (q and k in one call); eager CK/backends/eager/rope.py:129-143,178-189
 *   (rms_rope_split_half, rms_rope_split_half_).
 */
int xmh3_rope_heads_qk(void* q, void* q_out, void* k, void* k_out, int dtype, int64_t B, int64_t S, int64_t H,
                       int64_t head_dim, const int64_t* q_strides, const int64_t* q_out_strides,
                       const int64_t* k_strides, const int64_t* k_out_strides, const void* q_weight,
                       const void* k_weight, int weight_dtype, const void* freqs, int freqs_dtype,
                       const int64_t* freqs_strides, int rot_dim, float eps, int norm, int split_half,
                       xmh3_stream_t stream);

/*
 * The reference's per-head RMSNorm + RoPE launcher under its own name and
 * 46-argument list (7 pointers; batch, dim1, dim2, head_dim, rot_dim; the
 * table's three leading sizes; 4 strides each of q, k, q_out, k_out; 6 table
 * strides; the q / k weight strides; epsilon; input, table and weight dtype
 * codes; has_k; split_half; stream), so a ctypes caller with pinned argtypes
 * (h3serve/native_engine/model/single_qknorm_rope.py:36-66,158-187) binds
 * this library unchanged. Runs the kernels of xmh3_rope_heads_qk (q and k
 * with norm weights) or xmh3_rope_heads in either pair layout. Returns nothing, as the reference does: an argument
 * outside this build's support (a strided head dimension, weight or table
 * pair layout) launches nothing and sets xmh3_last_error().
 * Replaces: CK/backends/cuda/ops/rms_rope.cu:353-384 launch_rms_rope_kernel.
 */
void launch_rms_rope_kernel(const void* q, const void* k, const void* freqs, const void* q_scale,
                            const void* k_scale, void* q_out, void* k_out, int64_t batch, int64_t dim1,
                            int64_t dim2, int64_t head_dim, int64_t rot_dim, int64_t freqs_batch,
                            int64_t freqs_dim1, int64_t freqs_dim2, int64_t q_s0, int64_t q_s1, int64_t q_s2,
                            int64_t q_s3, int64_t k_s0, int64_t k_s1, int64_t k_s2, int64_t k_s3,
                            int64_t qo_s0, int64_t qo_s1, int64_t qo_s2, int64_t qo_s3, int64_t ko_s0,
                            int64_t ko_s1, int64_t ko_s2, int64_t ko_s3, int64_t f_s0, int64_t f_s1,
                            int64_t f_s2, int64_t f_s3, int64_t f_s4, int64_t f_s5, int64_t qs_stride,
                            int64_t ks_stride, float epsilon, int input_dtype_code, int freqs_dtype_code,
                            int scale_dtype_code, bool has_k, bool split_half, xmh3_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* XMH3_H */
