/*
 * Plain-C restatement of the integer/byte rules of the quantized DiT-block
 * path. TEST INFRASTRUCTURE ONLY: loaded by tests (ctypes) to pin the
 * torch-CPU oracle with a third, language-independent implementation.
 * Built with -ffp-contract=off -fno-fast-math so every fp32 operation rounds
 * once, in program order.
 *
 * Rules (CK = backends/turbo/vendor/comfy_kitchen in the reference):
 *   row quantizer   CK/backends/eager/quantization.py:815-826, 857-875
 *   its stochastic rounding (bf16 rows)
 *                   CK/backends/cuda/ops/int8_linear.cu:79-91, 186-195
 *   int8 GEMM       CK/backends/eager/quantization.py:749-783 (torch._int_mm)
 *   dequant         CK/backends/eager/quantization.py:1028-1054
 *   W4 decode       CK/backends/eager/w4a8_int8.py:344-363
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static float bf16_to_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static uint16_t f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* x: bf16 bits [M,K]; q: int8 [M,K]; s: fp32 [M] (the unrounded scale). */
void orc_quant_rows_bf16(const uint16_t* x, int64_t M, int64_t K, int8_t* q, float* s) {
    for (int64_t m = 0; m < M; ++m) {
        const uint16_t* row = x + m * K;
        float amax = 0.0f;
        for (int64_t k = 0; k < K; ++k) {
            float a = fabsf(bf16_to_f32(row[k]));
            if (a > amax) amax = a;
        }
        float scale = amax / 127.0f;
        if (scale < 1e-30f) scale = 1e-30f;
        s[m] = scale;
        float sb = bf16_to_f32(f32_to_bf16(scale));
        if (sb == 0.0f) sb = 1.17549435e-38f;
        for (int64_t k = 0; k < K; ++k) {
            float v = bf16_to_f32(row[k]) / sb;
            float vb = bf16_to_f32(f32_to_bf16(v));
            float r = nearbyintf(vb);
            if (r > 127.0f) r = 127.0f;
            if (r < -128.0f) r = -128.0f;
            q[m * K + k] = (int8_t)r;
        }
    }
}

/* The PCG-RXS-M-XS output hash keying the stochastic rounding noise. */
static uint32_t pcg32_output_hash(uint32_t x) {
    uint32_t state = x * 747796405u + 2891336453u;
    uint32_t word = ((state >> ((state >> 28u) + 4u)) ^ state) * 277803737u;
    return (word >> 22u) ^ word;
}

void orc_pcg_hash(const uint32_t* x, int64_t n, uint32_t* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = pcg32_output_hash(x[i]);
}

/* As orc_quant_rows_bf16 with stochastic rounding: element (m, k) gets
 * u = (hash(lo32(key) ^ hi32(key)) >> 8) * 2^-24, key = m*K + k + seed,
 * n = bf16(u), code = floor(bf16(v + n)) with the sum added in fp32 and then
 * rounded to bf16. */
void orc_quant_rows_sr_bf16(const uint16_t* x, int64_t M, int64_t K, uint64_t seed, int8_t* q, float* s) {
    for (int64_t m = 0; m < M; ++m) {
        const uint16_t* row = x + m * K;
        float amax = 0.0f;
        for (int64_t k = 0; k < K; ++k) {
            float a = fabsf(bf16_to_f32(row[k]));
            if (a > amax) amax = a;
        }
        float scale = amax / 127.0f;
        if (scale < 1e-30f) scale = 1e-30f;
        s[m] = scale;
        float sb = bf16_to_f32(f32_to_bf16(scale));
        if (sb == 0.0f) sb = 1.17549435e-38f;
        for (int64_t k = 0; k < K; ++k) {
            float vb = bf16_to_f32(f32_to_bf16(bf16_to_f32(row[k]) / sb));
            uint64_t key = (uint64_t)(m * K + k) + seed;
            uint32_t h = pcg32_output_hash((uint32_t)key ^ (uint32_t)(key >> 32));
            float u = (float)(h >> 8) * 0x1p-24f;
            float nb = bf16_to_f32(f32_to_bf16(u));
            float r = floorf(bf16_to_f32(f32_to_bf16(vb + nb)));
            if (r > 127.0f) r = 127.0f;
            if (r < -128.0f) r = -128.0f;
            q[m * K + k] = (int8_t)r;
        }
    }
}

/* acc[M,N] = a[M,K] . w[N,K]^T in int32 (the sums never exceed 2^31 for
 * K <= 131072 with int8 operands). */
void orc_int_mm(const int8_t* a, const int8_t* w, int64_t M, int64_t N, int64_t K, int32_t* acc) {
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) {
            int64_t t = 0;
            for (int64_t k = 0; k < K; ++k) t += (int64_t)a[m * K + k] * (int64_t)w[n * K + k];
            acc[m * N + n] = (int32_t)t;
        }
}

/* out = bf16(float(acc) * (sx[m] * sw[n or 0])) */
void orc_dequant_bf16(const int32_t* acc, const float* sx, const float* sw, int sw_per_channel,
                      int64_t M, int64_t N, uint16_t* out) {
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) {
            float scl = sx[m] * sw[sw_per_channel ? n : 0];
            float v = (float)acc[m * N + n] * scl;
            out[m * N + n] = f32_to_bf16(v);
        }
}

/* packed [N, K/2] (low nibble = even k), s_rel fp32 [N, K/G] -> int8 [N, K] */
void orc_w4_decode(const uint8_t* packed, const float* s_rel, int64_t N, int64_t K, int64_t G,
                   int8_t* out) {
    int64_t groups = K / G;
    for (int64_t n = 0; n < N; ++n)
        for (int64_t k = 0; k < K; ++k) {
            uint8_t b = packed[n * (K / 2) + k / 2];
            int code = (k & 1) ? (b >> 4) & 0xF : b & 0xF;
            float v = (float)(code - 8) * s_rel[n * groups + k / G];
            float r = nearbyintf(v);
            if (r > 127.0f) r = 127.0f;
            if (r < -127.0f) r = -127.0f;
            out[n * K + k] = (int8_t)r;
        }
}
