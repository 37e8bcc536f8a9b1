// int8 x int8 -> int32 GEMM on gfx950 MFMA with fused epilogues.
//
//   acc[m,n] = sum_k A[m,k] * B[n,k]        (A: [M,K] row-major activations,
//                                             B: [N,K] row-major weights)
// Epilogues (the reference's dequant, CK/backends/eager/quantization.py:1028-1054,
// CK = backends/turbo/vendor/comfy_kitchen):
//   EPI_DEQUANT : out = T(float(acc) * (sx[m] * sw[n])) (+ bias in T)
//   EPI_GELU    : h = bf16(...as above...); g = bf16(gelu_tanh(h)); store g and
//                 atomically fold max|g| per row into row_amax (fp32 bits) --
//                 fc1 of the fused MLP, feeding the per-token requant of fc2
//   EPI_INT32   : raw int32 accumulators (parity of the contraction itself)
//   EPI_GATED   : y = T(...as EPI_DEQUANT...); residual[m,n] =
//                 T(residual[m,n] + y * T(gate[gate_rows[m], n])) in place --
//                 fc2 of the H3 block with its AdaLN-gated residual update
//                 (h3serve/native_engine/model/fused_mlp.py:396-426,
//                 layers.py:937-953: int8_linear, then addcmul_ per segment;
//                 the product of two 16-bit floats is exact in fp32, so the
//                 only rounding before T is the add)
//
// Tiling: 256x256 block tile. The main kernel (K % 256 == 0,
// gemm_i8_pp_kernel) runs 8 waves, two per SIMD, that alternate between an
// MFMA phase and a memory phase (LDS refill by direct-to-LDS DMA, fragment
// reads), each wave owning a 128x64 sub-tile of v_mfma_i32_16x16x64_i8
// accumulators. Other K use 4-wave kernels (128x128 per wave, 256 AGPRs):
// DMA-fed for K % 128 == 0, register-staged otherwise. LDS tiles hold
// XOR-swizzled 16-byte chunks so ds_read_b128 is conflict-free. Workgroups
// are remapped so each XCD (own L2) walks a contiguous, GROUP_M-swizzled band
// of tiles.
#pragma once

#include "common.hpp"
#include "tile_map.hpp"
#include "w4_lut.hpp"

#include <type_traits>
#include <utility>

namespace xmh3 {

typedef int v4i __attribute__((ext_vector_type(4)));

// Compile-time loop: f(std::integral_constant<int, I>{}) for I in [0, N).
// Accumulator blocks are addressed only through these constants, so they can
// never become a dynamically indexed (scratch) array.
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

enum Epi : int { EPI_DEQUANT = 0, EPI_GELU = 1, EPI_INT32 = 2, EPI_GATED = 3 };

struct GemmArgs {
  const int8_t* A;
  const int8_t* B;
  int64_t lda, ldb;  // bytes
  int M, N, K;
  const float* sx;   // [M]
  const float* sw;   // [N] or [1]
  int sw_per_channel;
  const void* bias;  // [N] in the output dtype, nullable
  void* out;
  int64_t ldo;       // elements
  uint32_t* row_amax;
  int tiles_m, tiles_n;
  // EPI_GATED: out is the residual (read and written in place)
  const void* gate;            // [rows, N]: fp32 or the output dtype
  int64_t ldg;                 // elements
  int gate_f32;
  const int32_t* gate_rows;    // [M], clamped into [0, gate_nrows)
  int gate_nrows;
  int row_stores;              // dequant epilogue may store whole rows (N, ldo % 8 == 0, out 16-B aligned)
  // W4 weights (gemm_i8_pp_kernel<..., true>): B is the packed int4 [N, K/2]
  // (row stride ldb bytes) decoded in LDS with s_rel [N, K/128] (row stride
  // srel_ld elements, bf16 or fp32); sw is s_channel
  const void* srel;
  int64_t srel_ld;
  int srel_bf16;
};

constexpr int BM = 256, BN = 256, NTHREADS = 256;

// XOR swizzle of the 16-byte chunk index inside an LDS row of BK bytes.
template <int BK>
__device__ __forceinline__ int swz(int row, int chunk) {
  if constexpr (BK == 64) return chunk ^ ((row >> 1) & 3);
  else return chunk ^ (row & 7);
}

// 4 consecutive outputs -> one 8- or 16-byte store
__device__ __forceinline__ void store4(uint16_t* p, const float* v, BF16T) {
  *reinterpret_cast<uint2*>(p) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
}
__device__ __forceinline__ void store4(uint16_t* p, const float* v, F16T) {
  uint2 w;
  w.x = f32_to_f16(v[0]) | (f32_to_f16(v[1]) << 16);
  w.y = f32_to_f16(v[2]) | (f32_to_f16(v[3]) << 16);
  *reinterpret_cast<uint2*>(p) = w;
}
__device__ __forceinline__ void store4(float* p, const float* v, F32T) {
  *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
}

// Epilogue shared by the main loops. Lane holds, for accumulator block (i, j)
// of a wave sub-tile at (row0, col0): row m = row0 + i*16 + lane%16, columns
// n = col0 + j*16 + 4*(lane/16) + {0..3}. Straight-line code only
// (compile-time block indices, guards as predicates) so the accumulators stay
// in registers. The row and column scales of the sub-tile are all loaded in
// one batch when the main loop ends (the fragment registers are free then), so
// the epilogue pays one memory latency instead of one per output element.
//
// An epilogue reads its scales through a scale source: row(i) is the row
// scale of row em + 16 i, col4(j, w) the column scales of columns
// en + 16 j + {0..3}, bias4<TO>(p, n, j, b) the bias there as a float (value
// in TO); em = row0 + lane % 16 and en = col0 + 4 (lane / 16).
template <int NI = 8, int NJ = 8>
struct EpiScalesT {
  float sx[NI];      // rows m = em + 16 i
  float sw[NJ][4];   // columns n = en + 16 j + r
  __device__ __forceinline__ float row(int i) const { return sx[i]; }
  __device__ __forceinline__ void col4(int j, float (&w)[4]) const {
#pragma unroll
    for (int r = 0; r < 4; ++r) w[r] = sw[j][r];
  }
  template <typename TO>
  __device__ __forceinline__ void bias4(const GemmArgs& p, int n, int, float (&b)[4]) const {
    const typename TO::storage* brow = static_cast<const typename TO::storage*>(p.bias);
#pragma unroll
    for (int r = 0; r < 4; ++r) b[r] = TO::load(brow[min(n + r, p.N - 1)]);
  }
};
using EpiScales = EpiScalesT<8, 8>;

// The same scales staged once per wave in LDS (the ping-pong kernel, whose
// 128 VGPRs per lane cannot also hold 24 scales and 16 bias values through
// the epilogue): [128] row scales | [64] column scales | [64] bias (float),
// one 1 KiB region per wave, written and read by that wave only.
struct LdsScales {
  const float* base;
  int m16, c4;
  __device__ __forceinline__ float row(int i) const { return base[16 * i + m16]; }
  __device__ __forceinline__ void col4(int j, float (&w)[4]) const {
    const float4 v = *reinterpret_cast<const float4*>(base + 128 + 16 * j + c4);
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
  }
  template <typename TO>
  __device__ __forceinline__ void bias4(const GemmArgs&, int, int j, float (&b)[4]) const {
    const float4 v = *reinterpret_cast<const float4*>(base + 192 + 16 * j + c4);
    b[0] = v.x; b[1] = v.y; b[2] = v.z; b[3] = v.w;
  }
};
constexpr int LDS_SCALES_BYTES = 1024;

// Stage a 128 x 64 wave sub-tile's scales (and bias) at dst: four loads per
// lane (indices clamped into range; rows and columns past the end are never
// stored) in place of 24 (+16) per lane.
template <int EPI, typename TO>
__device__ __forceinline__ LdsScales stage_scales(const GemmArgs& p, int row0, int col0, int lane, float* dst) {
  if constexpr (EPI != EPI_INT32) {
    const float a = p.sx[min(row0 + lane, p.M - 1)];
    const float b = p.sx[min(row0 + 64 + lane, p.M - 1)];
    const float w = p.sw[p.sw_per_channel ? min(col0 + lane, p.N - 1) : 0];
    float bv = 0.0f;
    if (p.bias) bv = TO::load(static_cast<const typename TO::storage*>(p.bias)[min(col0 + lane, p.N - 1)]);
    dst[lane] = a;
    dst[64 + lane] = b;
    dst[128 + lane] = w;
    dst[192 + lane] = bv;
  }
  // a wave's LDS operations execute in order; the reads of other lanes'
  // values must stay below these writes
  asm volatile("" ::: "memory");
  return LdsScales{dst, lane & 15, 4 * (lane >> 4)};
}

// (row0, col0): origin of the wave's NI*16 x NJ*16 sub-tile
template <int EPI, int NI, int NJ>
__device__ __forceinline__ void load_scales_t(const GemmArgs& p, int row0, int col0, int lane,
                                              EpiScalesT<NI, NJ>& sc) {
  // Branch-free: indices are clamped into range (rows and columns past the
  // end are never stored), so every load is issued up front in one batch
  // instead of being sunk into a conditional block next to its use.
  if constexpr (EPI != EPI_INT32) {
    const int em = row0 + (lane & 15);
    const int en = col0 + 4 * (lane >> 4);
    const int nmask = p.sw_per_channel ? -1 : 0;   // per-tensor scale: index 0
#pragma unroll
    for (int i = 0; i < NI; ++i) sc.sx[i] = p.sx[min(em + i * 16, p.M - 1)];
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) sc.sw[j][r] = p.sw[min(en + j * 16 + r, p.N - 1) & nmask];
  }
}

template <int EPI>
__device__ __forceinline__ void load_scales(const GemmArgs& p, int m0, int n0, int wm, int wn, int lane,
                                            EpiScales& sc) {
  load_scales_t<EPI, 8, 8>(p, m0 + wm * 128, n0 + wn * 128, lane, sc);
}

template <int EPI, typename TO, bool VEC_OUT, bool BIAS, int NI, int NJ, typename SC>
__device__ __forceinline__ void epilogue_body(const GemmArgs& p, v4i (&acc)[NI][NJ], const SC& sc,
                                              int row0, int col0, int lane) {
  const int em = row0 + (lane & 15);
  const int en = col0 + 4 * (lane >> 4);
  static_for<NI>([&](auto I) {
    constexpr int i = I;
    const int m = em + i * 16;
    const bool mok = m < p.M;
    float amax = 0.0f;
    float sxm = 0.0f;
    if constexpr (EPI != EPI_INT32) sxm = sc.row(i);
    static_for<NJ>([&](auto J) {
      constexpr int j = J;
      const int n = en + j * 16;
      if constexpr (EPI == EPI_INT32) {
        int32_t* orow = static_cast<int32_t*>(p.out) + (int64_t)m * p.ldo;
        if (mok) {
          if (VEC_OUT && n + 3 < p.N) {
            *reinterpret_cast<v4i*>(orow + n) = acc[i][j];
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r)
              if (n + r < p.N) orow[n + r] = acc[i][j][r];
          }
        }
      } else {
        typename TO::storage* orow = static_cast<typename TO::storage*>(p.out) + (int64_t)m * p.ldo;
        float v[4], w[4], bv[4];
        sc.col4(j, w);
        if constexpr (BIAS) sc.template bias4<TO>(p, n, j, bv);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const bool nok = n + r < p.N;
          float y = (float)acc[i][j][r] * (sxm * w[r]);
          // the stores round to TO once; the bias add and GELU need the value
          // in TO first (the reference materialises it there)
          if constexpr (BIAS || EPI == EPI_GELU) y = TO::round(y);
          if constexpr (BIAS) y = TO::round(y + bv[r]);
          if constexpr (EPI == EPI_GELU) {
            y = TO::round(gelu_tanh_f32(y));
            amax = fmaxf(amax, nok ? fabsf(y) : 0.0f);
          }
          v[r] = y;
        }
        if (mok) {
          if (VEC_OUT && n + 3 < p.N) {
            store4(orow + n, v, TO{});
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r)
              if (n + r < p.N) orow[n + r] = (typename TO::storage)TO::store(v[r]);
          }
        }
      }
    });
    if constexpr (EPI == EPI_GELU) {
      amax = fmaxf(amax, __shfl_xor(amax, 16, 64));
      amax = fmaxf(amax, __shfl_xor(amax, 32, 64));
      if (lane < 16 && mok) atomicMax(p.row_amax + m, __float_as_uint(amax));
    }
  });
}

// EPI_GATED: the residual and gate values of row block I+1 are fetched while
// block I is computed and stored (the residual is read and written by the
// same lane, so its loads are issued explicitly ahead of the stores rather
// than left to the compiler, which cannot move loads above stores to the same
// buffer). Host contract: N, ldo and ldg are multiples of 4 and the residual
// and gate rows 8- (16- for an fp32 gate) byte aligned, so every column block
// of 4 is one vector load; rows and columns past the end are clamped for the
// loads and not stored.
template <typename TO, bool BIAS, int NI, int NJ, typename SC>
__device__ __forceinline__ void epilogue_gated(const GemmArgs& p, v4i (&acc)[NI][NJ], const SC& sc,
                                               int row0, int col0, int lane) {
  using S = typename TO::storage;
  const int em = row0 + (lane & 15);
  const int en = col0 + 4 * (lane >> 4);
  S* const res_base = static_cast<S*>(p.out);
  uint2 res[2][NJ];
  float gt[2][NJ][4];
  auto fetch = [&](auto I) __attribute__((always_inline)) {
    constexpr int i = I, b = i & 1;
    const int m = min(em + i * 16, p.M - 1);
    const int64_t grow = min(max(p.gate_rows[m], 0), p.gate_nrows - 1);
    const S* rrow = res_base + (int64_t)m * p.ldo;
    static_for<NJ>([&](auto J) {
      constexpr int j = J;
      const int n = min(en + j * 16, p.N - 4);
      res[b][j] = *reinterpret_cast<const uint2*>(rrow + n);
      if (p.gate_f32) {
        const float4 g4 = *reinterpret_cast<const float4*>(static_cast<const float*>(p.gate) + grow * p.ldg + n);
        gt[b][j][0] = g4.x; gt[b][j][1] = g4.y; gt[b][j][2] = g4.z; gt[b][j][3] = g4.w;
      } else {
        const uint2 g2 = *reinterpret_cast<const uint2*>(static_cast<const S*>(p.gate) + grow * p.ldg + n);
        gt[b][j][0] = TO::load(g2.x & 0xffffu); gt[b][j][1] = TO::load(g2.x >> 16);
        gt[b][j][2] = TO::load(g2.y & 0xffffu); gt[b][j][3] = TO::load(g2.y >> 16);
      }
    });
  };
  fetch(std::integral_constant<int, 0>{});
  static_for<NI>([&](auto I) {
    constexpr int i = I, b = i & 1;
    if constexpr (i + 1 < NI) fetch(std::integral_constant<int, i + 1>{});
    const int m = em + i * 16;
    const bool mok = m < p.M;
    const float sxm = sc.row(i);
    S* orow = res_base + (int64_t)m * p.ldo;
    static_for<NJ>([&](auto J) {
      constexpr int j = J;
      const int n = en + j * 16;
      const uint32_t rw[2] = {res[b][j].x, res[b][j].y};
      float v[4], w[4], bv[4];
      sc.col4(j, w);
      if constexpr (BIAS) sc.template bias4<TO>(p, n, j, bv);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float y = TO::round((float)acc[i][j][r] * (sxm * w[r]));
        if constexpr (BIAS) y = TO::round(y + bv[r]);
        const float g = TO::round(gt[b][j][r]);
        const float rv = TO::load((rw[r >> 1] >> (16 * (r & 1))) & 0xffffu);
        v[r] = TO::round(rv + y * g);
      }
      if (mok && n < p.N) store4(orow + n, v, TO{});
    });
  });
}

// The bias test is hoisted out of the element loop (a uniform branch per
// element otherwise).
template <int EPI, typename TO, bool VEC_OUT, int NI, int NJ, typename SC>
__device__ __forceinline__ void epilogue_t(const GemmArgs& p, v4i (&acc)[NI][NJ], const SC& sc,
                                           int row0, int col0, int lane) {
  if constexpr (EPI == EPI_GATED) {
    if (p.bias)
      epilogue_gated<TO, true>(p, acc, sc, row0, col0, lane);
    else
      epilogue_gated<TO, false>(p, acc, sc, row0, col0, lane);
  } else {
    if (EPI != EPI_INT32 && p.bias)
      epilogue_body<EPI, TO, VEC_OUT, true>(p, acc, sc, row0, col0, lane);
    else
      epilogue_body<EPI, TO, VEC_OUT, false>(p, acc, sc, row0, col0, lane);
  }
}

template <int EPI, typename TO, bool VEC_OUT>
__device__ __forceinline__ void epilogue(const GemmArgs& p, v4i (&acc)[8][8], const EpiScales& sc, int m0,
                                         int n0, int wm, int wn, int lane) {
  epilogue_t<EPI, TO, VEC_OUT, 8, 8>(p, acc, sc, m0 + wm * 128, n0 + wn * 128, lane);
}

template <int BK, int EPI, typename TO, bool VEC_OUT>
__global__ __launch_bounds__(NTHREADS, 1) void gemm_i8_kernel(GemmArgs p) {
  constexpr int CPR = BK / 16;                 // 16-byte chunks per tile row
  constexpr int TILE_BYTES = BM * BK;          // A tile == B tile size
  constexpr int LOADS = TILE_BYTES / 16 / NTHREADS;  // 16-byte loads per thread per operand
  constexpr int KSUB = BK / 64;                // MFMA k-steps per BK
  __shared__ __attribute__((aligned(16))) int8_t lds[2][2][TILE_BYTES];

  int tm, tn;
  tile_coords(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // global load coordinates (same for A and B)
  int ld_row[LOADS], ld_chunk[LOADS];
#pragma unroll
  for (int i = 0; i < LOADS; ++i) {
    const int c = tid + NTHREADS * i;
    ld_row[i] = c / CPR;
    ld_chunk[i] = c % CPR;
  }
  const int8_t* a_ptr[LOADS];
  const int8_t* b_ptr[LOADS];
  bool a_ok[LOADS], b_ok[LOADS];
#pragma unroll
  for (int i = 0; i < LOADS; ++i) {
    const int ar = m0 + ld_row[i], br = n0 + ld_row[i];
    a_ok[i] = ar < p.M;
    b_ok[i] = br < p.N;
    a_ptr[i] = p.A + (int64_t)(a_ok[i] ? ar : 0) * p.lda + ld_chunk[i] * 16;
    b_ptr[i] = p.B + (int64_t)(b_ok[i] ? br : 0) * p.ldb + ld_chunk[i] * 16;
  }
  int lds_off[LOADS];
#pragma unroll
  for (int i = 0; i < LOADS; ++i) lds_off[i] = ld_row[i] * BK + swz<BK>(ld_row[i], ld_chunk[i]) * 16;

  uint4 ra[LOADS], rb[LOADS];
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const bool kok = (k0 + ld_chunk[i] * 16) < p.K;
      ra[i] = (a_ok[i] && kok) ? *reinterpret_cast<const uint4*>(a_ptr[i] + k0) : make_uint4(0, 0, 0, 0);
      rb[i] = (b_ok[i] && kok) ? *reinterpret_cast<const uint4*>(b_ptr[i] + k0) : make_uint4(0, 0, 0, 0);
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      *reinterpret_cast<uint4*>(&lds[buf][0][lds_off[i]]) = ra[i];
      *reinterpret_cast<uint4*>(&lds[buf][1][lds_off[i]]) = rb[i];
    }
  };

  v4i acc[8][8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = v4i{0, 0, 0, 0};

  // fragment read offsets: row = base + lane%16, chunk = kk*4 + lane/16
  const int frow = lane & 15, fchunk = lane >> 4;

  const int ksteps = (p.K + BK - 1) / BK;
  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < ksteps; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < ksteps) gload((kt + 1) * BK);
#pragma unroll
    for (int kk = 0; kk < KSUB; ++kk) {
      v4i af[8], bf[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int r = wm * 128 + i * 16 + frow;
        af[i] = *reinterpret_cast<const v4i*>(&lds[cur][0][r * BK + swz<BK>(r, kk * 4 + fchunk) * 16]);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int r = wn * 128 + j * 16 + frow;
        bf[j] = *reinterpret_cast<const v4i*>(&lds[cur][1][r * BK + swz<BK>(r, kk * 4 + fchunk) * 16]);
      }
      static_for<8>([&](auto I) {
        static_for<8>([&](auto J) {
          acc[I][J] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bf[J], af[I], acc[I][J], 0, 0, 0);
        });
      });
    }
    if (kt + 1 < ksteps) sstore(cur ^ 1);
    __syncthreads();
  }

  EpiScales sc;
  load_scales<EPI>(p, m0, n0, wm, wn, lane, sc);
  epilogue<EPI, TO, VEC_OUT>(p, acc, sc, m0, n0, wm, wn, lane);
}

// ---------------------------------------------------------------------------
// main loop v2 (K % 128 == 0): global -> LDS by DMA (global_load_lds_dwordx4),
// 4 LDS stages of BK = 64, loads issued up to 4 K-steps ahead, no VGPR staging.
//
// Stage s holds the A tile [256 rows][64 B] at offset 0 and the B tile at
// 16 KiB, each row's four 16-byte chunks XOR-swizzled (chunk ^ ((row>>1)&3)).
// A DMA instruction writes 1 KiB contiguous (lane l -> byte 16*l), i.e. 16
// rows; the swizzle is applied on the global side by choosing which chunk
// each lane fetches. Rows past M or N are clamped to the last valid row (their
// products only reach outputs that are never stored).
//
// Synchronisation per K-step t: each wave waits (s_waitcnt) until its own
// fragment reads of stage t are in registers and its DMA for stage t+1 has
// landed, then s_barrier (no fence, so the loads of later stages stay in
// flight); after the barrier no wave reads stage t's buffer any more, so it
// takes stage t+4.
// ---------------------------------------------------------------------------
#ifndef XMH3_DMA_STAGES
#define XMH3_DMA_STAGES 3
#endif
#ifndef XMH3_DMA_SCHED
#define XMH3_DMA_SCHED 1
#endif
constexpr int DMA_BK = 64, DMA_STAGES = XMH3_DMA_STAGES, DMA_STAGE_BYTES = 2 * BM * DMA_BK;
typedef __attribute__((address_space(3))) void lds_void_t;

// s_waitcnt with vmcnt = 8 * n (8 DMA instructions per thread per stage) and
// the expcnt / lgkmcnt fields at their maximum (no wait on them)
template <int N>
__device__ __forceinline__ void wait_vm_n() {
  constexpr int v = 8 * N;
  __builtin_amdgcn_s_waitcnt((v & 15) | ((v >> 4) << 14) | (7 << 4) | (15 << 8));
}
__device__ __forceinline__ void wait_vm(int outstanding_stages) {
  if (outstanding_stages >= 4) wait_vm_n<4>();
  else if (outstanding_stages == 3) wait_vm_n<3>();
  else if (outstanding_stages == 2) wait_vm_n<2>();
  else if (outstanding_stages == 1) wait_vm_n<1>();
  else wait_vm_n<0>();
}
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xc07f); }

template <int EPI, typename TO, bool VEC_OUT>
__global__ __launch_bounds__(NTHREADS, 1) void gemm_i8_dma_kernel(GemmArgs p) {
  __shared__ __attribute__((aligned(1024))) int8_t lds[DMA_STAGES][DMA_STAGE_BYTES];

  int tm, tn;
  tile_coords(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave >> 1, wn = wave & 1;

  // DMA sources: wave w fills 16-row blocks b = 4w + i (i < 4) of A and B.
  // Uniform 64-bit bases + per-lane 32-bit offsets (the host guarantees the
  // operands span < 2^31 bytes), so each DMA is one saddr+voffset load.
  const int8_t* a_base = p.A + (int64_t)m0 * p.lda;
  const int8_t* b_base = p.B + (int64_t)n0 * p.ldb;
  uint32_t a_off_g[4], b_off_g[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = (wave * 4 + i) * 16 + (lane >> 2);
    const int c = (lane & 3) ^ ((r >> 1) & 3);
    a_off_g[i] = (uint32_t)(min(r, p.M - 1 - m0) * (int)p.lda + c * 16);
    b_off_g[i] = (uint32_t)(min(r, p.N - 1 - n0) * (int)p.ldb + c * 16);
  }
  auto issue = [&](int kslice, int slot) __attribute__((always_inline)) {
    int8_t* base = &lds[slot % DMA_STAGES][0];
    const int8_t* ab = a_base + (int64_t)kslice * DMA_BK;
    const int8_t* bb = b_base + (int64_t)kslice * DMA_BK;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      __builtin_amdgcn_global_load_lds(ab + a_off_g[i], (lds_void_t*)(base + (wave * 4 + i) * 1024), 16, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      __builtin_amdgcn_global_load_lds(bb + b_off_g[i], (lds_void_t*)(base + BM * DMA_BK + (wave * 4 + i) * 1024),
                                       16, 0, 0);
  };

  v4i acc[8][8];
  static_for<8>([&](auto I) { static_for<8>([&](auto J) { acc[I][J] = v4i{0, 0, 0, 0}; }); });

  // fragment offsets within a stage: row = base + lane%16, logical chunk lane/16
  const int frow = lane & 15, fchunk = lane >> 4;
  int a_off[8], b_off[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int ra = wm * 128 + i * 16 + frow, rb = wn * 128 + i * 16 + frow;
    a_off[i] = ra * DMA_BK + ((fchunk ^ ((ra >> 1) & 3)) * 16);
    b_off[i] = BM * DMA_BK + rb * DMA_BK + ((fchunk ^ ((rb >> 1) & 3)) * 16);
  }
  // Fragments are double-buffered in registers: while the MFMAs of step t run
  // on one set, the LDS reads of step t+1 fill the other.
  auto load_frags = [&](int t, v4i (&af)[8], v4i (&bf)[8]) __attribute__((always_inline)) {
    const int8_t* st = &lds[t % DMA_STAGES][0];
#pragma unroll
    for (int j = 0; j < 8; ++j) bf[j] = *reinterpret_cast<const v4i*>(st + b_off[j]);
#pragma unroll
    for (int i = 0; i < 8; ++i) af[i] = *reinterpret_cast<const v4i*>(st + a_off[i]);
  };
  auto mfmas = [&](v4i (&af)[8], v4i (&bf)[8]) __attribute__((always_inline)) {
    static_for<8>([&](auto I) {
      static_for<8>([&](auto J) {
        acc[I][J] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bf[J], af[I], acc[I][J], 0, 0, 0);
      });
    });
  };
  v4i fa0[8], fb0[8], fa1[8], fb1[8];

  // Every step has the same branch-free body, so the scheduler can interleave
  // the DMA and the LDS reads with the MFMAs. In the last STAGES steps the DMA
  // re-fetches the final K-slice into buffers that are never read again, and
  // the last step's fragment reads fetch data that is never used; both stay in
  // bounds. ksteps is even (host: K % 128 == 0), so the 2x unrolled loop has
  // no tail.
  const int ksteps = p.K / DMA_BK;
#pragma unroll
  for (int s = 0; s < DMA_STAGES; ++s) issue(min(s, ksteps - 1), s);
  wait_vm_n<DMA_STAGES - 1>();
  asm volatile("s_barrier" ::: "memory");
  load_frags(0, fa0, fb0);

  // Step t: [own fragment reads of step t done] + [own DMA of stage t+1
  // landed] -> barrier (no wave reads stage t's buffer any more, so it takes
  // stage t+STAGES) -> refill -> reads of step t+1 -> MFMAs of step t.
  auto step = [&](int t, v4i (&af)[8], v4i (&bf)[8], v4i (&an)[8], v4i (&bn)[8]) __attribute__((always_inline)) {
    wait_lgkm0();
    wait_vm_n<DMA_STAGES - 2>();
    asm volatile("s_barrier" ::: "memory");
    issue(min(t + DMA_STAGES, ksteps - 1), t + DMA_STAGES);
    load_frags(t + 1, an, bn);
    mfmas(af, bf);
#if XMH3_DMA_SCHED
    static_for<8>([&](auto) {
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // one DMA
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // two fragment reads
      __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);  // eight MFMAs
    });
#endif
  };
  for (int t = 0; t < ksteps; t += 2) {
    step(t, fa0, fb0, fa1, fb1);
    step(t + 1, fa1, fb1, fa0, fb0);
  }
  wait_vm_n<0>();  // no DMA may land after the workgroup's LDS is released
  EpiScales sc;
  load_scales<EPI>(p, m0, n0, wm, wn, lane, sc);
  epilogue<EPI, TO, VEC_OUT>(p, acc, sc, m0, n0, wm, wn, lane);
}

// ---------------------------------------------------------------------------
// ping-pong main loop (K % 256 == 0): 8 waves, two per SIMD, in two groups
// that alternate roles at every workgroup barrier. Waves 0-3 (group P) and
// 4-7 (group Q) share SIMDs pairwise (the dispatcher places wave w on SIMD
// w % 4): while one group issues its 64 MFMAs of a K-step (128 bytes of K),
// the other refills LDS and reads its fragments of the same K-step, so each
// SIMD's MFMA pipe is fed by one wave or the other. Each wave owns a 128 x 64
// sub-tile (rows 128*(w&1), columns 64*(w>>1)): 8 x 4 accumulators of
// v_mfma_i32_16x16x64_i8 in 128 AGPRs, 96 VGPRs of fragments.
//
// LDS (160 KiB). int8 weights: the B tile (256 rows x 128 bytes = 32 KiB per
// K-step) in a ring of three buffers at [0, 96K), the A tile in two buffers
// at [96K, 160K). A 16-byte chunk c of row r sits at slot c ^ (r & 7)
// (conflict-free ds_read_b128). The DMA is buffer_load_dwordx4 ... lds, 8
// whole 128-byte rows per instruction, rows past M or N clamped to the last
// valid row (their products reach no stored output).
//
// Phases (P one phase ahead of Q; both groups run 1 + 2T barriers):
//   P, memory phase of step t : A slice t+1 -> A buffer (t+1)&1, read step t
//   P, MFMA phase of step t   : 64 MFMAs (the last 4 after the barrier that
//                               ends the phase), A slice t+1 landed
//   Q, memory phase of step t : B slice t+2 -> B buffer (t+2)%3, read step t,
//                               B slice t+1 landed
//   Q, MFMA phase of step t   : 64 MFMAs
// so each memory phase carries 8 DMA and 24 fragment reads per wave, A
// slices are issued two phases and B slices three phases before they are
// read.
//
// W4 weights (group 128 = one K-step): the B ring holds the decoded int8
// tile in two buffers at [0, 64K) and A is at [64K, 128K). Wave w owns B rows
// 32w .. 32w+31: their packed int4 slice (64 bytes per row and step) and
// s_rel dwords are staged by DMA in the wave's own part of [128K, 146K). In
// its memory phase of step t the wave first decodes slice t+1 through the
// rows' 16-entry level tables (w4_lut.hpp) into the int8 B buffer (t+1)&1
// (P's half in phase 2t, Q's in 2t+1, both before the barrier that opens P's
// reads of step t+1), then stages slice t+2 in the buffer it has just read
// and issues its A refill. Decoding before issuing keeps the only DMA still
// in flight at the decode the one it waits for. The MFMA side and the
// epilogue are those of int8 weights, with s_channel as the per-channel
// scale.
// ---------------------------------------------------------------------------
constexpr int PP_BK = 128;                 // K bytes per step
constexpr int PP_THREADS = 512;
constexpr int PP_TILE = BM * PP_BK;        // 32 KiB: one operand tile of one step
constexpr int PP_LDS = 5 * PP_TILE;        // 160 KiB
constexpr int PP_TAIL = 4;                 // MFMAs of P's phase issued after its barrier
constexpr int PP_SLICE = 16 * 144;         // per-wave epilogue transpose slice
constexpr int PP_W4_PK0 = 4 * PP_TILE;     // W4: packed B slice staging (16 KiB)
constexpr int PP_W4_SR0 = PP_W4_PK0 + BN * PP_BK / 2;   // W4: s_rel staging (256 bytes per wave)
template <bool W4>
constexpr int pp_a0() { return W4 ? 2 * PP_TILE : 3 * PP_TILE; }   // A ring

// Raw buffer resource over [base, base + bytes): word 3 is the gfx9 data format
// for untyped dword access.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t raw_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// s_waitcnt vmcnt(N) with expcnt / lgkmcnt at their maximum (no wait on them)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

__device__ __forceinline__ void s_barrier() { asm volatile("s_barrier" ::: "memory"); }

// Dequant epilogue with whole-line stores: the wave's 128 x 64 sub-tile goes
// through an LDS slice 16 rows at a time (row stride 144 bytes) and is read
// back so that 8 consecutive lanes hold one row's 128 bytes: every
// global_store_dwordx4 then writes 8 whole rows, where the MFMA layout's
// 8-byte pieces would touch 16 lines a quarter each (measured: 9 % of the
// 720p fc1 GEMM). Values are computed as in epilogue_body (dequant, optional
// bias in TO, one rounding to TO). Host contract: N % 8 == 0, ldo % 8 == 0,
// out 16-byte aligned.
template <typename TO, bool BIAS>
__device__ __forceinline__ void epilogue_rows_lds(const GemmArgs& p, v4i (&acc)[8][4], const LdsScales& sc,
                                                  int row0, int col0, int lane, int8_t* slice) {
  using S = typename TO::storage;
  const int q = lane >> 4, m16 = lane & 15;
  const int rr = lane >> 3, ch = lane & 7;
  const int col = col0 + ch * 8;
  int8_t* wr = slice + m16 * 144 + 8 * q;
  const int8_t* rd = slice + rr * 144 + ch * 16;
  static_for<8>([&](auto I) {
    constexpr int i = I;
    const float sxm = sc.row(i);
    static_for<4>([&](auto J) {
      constexpr int j = J;
      float v[4], sw[4], bv[4];
      sc.col4(j, sw);
      if constexpr (BIAS) sc.template bias4<TO>(p, 0, j, bv);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float y = (float)acc[i][j][r] * (sxm * sw[r]);
        if constexpr (BIAS) y = TO::round(TO::round(y) + bv[r]);
        v[r] = y;
      }
      uint2 w;
      w.x = TO::store2(v[0], v[1]);
      w.y = TO::store2(v[2], v[3]);
      *reinterpret_cast<uint2*>(wr + 32 * j) = w;
    });
    // the wave's LDS operations execute in order; keep the compiler from
    // moving the reads above the writes of other lanes
    asm volatile("" ::: "memory");
    const uint4 o0 = *reinterpret_cast<const uint4*>(rd);
    const uint4 o1 = *reinterpret_cast<const uint4*>(rd + 8 * 144);
    asm volatile("" ::: "memory");
    const int m = row0 + i * 16 + rr;
    if (col < p.N) {
      if (m < p.M) *reinterpret_cast<uint4*>(static_cast<S*>(p.out) + (int64_t)m * p.ldo + col) = o0;
      if (m + 8 < p.M) *reinterpret_cast<uint4*>(static_cast<S*>(p.out) + (int64_t)(m + 8) * p.ldo + col) = o1;
    }
  });
}

template <int EPI, typename TO, bool VEC_OUT, bool W4>
__global__ __launch_bounds__(PP_THREADS, 1) void gemm_i8_pp_kernel(GemmArgs p) {
  __shared__ __attribute__((aligned(1024))) int8_t lds[PP_LDS];
  constexpr int A0 = pp_a0<W4>();

  int tm, tn;
  tile_coords(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave & 1, wn = wave >> 1;
  const bool grp_p = wave < 4;
  const int rows_a = min(BM, p.M - m0), rows_b = min(BN, p.N - n0);
  const int lda = (int)p.lda, ldb = (int)p.ldb;
  // int8 weights: P waves DMA the A tile, Q waves the B tile, rows
  // 64*dw .. 64*dw + 63. W4: P waves DMA A, every wave its packed B rows.
  const int dw = wave & 3;
  const __amdgpu_buffer_rsrc_t rsrc = (grp_p || W4) ? raw_rsrc(p.A + (int64_t)m0 * p.lda, (uint32_t)(rows_a * lda))
                                                    : raw_rsrc(p.B + (int64_t)n0 * p.ldb, (uint32_t)(rows_b * ldb));
  const uint32_t lim = (uint32_t)(((grp_p || W4) ? rows_a : rows_b) - 1);
  const uint32_t ld = (uint32_t)((grp_p || W4) ? lda : ldb);
  // lane l of DMA instruction g fetches row r0 + 8g (clamped), 16-byte chunk
  // (l & 7) ^ (row & 7), landing at byte 16 l of the instruction's 1 KiB
  const int r0 = dw * 64 + (lane >> 3);
  const uint32_t c16 = (uint32_t)(((lane & 7) ^ ((lane >> 3) & 7)) * 16);
  // The offsets are formed right before each DMA (volatile asm, so the
  // compiler cannot hoist the 8 of them into live registers and spill).
  auto dma_off = [&](auto G) __attribute__((always_inline)) {
    constexpr int g = decltype(G)::value;
    uint32_t v;
    asm volatile("v_add_u32 %0, %1, %2\n\tv_min_u32 %0, %0, %3\n\tv_mad_u32_u24 %0, %0, %4, %5"
                 : "=&v"(v) : "i"(8 * g), "v"(r0), "s"(lim), "s"(ld), "v"(c16));
    return v;
  };
  // this wave's 64 rows of K-slice kslice -> the operand buffer at buf_off
  auto issue = [&](int kslice, int buf_off) __attribute__((always_inline)) {
    const int soff = kslice * PP_BK;
    int8_t* base = lds + buf_off + dw * 8192;
    static_for<8>([&](auto G) {
      constexpr int g = decltype(G)::value;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void_t*)(base + g * 1024), 16, dma_off(G), soff, 0, 0);
    });
  };

  // W4: wave w's packed rows 32w .. 32w+31 (64 bytes each per step), two DMA
  // of 16 rows, and one dword DMA of the rows' s_rel (lane l: row 32w + l;
  // a bf16 value is read in its 4-byte aligned dword, which lies in the same
  // page as the value). The decoding lane's row is 32w + lane/2, its half of
  // the row's 128 codes lane & 1.
  const int w4_row = 32 * wave + (lane >> 1), w4_half = lane & 1;
  __amdgpu_buffer_rsrc_t rsrc_w4, rsrc_sr;
  uint32_t pk_off[2] = {0, 0}, sr_off = 0;
  int sr_esize = 4;
  if constexpr (W4) {
    rsrc_w4 = raw_rsrc(p.B + (int64_t)n0 * p.ldb, (uint32_t)(rows_b * ldb));
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      const int r = 32 * wave + 16 * g + (lane >> 2);
      pk_off[g] = (uint32_t)(min(r, rows_b - 1) * ldb + (lane & 3) * 16);
    }
    sr_esize = p.srel_bf16 ? 2 : 4;
    // based at s_rel itself (4-byte aligned, host-checked) so that each
    // dword offset below is 4-byte aligned in memory
    const uint32_t sr_bytes = (uint32_t)(((int64_t)(n0 + rows_b) * p.srel_ld * sr_esize + 3) & ~3LL);
    rsrc_sr = raw_rsrc(p.srel, sr_bytes);
    sr_off = (uint32_t)((int64_t)(n0 + min(32 * wave + lane, rows_b - 1)) * p.srel_ld * sr_esize);
  }
  auto issue_w4 = [&](int kslice) __attribute__((always_inline)) {
    int8_t* base = lds + PP_W4_PK0 + wave * 2048;
#pragma unroll
    for (int g = 0; g < 2; ++g)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc_w4, (lds_void_t*)(base + g * 1024), 16, pk_off[g],
                                               kslice * (PP_BK / 2), 0, 0);
    const uint32_t e = sr_off + (uint32_t)(kslice * sr_esize);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc_sr, (lds_void_t*)(lds + PP_W4_SR0 + wave * 256), 4, e & ~3u, 0, 0,
                                             0);
  };
  // decode this lane's 64 codes of the staged slice kslice into B buffer bbuf
  auto decode_w4 = [&](int kslice, int bbuf) __attribute__((always_inline)) {
    const int8_t* src = lds + PP_W4_PK0 + wave * 2048 + (lane >> 1) * 64 + w4_half * 32;
    const uint4 p0 = *reinterpret_cast<const uint4*>(src);
    const uint4 p1 = *reinterpret_cast<const uint4*>(src + 16);
    const uint32_t sw = *reinterpret_cast<const uint32_t*>(lds + PP_W4_SR0 + wave * 256 + (lane >> 1) * 4);
    float s;
    if (p.srel_bf16) {
      // the value sits in the upper half of its dword when its element index is odd
      const bool upper = (((int64_t)(n0 + min(w4_row, rows_b - 1)) * p.srel_ld + kslice) & 1) != 0;
      s = bf16_to_f32(upper ? (sw >> 16) : (sw & 0xffffu));
    } else {
      s = __uint_as_float(sw);
    }
    uint32_t lut[4];
#pragma unroll
    for (int w = 0; w < 4; ++w)
      lut[w] = w4_entry4((float)(4 * w - 8), (float)(4 * w - 7), (float)(4 * w - 6), (float)(4 * w - 5), s);
    const uint32_t pw[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
    int8_t* dst = lds + bbuf * PP_TILE + w4_row * PP_BK;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint4 o = make_uint4(w4_lookup4<0x01010000u>(pw[2 * c], lut), w4_lookup4<0x03030202u>(pw[2 * c], lut),
                                 w4_lookup4<0x01010000u>(pw[2 * c + 1], lut),
                                 w4_lookup4<0x03030202u>(pw[2 * c + 1], lut));
      *reinterpret_cast<uint4*>(dst + (((4 * w4_half + c) ^ (w4_row & 7)) * 16)) = o;
    }
  };

  v4i acc[8][4];
  static_for<8>([&](auto I) { static_for<4>([&](auto J) { acc[I][J] = v4i{0, 0, 0, 0}; }); });

  // fragment (i or j, half h): row base + lane%16, logical chunk 4h + lane/16
  const int frow = lane & 15, fchunk = lane >> 4;
  const int fa_off = A0 + (wm * 128 + frow) * PP_BK;
  const int fb_off = (wn * 64 + frow) * PP_BK;
  const int sw0 = ((fchunk) ^ (frow & 7)) * 16, sw1 = ((4 + fchunk) ^ (frow & 7)) * 16;
  v4i fa[2][8], fb[2][4];
  auto load_frags = [&](auto ASTG, int bbuf) __attribute__((always_inline)) {
    constexpr int sa = decltype(ASTG)::value;
    const int8_t* pa = lds + fa_off + sa * PP_TILE;
    const int8_t* pb = lds + fb_off + bbuf * PP_TILE;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int sw = h ? sw1 : sw0;
#pragma unroll
      for (int j = 0; j < 4; ++j) fb[h][j] = *reinterpret_cast<const v4i*>(pb + sw + j * 16 * PP_BK);
#pragma unroll
      for (int i = 0; i < 8; ++i) fa[h][i] = *reinterpret_cast<const v4i*>(pa + sw + i * 16 * PP_BK);
    }
  };
  // MFMAs [BEG, END) of a step (index h*32 + i*4 + j). They are inline asm
  // with the accumulator tied in place ("+a"): with the builtin the register
  // allocator rotates the accumulator tuples through copies every pass. The
  // step's last MFMA carries, inside the same asm statement, the wait states
  // a VALU read of its accumulators needs, skipped by a scalar branch unless
  // this is the tile's last step: the hazard is invisible to the compiler,
  // which may place accumulator copies or spills right after the loop, and
  // the other steps only pay a branch that executes under the MFMAs still in
  // the pipe.
  auto mfmas = [&](int last, auto BEG, auto END) __attribute__((always_inline)) {
    constexpr int b = decltype(BEG)::value, e = decltype(END)::value;
    static_for<2>([&](auto H) {
      static_for<8>([&](auto I) {
        static_for<4>([&](auto J) {
          constexpr int idx = H * 32 + I * 4 + J;
          if constexpr (idx >= b && idx < e) {
            v4i& c = acc[I][J];
            const v4i& xb = fb[H][J];
            const v4i& xa = fa[H][I];
            const int lst = __builtin_amdgcn_readfirstlane(last);   // an SGPR operand in every variant
            if constexpr (idx == 63)
              asm volatile(
                  "v_mfma_i32_16x16x64_i8 %0, %1, %2, %0\n\t"
                  "s_cmp_eq_u32 %3, 0\n\t"
                  "s_cbranch_scc1 1f\n\t"
                  "s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n"
                  "1:"
                  : "+a"(c) : "v"(xb), "v"(xa), "s"(lst) : "scc");
            else
              asm volatile("v_mfma_i32_16x16x64_i8 %0, %1, %2, %0" : "+a"(c) : "v"(xb), "v"(xa));
          }
        });
      });
    });
  };
  using C0 = std::integral_constant<int, 0>;
  using C1 = std::integral_constant<int, 1>;
  using M0 = std::integral_constant<int, 0>;
  using MT = std::integral_constant<int, 64 - PP_TAIL>;
  using M64 = std::integral_constant<int, 64>;
  const int ksteps = p.K / PP_BK;  // even, >= 2 (host: K % 256 == 0)

  // W4 prologue (every wave; P also its A slice 0): stage and decode slice 0
  // into B buffer 0, then stage slice 1.
  if constexpr (W4) {
    if (grp_p) issue(0, A0);
    issue_w4(0);
    wait_vmcnt<0>();
    decode_w4(0, 0);
    wait_lgkm0();
    issue_w4(min(1, ksteps - 1));
  }

  // Past the end the DMA re-fetches the last slice into buffers nobody reads
  // any more; everything stays in bounds.
  if (grp_p) {
    if constexpr (!W4) {
      issue(0, A0);
      wait_vmcnt<0>();
    }
    s_barrier();
    int bbuf = 0;
    auto step = [&](int t, auto ASTG) __attribute__((always_inline)) {
      constexpr int sa = decltype(ASTG)::value;
      const int last = __builtin_amdgcn_readfirstlane(t + 1 == ksteps);
      if constexpr (W4) {
        wait_vmcnt<0>();         // staged slice t+1 (already landed from step 1 on)
        decode_w4(min(t + 1, ksteps - 1), sa ^ 1);
        wait_lgkm0();
        issue_w4(min(t + 2, ksteps - 1));
      }
      issue(min(t + 1, ksteps - 1), A0 + (sa ^ 1) * PP_TILE);
      load_frags(ASTG, W4 ? sa : bbuf);
      if constexpr (!W4) bbuf = bbuf == 2 ? 0 : bbuf + 1;
      wait_lgkm0();
      s_barrier();
      mfmas(last, M0{}, MT{});
      wait_vmcnt<0>();           // A slice t+1 landed (W4: and the staged slice t+2)
      s_barrier();
      mfmas(last, MT{}, M64{});
    };
    for (int t = 0; t < ksteps; t += 2) {
      step(t, C0{});
      step(t + 1, C1{});
    }
  } else {
    if constexpr (!W4) {
      issue(0, 0);
      issue(min(1, ksteps - 1), PP_TILE);
      wait_vmcnt<0>();
    }
    s_barrier();
    int bbuf = 0, bnext = 2;
    // the barrier opening step t closes Q's MFMA phase of step t-1 (for
    // t = 0: P's first memory phase)
    auto step = [&](int t, auto ASTG) __attribute__((always_inline)) {
      constexpr int sa = decltype(ASTG)::value;
      s_barrier();
      if constexpr (W4) {
        wait_vmcnt<0>();         // staged slice t+1 landed
        decode_w4(min(t + 1, ksteps - 1), sa ^ 1);
        wait_lgkm0();
        issue_w4(min(t + 2, ksteps - 1));
        load_frags(ASTG, sa);
        wait_lgkm0();
      } else {
        issue(min(t + 2, ksteps - 1), bnext * PP_TILE);
        bnext = bnext == 2 ? 0 : bnext + 1;
        load_frags(ASTG, bbuf);
        bbuf = bbuf == 2 ? 0 : bbuf + 1;
        wait_lgkm0();
        wait_vmcnt<8>();         // slice t+1 landed; the 8 DMA of slice t+2 may stay in flight
      }
      s_barrier();
      mfmas(__builtin_amdgcn_readfirstlane(t + 1 == ksteps), M0{}, M64{});
    };
    for (int t = 0; t < ksteps; t += 2) {
      step(t, C0{});
      step(t + 1, C1{});
    }
  }
  wait_vmcnt<0>();  // no DMA may land after the workgroup's LDS is released
  const int row0 = m0 + wm * 128, col0 = n0 + wn * 64;
  // The A ring is idle once P has passed its last barrier (every A DMA has
  // landed and Q's last reads of it are done), so each wave's scale region
  // and transpose slice live there; the last refills of the other rings may
  // still be landing.
  static_assert(8 * PP_SLICE + 8 * LDS_SCALES_BYTES <= 2 * PP_TILE, "epilogue LDS exceeds the A ring");
  const LdsScales sc = stage_scales<EPI, TO>(
      p, row0, col0, lane, reinterpret_cast<float*>(lds + A0 + 8 * PP_SLICE + wave * LDS_SCALES_BYTES));
  if constexpr (EPI == EPI_DEQUANT && !std::is_same<TO, F32T>::value) {
    if (p.row_stores) {
      int8_t* slice = lds + A0 + wave * PP_SLICE;
      if (p.bias)
        epilogue_rows_lds<TO, true>(p, acc, sc, row0, col0, lane, slice);
      else
        epilogue_rows_lds<TO, false>(p, acc, sc, row0, col0, lane, slice);
      return;
    }
  }
  epilogue_t<EPI, TO, VEC_OUT, 8, 4>(p, acc, sc, row0, col0, lane);
}

// ---------------------------------------------------------------------------
// host launcher: picks the main loop for K and alignment. Instantiated per
// (epilogue, output type) in the gemm_i8_*.hip translation units, so the
// kernel families compile in parallel.
// ---------------------------------------------------------------------------
template <int BK, int EPI, typename TO>
inline int launch_gemm_T(GemmArgs& a, bool vec, hipStream_t st) {
  dim3 grid((unsigned)(a.tiles_m * a.tiles_n));
  const bool spans_ok = (int64_t)a.M * a.lda < (1LL << 31) && (int64_t)a.N * a.ldb < (1LL << 31);
  // the gated epilogue always has aligned vector rows (host contract): its
  // scalar-row variants are not instantiated
  constexpr bool only_vec = EPI == EPI_GATED;
  if (a.K % (2 * PP_BK) == 0 && spans_ok) {
    if (vec || only_vec)
      hipLaunchKernelGGL((gemm_i8_pp_kernel<EPI, TO, true, false>), grid, dim3(PP_THREADS), 0, st, a);
    else if constexpr (!only_vec)
      hipLaunchKernelGGL((gemm_i8_pp_kernel<EPI, TO, false, false>), grid, dim3(PP_THREADS), 0, st, a);
    return check_launch("gemm_i8_pp_kernel");
  }
  if (a.K % (2 * DMA_BK) == 0 && spans_ok) {
    if (vec || only_vec)
      hipLaunchKernelGGL((gemm_i8_dma_kernel<EPI, TO, true>), grid, dim3(NTHREADS), 0, st, a);
    else if constexpr (!only_vec)
      hipLaunchKernelGGL((gemm_i8_dma_kernel<EPI, TO, false>), grid, dim3(NTHREADS), 0, st, a);
    return check_launch("gemm_i8_dma_kernel");
  }
  if (vec || only_vec)
    hipLaunchKernelGGL((gemm_i8_kernel<BK, EPI, TO, true>), grid, dim3(NTHREADS), 0, st, a);
  else if constexpr (!only_vec)
    hipLaunchKernelGGL((gemm_i8_kernel<BK, EPI, TO, false>), grid, dim3(NTHREADS), 0, st, a);
  return check_launch("gemm_i8_kernel");
}

template <int EPI, typename TO>
int launch_gemm(GemmArgs& a, bool vec, hipStream_t st);

// W4 weights: K % 256 == 0, group 128, operand spans < 2^31 (host checks)
template <int EPI, typename TO>
inline int launch_gemm_w4_T(GemmArgs& a, hipStream_t st) {
  dim3 grid((unsigned)(a.tiles_m * a.tiles_n));
  hipLaunchKernelGGL((gemm_i8_pp_kernel<EPI, TO, true, true>), grid, dim3(PP_THREADS), 0, st, a);
  return check_launch("gemm_i8_pp_kernel (W4)");
}

#define XMH3_INSTANTIATE_GEMM(EPI, TO)                                      \
  template <>                                                             \
  int launch_gemm<EPI, TO>(GemmArgs & a, bool vec, hipStream_t st) {      \
    return launch_gemm_T<128, EPI, TO>(a, vec, st);                       \
  }

}  // namespace xmh3
