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
// Tiling: 256x256 block tile, 4 waves in a 2x2 grid, each wave owning a
// 128x128 sub-tile held as 8x8 accumulators of v_mfma_i32_16x16x64_i8 (256
// AGPRs). K advances BK bytes per step; A and B tiles are staged through LDS
// (double buffered, XOR-swizzled 16-byte chunks so ds_read_b128 is
// conflict-free), with the next step's global loads in flight while the
// current step's MFMAs run. Workgroups are remapped so each XCD (own L2)
// walks a contiguous, GROUP_M-swizzled band of tiles.
#include "common.hpp"

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
};

#ifndef XMH3_GROUP_M
#define XMH3_GROUP_M 4
#endif
#ifndef XMH3_NUM_XCD
#define XMH3_NUM_XCD 8
#endif
constexpr int BM = 256, BN = 256, NTHREADS = 256;
constexpr int GROUP_M = XMH3_GROUP_M;   // M-tiles per swizzle group
constexpr int NUM_XCD = XMH3_NUM_XCD;   // XCDs workgroups are dealt over

// XOR swizzle of the 16-byte chunk index inside an LDS row of BK bytes.
template <int BK>
__device__ __forceinline__ int swz(int row, int chunk) {
  if constexpr (BK == 64) return chunk ^ ((row >> 1) & 3);
  else return chunk ^ (row & 7);
}

// Map the hardware workgroup id to (tile_m, tile_n): contiguous logical tile
// ranges per XCD (workgroups are dealt round-robin over the XCDs), then a
// GROUP_M swizzle inside the logical order.
__device__ __forceinline__ void tile_coords(int pid, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int total = tiles_m * tiles_n;
  const int q = total / NUM_XCD, r = total % NUM_XCD;
  const int x = pid % NUM_XCD, j = pid / NUM_XCD;
  const int logical = (x < r) ? x * (q + 1) + j : r * (q + 1) + (x - r) * q + j;
  const int in_group = GROUP_M * tiles_n;
  const int group = logical / in_group;
  const int first_m = group * GROUP_M;
  const int gsize = min(tiles_m - first_m, GROUP_M);
  const int rem = logical - group * in_group;
  tm = first_m + rem % gsize;
  tn = rem / gsize;
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
template <int NI = 8, int NJ = 8>
struct EpiScalesT {
  float sx[NI];      // rows m = em + 16 i
  float sw[NJ][4];   // columns n = en + 16 j + r
};
using EpiScales = EpiScalesT<8, 8>;

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

template <int EPI, typename TO, bool VEC_OUT, bool BIAS, int NI, int NJ>
__device__ __forceinline__ void epilogue_body(const GemmArgs& p, v4i (&acc)[NI][NJ], const EpiScalesT<NI, NJ>& sc,
                                              int row0, int col0, int lane) {
  const int em = row0 + (lane & 15);
  const int en = col0 + 4 * (lane >> 4);
  static_for<NI>([&](auto I) {
    constexpr int i = I;
    const int m = em + i * 16;
    const bool mok = m < p.M;
    float amax = 0.0f;
    float sxm = 0.0f;
    if constexpr (EPI != EPI_INT32) sxm = sc.sx[i];
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
        const typename TO::storage* brow = static_cast<const typename TO::storage*>(p.bias);
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const bool nok = n + r < p.N;
          float y = (float)acc[i][j][r] * (sxm * sc.sw[j][r]);
          // the stores round to TO once; the bias add and GELU need the value
          // in TO first (the reference materialises it there)
          if constexpr (BIAS || EPI == EPI_GELU) y = TO::round(y);
          if constexpr (BIAS) y = TO::round(y + TO::load(brow[min(n + r, p.N - 1)]));
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
template <typename TO, bool BIAS, int NI, int NJ>
__device__ __forceinline__ void epilogue_gated(const GemmArgs& p, v4i (&acc)[NI][NJ], const EpiScalesT<NI, NJ>& sc,
                                               int row0, int col0, int lane) {
  using S = typename TO::storage;
  const int em = row0 + (lane & 15);
  const int en = col0 + 4 * (lane >> 4);
  S* const res_base = static_cast<S*>(p.out);
  const S* const brow = static_cast<const S*>(p.bias);
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
    const float sxm = sc.sx[i];
    S* orow = res_base + (int64_t)m * p.ldo;
    static_for<NJ>([&](auto J) {
      constexpr int j = J;
      const int n = en + j * 16;
      const uint32_t rw[2] = {res[b][j].x, res[b][j].y};
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float y = TO::round((float)acc[i][j][r] * (sxm * sc.sw[j][r]));
        if constexpr (BIAS) y = TO::round(y + TO::load(brow[min(n + r, p.N - 1)]));
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
template <int EPI, typename TO, bool VEC_OUT, int NI, int NJ>
__device__ __forceinline__ void epilogue_t(const GemmArgs& p, v4i (&acc)[NI][NJ], const EpiScalesT<NI, NJ>& sc,
                                           int row0, int col0, int lane) {
  if constexpr (EPI == EPI_GATED) {
    if (p.bias)
      epilogue_gated<TO, true, NI, NJ>(p, acc, sc, row0, col0, lane);
    else
      epilogue_gated<TO, false, NI, NJ>(p, acc, sc, row0, col0, lane);
  } else {
    if (EPI != EPI_INT32 && p.bias)
      epilogue_body<EPI, TO, VEC_OUT, true, NI, NJ>(p, acc, sc, row0, col0, lane);
    else
      epilogue_body<EPI, TO, VEC_OUT, false, NI, NJ>(p, acc, sc, row0, col0, lane);
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
// main loop v5 (K % 256 == 0): K-steps of 128 bytes, two LDS stages of
// 64 KiB (A tile [256][128] at 0, B tile at 32 KiB), each DMA instruction
// (buffer_load_dwordx4 ... lds) fetching 8 whole 128-byte rows, i.e. full
// cache lines: with 64-byte row pieces the same bytes cost twice the L1/L2
// transactions, and that request rate, not the MFMAs, set the loop's pace.
// A 16-byte chunk c of row r sits in LDS slot c ^ (r & 7) (ds_read_b128
// conflict-free). Each K-step runs as two 64-byte sub-steps whose fragments
// are double-buffered in VGPRs: X holds the k0 half, Y the k1 half.
//
//   step t (stage t&1):
//     sub 0: [X = (t, k0) ready]  read Y = (t, k1)       | MFMAs on X
//     sub 1: [Y ready, slice t+1 landed] barrier -> DMA slice t+2 into stage
//            t&1 (every wave has finished reading it) ; read X = (t+1, k0)
//            from stage (t+1)&1                          | MFMAs on Y
// A slice is therefore issued one full K-step (128 MFMAs per wave) before it
// is first read. The DMA goes through a buffer resource based at the
// workgroup's first row, so the K advance is a scalar offset; rows past M
// or N are clamped to the last valid row (their products reach no stored
// output).
// ---------------------------------------------------------------------------
constexpr int V5_BK = 128, V5_STAGE_BYTES = 2 * BM * V5_BK;

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

template <int EPI, typename TO, bool VEC_OUT>
__global__ __launch_bounds__(NTHREADS, 1) void gemm_i8_v5_kernel(GemmArgs p) {
  __shared__ __attribute__((aligned(1024))) int8_t lds[2 * V5_STAGE_BYTES];

  int tm, tn;
  tile_coords(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int rows_a = min(BM, p.M - m0), rows_b = min(BN, p.N - n0);
  const int lda = (int)p.lda, ldb = (int)p.ldb;
  const __amdgpu_buffer_rsrc_t ra = raw_rsrc(p.A + (int64_t)m0 * p.lda, (uint32_t)(rows_a * lda));
  const __amdgpu_buffer_rsrc_t rb = raw_rsrc(p.B + (int64_t)n0 * p.ldb, (uint32_t)(rows_b * ldb));

  // DMA: wave w fills 8-row blocks 8w + i (i < 8) of A and B; lane l fetches
  // row 8*(8w+i) + l/8, chunk (l&7) ^ (row&7), landing at LDS byte 16*l of
  // the block's 1 KiB.
  uint32_t voa[8], vob[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = (wave * 8 + i) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ (r & 7);
    voa[i] = (uint32_t)(min(r, rows_a - 1) * lda + c * 16);
    vob[i] = (uint32_t)(min(r, rows_b - 1) * ldb + c * 16);
  }
  // DMA pair g (A and B block 8*wave + g) of K-slice kslice into stage STG
  auto issue_pair = [&](int g, int kslice, auto STG) __attribute__((always_inline)) {
    constexpr int s = decltype(STG)::value;
    const int soff = kslice * V5_BK;
    int8_t* base = lds + s * V5_STAGE_BYTES + wave * 8192 + g * 1024;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void_t*)base, 16, voa[g], soff, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_void_t*)(base + BM * V5_BK), 16, vob[g], soff, 0, 0);
  };
  auto issue = [&](int kslice, auto STG) __attribute__((always_inline)) {
#pragma unroll
    for (int g = 0; g < 8; ++g) issue_pair(g, kslice, STG);
  };

  v4i acc[8][8];
  static_for<8>([&](auto I) { static_for<8>([&](auto J) { acc[I][J] = v4i{0, 0, 0, 0}; }); });

  // Fragment (i, half h): row wm*128 + 16 i + lane%16, logical chunk
  // 4h + lane/16; the swizzle term row&7 = lane&7, so every fragment of a
  // stage is one per-lane base plus a constant.
  const int frow = lane & 15, fchunk = lane >> 4;
  const int8_t* fa_base = lds + (wm * 128 + frow) * V5_BK;
  const int8_t* fb_base = lds + BM * V5_BK + (wn * 128 + frow) * V5_BK;
  const int sw0 = ((fchunk) ^ (frow & 7)) * 16, sw1 = ((4 + fchunk) ^ (frow & 7)) * 16;
  auto load_pair = [&](auto STG, auto HALF, int g, v4i (&af)[8], v4i (&bf)[8]) __attribute__((always_inline)) {
    constexpr int s = decltype(STG)::value;
    constexpr int h = decltype(HALF)::value;
    const int sw = h ? sw1 : sw0;
    bf[g] = *reinterpret_cast<const v4i*>(fb_base + sw + s * V5_STAGE_BYTES + g * 16 * V5_BK);
    af[g] = *reinterpret_cast<const v4i*>(fa_base + sw + s * V5_STAGE_BYTES + g * 16 * V5_BK);
  };
  auto load_frags = [&](auto STG, auto HALF, v4i (&af)[8], v4i (&bf)[8]) __attribute__((always_inline)) {
#pragma unroll
    for (int g = 0; g < 8; ++g) load_pair(STG, HALF, g, af, bf);
  };
  // The MFMA is written as inline asm with the accumulator tied in place
  // ("+a"): with the builtin, the register allocator rotates the 64
  // accumulator tuples through copies on every pass of the pipelined loop.
  // Hazards the compiler cannot see through the asm: the accumulators are
  // written by VALU long before the first MFMA (prologue), and the epilogue
  // reads them only after explicit wait states (below).
  auto mfma_row = [&](auto I, v4i (&af)[8], v4i (&bf)[8]) __attribute__((always_inline)) {
    static_for<8>([&](auto J) {
      v4i& c = acc[I][J];
      const v4i& xb = bf[J];
      const v4i& xa = af[I];
      asm volatile("v_mfma_i32_16x16x64_i8 %0, %1, %2, %0" : "+a"(c) : "v"(xb), "v"(xa));
    });
  };
  v4i xa[8], xb[8], ya[8], yb[8];
  using C0 = std::integral_constant<int, 0>;
  using C1 = std::integral_constant<int, 1>;

  const int ksteps = p.K / V5_BK;  // even (host: K % 256 == 0)
  issue(0, C0{});
  issue(min(1, ksteps - 1), C1{});
  wait_vmcnt<16>();
  asm volatile("s_barrier" ::: "memory");
  load_frags(C0{}, C0{}, xa, xb);

  // Past the end the DMA re-fetches the last slice and the reads fetch unused
  // data; both stay in bounds.
  // The memory operations are spread over the MFMA stream in groups of 8
  // MFMAs, pinned by scheduling barriers, so no burst of loads holds up MFMA
  // issue. Two barriers per K-step: A (stage t&1 is read by nobody any more)
  // early in sub-step 0, so the DMA of slice t+2 starts 1.5 K-steps before
  // its first read; B (slice t+1 has landed in every wave) at sub-step 1.
  // DMA pairs 0-5 go out in sub-step 0 after barrier A, pairs 6-7 in sub-step
  // 1, so vmcnt <= 12 at B means slice t+1 is complete.
#ifndef XMH3_V5_AROWS
#define XMH3_V5_AROWS 3
#endif
#ifndef XMH3_V5_XEARLY
#define XMH3_V5_XEARLY 0
#endif
  // AROWS MFMA rows on X run before barrier A (time for the Y reads to land);
  // the remaining rows carry the first 8 - AROWS DMA pairs of slice t+2
  constexpr int AROWS = XMH3_V5_AROWS, PRE = 8 - AROWS;
  auto step = [&](int t, auto STG) __attribute__((always_inline)) {
    constexpr int s = decltype(STG)::value;
    const int knext = min(t + 2, ksteps - 1);
    wait_lgkm0();                       // X = (t, k0) in registers
    load_frags(STG, C1{}, ya, yb);      // Y = (t, k1): the last reads of stage s
    static_for<AROWS>([&](auto I) { mfma_row(I, xa, xb); });
    __builtin_amdgcn_sched_barrier(0);
    wait_lgkm0();
    asm volatile("s_barrier" ::: "memory");   // A
    static_for<PRE>([&](auto G) {
      issue_pair(G, knext, STG);
      mfma_row(std::integral_constant<int, G + AROWS>{}, xa, xb);
      __builtin_amdgcn_sched_barrier(0);
    });
    wait_vmcnt<2 * PRE>();
    asm volatile("s_barrier" ::: "memory");   // B
    static_for<8>([&](auto G) {
      if constexpr (G >= PRE) issue_pair(G, knext, STG);
#if XMH3_V5_XEARLY
      // next step's X fragments two pairs per row over the first half
      if constexpr (G < 4) {
        load_pair(std::integral_constant<int, s ^ 1>{}, C0{}, 2 * G, xa, xb);
        load_pair(std::integral_constant<int, s ^ 1>{}, C0{}, 2 * G + 1, xa, xb);
      }
#else
      load_pair(std::integral_constant<int, s ^ 1>{}, C0{}, G, xa, xb);
#endif
      mfma_row(G, ya, yb);
      __builtin_amdgcn_sched_barrier(0);
    });
  };
  for (int t = 0; t < ksteps; t += 2) {
    step(t, C0{});
    step(t + 1, C1{});
  }
  // the last MFMA's result must be written back before VALU reads it
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  wait_vmcnt<0>();  // no DMA may land after the workgroup's LDS is released
  EpiScales sc;
  load_scales<EPI>(p, m0, n0, wm, wn, lane, sc);
  epilogue<EPI, TO, VEC_OUT>(p, acc, sc, m0, n0, wm, wn, lane);
}

#ifndef XMH3_GEMM_KERNELS_ONLY
// ---------------------------------------------------------------------------
// host launcher
// ---------------------------------------------------------------------------
template <int BK, int EPI, typename TO>
static int launch_gemm_T(GemmArgs& a, bool vec, hipStream_t st) {
  dim3 grid((unsigned)(a.tiles_m * a.tiles_n));
  const bool spans_ok = (int64_t)a.M * a.lda < (1LL << 31) && (int64_t)a.N * a.ldb < (1LL << 31);
#ifndef XMH3_GEMM_V5
#define XMH3_GEMM_V5 1
#endif
  // the gated epilogue always has aligned vector rows (host contract): its
  // scalar-row variants are not instantiated
  constexpr bool only_vec = EPI == EPI_GATED;
  if (XMH3_GEMM_V5 && a.K % (2 * V5_BK) == 0 && spans_ok) {
    if (vec || only_vec)
      hipLaunchKernelGGL((gemm_i8_v5_kernel<EPI, TO, true>), grid, dim3(NTHREADS), 0, st, a);
    else if constexpr (!only_vec)
      hipLaunchKernelGGL((gemm_i8_v5_kernel<EPI, TO, false>), grid, dim3(NTHREADS), 0, st, a);
    return check_launch("gemm_i8_v5_kernel");
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
  // BK=128 needs 128 KiB of LDS (2 stages x 2 operands x 32 KiB)
  switch (epilogue) {
    case EPI_INT32:
      return launch_gemm_T<128, EPI_INT32, F32T>(a, vec, st);
    case EPI_GELU:
      return launch_gemm_T<128, EPI_GELU, BF16T>(a, vec, st);
    case EPI_DEQUANT:
      if (out_dtype == DT_BF16) return launch_gemm_T<128, EPI_DEQUANT, BF16T>(a, vec, st);
      if (out_dtype == DT_F16) return launch_gemm_T<128, EPI_DEQUANT, F16T>(a, vec, st);
      if (out_dtype == DT_F32) return launch_gemm_T<128, EPI_DEQUANT, F32T>(a, vec, st);
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
  a.tiles_m = (int)((M + BM - 1) / BM);
  a.tiles_n = (int)((N + BN - 1) / BN);
  XMH3_REQUIRE((int64_t)a.tiles_m * a.tiles_n < (1LL << 31), "int8_gemm_gated_residual: grid too large");
  if (res_dtype == DT_BF16) return launch_gemm_T<128, EPI_GATED, BF16T>(a, true, st);
  return launch_gemm_T<128, EPI_GATED, F16T>(a, true, st);
}

#endif  // XMH3_GEMM_KERNELS_ONLY
}  // namespace xmh3

#ifndef XMH3_GEMM_KERNELS_ONLY
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
#endif
