// Memory-bound normalisation / rotary kernels for gfx950.
//
// Cooperative family (the measured paths): a row split over the waves of a
// block, one block per CU streaming row groups with two groups of loads in
// flight, the reference-order reduction assembled through LDS:
//   * norm_rope_coop_kernel : norm_rope of Q and K rows, width % 1024 == 0
//   * adaln_coop_kernel     : rms_adaln of bf16 rows with bf16 modulation
//   * qk_coop_kernel        : per-head rms_norm + full split-half rotation of
//                             64/96/128-wide heads, Q and K in one launch
// Row-span family (one wave64 per token row, the row held in VGPRs, 16-byte
// loads and stores, wave reduction of the sum of squares, no LDS), for the
// widths, dtypes and modulation forms the cooperative kernels do not take:
//   * norm_rope  : out = rope_split_half(rms_adaln(x, scale, shift, eps), freqs)
//                  for Q and K of one token in the same wave (the table row is
//                  read once for both); RMS over the full row, rotation per
//                  head. (CK/backends/eager/adaln.py:17-20 then
//                  CK/backends/eager/rope.py:39-42)
//   * rms_adaln  : rms_norm(x [* weight]) * (1 + scale[r]) + shift[r] with the
//                  modulation row r = row_map[token] or token / group
//                  (CK/backends/eager/adaln.py:17-20,
//                   h3serve/native_engine/model/kernels.py:7623-7634)
// Head-span family (a power-of-two group of lanes per (token, head)), for
// the rotary calls the cooperative QK kernel does not take:
//   * rms_rope_split_half : per-head rms_norm with weight, split-half rotation
//                  of the first rot_dim dims, tail norm-only, in place on
//                  strided [B,S,H,D] (CK/backends/eager/rope.py:67-92,178-189)
//   * rope_split_half     : the rotation alone (CK/backends/eager/rope.py:39-48)
//
// Rounding points follow the eager op order exactly: rms_norm rounds once to
// x's dtype ((x*rrms)*w in fp32); 1+scale, the product and the sum each round
// to the promoted dtype; the rotation's two products and their sum round to the
// table's dtype, then the result rounds to x's dtype. No FMA contraction
// (-ffp-contract=off); the only fused multiply-add is in the sum of squares of
// 16-bit inputs, where the square is exact and fusing changes no bit.
// CK = backends/turbo/vendor/comfy_kitchen.
#include "common.hpp"

#include <algorithm>
#include <type_traits>

namespace xmh3 {

// 8 x 16-bit or 8 x fp32 values as raw storage
template <typename T> struct V8;
template <> struct V8<BF16T> { uint4 v; };
template <> struct V8<F16T> { uint4 v; };
template <> struct V8<F32T> { uint4 v[2]; };

template <typename T>
__device__ __forceinline__ void ld8(const void* base, int64_t idx, V8<T>& d) {
  const typename T::storage* p = static_cast<const typename T::storage*>(base) + idx;
  if constexpr (sizeof(typename T::storage) == 2) d.v = *reinterpret_cast<const uint4*>(p);
  else { d.v[0] = *reinterpret_cast<const uint4*>(p); d.v[1] = *reinterpret_cast<const uint4*>(p + 4); }
}
template <typename T>
__device__ __forceinline__ void st8(void* base, int64_t idx, const V8<T>& d) {
  typename T::storage* p = static_cast<typename T::storage*>(base) + idx;
  if constexpr (sizeof(typename T::storage) == 2) *reinterpret_cast<uint4*>(p) = d.v;
  else { *reinterpret_cast<uint4*>(p) = d.v[0]; *reinterpret_cast<uint4*>(p + 4) = d.v[1]; }
}
template <typename T>
__device__ __forceinline__ float g8(const V8<T>& d, int j) {
  if constexpr (sizeof(typename T::storage) == 2) {
    uint32_t w = (&d.v.x)[j >> 1];
    return T::load((j & 1) ? (w >> 16) : (w & 0xffffu));
  } else {
    return __uint_as_float((&d.v[j >> 2].x)[j & 3]);
  }
}
// 8 fp32 values rounded to T's storage, two per conversion for 16-bit T
template <typename T>
__device__ __forceinline__ V8<T> pack8(const float* y) {
  V8<T> d;
  if constexpr (sizeof(typename T::storage) == 2) {
    d.v = make_uint4(T::store2(y[0], y[1]), T::store2(y[2], y[3]), T::store2(y[4], y[5]),
                     T::store2(y[6], y[7]));
  } else {
    d.v[0] = make_uint4(__float_as_uint(y[0]), __float_as_uint(y[1]), __float_as_uint(y[2]),
                        __float_as_uint(y[3]));
    d.v[1] = make_uint4(__float_as_uint(y[4]), __float_as_uint(y[5]), __float_as_uint(y[6]),
                        __float_as_uint(y[7]));
  }
  return d;
}

// type promotion of (x dtype, modulation dtype) as torch does for x * (1 + s)
template <typename TX, typename TM> struct Promote { using type = TX; };
template <> struct Promote<BF16T, F32T> { using type = F32T; };
template <> struct Promote<F16T, F32T> { using type = F32T; };
template <> struct Promote<BF16T, F16T> { using type = F32T; };
template <> struct Promote<F16T, BF16T> { using type = F32T; };

// one rotated pair in the table dtype TF, result rounded to TO
template <typename TF, typename TO>
__device__ __forceinline__ void rotate_pair(float a0, float a1, float f00, float f01, float f10,
                                            float f11, float& r0, float& r1) {
  const float x0 = TF::round(a0), x1 = TF::round(a1);  // x.to(freqs.dtype)
  r0 = TO::round(TF::round(TF::round(f00 * x0) + TF::round(f01 * x1)));
  r1 = TO::round(TF::round(TF::round(f10 * x0) + TF::round(f11 * x1)));
}

// The interleaved form (CK/backends/eager/rope.py:10-16): out = f[., 0] * x0,
// then out.addcmul_(f[., 1], x1), which torch's CPU kernel evaluates as one
// fused multiply-add in the table dtype (for 16-bit tables the product is
// exact in fp32, so the fp32 fma rounded to TF is the same value).
template <typename TF, typename TO>
__device__ __forceinline__ void rotate_pair_fma(float a0, float a1, float f00, float f01, float f10,
                                                float f11, float& r0, float& r1) {
  const float x0 = TF::round(a0), x1 = TF::round(a1);  // x.to(freqs.dtype)
  r0 = TO::round(TF::round(__builtin_fmaf(f01, x1, TF::round(f00 * x0))));
  r1 = TO::round(TF::round(__builtin_fmaf(f11, x1, TF::round(f10 * x0))));
}

// table entries for 8 consecutive pairs: [pair][2][2] in TF
template <typename TF>
struct Tab8 { float f[8][4]; };

// the first 4 pairs only (16 consecutive elements from idx)
template <typename TF>
__device__ __forceinline__ void load_tab4(const void* base, int64_t idx, Tab8<TF>& t) {
  V8<TF> raw[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) ld8<TF>(base, idx + q * 8, raw[q]);
#pragma unroll
  for (int p = 0; p < 4; ++p)
#pragma unroll
    for (int e = 0; e < 4; ++e) t.f[p][e] = g8<TF>(raw[(p * 4 + e) >> 3], (p * 4 + e) & 7);
}

template <typename TF>
__device__ __forceinline__ void load_tab8(const void* base, int64_t idx, Tab8<TF>& t) {
  // idx: element index of pair p0's f00; 32 consecutive elements
  V8<TF> raw[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) ld8<TF>(base, idx + q * 8, raw[q]);
#pragma unroll
  for (int p = 0; p < 8; ++p)
#pragma unroll
    for (int e = 0; e < 4; ++e) t.f[p][e] = g8<TF>(raw[(p * 4 + e) >> 3], (p * 4 + e) & 7);
}

// ---------------------------------------------------------------------------
// row-span kernel
// ---------------------------------------------------------------------------
struct RowArgs {
  const void* x0; void* o0;       // first tensor (Q, or the only one)
  const void* x1; void* o1;       // optional second tensor (K), same shape
  int64_t ldx, ldo, rows, D;
  const void* weight;             // [D] in TX, nullable
  const void* scale; const void* shift;  // [R, D] in TM (ADALN)
  int64_t mod_ld;                 // row stride of scale/shift
  const int32_t* row_map;         // nullable
  int64_t mod_group;              // token -> modulation row = token / mod_group
  const void* freqs;              // ROPE: [rows or 1, head_dim/2, 2, 2] in TF
  int64_t freqs_row_stride;       // elements; 0 = one table row for all tokens
  int head_dim;
  float eps;
};

// Modulation row of a token under a row map: entries are clamped into the
// table's mod_rows rows, so a bad map can never read outside the scale/shift
// tables (callers validate the map; the H3 segment helper does on the host).
__device__ __forceinline__ int64_t map_row(int32_t r, int64_t mod_rows) {
  return r < 0 ? 0 : (r >= mod_rows ? mod_rows - 1 : (int64_t)r);
}

// ---------------------------------------------------------------------------
// Sum of squares of a row in the reference's reduction order.
//
// The reference normalises with torch's F.rms_norm on the CPU: mean =
// sum(x*x) / D, where the sum is ATen's vectorised cascade sum. For a
// contiguous fp32 row it runs as 8-lane vectors read 4 at a time into 4
// accumulator rows -- 32 independent chains, chain L summing the squares at
// positions 32*i + L -- each chain adding in chunks of 16 that feed a 4-level
// cascade (acc1 += chunk; every 256 steps acc2 += acc1; every 4096 acc3 +=
// acc2), a remainder added from zero, the levels folded ((a0+a1)+a2)+a3, the
// 4 rows added lane-wise ((r0+r1)+r2)+r3 and the 8 lanes left to right.
// Reproducing that order makes the GPU rms bit-identical to the reference's.
//
// When D/8 is not a multiple of 4, the 1-3 leftover 8-lane vectors are added
// to accumulator row 0 (chains 0..7) after the cascade, before the rows are
// combined. The row is staged in a per-wave LDS buffer; chain L runs on lane L
// for the even chunks and on lane L+32 for the odd ones. Requires D % 8 == 0
// and D < 2^17 (cascade step 16).
// ---------------------------------------------------------------------------
// c + v*v. For 16-bit inputs v*v is exact in fp32, so the fused form rounds
// identically to the reference's separate product and sum (one instruction
// instead of two); fp32 inputs keep the separate rounding of the product.
template <typename TX>
__device__ __forceinline__ float add_sq(float c, float v) {
  if constexpr (sizeof(typename TX::storage) == 2) return __builtin_fmaf(v, v, c);
  else return c + v * v;
}

struct IdentityIdx {
  __device__ int operator()(int p) const { return p; }
};

template <typename TX, typename Idx = IdentityIdx>
__device__ __forceinline__ float ref_order_sumsq(const typename TX::storage* row, int D, int lane,
                                                 Idx idx = Idx{}) {
  const int L = lane & 31, h = lane >> 5;
  const int steps = D >> 5;
  const int nchunks = steps >> 4;
  float acc1 = 0.0f, acc2 = 0.0f, acc3 = 0.0f;
  auto apply = [&](float c, int i_end) {
    acc1 = acc1 + c;
    if ((i_end & (15 << 4)) == 0) {
      acc2 = acc2 + acc1;
      acc1 = 0.0f;
      if ((i_end & (15 << 8)) == 0) {
        acc3 = acc3 + acc2;
        acc2 = 0.0f;
      }
    }
  };
  for (int jj = 0; jj < nchunks; jj += 2) {
    const int j = jj + h;
    float c = 0.0f;
    if (j < nchunks) {
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const float v = TX::load(row[idx(j * 512 + u * 32 + L)]);
        c = add_sq<TX>(c, v);
      }
    }
    const float c_odd = __shfl(c, L + 32, 64);
    if (h == 0) {
      apply(c, (jj + 1) * 16);
      if (jj + 1 < nchunks) apply(c_odd, (jj + 2) * 16);
    }
  }
  float acc0 = 0.0f;
  for (int i = nchunks * 16; i < steps; ++i) {
    const float v = TX::load(row[idx(i * 32 + L)]);
    acc0 = add_sq<TX>(acc0, v);
  }
  float tot = ((acc0 + acc1) + acc2) + acc3;
  for (int q = steps * 4; q < (D >> 3); ++q) {   // leftover vectors -> row 0
    const float v = TX::load(row[idx(q * 8 + (L & 7))]);
    if (L < 8) tot = add_sq<TX>(tot, v);
  }
  const int v8 = lane & 7;
  const float r0 = __shfl(tot, v8, 64), r1 = __shfl(tot, v8 + 8, 64);
  const float r2 = __shfl(tot, v8 + 16, 64), r3 = __shfl(tot, v8 + 24, 64);
  const float pv = ((r0 + r1) + r2) + r3;
  float fin = 0.0f;
#pragma unroll
  for (int v = 0; v < 8; ++v) fin = fin + __shfl(pv, v, 64);
  return fin;
}

// Row-span kernel (one wave per token row; the rows of Q and K of a token in
// the same wave). ROPE: items are (8 at head offset i, 8 at i + head_dim/2),
// IPH per head; otherwise items are 8 consecutive elements; NSTEP steps of 64
// items per row, all held in VGPRs (16-byte loads and stores). The rows are
// also staged in LDS (WPB waves per block, two row buffers each) for the
// reference-order reduction. D % 8 == 0.
template <typename TX, typename TM, typename TF, bool ROPE, bool ADALN, bool WEIGHT, int IPH, int NSTEP>
__global__ __launch_bounds__(256) void rowspan_exact_kernel(RowArgs a) {
  using TO = typename std::conditional<ADALN, typename Promote<TX, TM>::type, TX>::type;
  using S = typename TX::storage;
  extern __shared__ __attribute__((aligned(16))) uint8_t dyn_lds[];
  constexpr int EPI = ROPE ? 16 : 8;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + wave;
  if (row >= a.rows) return;
  const int64_t items = a.D / EPI;
  const int nt = a.x1 ? 2 : 1;
  S* lrow = reinterpret_cast<S*>(dyn_lds) + (int64_t)wave * nt * a.D;

  auto item_off = [&](int64_t u, int64_t& o0, int64_t& o1) {
    if constexpr (ROPE) {
      const int64_t head = u / IPH;
      const int it = (int)(u - head * IPH);
      o0 = head * a.head_dim + it * 8;
      o1 = o0 + (a.head_dim >> 1);
    } else {
      o0 = u * 8;
      o1 = 0;
    }
  };

  // load every row of this token into registers and stage it in LDS
  V8<TX> v[2][NSTEP][ROPE ? 2 : 1];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    if (t >= nt) break;
    const void* xb = t ? a.x1 : a.x0;
#pragma unroll
    for (int s = 0; s < NSTEP; ++s) {
      const int64_t u = (int64_t)s * 64 + lane;
      if (u < items) {
        int64_t o0, o1;
        item_off(u, o0, o1);
        ld8<TX>(xb, row * a.ldx + o0, v[t][s][0]);
        st8<TX>(lrow + t * a.D, o0, v[t][s][0]);
        if constexpr (ROPE) {
          ld8<TX>(xb, row * a.ldx + o1, v[t][s][1]);
          st8<TX>(lrow + t * a.D, o1, v[t][s][1]);
        }
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): this wave's LDS stores done
  __builtin_amdgcn_wave_barrier();
  float rr[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    rr[t] = 1.0f;
    if (t < nt) {
      const float tot = ref_order_sumsq<TX>(lrow + t * a.D, (int)a.D, lane);
      rr[t] = 1.0f / sqrtf(tot / (float)a.D + a.eps);
    }
  }

  int64_t mrow = 0;
  if constexpr (ADALN) mrow = a.row_map ? map_row(a.row_map[row], a.mod_group) : row / a.mod_group;
  Tab8<TF> tab;
  const int64_t trow = a.freqs_row_stride ? row * a.freqs_row_stride : 0;
  bool tab_loaded = false;

  // weight / scale / shift of the items of step s, loaded one step ahead: the
  // compiler may not move a load above the previous step's stores (the output
  // could alias them), so the prefetch is explicit
  constexpr int NH = ROPE ? 2 : 1;
  struct Mod { V8<TX> w[NH]; V8<TM> sc[NH], sh[NH]; };
  auto fetch_mod = [&](int s, Mod& m) __attribute__((always_inline)) {
    const int64_t u = (int64_t)s * 64 + lane;
    if (u >= items) return;
    int64_t o0, o1;
    item_off(u, o0, o1);
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      const int64_t col = h ? o1 : o0;
      if constexpr (WEIGHT) ld8<TX>(a.weight, col, m.w[h]);
      if constexpr (ADALN) {
        ld8<TM>(a.scale, mrow * a.mod_ld + col, m.sc[h]);
        ld8<TM>(a.shift, mrow * a.mod_ld + col, m.sh[h]);
      }
    }
  };
  Mod mod[2];
  fetch_mod(0, mod[0]);

#pragma unroll
  for (int s = 0; s < NSTEP; ++s) {
    if (s + 1 < NSTEP) fetch_mod(s + 1, mod[(s + 1) & 1]);
    const Mod& m = mod[s & 1];
    const int64_t u = (int64_t)s * 64 + lane;
    if (u >= items) continue;
    int64_t o0, o1;
    item_off(u, o0, o1);
    if constexpr (ROPE) {
      if (!tab_loaded || (64 % IPH) != 0) {
        load_tab8<TF>(a.freqs, trow + (int64_t)(u % IPH) * 8 * 4, tab);
        tab_loaded = true;
      }
    }
    float y[2][NH][8];
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      float w8[8], t8[8], sh8[8];
      if constexpr (WEIGHT) {
#pragma unroll
        for (int j = 0; j < 8; ++j) w8[j] = g8<TX>(m.w[h], j);
      }
      if constexpr (ADALN) {
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
          t8[j] = 1.0f + g8<TM>(m.sc[h], j);          // (1 + scale) in scale's dtype
          t8[j + 1] = 1.0f + g8<TM>(m.sc[h], j + 1);
          TM::round2(t8[j], t8[j + 1]);
          sh8[j] = g8<TM>(m.sh[h], j);
          sh8[j + 1] = g8<TM>(m.sh[h], j + 1);
        }
      }
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        if (t >= nt) break;
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
          float n0 = g8<TX>(v[t][s][h], j) * rr[t], n1 = g8<TX>(v[t][s][h], j + 1) * rr[t];
          if constexpr (WEIGHT) { n0 = n0 * w8[j]; n1 = n1 * w8[j + 1]; }
          TX::round2(n0, n1);                      // rms_norm output in x's dtype
          if constexpr (ADALN) {
            n0 = n0 * t8[j]; n1 = n1 * t8[j + 1];
            TO::round2(n0, n1);
            n0 = n0 + sh8[j]; n1 = n1 + sh8[j + 1];
            TO::round2(n0, n1);
          }
          y[t][h][j] = n0;
          y[t][h][j + 1] = n1;
        }
      }
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      if (t >= nt) break;
      if constexpr (ROPE) {
        static_assert(std::is_same<TO, TX>::value, "rope path keeps x's dtype");
        uint32_t w0[4], w1[4];
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
          float p0[2], p1[2];
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const float a0 = TF::round(y[t][0][j + e]), a1 = TF::round(y[t][1][j + e]);
            const float* f = tab.f[j + e];
            p0[e] = TF::round(TF::round(f[0] * a0) + TF::round(f[1] * a1));
            p1[e] = TF::round(TF::round(f[2] * a0) + TF::round(f[3] * a1));
          }
          w0[j >> 1] = TX::store2(p0[0], p0[1]);
          w1[j >> 1] = TX::store2(p1[0], p1[1]);
        }
        S* ob = static_cast<S*>(t ? a.o1 : a.o0) + row * a.ldo;
        *reinterpret_cast<uint4*>(ob + o0) = make_uint4(w0[0], w0[1], w0[2], w0[3]);
        *reinterpret_cast<uint4*>(ob + o1) = make_uint4(w1[0], w1[1], w1[2], w1[3]);
      } else {
        st8<TO>(t ? a.o1 : a.o0, row * a.ldo + o0, pack8<TO>(y[t][0]));
      }
    }
  }
}

// ---------------------------------------------------------------------------
// LDS placement of a staged row: element p of head h = p / 128 sits in half
// ((p / 64) & 1) ^ flip(h) of the head's 256 bytes. flip alternates between
// the heads one 64-lane access touches (8 consecutive heads for the 16-byte
// items, heads 4 apart for the two lane halves of the ordered reduction), so
// both kinds of access spread over all 64 banks.
__device__ __forceinline__ int row_flip(int h) { return (h ^ (h >> 2)) & 1; }
struct SwizzledRowIdx {
  __device__ int operator()(int p) const {
    const int h = p >> 7;
    return (p & ~127) | ((((p >> 6) & 1) ^ row_flip(h)) << 6) | (p & 63);
  }
};

// ---------------------------------------------------------------------------
// Cooperative norm-rope: a row is split over P = D / 1024 waves; wave p of a
// row owns the 1024 consecutive elements (8 heads) [1024 p, 1024 p + 1024).
// A block of R * P waves takes the R consecutive rows of a row group per
// iteration; the rows are ordered all Q rows, then all K rows (row r: tensor
// r / tokens), and the blocks (one per CU) visit groups blockIdx.x,
// + gridDim.x, ..., so the accesses in flight at any time cover one dense
// window of one tensor. A plain copy of the same bytes measured 168 us in
// this form; a wave per whole row (the waves' accesses spread over as many
// rows as waves) took 190 us, a block per token with its Q and K rows
// 179 us, and more blocks per CU were slower. R rows per block keep R rows'
// reductions and element passes in flight at once (one row per block left
// the CU latency-bound: 278 us).
//
// The reference-order sum of squares (ref_order_sumsq) is a fold over chunks
// of 512 positions: chain L adds the 16 squares at 512 j + 32 u + L from zero
// (u = 0..15) and folds the chunk sum into its cascade. A part holds chunks
// 2 p and 2 p + 1 whole, so each wave computes its 2 x 32 chunk sums from its
// staged part, the block shares them in LDS, and after one barrier one wave
// of the row folds the row's 2P chunk sums in order and combines the chains
// as ref_order_sumsq does (bit-identical rrms) and publishes the rrms, which
// the row's waves use after the next iteration's barrier. D % 1024 == 0
// leaves no partial chunk and no leftover vector.
//
// Two rows are prefetched in registers (2 items of 16 bytes per lane per row,
// plus the row's table row, 16 bytes per lane). Staging, chunk sums and rrms
// live in two parity slots and table rows in three, so one barrier per row
// suffices: a slot is rewritten after every wave has passed the barrier that
// follows its last read. The barrier waits for LDS only (__syncthreads would
// also wait for the prefetched loads).
// LDS: 8 D (modulation, ADALN) + 4 KB per wave (staging) + 2 * R * 2P * 32
// floats (chunk sums) + 3 R table rows + 2 R floats (rrms).
// ---------------------------------------------------------------------------
template <typename TX, typename TF, bool ADALN, int P>
__global__ __launch_bounds__(1024) void norm_rope_coop_kernel(RowArgs a, int nt) {
  using S = typename TX::storage;
  using SF = typename TF::storage;
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  static_assert(sizeof(S) == 2, "16-bit rows");
  constexpr int HD = 128, IPH = HD / 16, D = P * 1024, NCH = 2 * P;
  constexpr int TAB_BYTES = (HD / 2) * 4 * (int)sizeof(SF);
  constexpr int TAB_CHUNKS = TAB_BYTES / 16;
  constexpr int CPG = TAB_CHUNKS / IPH;                          // 16-byte pieces per 8-pair group
  constexpr int EPC = 16 / (int)sizeof(SF);
  extern __shared__ __attribute__((aligned(16))) uint8_t dyn_lds[];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int R = (blockDim.x >> 6) / P;                                 // rows per block iteration
  const int sub = w / P, part = w - sub * P;
  f32x4* lt = reinterpret_cast<f32x4*>(dyn_lds);
  f32x4* ls = lt + D / 4;
  uint8_t* p0 = dyn_lds + (ADALN ? 8 * D : 0);
  S* stage = reinterpret_cast<S*>(p0 + w * 4096);                     // [2][1024] per wave
  float* sums = reinterpret_cast<float*>(p0 + R * P * 4096);           // [2][R][NCH][32]
  u32x4* tabs = reinterpret_cast<u32x4*>(sums + 2 * R * NCH * 32);     // [3][R][TAB_CHUNKS]
  float* rrs = reinterpret_cast<float*>(tabs + 3 * R * TAB_CHUNKS);    // [2][R]

  if constexpr (ADALN) {
    // t = round_TX(1 + scale), sh = shift, as fp32, lane-major: float4
    // (((part * 2 + half) * 2 + quad) * 64 + lane) holds the columns of item
    // half of that lane in that part, + 4 * quad .. + 3
    const S* sc = static_cast<const S*>(a.scale);
    const S* sh = static_cast<const S*>(a.shift);
    for (int i = threadIdx.x; i < D / 4; i += blockDim.x) {
      const int l = i & 63, q = (i >> 6) & 1, hf = (i >> 7) & 1, st = i >> 8;
      const int u = st * 64 + l;
      const int col = (u / IPH) * HD + hf * (HD / 2) + (u % IPH) * 8 + q * 4;
      f32x4 tv, sv;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        tv[e] = TX::round(1.0f + TX::load(sc[col + e]));
        sv[e] = TX::load(sh[col + e]);
      }
      lt[i] = tv;
      ls[i] = sv;
    }
  }
  __syncthreads();

  // 32-bit row and group indices (the launcher checks rows * nt < 2^30); the
  // wave takes row gg * R + sub of groups gg = blockIdx.x + it * G
  const int ntok = (int)a.rows, nrows = ntok * nt, ngroups = (nrows + R - 1) / R;
  const int G = gridDim.x;
  if ((int)blockIdx.x >= ngroups) return;   // uniform per block
  const int iters = (ngroups - (int)blockIdx.x + G - 1) / G;
  auto row_of = [&](int it) {
    it = it < iters ? it : iters - 1;       // past the block's last iteration: that one again
    const int row = ((int)blockIdx.x + it * G) * R + sub;
    return row < nrows ? row : nrows - 1;   // past the end: the last row again
  };

  const int qh = lane / IPH, it8 = (lane % IPH) * 8;
  const int o0 = part * 1024 + qh * HD + it8;                         // item 0; item 1 at + 64
  const int sl0 = qh * HD + (row_flip(qh) << 6) + it8;                 // staged (SwizzledRowIdx)
  const int sl1 = qh * HD + ((row_flip(qh) ^ 1) << 6) + it8;
  const int tab_lane = min(lane, TAB_CHUNKS - 1);
  // table piece c = tab_lane goes to slot (c % CPG) * 8 + c / CPG, so the
  // lanes of one 8-pair group read consecutive slots
  const int tab_slot = (tab_lane % CPG) * IPH + tab_lane / CPG;

  // this wave's row of iteration it; rows past the last are the last row
  // again, computed from loads issued before any store of their row group and
  // stored with identical bytes (so in-place calls stay exact), so that every
  // wave keeps the block's barriers and issues the same memory operations on
  // every path (the compiler's waits then leave the prefetch in flight)
  auto issue = [&](int it, u32x4 (&bx)[2], u32x4& bt) __attribute__((always_inline)) {
    const int row = row_of(it);
    const int tok = row < ntok ? row : row - ntok;
    const S* xb = static_cast<const S*>(row < ntok ? a.x0 : a.x1) + (int64_t)tok * a.ldx + o0;
    bx[0] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(xb));
    bx[1] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(xb + HD / 2));
    const SF* tb = static_cast<const SF*>(a.freqs) + (a.freqs_row_stride ? (int64_t)tok * a.freqs_row_stride : 0);
    bt = *reinterpret_cast<const u32x4*>(tb + tab_lane * EPC);
  };

  // Iteration it: front(it) stages row_of(it), prefetches iteration it + 2,
  // publishes its chunk sums and, after the barrier, one wave of the row
  // (part rpart) folds them into the row's rrms; back(it - 1) then runs the
  // element pass of the previous iteration's row, whose rrms that wave
  // published before this barrier. Only one wave per row folds, combines and
  // divides (every wave doing it cost 3-5 % of the kernel), with no extra
  // barrier: the element pass trails the reduction by one iteration. Slots:
  // staging and rrms in two (parity), table rows in three (written before the
  // barrier of iteration it, read after that of it + 1, rewritten before that
  // of it + 3).
  //
  // Folding waves are placed by SIMD load: waves are dealt to the CU's four
  // SIMDs in turn (wave w on SIMD w % 4), and row by row the fold goes to the
  // row's wave on the least loaded SIMD, a wave counting 4 and a fold 1. A
  // block of 15 waves (P = 5, R = 3) leaves SIMD 3 one wave short, and its
  // three folds all go there (folding on part 0 put them on SIMDs 0-2 and
  // measured 2-3 % slower); with 12 waves (P = 3, R = 4) the four folds go
  // to four different SIMDs (107.1 us at 25200 x 3072 against 107.8 us with
  // all four on SIMD 3: there the spread hardly matters). The choice only
  // moves work; any wave of the row gives the same bits.
  int par = 0, tsl = 0;
  int rpart = 0;
  {
    // SIMD loads in four scalars (no indexed array, so nothing goes to scratch)
    const int nw = R * P;
    int l0 = 4 * ((nw + 3) / 4), l1 = 4 * ((nw + 2) / 4), l2 = 4 * ((nw + 1) / 4), l3 = 4 * (nw / 4);
    auto load_of = [&](int s) { return s == 0 ? l0 : s == 1 ? l1 : s == 2 ? l2 : l3; };
    for (int r = 0; r <= sub; ++r) {
      int best = 0;
      for (int p = 1; p < P; ++p)
        if (load_of((r * P + p) & 3) < load_of((r * P + best) & 3)) best = p;
      const int s = (r * P + best) & 3;
      l0 += s == 0; l1 += s == 1; l2 += s == 2; l3 += s == 3;
      rpart = best;
    }
  }
  auto front = [&](int it, u32x4 (&bx)[2], u32x4& bt) __attribute__((always_inline)) {
    S* sg = stage + par * 1024;
    const int slot = par * R + sub;
    *reinterpret_cast<u32x4*>(sg + sl0) = bx[0];
    *reinterpret_cast<u32x4*>(sg + sl1) = bx[1];
    if (part == 0 && lane < TAB_CHUNKS) tabs[(tsl * R + sub) * TAB_CHUNKS + tab_slot] = bt;
    __builtin_amdgcn_sched_barrier(0);
    issue(it + 2, bx, bt);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): this wave's staging stores done
    __builtin_amdgcn_wave_barrier();
    {
      // chunk 2 part + h of chain L: 16 squares in order, from zero
      const int L = lane & 31, h = lane >> 5;
      float c = 0.0f;
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const float v = TX::load(sg[SwizzledRowIdx{}(h * 512 + u * 32 + L)]);
        c = add_sq<TX>(c, v);
      }
      sums[(slot * NCH + 2 * part + h) * 32 + L] = c;
    }
    // publish the chunk sums (and wave 0's table row) to the block
    __builtin_amdgcn_s_waitcnt(0xc07f);
    asm volatile("s_barrier" ::: "memory");
    if (part == rpart) {
      // the reference order: fold the row's chunk sums, then the chains
      const int L = lane & 31;
      const float* cs = sums + slot * NCH * 32 + L;
      float acc1 = 0.0f, acc2 = 0.0f, acc3 = 0.0f;
#pragma unroll
      for (int j = 0; j < NCH; ++j) {
        acc1 = acc1 + cs[j * 32];
        const int i_end = (j + 1) * 16;
        if ((i_end & (15 << 4)) == 0) {
          acc2 = acc2 + acc1;
          acc1 = 0.0f;
          if ((i_end & (15 << 8)) == 0) {
            acc3 = acc3 + acc2;
            acc2 = 0.0f;
          }
        }
      }
      const float tot = ((0.0f + acc1) + acc2) + acc3;
      const int v8 = lane & 7;
      const float r0 = __shfl(tot, v8, 64), r1 = __shfl(tot, v8 + 8, 64);
      const float r2 = __shfl(tot, v8 + 16, 64), r3 = __shfl(tot, v8 + 24, 64);
      const float pv = ((r0 + r1) + r2) + r3;
      float fin = 0.0f;
#pragma unroll
      for (int v = 0; v < 8; ++v) fin = fin + __shfl(pv, v, 64);
      if (lane == 0) rrs[slot] = 1.0f / sqrtf(fin / (float)D + a.eps);
    }
  };
  // element pass of row_of(it), staged by the previous front()
  auto back = [&](int it) __attribute__((always_inline)) {
    const int row = row_of(it);
    const int pp = par ^ 1, ts = tsl == 0 ? 2 : tsl - 1;
    const S* sg = stage + pp * 1024;
    const float rr = rrs[pp * R + sub];
    // this lane's 8 pairs (it8 .. it8 + 7) of the token's table row
    Tab8<TF> tab;
    {
      SF el[CPG * EPC];
#pragma unroll
      for (int j = 0; j < CPG; ++j) {
        const u32x4 v = tabs[(ts * R + sub) * TAB_CHUNKS + j * IPH + (lane % IPH)];
#pragma unroll
        for (int e = 0; e < EPC; ++e) {
          if constexpr (sizeof(SF) == 4) el[j * EPC + e] = __uint_as_float(v[e]);
          else el[j * EPC + e] = (SF)((v[e >> 1] >> ((e & 1) * 16)) & 0xffffu);
        }
      }
#pragma unroll
      for (int pp2 = 0; pp2 < 8; ++pp2)
#pragma unroll
        for (int e = 0; e < 4; ++e) tab.f[pp2][e] = TF::load(el[pp2 * 4 + e]);
    }
    float y[2][8];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      V8<TX> xv;
      xv.v = *reinterpret_cast<const uint4*>(sg + (h ? sl1 : sl0));
      float t8[8], sh8[8];
      if constexpr (ADALN) {
        const int i0 = ((part * 2 + h) * 2) * 64 + lane;
        const f32x4 ta = lt[i0], tb2 = lt[i0 + 64], sa = ls[i0], sb = ls[i0 + 64];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          t8[e] = ta[e]; t8[e + 4] = tb2[e];
          sh8[e] = sa[e]; sh8[e + 4] = sb[e];
        }
      }
#pragma unroll
      for (int j = 0; j < 8; j += 2) {
        float n0 = g8<TX>(xv, j) * rr, n1 = g8<TX>(xv, j + 1) * rr;
        TX::round2(n0, n1);                      // rms_norm output in x's dtype
        if constexpr (ADALN) {
          n0 = n0 * t8[j]; n1 = n1 * t8[j + 1];
          TX::round2(n0, n1);
          n0 = n0 + sh8[j]; n1 = n1 + sh8[j + 1];
          TX::round2(n0, n1);
        }
        y[h][j] = n0;
        y[h][j + 1] = n1;
      }
    }
    uint32_t w0[4], w1[4];
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
      float q0[2], q1[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const float a0 = TF::round(y[0][j + e]), a1 = TF::round(y[1][j + e]);
        const float* f = tab.f[j + e];
        q0[e] = TF::round(TF::round(f[0] * a0) + TF::round(f[1] * a1));
        q1[e] = TF::round(TF::round(f[2] * a0) + TF::round(f[3] * a1));
      }
      w0[j >> 1] = TX::store2(q0[0], q0[1]);
      w1[j >> 1] = TX::store2(q1[0], q1[1]);
    }
    {
      const int tok = row < ntok ? row : row - ntok;
      S* ob = static_cast<S*>(row < ntok ? a.o0 : a.o1) + (int64_t)tok * a.ldo + o0;
      __builtin_nontemporal_store(u32x4{w0[0], w0[1], w0[2], w0[3]}, reinterpret_cast<u32x4*>(ob));
      __builtin_nontemporal_store(u32x4{w1[0], w1[1], w1[2], w1[3]}, reinterpret_cast<u32x4*>(ob + HD / 2));
    }
  };
  auto next = [&]() __attribute__((always_inline)) {
    // LDS work of this iteration done before the slots turn over
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    par ^= 1;
    tsl = tsl == 2 ? 0 : tsl + 1;
  };

  // Two row groups in flight, in two register buffers taken in turn. The
  // first two iterations are peeled off the loop (the first has no element
  // pass) and the loop body is two whole iterations with its only exit at the
  // bottom: the loop head is then reached with the other buffer's loads
  // outstanding after the buffer it consumes, so the compiler's waits there
  // leave the prefetched group in flight (a path with fewer operations
  // outstanding makes those waits drain the prefetch). The peeled path has
  // one group of stores fewer than the back edge, so on the back edge the
  // head also waits for the stores of two iterations back, older than the
  // prefetch; peeling a third iteration removes that wait and measured 1-2 %
  // slower. A count that leaves the last pair half full ends with one extra
  // iteration that redoes the block's last one: its loads were issued before
  // that row's stores, so it stores identical bytes, also in place. A last
  // barrier publishes the last row's rrms for its element pass.
  u32x4 x0[2], x1[2], t0, t1;
  issue(0, x0, t0);
  issue(1, x1, t1);
  __builtin_amdgcn_sched_barrier(0);
  front(0, x0, t0);
  next();
  front(1, x1, t1);
  back(0);
  next();
  for (int it = 2; it < iters; it += 2) {
    front(it, x0, t0);
    back(it - 1);
    next();
    front(it + 1, x1, t1);
    back(it);
    next();
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);
  asm volatile("s_barrier" ::: "memory");
  back(iters - 1);
  __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): no load lands after the wave ends
}

// ---------------------------------------------------------------------------
// Pipelined rms_adaln (row-span, no rotation) for 16-bit rows whose
// modulation has the rows' dtype.
//
// Block b owns the contiguous rows [b * chunk, (b + 1) * chunk); its waves take
// rows first + wave, first + wave + WPB, ..., two rows ahead (loads of rows
// i + 1 and i + 2 in flight in two register buffers while row i is
// reduced, modulated and stored). The block caches in LDS round(1 + scale), shift
// and the norm weight of its first row's modulation row; a row with another
// modulation row (a block that straddles a segment or sample boundary) reads
// its modulation from global memory, which costs that row the prefetch
// overlap. Item slots u = s * 64 + lane (s < NSTEP) are clamped to the last
// item, so every lane issues the same unpredicated loads and stores (a
// clamped lane recomputes and rewrites the last item's identical bytes).
//
// LDS: 3 * D * sizeof(x) (t, shift, weight) + WPB * D * sizeof(x).
// ---------------------------------------------------------------------------
template <typename TX, bool WEIGHT, int NSTEP>
__global__ __launch_bounds__(512) void adaln_pipe_kernel(RowArgs a, int64_t chunk) {
  using S = typename TX::storage;
  static_assert(sizeof(S) == 2, "16-bit rows");
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  extern __shared__ __attribute__((aligned(16))) uint8_t dyn_lds[];
  const int D = (int)a.D, items = D >> 3;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wpb = blockDim.x >> 6;
  S* lt = reinterpret_cast<S*>(dyn_lds);
  S* lsh = lt + D;
  S* lw = lsh + D;
  S* lrow = lw + D + wave * D;
  const int64_t first = (int64_t)blockIdx.x * chunk;
  const int64_t last = first + chunk < a.rows ? first + chunk : a.rows;
  if (first >= last) return;   // the whole block
  auto mod_row = [&](int64_t row) -> int64_t {
    return a.row_map ? map_row(a.row_map[row], a.mod_group) : row / a.mod_group;
  };
  const int64_t m0 = mod_row(first);
  {
    const S* sc = static_cast<const S*>(a.scale) + m0 * a.mod_ld;
    const S* sh = static_cast<const S*>(a.shift) + m0 * a.mod_ld;
    for (int i = threadIdx.x; i < items; i += blockDim.x) {
      V8<TX> vs, vh;
      ld8<TX>(sc, (int64_t)i * 8, vs);
      ld8<TX>(sh, (int64_t)i * 8, vh);
      float t[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) t[j] = TX::round(1.0f + g8<TX>(vs, j));   // (1 + scale) in its dtype
      st8<TX>(lt, (int64_t)i * 8, pack8<TX>(t));
      st8<TX>(lsh, (int64_t)i * 8, vh);
      if constexpr (WEIGHT) {
        V8<TX> vw;
        ld8<TX>(a.weight, (int64_t)i * 8, vw);
        st8<TX>(lw, (int64_t)i * 8, vw);
      }
    }
    __syncthreads();
  }
  int64_t r = first + wave;
  if (r >= last) return;
  const int64_t stride = wpb;
  auto col = [&](int s) { const int u = s * 64 + lane; return (u < items ? u : items - 1) * 8; };

  auto issue = [&](int64_t row, u32x4 (&bx)[NSTEP]) __attribute__((always_inline)) {
    row = row < last ? row : last - 1;   // past the block's rows: re-read the last, never processed
    const S* xb = static_cast<const S*>(a.x0) + row * a.ldx;
#pragma unroll
    for (int s = 0; s < NSTEP; ++s)   // streamed once: non-temporal
      bx[s] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(xb + col(s)));
  };

  // one item: rms_norm (x * rrms * w, rounded to x's dtype), then * t and
  // + shift, each rounded, as the eager op order does
  auto element = [&](int s, float rr, const float* t8, const float* sh8, S* ob) __attribute__((always_inline)) {
    V8<TX> xv, wv;
    xv.v = *reinterpret_cast<const uint4*>(lrow + col(s));
    if constexpr (WEIGHT) wv.v = *reinterpret_cast<const uint4*>(lw + col(s));
    float y[8];
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
      float n0 = g8<TX>(xv, j) * rr, n1 = g8<TX>(xv, j + 1) * rr;
      if constexpr (WEIGHT) { n0 = n0 * g8<TX>(wv, j); n1 = n1 * g8<TX>(wv, j + 1); }
      TX::round2(n0, n1);
      n0 = n0 * t8[j]; n1 = n1 * t8[j + 1];
      TX::round2(n0, n1);
      n0 = n0 + sh8[j]; n1 = n1 + sh8[j + 1];
      TX::round2(n0, n1);
      y[j] = n0;
      y[j + 1] = n1;
    }
    const V8<TX> ov = pack8<TX>(y);
    __builtin_nontemporal_store(u32x4{ov.v.x, ov.v.y, ov.v.z, ov.v.w}, reinterpret_cast<u32x4*>(ob + col(s)));
  };

  auto process = [&](int64_t row, u32x4 (&bx)[NSTEP]) __attribute__((always_inline)) {
#pragma unroll
    for (int s = 0; s < NSTEP; ++s) *reinterpret_cast<u32x4*>(lrow + col(s)) = bx[s];
    // the buffer is free again: loads of row i+2, kept in program order
    // (ahead of this row's stores) so the next wait can leave them in flight
    __builtin_amdgcn_sched_barrier(0);
    issue(row + 2 * stride, bx);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): this wave's LDS stores done
    __builtin_amdgcn_wave_barrier();
    const float tot = ref_order_sumsq<TX>(lrow, D, lane);
    const float rr = 1.0f / sqrtf(tot / (float)D + a.eps);
    const int64_t m = mod_row(row);
    S* ob = static_cast<S*>(a.o0) + row * a.ldo;
    if (m == m0) {
#pragma unroll
      for (int s = 0; s < NSTEP; ++s) {
        V8<TX> vt, vh;
        vt.v = *reinterpret_cast<const uint4*>(lt + col(s));
        vh.v = *reinterpret_cast<const uint4*>(lsh + col(s));
        float t8[8], sh8[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) { t8[j] = g8<TX>(vt, j); sh8[j] = g8<TX>(vh, j); }
        element(s, rr, t8, sh8, ob);
      }
    } else {
      const S* sc = static_cast<const S*>(a.scale) + m * a.mod_ld;
      const S* sh = static_cast<const S*>(a.shift) + m * a.mod_ld;
#pragma unroll
      for (int s = 0; s < NSTEP; ++s) {
        V8<TX> vs, vh;
        ld8<TX>(sc, col(s), vs);
        ld8<TX>(sh, col(s), vh);
        float t8[8], sh8[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) { t8[j] = TX::round(1.0f + g8<TX>(vs, j)); sh8[j] = g8<TX>(vh, j); }
        element(s, rr, t8, sh8, ob);
      }
    }
    // the next row's staging overwrites this wave's LDS slice: every lane's
    // reads of it must be done
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
  };

  // first row peeled off the loop so that the loop is entered with the
  // memory operations of its back edge in flight
  u32x4 x0[NSTEP], x1[NSTEP];
  issue(r, x0);
  issue(r + stride, x1);
  __builtin_amdgcn_sched_barrier(0);
  process(r, x0);
  r += stride;
  while (r < last) {
    process(r, x1);
    r += stride;
    if (r >= last) break;
    process(r, x0);
    r += stride;
  }
  __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): no load lands after the wave ends
}

// ---------------------------------------------------------------------------
// Cooperative rms_adaln for 16-bit rows whose modulation has the rows'
// dtype, on the plan of the cooperative norm-rope kernel: a row is split
// into W parts of PS = 512 CPP elements (the last part may be shorter), one
// wave per part; a block of R * W waves takes the R consecutive rows of a
// row group per iteration, one block per CU, the blocks visiting groups
// blockIdx.x, + gridDim.x, ... (one dense window of rows in flight).
//
// The reference-order sum of squares (ref_order_sumsq): full chunks j of 512
// positions give chain sums c_j (16 squares from zero), folded in order into
// the acc1 / acc2 / acc3 cascade; the rem = D / 32 - 16 * nchunks i-steps
// past the last full chunk are summed from zero into acc0 (by the wave whose
// part holds them: host-checked to be one part), and D % 32 == 0 leaves no
// leftover vector. Each wave writes its chunk sums (and acc0), and after an
// LDS-only barrier every wave of the row folds them in the reference order:
// bit-identical rrms.
//
// Per lane: CPP items of 8 elements at part offsets 512 k + 8 lane (clamped
// to the row's last item past the end, and rows past the last to the last
// row: every load and store is unpredicated, a clamped item rewrites its
// source item's identical output, computed from loads issued before any
// store of that row group, so in-place calls stay exact), the norm weight of
// those items held as fp32 for the whole kernel, round(1 + scale) and shift
// of the current modulation row held as fp32 until a row of another
// modulation row comes (segment or sample boundaries). PF row groups are
// prefetched into registers. LDS: per wave a staged part (512-element blocks
// padded by 64 bytes, so the two halves of a wave's ordered reads fall in
// different banks), chunk sums and acc0 in two parity slots.
//
// The kernel is VALU-heavy for a streaming kernel (about 10 VALU operations
// per element at 64 lanes per CU per clock): the modulation is unpacked once,
// the last rounding is the output packing, and every memory operation is
// issued on every path so that the compiler's waits leave the prefetch in
// flight (a conditional load or store anywhere in the loop makes them wait
// for everything).
// ---------------------------------------------------------------------------
template <typename TX, bool WEIGHT, int CPP, int PF>
__global__ __launch_bounds__(768) void adaln_coop_kernel(RowArgs a, int W) {
  using S = typename TX::storage;
  static_assert(sizeof(S) == 2, "16-bit rows");
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  constexpr int PS = 512 * CPP, SLICE = PS + 32 * CPP;      // staged elements per wave (padded)
  extern __shared__ __attribute__((aligned(16))) uint8_t dyn_lds[];
  const int D = (int)a.D;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int R = (blockDim.x >> 6) / W;
  const int sub = w / W, part = w - sub * W;
  const int steps = D >> 5, nchunks = steps >> 4, rem = steps - nchunks * 16;
  S* stage = reinterpret_cast<S*>(dyn_lds) + w * SLICE;
  float* sums = reinterpret_cast<float*>(dyn_lds + (size_t)R * W * SLICE * sizeof(S));   // [2][R][nchunks][32]
  float* acc0s = sums + 2 * R * nchunks * 32;                                              // [2][R][32]
  const int base = part * PS;
  const int last_item = D - 8;
  auto col = [&](int k) { const int c = base + k * 512 + lane * 8; return c < D ? c : last_item; };
  auto spos = [&](int p) { return p + (p >> 9) * 32; };     // padded staging position of part offset p

  // weight, round(1 + scale) and shift held as fp32 (unpacked once)
  float wf[CPP][8], tf[CPP][8], shf[CPP][8];
  if constexpr (WEIGHT) {
#pragma unroll
    for (int k = 0; k < CPP; ++k) {
      V8<TX> wv;
      ld8<TX>(a.weight, col(k), wv);
#pragma unroll
      for (int j = 0; j < 8; ++j) wf[k][j] = g8<TX>(wv, j);
    }
  }
  int64_t mcur = -1;
  auto load_mod = [&](int64_t m) __attribute__((always_inline)) {
    const S* sc = static_cast<const S*>(a.scale) + m * a.mod_ld;
    const S* sh = static_cast<const S*>(a.shift) + m * a.mod_ld;
#pragma unroll
    for (int k = 0; k < CPP; ++k) {
      V8<TX> vs, vh;
      ld8<TX>(sc, col(k), vs);
      ld8<TX>(sh, col(k), vh);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        tf[k][j] = TX::round(1.0f + g8<TX>(vs, j));   // (1 + scale) in its dtype
        shf[k][j] = g8<TX>(vh, j);
      }
    }
    mcur = m;
  };

  // 32-bit row and group indices (the launcher checks rows < 2^30). The wave
  // takes row gg * R + sub of groups gg = blockIdx.x + it * G, it = 0, 1, ...
  const int nrows = (int)a.rows, ngroups = (nrows + R - 1) / R;
  const int G = gridDim.x;
  if ((int)blockIdx.x >= ngroups) return;   // uniform per block
  const int iters = (ngroups - (int)blockIdx.x + G - 1) / G;
  auto row_of = [&](int it) {
    const int row = ((int)blockIdx.x + it * G) * R + sub;
    return row < nrows ? row : nrows - 1;   // past the end: the last row again
  };

  // Modulation rows of this wave's rows, 64 iterations at a time: lane l
  // holds that of iteration it0 + l. The refill consumes its load inside its
  // branch, so no load of it is pending past the branch, and the loop's waits
  // count only the row loads and stores.
  int mtab = 0;
  const int mod_group = (int)a.mod_group;   // < 2^31 (launcher)
  auto fill = [&](int it0) __attribute__((always_inline)) {
    const int row = row_of(it0 + lane < iters ? it0 + lane : iters - 1);
    if (a.row_map) {
      const int r = a.row_map[row];
      mtab = r < 0 ? 0 : (r >= mod_group ? mod_group - 1 : r);   // clamped into the table
    } else {
      mtab = row / mod_group;
    }
  };

  auto issue = [&](int it, u32x4 (&bx)[CPP]) __attribute__((always_inline)) {
    const S* xb = static_cast<const S*>(a.x0) + (int64_t)row_of(it < iters ? it : iters - 1) * a.ldx;
#pragma unroll
    for (int k = 0; k < CPP; ++k)   // streamed once: non-temporal
      bx[k] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(xb + col(k)));
  };

  int par = 0;
  auto process = [&](int it, u32x4 (&bx)[CPP]) __attribute__((always_inline)) {
    const int row = row_of(it);
    const int slot = par * R + sub;
#pragma unroll
    for (int k = 0; k < CPP; ++k) *reinterpret_cast<u32x4*>(stage + spos(k * 512 + lane * 8)) = bx[k];
    __builtin_amdgcn_sched_barrier(0);
    issue(it + PF, bx);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): this wave's staging stores done
    __builtin_amdgcn_wave_barrier();
    {
      const int L = lane & 31, h = lane >> 5;
#pragma unroll
      for (int q = 0; q < CPP; q += 2) {
        const int j = part * CPP + q + h;                     // this lane's chunk
        if (q + h < CPP && j < nchunks) {
          float c = 0.0f;
#pragma unroll
          for (int u = 0; u < 16; ++u) c = add_sq<TX>(c, TX::load(stage[(q + h) * 544 + u * 32 + L]));
          sums[(slot * nchunks + j) * 32 + L] = c;
        }
      }
      if (rem && base <= nchunks * 512 && nchunks * 512 < base + PS && h == 0) {
        // the i-steps past the last full chunk (this part holds them)
        float c0 = 0.0f;
        const int p0 = nchunks * 512 - base;
        const S* rp = stage + spos(p0) + L;   // one 512-element block
        for (int i = 0; i < rem; ++i) c0 = add_sq<TX>(c0, TX::load(rp[i * 32]));
        acc0s[slot * 32 + L] = c0;
      }
    }
    // publish the sums to the block (LDS only: the prefetched rows stay in flight)
    __builtin_amdgcn_s_waitcnt(0xc07f);
    asm volatile("s_barrier" ::: "memory");
    float rr;
    {
      const int L = lane & 31;
      const float* cs = sums + slot * nchunks * 32 + L;
      float acc1 = 0.0f, acc2 = 0.0f, acc3 = 0.0f;
      for (int j = 0; j < nchunks; ++j) {
        acc1 = acc1 + cs[j * 32];
        const int i_end = (j + 1) * 16;
        if ((i_end & (15 << 4)) == 0) {
          acc2 = acc2 + acc1;
          acc1 = 0.0f;
          if ((i_end & (15 << 8)) == 0) {
            acc3 = acc3 + acc2;
            acc2 = 0.0f;
          }
        }
      }
      const float acc0 = rem ? acc0s[slot * 32 + L] : 0.0f;
      const float tot = ((acc0 + acc1) + acc2) + acc3;
      const int v8 = lane & 7;
      const float r0 = __shfl(tot, v8, 64), r1 = __shfl(tot, v8 + 8, 64);
      const float r2 = __shfl(tot, v8 + 16, 64), r3 = __shfl(tot, v8 + 24, 64);
      const float pv = ((r0 + r1) + r2) + r3;
      float fin = 0.0f;
#pragma unroll
      for (int v = 0; v < 8; ++v) fin = fin + __shfl(pv, v, 64);
      rr = 1.0f / sqrtf(fin / (float)D + a.eps);
    }
    if ((it & 63) == 0) fill(it);
    const int64_t m = __builtin_amdgcn_readlane(mtab, it & 63);
    if (m != mcur) load_mod(m);
    S* ob = static_cast<S*>(a.o0) + (int64_t)row * a.ldo;
#pragma unroll
    for (int k = 0; k < CPP; ++k) {
      V8<TX> xv;
      xv.v = *reinterpret_cast<const uint4*>(stage + spos(k * 512 + lane * 8));
      float y[8];
#pragma unroll
      for (int j = 0; j < 8; j += 2) {
        float n0 = g8<TX>(xv, j) * rr, n1 = g8<TX>(xv, j + 1) * rr;
        if constexpr (WEIGHT) { n0 = n0 * wf[k][j]; n1 = n1 * wf[k][j + 1]; }
        TX::round2(n0, n1);
        n0 = n0 * tf[k][j]; n1 = n1 * tf[k][j + 1];
        TX::round2(n0, n1);
        y[j] = n0 + shf[k][j];          // the packing below is its rounding
        y[j + 1] = n1 + shf[k][j + 1];
      }
      const V8<TX> ov = pack8<TX>(y);
      // unpredicated: a clamped item (past the row's end, or a row past the
      // last) rewrites its source item's output with identical bytes
      __builtin_nontemporal_store(u32x4{ov.v.x, ov.v.y, ov.v.z, ov.v.w}, reinterpret_cast<u32x4*>(ob + col(k)));
    }
    // the next row's staging overwrites this wave's slice
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    par ^= 1;
  };

  // PF groups in flight, in PF register buffers taken in turn (iteration it
  // in buffer it % PF). The first iteration is peeled off the loop, the loop
  // body is PF whole iterations with its only exit at the bottom and the
  // last (iters - 1) % PF iterations follow it: the loop head is then reached
  // only with the other buffers' loads, one prefetch and its stores
  // outstanding (as on the back edge, save for older stores), so the waits
  // the compiler places there leave the prefetched groups in flight.
  u32x4 xb[PF][CPP];
#pragma unroll
  for (int i = 0; i < PF; ++i) issue(i, xb[i]);
  __builtin_amdgcn_sched_barrier(0);
  process(0, xb[0]);
  int it = 1;
  for (; it + PF <= iters; it += PF) {
#pragma unroll
    for (int i = 1; i <= PF; ++i) process(it + i - 1, xb[i % PF]);
  }
#pragma unroll
  for (int i = 1; i < PF; ++i)
    if (it + i - 1 < iters) process(it + i - 1, xb[i % PF]);
  __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): no load lands after the wave ends
}

// ---------------------------------------------------------------------------
// head-span kernel: LPH lanes per (b, s, h) head
// ---------------------------------------------------------------------------
// Division of non-negative 64-bit values by a launch-invariant divisor d >= 1
// with a precomputed multiplier (Granlund & Montgomery, "Division by
// invariant integers using multiplication", PLDI 1994, the round-up form):
// l = ceil(log2 d), m = floor(2^64 (2^l - d) / d) + 1,
// q = (t + ((n - t) >> 1)) >> (l - 1) with t = mulhi(m, n); d == 1 is q = n.
struct FastDivU64 {
  uint64_t d, m;
  int l;
  static FastDivU64 make(uint64_t d) {
    FastDivU64 f{d, 0, 0};
    while (f.l < 64 && (uint64_t(1) << f.l) < d) ++f.l;
    if (d > 1) {
      const unsigned __int128 two_l = (unsigned __int128)1 << f.l;
      f.m = (uint64_t)((((two_l - d) << 64) / d) + 1);
    }
    return f;
  }
  __device__ __forceinline__ uint64_t div(uint64_t n) const {
    if (d == 1) return n;
    const uint64_t t = __umul64hi(m, n);
    return (t + ((n - t) >> 1)) >> (l - 1);
  }
};

struct HeadArgs {
  void* x; void* out;                 // out may alias x (in place)
  int64_t B, S, H, D;
  FastDivU64 divS, divH;              // by S and by H
  int64_t sb, ss, sh;                 // element strides of x
  int64_t ob, os, oh;                 // element strides of out
  const void* weight;                 // [D] (NORM)
  const void* freqs;
  int64_t fb, fs, fh;                 // table strides (0 = broadcast), pairs contiguous
  int rot;                            // rotated prefix
  float eps;
  // a second tensor of the same shape and strides (the cooperative QK
  // kernel, nt = 2): its input, output and norm weight
  void* x1; void* out1;
  const void* weight1;
};

// TABL: the table is shared by the heads of a token (head stride 0) and the
// block's heads span at most 8 tokens; the block stages those table rows in
// LDS once instead of every pair lane reading its 128 bytes from L2.
// Pair lane s owns TAB_CPL 16-byte chunks of a staged row; its chunk k is
// stored at slot (k - s) mod TAB_CPL of its segment, so at each read step the
// lanes of a group touch different banks.
template <typename TF>
constexpr int tab_cpl() { return 8 * 4 * (int)sizeof(typename TF::storage) / 16; }
template <typename TF>
__device__ __forceinline__ int tab_slot(int c) {   // chunk c of a row -> stored chunk
  constexpr int CPL = tab_cpl<TF>();
  const int seg = c / CPL, k = c - seg * CPL;
  return seg * CPL + ((k - seg) & (CPL - 1));
}
template <typename TF>
__device__ __forceinline__ void lds_tab8(const uint8_t* row, int seg, Tab8<TF>& t) {
  constexpr int CPL = tab_cpl<TF>();
  const uint8_t* p = row + seg * CPL * 16;
  uint4 raw[CPL];
#pragma unroll
  for (int k = 0; k < CPL; ++k) raw[k] = *reinterpret_cast<const uint4*>(p + ((k - seg) & (CPL - 1)) * 16);
#pragma unroll
  for (int pp = 0; pp < 8; ++pp)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int idx = pp * 4 + e;     // element of the lane's 32
      if constexpr (sizeof(typename TF::storage) == 4) {
        t.f[pp][e] = __uint_as_float((&raw[idx >> 2].x)[idx & 3]);
      } else {
        const uint32_t w = (&raw[idx >> 3].x)[(idx & 7) >> 1];
        t.f[pp][e] = TF::load((idx & 1) ? (w >> 16) : (w & 0xffffu));
      }
    }
}

constexpr int HEAD_TAB_ROWS = 8, HEAD_TAB_ROW_BYTES = 1024;   // rot <= 128, fp32

// SPLIT: pairs (i, i + rot/2), items of 8 at head offsets i and i + rot/2;
// otherwise interleaved pairs (2i, 2i + 1), an item is 8 consecutive elements
// (4 pairs) and the table rows are read directly.
template <typename TX, typename TW, typename TF, bool NORM, int LPH, bool TABL, bool SPLIT>
__global__ __launch_bounds__(256) void headspan_kernel(HeadArgs a) {
  static_assert(SPLIT || !TABL, "the LDS table staging serves the split-half layout");
  const int lane = threadIdx.x & 63;
  const int64_t head = (int64_t)blockIdx.x * (256 / LPH) + threadIdx.x / LPH;
  const int it = threadIdx.x % LPH;
  const int64_t nheads = a.B * a.S * a.H;
  // keep whole-group participation in the shuffles: out-of-range groups
  // compute on a clamped head and skip the stores
  const bool live = head < nheads;
  const int64_t hd = live ? head : 0;
  const int64_t bs = (int64_t)a.divH.div((uint64_t)hd), h = hd - bs * a.H;
  const int64_t b = (int64_t)a.divS.div((uint64_t)bs), s = bs - b * a.S;
  const int half = a.rot >> 1;
  const int pair_items = SPLIT ? half / 8 : a.rot / 8;
  const int tail_items = (int)((a.D - a.rot) / 8);
  const bool is_pair = it < pair_items;
  const bool is_tail = !is_pair && it < pair_items + tail_items;
  int64_t c0 = 0, c1 = 0;
  if (is_pair) { c0 = it * 8; c1 = c0 + half; }
  else if (is_tail) { c0 = a.rot + (int64_t)(it - pair_items) * 8; }
  const bool two = SPLIT && is_pair;          // the item's second 8 elements
  const int64_t xoff = b * a.sb + s * a.ss + h * a.sh;
  const int64_t ooff = b * a.ob + s * a.os + h * a.oh;

  V8<TX> v0, v1;
  if (is_pair || is_tail) {
    ld8<TX>(a.x, xoff + c0, v0);
    if (two) ld8<TX>(a.x, xoff + c1, v1);
  }
  // the norm weight and the table do not depend on the reduction: their loads
  // go out with the row's, so the element pass waits on one memory latency
  V8<TW> wv0, wv1;
  Tab8<TF> tab;
  if constexpr (NORM) {
    if (is_pair || is_tail) {
      ld8<TW>(a.weight, c0, wv0);
      if (two) ld8<TW>(a.weight, c1, wv1);
    }
  }
  if constexpr (TABL) {
    __shared__ __attribute__((aligned(16))) uint8_t tabs[HEAD_TAB_ROWS * HEAD_TAB_ROW_BYTES];
    constexpr int G = 256 / LPH;
    const int64_t first = (int64_t)blockIdx.x * G;
    const int64_t last = (first + G < nheads ? first + G : nheads) - 1;
    const int64_t bs0 = (int64_t)a.divH.div((uint64_t)first);
    const int nrow = (int)((int64_t)a.divH.div((uint64_t)last) - bs0 + 1);   // <= HEAD_TAB_ROWS (host)
    const int row_bytes = half * 4 * (int)sizeof(typename TF::storage);
    const int chunks = row_bytes / 16;
    for (int i = threadIdx.x; i < nrow * chunks; i += 256) {
      const int rrow = i / chunks, c = i - rrow * chunks;
      const int64_t bsr = bs0 + rrow, br = (int64_t)a.divS.div((uint64_t)bsr), sr = bsr - br * a.S;
      const uint8_t* src = static_cast<const uint8_t*>(a.freqs) +
                           (br * a.fb + sr * a.fs) * (int64_t)sizeof(typename TF::storage);
      *reinterpret_cast<uint4*>(tabs + rrow * HEAD_TAB_ROW_BYTES + tab_slot<TF>(c) * 16) =
          *reinterpret_cast<const uint4*>(src + c * 16);
    }
    __syncthreads();
    if (is_pair && live)
      lds_tab8<TF>(tabs + (bs - bs0) * HEAD_TAB_ROW_BYTES, it, tab);
  } else if constexpr (SPLIT) {
    if (is_pair) load_tab8<TF>(a.freqs, b * a.fb + s * a.fs + h * a.fh + (int64_t)it * 8 * 4, tab);
  } else {
    if (is_pair) load_tab4<TF>(a.freqs, b * a.fb + s * a.fs + h * a.fh + (int64_t)it * 4 * 4, tab);
  }
  float rr = 1.0f;
  if constexpr (NORM) {
    // per-head sum of squares in the reference's order (see ref_order_sumsq):
    // the head is staged in LDS, lane g of the group walks chains
    // L = g, g + LPH, ... (32 chains, each over positions 32*i + L), then the
    // chain totals are combined row-wise and lane by lane.
    // rows padded by 16 bytes: the groups of a wave start 4 banks apart
    constexpr int HROW = 16 * LPH + 16 / (int)sizeof(typename TX::storage);
    __shared__ __attribute__((aligned(16))) typename TX::storage heads[256 / LPH][HROW];
    typename TX::storage* hrow = heads[threadIdx.x / LPH];
    if (is_pair || is_tail) {
      st8<TX>(hrow, c0, v0);
      if (two) st8<TX>(hrow, c1, v1);
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    constexpr int NCH = LPH >= 32 ? 1 : 32 / LPH;
    const int D = (int)a.D, steps = D >> 5;
    float tch[NCH];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int L = it + c * LPH;
      float acc = 0.0f;
      if (L < 32) {
        // D <= 16 * LPH (host), so at most LPH / 2 steps of 32 and 3 leftover
        // vectors: fully unrolled, every read is issued before the first add
        constexpr int MAXS = LPH / 2 < 16 ? LPH / 2 : 16;
#pragma unroll
        for (int i = 0; i < MAXS; ++i) {
          if (i < steps) {
            const float x = TX::load(hrow[i * 32 + L]);
            acc = add_sq<TX>(acc, x);
          }
        }
#pragma unroll
        for (int e = 0; e < 3; ++e) {  // leftover 8-lane vectors -> row 0
          const int q = steps * 4 + e;
          if (q < (D >> 3)) {
            const float x = TX::load(hrow[q * 8 + (L & 7)]);
            if (L < 8) acc = add_sq<TX>(acc, x);
          }
        }
      }
      tch[c] = acc;
    }
    const int gbase = lane - (lane % LPH);
    float fin = 0.0f;
    if constexpr (LPH <= 8) {
      // chain L = v + 8r sits on lane v % LPH, slot L / LPH: the 4-row sum of
      // lane-vector v is local to one lane; only the 8 row sums travel
      constexpr int NV = 8 / LPH;
      float rs[NV];
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        float r = tch[k];
#pragma unroll
        for (int q = 1; q < 4; ++q) r = r + tch[k + q * NV];
        rs[k] = r;     // lane-vector v = it + k * LPH
      }
#pragma unroll
      for (int v = 0; v < 8; ++v) fin = fin + __shfl(rs[v / LPH], gbase + (v % LPH), 64);
    } else {
#pragma unroll
      for (int v = 0; v < 8; ++v) {
        float rsum = 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int L = v + 8 * r;
          const float t = __shfl(tch[(L / LPH) < NCH ? (L / LPH) : 0], gbase + (L % LPH), 64);
          rsum = r ? rsum + t : t;
        }
        fin = fin + rsum;
      }
    }
    rr = 1.0f / sqrtf(fin / (float)a.D + a.eps);
  }
  if (!live || !(is_pair || is_tail)) return;

  // element pass in fp32: each element is unpacked once, rounded where the
  // eager op order rounds, and packed two per conversion on the way out (the
  // pack rounds to x's dtype, which is the rotation's last rounding)
  float y0[8], y1[8];
  auto normalise = [&](const V8<TX>& vv, const V8<TW>& wv, float* y) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      y[j] = g8<TX>(vv, j);
      if constexpr (NORM) y[j] = TX::round((y[j] * rr) * g8<TW>(wv, j));
    }
  };
  normalise(v0, wv0, y0);
  if constexpr (!SPLIT) {
    if (is_pair) {
      float r0[8];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        rotate_pair_fma<TF, F32T>(y0[2 * j], y0[2 * j + 1], tab.f[j][0], tab.f[j][1], tab.f[j][2], tab.f[j][3],
                                  r0[2 * j], r0[2 * j + 1]);
      st8<TX>(a.out, ooff + c0, pack8<TX>(r0));
      return;
    }
  }
  if (two) {
    normalise(v1, wv1, y1);
    float r0[8], r1[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      rotate_pair<TF, F32T>(y0[j], y1[j], tab.f[j][0], tab.f[j][1], tab.f[j][2], tab.f[j][3], r0[j], r1[j]);
    st8<TX>(a.out, ooff + c0, pack8<TX>(r0));
    st8<TX>(a.out, ooff + c1, pack8<TX>(r1));
  } else if constexpr (NORM) {
    st8<TX>(a.out, ooff + c0, pack8<TX>(y0));
  } else {
    st8<TX>(a.out, ooff + c0, v0);      // pass-through dims keep their bits
  }
}

// ---------------------------------------------------------------------------
// Cooperative per-head RMSNorm + full split-half rotation of [B, S, H, D]
// heads (the QK norm-rope), D = 64, 96 or 128, 16-bit values, one table row
// per token (head stride 0). A token row of H heads is split into P parts of
// HPW = 64 / LPH heads (LPH = D / 16 lanes per head, lane p holding the items
// at head offsets 8 p and 8 p + D / 2; lanes past HPW * LPH, and the heads
// past H of the last part, redo the part's last head), one wave per part; a
// block of R * P waves takes R consecutive tokens per iteration, one block
// per CU, the blocks visiting token groups blockIdx.x, + gridDim.x, ...: one
// dense window of the tensor in flight, as in the cooperative norm-rope.
// Wave p of a token loads the p-th slice of the token's table row, the block
// shares the row in LDS (one LDS-only barrier per iteration, the table in
// two parity slots), so each row is read once per token rather than once per
// wave. The sum of squares of a head stays in its wave: HPW x 8 jobs, job
// (head, v) summing the chains v, v + 8, v + 16, v + 24 (each D / 32 squares
// from zero, the reference order of ref_order_sumsq with no full chunk and
// no leftover vector) into ((c_v + c_v+8) + c_v+16) + c_v+24, and a head's
// lanes add its 8 job results in order from zero: bit-identical rrms.
// Every path issues the same loads and stores (clamped rows, heads and
// iterations recompute from loads issued before any store of theirs and
// store identical bytes, so in-place calls stay exact).
// ---------------------------------------------------------------------------
template <typename TX, typename TW, typename TF, int D>
__global__ __launch_bounds__(768) void qk_coop_kernel(HeadArgs a, int P, int nt) {
  using S = typename TX::storage;
  using SF = typename TF::storage;
  static_assert(sizeof(S) == 2, "16-bit heads");
  static_assert(D == 64 || D == 96 || D == 128, "head width");
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  constexpr int LPH = D / 16, HPW = 64 / LPH, HALF = D / 2, STEPS = D / 32;
  constexpr int HROW = D + 8;                         // staged head (elements), rows 16 bytes apart in banks
  constexpr int RB = HALF * 4 * (int)sizeof(SF);      // table row bytes
  constexpr int RCH = RB / 16;                        // its 16-byte chunks
  constexpr int NJOB = HPW * 8;
  constexpr int WSLICE = HPW * HROW * 2 + NJOB * 4;   // LDS bytes per wave
  extern __shared__ __attribute__((aligned(16))) uint8_t dyn_lds[];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int R = (blockDim.x >> 6) / P;
  const int sub = w / P, part = w - sub * P;
  S* xs = reinterpret_cast<S*>(dyn_lds + w * WSLICE);                 // [HPW][HROW]
  float* rs = reinterpret_cast<float*>(dyn_lds + w * WSLICE + HPW * HROW * 2);
  uint8_t* tabs = dyn_lds + R * P * WSLICE;                            // [2][R][RB]
  const int slot0 = lane / LPH, p = lane - slot0 * LPH;
  const int c0 = 8 * p, c1 = c0 + HALF;
  // the lane's head within the token (past the part or the token: the last)
  const int hl = min(part * HPW + min(slot0, HPW - 1), (int)a.H - 1);
  const int hslot = hl - part * HPW;                                   // its staged row
  const int cpw = (RCH + P - 1) / P;                                   // table chunks per wave
  const int tch = min(part * cpw + min(lane, cpw - 1), RCH - 1);       // this lane's chunk
  // Global loads and stores move whole 16-byte chunks in memory order (lane
  // l: chunks l and 64 + l of the part, CPH per head), so each instruction
  // covers whole cache lines; the pairs are formed in LDS. Chunks past the
  // part's heads (or past H) redo the part's last chunk.
  constexpr int CPH = D / 8, NCHK = HPW * CPH;
  int ch_head[2], ch_off[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int c = min(lane + 64 * i, NCHK - 1);
    const int hh = min(part * HPW + c / CPH, (int)a.H - 1);
    ch_head[i] = hh;
    ch_off[i] = (hh - part * HPW) * HROW + (hh == part * HPW + c / CPH ? c % CPH : CPH - 1) * 8;
  }

  // the lane's norm weights of both tensors (the second: the first again
  // when nt = 1)
  float wq[2][8], wk[2][8];
  {
    V8<TW> v[4];
    ld8<TW>(a.weight, c0, v[0]);
    ld8<TW>(a.weight, c1, v[1]);
    ld8<TW>(nt > 1 ? a.weight1 : a.weight, c0, v[2]);
    ld8<TW>(nt > 1 ? a.weight1 : a.weight, c1, v[3]);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      wq[0][j] = g8<TW>(v[0], j); wq[1][j] = g8<TW>(v[1], j);
      wk[0][j] = g8<TW>(v[2], j); wk[1][j] = g8<TW>(v[3], j);
    }
  }

  // 32-bit row indices (the launcher checks nt B S < 2^30); rows are the
  // tokens of the first tensor, then those of the second
  const int ntok = (int)(a.B * a.S), nrows = ntok * nt, ngroups = (nrows + R - 1) / R;
  const int G = gridDim.x;
  if ((int)blockIdx.x >= ngroups) return;   // uniform per block
  const int iters = (ngroups - (int)blockIdx.x + G - 1) / G;
  // row of this wave in iteration it (past the block's last iteration: that
  // one again; past the last row: the last row)
  auto row_of = [&](int it) {
    it = it < iters ? it : iters - 1;
    const int r = ((int)blockIdx.x + it * G) * R + sub;
    return r < nrows ? r : nrows - 1;
  };
  struct Tok { const S* x; S* o; const uint8_t* t; bool second; };
  auto tok_at = [&](int r) __attribute__((always_inline)) {
    const bool second = r >= ntok;
    const int t = second ? r - ntok : r;
    const int64_t b = (int64_t)a.divS.div((uint64_t)t), s = (int64_t)t - b * a.S;
    Tok k;
    k.x = static_cast<const S*>(second ? a.x1 : a.x) + b * a.sb + s * a.ss;
    k.o = static_cast<S*>(second ? a.out1 : a.out) + b * a.ob + s * a.os;
    k.t = static_cast<const uint8_t*>(a.freqs) + (b * a.fb + s * a.fs) * (int64_t)sizeof(SF);
    k.second = second;
    return k;
  };

  auto issue = [&](int it, u32x4 (&bx)[2], u32x4& bt) __attribute__((always_inline)) {
    const Tok tk = tok_at(row_of(it));
    const S* xp = tk.x;
#pragma unroll
    for (int i = 0; i < 2; ++i)
      bx[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
          xp + (int64_t)ch_head[i] * a.sh + (ch_off[i] - (ch_head[i] - part * HPW) * HROW)));
    bt = *reinterpret_cast<const u32x4*>(tk.t + tch * 16);
  };

  int par = 0;
  auto process = [&](int it, u32x4 (&bx)[2], u32x4& bt) __attribute__((always_inline)) {
    uint8_t* trow = tabs + (par * R + sub) * RB;
    *reinterpret_cast<u32x4*>(&xs[ch_off[0]]) = bx[0];
    *reinterpret_cast<u32x4*>(&xs[ch_off[1]]) = bx[1];
    *reinterpret_cast<u32x4*>(trow + tch * 16) = bt;
    __builtin_amdgcn_sched_barrier(0);
    issue(it + 2, bx, bt);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): the staging stores are done
    __builtin_amdgcn_wave_barrier();
    // job pairs (head, v), (head, v + 1), v even: each 32-bit read holds
    // the elements of chains v + 8 g and v + 1 + 8 g; NJOB / 2 <= 64 lanes
    static_assert(NJOB / 2 <= 64, "one round of job pairs");
    if (lane < NJOB / 2) {
      const S* hr = xs + (lane >> 2) * HROW;
      const int v = (lane & 3) * 2;
      float r0 = 0.0f, r1 = 0.0f;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float c0 = 0.0f, c1 = 0.0f;
#pragma unroll
        for (int i = 0; i < STEPS; ++i) {
          const uint32_t w2 = *reinterpret_cast<const uint32_t*>(hr + i * 32 + v + 8 * g);
          c0 = add_sq<TX>(c0, TX::load(w2 & 0xffffu));
          c1 = add_sq<TX>(c1, TX::load(w2 >> 16));
        }
        r0 = g ? r0 + c0 : c0;
        r1 = g ? r1 + c1 : c1;
      }
      *reinterpret_cast<float2*>(rs + (lane >> 2) * 8 + v) = make_float2(r0, r1);
    }
    // publish the job results and the table slices (LDS only: the
    // prefetched rows stay in flight)
    __builtin_amdgcn_s_waitcnt(0xc07f);
    asm volatile("s_barrier" ::: "memory");
    float fin = 0.0f;
#pragma unroll
    for (int v = 0; v < 8; ++v) fin = fin + rs[hslot * 8 + v];
    const float rr = 1.0f / sqrtf(fin / (float)D + a.eps);
    V8<TX> v0, v1;
    v0.v = *reinterpret_cast<const uint4*>(&xs[hslot * HROW + c0]);
    v1.v = *reinterpret_cast<const uint4*>(&xs[hslot * HROW + c1]);
    const SF* tp = reinterpret_cast<const SF*>(trow) + c0 * 4;   // pair c0's entries
    const Tok tk = tok_at(row_of(it));
    float r0[8], r1[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float y0 = TX::round((g8<TX>(v0, j) * rr) * (tk.second ? wk[0][j] : wq[0][j]));
      const float y1 = TX::round((g8<TX>(v1, j) * rr) * (tk.second ? wk[1][j] : wq[1][j]));
      rotate_pair<TF, F32T>(y0, y1, TF::load(tp[4 * j]), TF::load(tp[4 * j + 1]), TF::load(tp[4 * j + 2]),
                            TF::load(tp[4 * j + 3]), r0[j], r1[j]);
    }
    // the rotated pairs back into the staged heads, then out in memory order
    const V8<TX> o0 = pack8<TX>(r0), o1 = pack8<TX>(r1);
    *reinterpret_cast<uint4*>(&xs[hslot * HROW + c0]) = o0.v;
    *reinterpret_cast<uint4*>(&xs[hslot * HROW + c1]) = o1.v;
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    S* op = tk.o;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint4 v = *reinterpret_cast<const uint4*>(&xs[ch_off[i]]);
      __builtin_nontemporal_store(u32x4{v.x, v.y, v.z, v.w},
                                  reinterpret_cast<u32x4*>(op + (int64_t)ch_head[i] * a.oh +
                                                           (ch_off[i] - (ch_head[i] - part * HPW) * HROW)));
    }
    // the next token's staging overwrites the wave's slice
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    par ^= 1;
  };

  // Two token groups in flight in two register buffers taken in turn: the
  // first iteration is peeled off, the loop body is two whole iterations
  // with its only exit at the bottom (an odd count ends with a redo of the
  // block's last iteration, whose loads precede that iteration's stores), so
  // the loop head is reached only with one buffer's loads, one prefetch and
  // its stores outstanding and the compiler's waits leave the prefetch in
  // flight.
  u32x4 x0[2], x1[2], t0, t1;
  issue(0, x0, t0);
  issue(1, x1, t1);
  __builtin_amdgcn_sched_barrier(0);
  process(0, x0, t0);
  for (int it = 1; it < iters; it += 2) {
    process(it, x1, t1);
    process(it + 1, x0, t0);
  }
  __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): no load lands after the wave ends
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
template <typename TX, typename TM, typename TF, bool ROPE, bool ADALN, bool WEIGHT, int IPH, int N>
static int launch_row_n(RowArgs& a, hipStream_t st) {
  // one LDS row per tensor per wave; two waves per workgroup, so that several
  // workgroups share a CU's LDS (one wave per row and nothing else in flight:
  // the occupancy is what hides the memory latency)
  const size_t per_wave = (a.x1 ? 2 : 1) * (size_t)a.D * sizeof(typename TX::storage);
  const int wpb = (int)std::min<size_t>(2, (160 * 1024) / per_wave);
  if (a.D % 8 != 0 || a.D >= (1 << 17) || wpb < 1)
    return fail(XMH3_EUNSUPPORTED, "row-span kernel: width must be a multiple of 8 and below 2^17");
  auto kern = rowspan_exact_kernel<TX, TM, TF, ROPE, ADALN, WEIGHT, IPH, N>;
  static bool attr_set = false;
  if (!attr_set) {
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) !=
        hipSuccess)
      return fail(XMH3_EHIP, "row-span kernel: cannot raise the dynamic LDS limit");
    attr_set = true;
  }
  dim3 grid((unsigned)((a.rows + wpb - 1) / wpb));
  hipLaunchKernelGGL(kern, grid, dim3(64 * wpb), per_wave * wpb, st, a);
  return check_launch("rowspan_exact_kernel");
}

template <typename TX, typename TM, typename TF, bool ROPE, bool ADALN, bool WEIGHT, int IPH>
static int launch_row(RowArgs& a, hipStream_t st) {
  const int64_t items = a.D / (ROPE ? 16 : 8);
  const int64_t steps = (items + 63) / 64;
#define XMH3_R(N) \
  if (steps <= N) return launch_row_n<TX, TM, TF, ROPE, ADALN, WEIGHT, IPH, N>(a, st);
  if constexpr (ROPE) {
    XMH3_R(2) XMH3_R(4) XMH3_R(5) XMH3_R(8)
  } else {
    XMH3_R(2) XMH3_R(4) XMH3_R(8) XMH3_R(11) XMH3_R(16)
  }
#undef XMH3_R
  return fail(XMH3_EUNSUPPORTED, "row-span kernel: row too wide for the register path");
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

static int cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (!cached[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cached[dev] = n;
  }
  return cached[dev];
}

constexpr size_t LDS_BYTES = 160 * 1024;   // gfx950 LDS per workgroup

// Launch of the pipelined rms_adaln kernel, one block of rows per CU.
// Returns -1 (no launch) when the row does not fit its LDS plan.
template <typename TX, bool WEIGHT, int N>
static int launch_adaln_pipe_n(RowArgs& a, hipStream_t st) {
  const size_t row = (size_t)a.D * sizeof(typename TX::storage);
  if (4 * row > LDS_BYTES) return -1;
  const int wpb = (int)std::min<size_t>(8, (LDS_BYTES - 3 * row) / row);
  const size_t lds = (3 + (size_t)wpb) * row;
  auto kern = adaln_pipe_kernel<TX, WEIGHT, N>;
  static bool attr_set = false;
  if (!attr_set) {
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)LDS_BYTES) !=
        hipSuccess)
      return fail(XMH3_EHIP, "rms_adaln kernel: cannot raise the dynamic LDS limit");
    attr_set = true;
  }
  const int64_t cus = std::max(1, cu_count());
  const int64_t chunk = (a.rows + cus - 1) / cus;
  const int64_t grid = (a.rows + chunk - 1) / chunk;
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(64 * wpb), lds, st, a, chunk);
  return check_launch("adaln_pipe_kernel");
}

#ifndef XMH3_ADALN_CPP
#define XMH3_ADALN_CPP 2
#endif
#ifndef XMH3_ADALN_PF
#define XMH3_ADALN_PF 2
#endif
// Launch of the cooperative rms_adaln kernel: one block per CU of R rows of
// W = ceil(D / PS) waves (R * W <= 12). Returns -1 (no launch) when the row
// does not fit its plan (D % 32, the i-steps past the last full chunk split
// over two parts, LDS).
template <typename TX, bool WEIGHT>
static int launch_adaln_coop(RowArgs& a, hipStream_t st) {
  constexpr int CPP = XMH3_ADALN_CPP, PS = 512 * CPP, PF = XMH3_ADALN_PF;
  if (a.x1 || a.D % 32 != 0 || a.D > 16384 || a.rows >= (int64_t(1) << 30) ||
      a.mod_group >= (int64_t(1) << 31))
    return -1;
  const int D = (int)a.D, W = (D + PS - 1) / PS;
  const int nchunks = D / 512, rem = D / 32 - nchunks * 16;
  if (rem && (nchunks * 512) / PS != (D - 1) / PS) return -1;
  if (W > 12) return -1;
  const int R = std::max(1, 12 / W);
  const size_t lds = (size_t)R * W * (PS + 32 * CPP) * sizeof(typename TX::storage) +
                     (size_t)2 * R * nchunks * 32 * 4 + (size_t)2 * R * 32 * 4;
  if (lds > LDS_BYTES) return -1;
  auto kern = adaln_coop_kernel<TX, WEIGHT, CPP, PF>;
  static bool attr_set = false;
  if (!attr_set) {
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)LDS_BYTES) !=
        hipSuccess)
      return fail(XMH3_EHIP, "rms_adaln kernel: cannot raise the dynamic LDS limit");
    attr_set = true;
  }
  const int64_t cus = std::max(1, cu_count());
  const int64_t grid = std::min<int64_t>((a.rows + R - 1) / R, cus);
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(64 * W * R), lds, st, a, W);
  return check_launch("adaln_coop_kernel");
}

template <typename TX, bool WEIGHT>
static int launch_adaln_pipe(RowArgs& a, hipStream_t st) {
  if (a.x1 || a.D % 8 != 0 || a.D >= (1 << 17)) return -1;
  const int64_t steps = (a.D / 8 + 63) / 64;
#define XMH3_AP(N) \
  if (steps <= N) return launch_adaln_pipe_n<TX, WEIGHT, N>(a, st);
  XMH3_AP(2) XMH3_AP(4) XMH3_AP(6) XMH3_AP(8) XMH3_AP(10) XMH3_AP(11) XMH3_AP(12)
#undef XMH3_AP
  return -1;
}

#ifndef XMH3_COOP_ROWS
#define XMH3_COOP_ROWS 4
#endif
// Launch of the cooperative norm-rope kernel: one block per CU of R rows of
// D / 1024 waves (R * P <= 16, R <= 4). Returns -1 (no launch) when the row
// does not fit it.
template <typename TX, typename TF, bool ADALN, int P>
static int launch_coop_p(RowArgs& a, int nt, hipStream_t st) {
  if (a.rows * nt >= (int64_t(1) << 30)) return -1;   // 32-bit row indices
  const int R = std::max(1, std::min(XMH3_COOP_ROWS, 16 / P));
  const size_t lds = (ADALN ? 8 * (size_t)a.D : 0) + (size_t)R * P * 4096 + (size_t)2 * R * 2 * P * 32 * 4 +
                     3 * (size_t)R * 64 * 4 * sizeof(typename TF::storage) + 2 * (size_t)R * 4;
  if (lds > LDS_BYTES) return -1;
  auto kern = norm_rope_coop_kernel<TX, TF, ADALN, P>;
  static bool attr_set = false;
  if (!attr_set) {
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)LDS_BYTES) !=
        hipSuccess)
      return fail(XMH3_EHIP, "norm-rope kernel: cannot raise the dynamic LDS limit");
    attr_set = true;
  }
  const int64_t cus = std::max(1, cu_count());
  const int64_t grid = std::min<int64_t>((a.rows * nt + R - 1) / R, cus);
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(64 * P * R), lds, st, a, nt);
  return check_launch("norm_rope_coop_kernel");
}

template <typename TX, typename TF, bool ADALN>
static int launch_coop(RowArgs& a, int nt, hipStream_t st) {
  if (a.D % 1024 != 0) return -1;
  switch (a.D / 1024) {
    case 1: return launch_coop_p<TX, TF, ADALN, 1>(a, nt, st);
    case 2: return launch_coop_p<TX, TF, ADALN, 2>(a, nt, st);
    case 3: return launch_coop_p<TX, TF, ADALN, 3>(a, nt, st);
    case 4: return launch_coop_p<TX, TF, ADALN, 4>(a, nt, st);
    case 5: return launch_coop_p<TX, TF, ADALN, 5>(a, nt, st);
    case 6: return launch_coop_p<TX, TF, ADALN, 6>(a, nt, st);
    case 7: return launch_coop_p<TX, TF, ADALN, 7>(a, nt, st);
    case 8: return launch_coop_p<TX, TF, ADALN, 8>(a, nt, st);
    default: return -1;
  }
}

int norm_rope_rows(const void* x0, void* o0, const void* x1, void* o1, int dtype, int64_t rows,
                   int64_t D, int64_t ldx, int64_t ldo, const void* scale, const void* shift,
                   int mod_dtype, int64_t mod_ld, int64_t mod_group, const void* freqs,
                   int freqs_dtype, int64_t freqs_row_stride, int head_dim, float eps,
                   hipStream_t st) {
  XMH3_REQUIRE(rows >= 0 && D > 0, "norm_rope: bad sizes");
  if (rows == 0) return XMH3_OK;
  XMH3_REQUIRE(x0 && o0 && freqs, "norm_rope: null pointer");
  XMH3_REQUIRE((x1 == nullptr) == (o1 == nullptr), "norm_rope: second tensor needs both in and out");
  XMH3_REQUIRE(head_dim == 128, "norm_rope: head_dim must be 128");
  XMH3_REQUIRE(D % head_dim == 0, "norm_rope: row width must be a multiple of head_dim");
  XMH3_REQUIRE(ldx % 8 == 0 && ldo % 8 == 0, "norm_rope: strides must be multiples of 8");
  XMH3_REQUIRE(dtype == mod_dtype || (scale == nullptr && shift == nullptr),
               "norm_rope: scale/shift must have the dtype of x");
  XMH3_REQUIRE(aligned16(x0) && aligned16(o0) && (!x1 || (aligned16(x1) && aligned16(o1))) &&
                   aligned16(freqs),
               "norm_rope: pointers must be 16-byte aligned");
  XMH3_REQUIRE(mod_group >= 1, "norm_rope: modulation group must be >= 1");
  RowArgs a{};
  a.x0 = x0; a.o0 = o0; a.x1 = x1; a.o1 = o1; a.ldx = ldx; a.ldo = ldo; a.rows = rows; a.D = D;
  a.scale = scale; a.shift = shift; a.mod_ld = mod_ld; a.row_map = nullptr; a.mod_group = mod_group;
  a.freqs = freqs; a.freqs_row_stride = freqs_row_stride; a.head_dim = head_dim; a.eps = eps;
  const bool adaln = scale != nullptr;
  XMH3_REQUIRE(adaln == (shift != nullptr), "norm_rope: scale and shift go together");
  const size_t fsize = freqs_dtype == DT_F32 ? 4 : 2;
  XMH3_REQUIRE((freqs_row_stride * (int64_t)fsize) % 16 == 0, "norm_rope: table rows must be 16-byte aligned");
  // one modulation row for every token (or none): the cooperative kernel
  const bool one_mod_row = !adaln || mod_group >= rows;
  const int nt = x1 ? 2 : 1;
#define XMH3_NR(TX, TF)                                                         \
  {                                                                             \
    if (one_mod_row) {                                                          \
      const int rc = adaln ? launch_coop<TX, TF, true>(a, nt, st)               \
                           : launch_coop<TX, TF, false>(a, nt, st);             \
      if (rc >= 0) return rc;                                                   \
    }                                                                           \
    if (adaln) return launch_row<TX, TX, TF, true, true, false, 8>(a, st);      \
    return launch_row<TX, TX, TF, true, false, false, 8>(a, st);                \
  }
  if (dtype == DT_BF16 && freqs_dtype == DT_F32) XMH3_NR(BF16T, F32T)
  if (dtype == DT_BF16 && freqs_dtype == DT_BF16) XMH3_NR(BF16T, BF16T)
  if (dtype == DT_F16 && freqs_dtype == DT_F32) XMH3_NR(F16T, F32T)
  if (dtype == DT_F16 && freqs_dtype == DT_F16) XMH3_NR(F16T, F16T)
#undef XMH3_NR
  return fail(XMH3_EUNSUPPORTED, "norm_rope: dtype combination not supported (x bf16/fp16; table fp32 or x's dtype)");
}

int rms_adaln_rows(const void* x, void* out, int dtype, int64_t rows, int64_t D, int64_t ldx,
                   int64_t ldo, const void* weight, const void* scale, const void* shift,
                   int mod_dtype, int64_t mod_ld, const int32_t* row_map, int64_t mod_group,
                   float eps, hipStream_t st) {
  XMH3_REQUIRE(rows >= 0 && D > 0, "rms_adaln: bad sizes");
  if (rows == 0) return XMH3_OK;
  XMH3_REQUIRE(x && out && scale && shift, "rms_adaln: null pointer");
  XMH3_REQUIRE(D % 8 == 0 && ldx % 8 == 0 && ldo % 8 == 0 && mod_ld % 8 == 0,
               "rms_adaln: width and strides must be multiples of 8");
  XMH3_REQUIRE(aligned16(x) && aligned16(out) && aligned16(scale) && aligned16(shift) &&
                   (!weight || aligned16(weight)),
               "rms_adaln: pointers must be 16-byte aligned");
  XMH3_REQUIRE(mod_group >= 1, row_map ? "rms_adaln: the modulation table needs >= 1 row"
                                        : "rms_adaln: modulation group must be >= 1");
  RowArgs a{};
  a.x0 = x; a.o0 = out; a.ldx = ldx; a.ldo = ldo; a.rows = rows; a.D = D; a.weight = weight;
  a.scale = scale; a.shift = shift; a.mod_ld = mod_ld; a.row_map = row_map; a.mod_group = mod_group;
  a.eps = eps;
  if (dtype == DT_BF16 && mod_dtype == DT_BF16) {
    int rc = weight ? launch_adaln_coop<BF16T, true>(a, st) : launch_adaln_coop<BF16T, false>(a, st);
    if (rc != -1) return rc;
    rc = weight ? launch_adaln_pipe<BF16T, true>(a, st) : launch_adaln_pipe<BF16T, false>(a, st);
    if (rc != -1) return rc;
  }
#define XMH3_RA(TX, TM)                                                          \
  {                                                                              \
    if (weight) return launch_row<TX, TM, F32T, false, true, true, 1>(a, st);    \
    return launch_row<TX, TM, F32T, false, true, false, 1>(a, st);               \
  }
  if (dtype == DT_BF16 && mod_dtype == DT_BF16) XMH3_RA(BF16T, BF16T)
  if (dtype == DT_BF16 && mod_dtype == DT_F32) XMH3_RA(BF16T, F32T)
  if (dtype == DT_F16 && mod_dtype == DT_F16) XMH3_RA(F16T, F16T)
  if (dtype == DT_F16 && mod_dtype == DT_F32) XMH3_RA(F16T, F32T)
  if (dtype == DT_F32 && mod_dtype == DT_F32) XMH3_RA(F32T, F32T)
#undef XMH3_RA
  return fail(XMH3_EUNSUPPORTED, "rms_adaln: dtype combination not supported");
}

// Launch of the cooperative QK norm-rope when it serves the call (full
// rotation of 64-, 96- or 128-wide heads, one table row per token, at most 12
// parts per token); -1 otherwise.
template <typename TX, typename TW, typename TF>
static int launch_qk_coop(HeadArgs& a, hipStream_t st, int nt = 1) {
  const int64_t ntok = a.B * a.S;
  if (a.rot != a.D || a.fh != 0 || ntok * nt >= (int64_t(1) << 30)) return -1;
  auto go = [&](auto kern, int D) -> int {
    const int lph = D / 16, hpw = 64 / lph;
    const int P = (int)((a.H + hpw - 1) / hpw);
    if (P > 12) return -1;
    const int R = std::max(1, 12 / P);
    const size_t wslice = (size_t)hpw * (D + 8) * 2 + (size_t)hpw * 8 * 4;
    const size_t rb = (size_t)(D / 2) * 4 * sizeof(typename TF::storage);
    const size_t lds = (size_t)R * P * wslice + 2 * (size_t)R * rb;
    if (lds > LDS_BYTES) return -1;
    const int64_t grid = std::min<int64_t>((ntok * nt + R - 1) / R, std::max(1, cu_count()));
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(64 * P * R), lds, st, a, P, nt);
    return check_launch("qk_coop_kernel");
  };
  if (a.D == 64) return go(qk_coop_kernel<TX, TW, TF, 64>, 64);
  if (a.D == 96) return go(qk_coop_kernel<TX, TW, TF, 96>, 96);
  if (a.D == 128) return go(qk_coop_kernel<TX, TW, TF, 128>, 128);
  return -1;
}

template <typename TX, typename TW, typename TF, bool NORM, bool SPLIT>
static int launch_head(HeadArgs& a, int lph, hipStream_t st) {
  const int64_t nheads = a.B * a.S * a.H;
  if constexpr (NORM && SPLIT && sizeof(typename TX::storage) == 2) {
    if (const int rc = launch_qk_coop<TX, TW, TF>(a, st); rc != -1) return rc;
  }
  // table rows through LDS: shared by the heads of a token, at most
  // HEAD_TAB_ROWS tokens per block, rows of at most HEAD_TAB_ROW_BYTES
  auto tabl_ok = [&](int L) {
    const int64_t g = 256 / L;
    return SPLIT && a.fh == 0 && (int64_t)(a.rot / 2) * 4 * (int64_t)sizeof(typename TF::storage) <= HEAD_TAB_ROW_BYTES &&
           (g - 1) / a.H + 2 <= HEAD_TAB_ROWS;
  };
#define XMH3_H(L)                                                                               \
  if (lph == L) {                                                                               \
    dim3 grid((unsigned)((nheads + (256 / L) - 1) / (256 / L)));                                \
    hipLaunchKernelGGL((headspan_kernel<TX, TW, TF, NORM, L, false, SPLIT>), grid, dim3(256), 0, st, a); \
    return check_launch("headspan_kernel");                                                     \
  }
#define XMH3_HT(L)                                                                              \
  if (lph == L && tabl_ok(L)) {                                                                 \
    dim3 grid((unsigned)((nheads + (256 / L) - 1) / (256 / L)));                                \
    hipLaunchKernelGGL((headspan_kernel<TX, TW, TF, NORM, L, SPLIT, SPLIT>), grid, dim3(256), 0, st, a); \
    return check_launch("headspan_kernel");                                                     \
  }
  XMH3_HT(4) XMH3_HT(8) XMH3_HT(16)
  XMH3_H(1) XMH3_H(2) XMH3_H(4) XMH3_H(8) XMH3_H(16) XMH3_H(32) XMH3_H(64)
#undef XMH3_HT
#undef XMH3_H
  return fail(XMH3_EUNSUPPORTED, "head-span kernel: head too wide");
}

// Q and K with one table (the reference's launcher takes both): one launch
// of the cooperative QK kernel when both tensors have the same strides and
// it serves the call, else one call per tensor.
int rope_heads(void* x, void* out, int dtype, int64_t B, int64_t S, int64_t H, int64_t D,
               const int64_t* xstrides, const int64_t* ostrides, const void* weight,
               int weight_dtype, const void* freqs, int freqs_dtype, const int64_t* fstrides,
               int rot_dim, float eps, int norm, int split_half, hipStream_t st);
int rope_heads_qk(void* q, void* q_out, void* k, void* k_out, int dtype, int64_t B, int64_t S, int64_t H,
                  int64_t D, const int64_t* qstrides, const int64_t* qostrides, const int64_t* kstrides,
                  const int64_t* kostrides, const void* q_weight, const void* k_weight, int weight_dtype,
                  const void* freqs, int freqs_dtype, const int64_t* fstrides, int rot_dim, float eps,
                  int norm, int split_half, hipStream_t st) {
  bool same = true;
  for (int i = 0; i < 3; ++i) same = same && qstrides[i] == kstrides[i] && qostrides[i] == kostrides[i];
  const int rot = rot_dim ? rot_dim : (int)D;
  const bool b16 = dtype == DT_BF16 || dtype == DT_F16;
  if (same && norm && split_half && b16 && rot == D && fstrides[2] == 0 && B * S * H > 0 && q && k && q_out &&
      k_out && q_weight && k_weight && aligned16(k) && aligned16(k_out) && aligned16(k_weight) &&
      (weight_dtype == dtype || weight_dtype == DT_F32)) {
    // the first tensor's checks, and the arguments, come from rope_heads
    // with a launch-free probe: validate by building the same HeadArgs
    XMH3_REQUIRE(D > 0 && rot % 16 == 0 && D <= 512, "rope: bad head_dim");
    for (int i = 0; i < 3; ++i)
      XMH3_REQUIRE(qstrides[i] % 8 == 0 && qostrides[i] % 8 == 0 && fstrides[i] % 8 == 0,
                   "rope: strides must be multiples of 8 elements");
    XMH3_REQUIRE(aligned16(q) && aligned16(q_out) && aligned16(freqs) && aligned16(q_weight),
                 "rope: pointers must be 16-byte aligned");
    HeadArgs a{};
    a.x = q; a.out = q_out; a.B = B; a.S = S; a.H = H; a.D = D;
    a.sb = qstrides[0]; a.ss = qstrides[1]; a.sh = qstrides[2];
    a.ob = qostrides[0]; a.os = qostrides[1]; a.oh = qostrides[2];
    a.weight = q_weight; a.freqs = freqs; a.fb = fstrides[0]; a.fs = fstrides[1]; a.fh = fstrides[2];
    a.divS = FastDivU64::make((uint64_t)S); a.divH = FastDivU64::make((uint64_t)H);
    a.rot = rot; a.eps = eps;
    a.x1 = k; a.out1 = k_out; a.weight1 = k_weight;
    int rc = -1;
#define XMH3_QK(TX, TF)                                                                      \
    rc = weight_dtype == DT_F32 ? launch_qk_coop<TX, F32T, TF>(a, st, 2) : launch_qk_coop<TX, TX, TF>(a, st, 2);
    if (dtype == DT_BF16 && freqs_dtype == DT_F32) { XMH3_QK(BF16T, F32T) }
    else if (dtype == DT_BF16 && freqs_dtype == DT_BF16) { XMH3_QK(BF16T, BF16T) }
    else if (dtype == DT_F16 && freqs_dtype == DT_F32) { XMH3_QK(F16T, F32T) }
    else if (dtype == DT_F16 && freqs_dtype == DT_F16) { XMH3_QK(F16T, F16T) }
#undef XMH3_QK
    if (rc != -1) return rc;
  }
  const int rc = rope_heads(q, q_out, dtype, B, S, H, D, qstrides, qostrides, q_weight, weight_dtype, freqs,
                            freqs_dtype, fstrides, rot_dim, eps, norm, split_half, st);
  if (rc != XMH3_OK) return rc;
  return rope_heads(k, k_out, dtype, B, S, H, D, kstrides, kostrides, k_weight, weight_dtype, freqs, freqs_dtype,
                    fstrides, rot_dim, eps, norm, split_half, st);
}

int rope_heads(void* x, void* out, int dtype, int64_t B, int64_t S, int64_t H, int64_t D,
               const int64_t* xstrides, const int64_t* ostrides, const void* weight,
               int weight_dtype, const void* freqs, int freqs_dtype, const int64_t* fstrides,
               int rot_dim, float eps, int norm, int split_half, hipStream_t st) {
  XMH3_REQUIRE(B >= 0 && S >= 0 && H >= 0 && D > 0, "rope: bad sizes");
  if (B * S * H == 0) return XMH3_OK;
  const int rot = rot_dim ? rot_dim : (int)D;
  if (split_half)
    XMH3_REQUIRE(rot > 0 && rot <= D && rot % 16 == 0 && (D - rot) % 8 == 0,
                 "rope: rot_dim must be a multiple of 16 and (head_dim - rot_dim) a multiple of 8");
  else
    XMH3_REQUIRE(rot > 0 && rot <= D && rot % 8 == 0 && D % 8 == 0,
                 "rope: interleaved rot_dim and head_dim must be multiples of 8");
  XMH3_REQUIRE(x && out && freqs && (!norm || weight), "rope: null pointer");
  for (int i = 0; i < 3; ++i)
    XMH3_REQUIRE(xstrides[i] % 8 == 0 && ostrides[i] % 8 == 0 && fstrides[i] % 8 == 0,
                 "rope: strides must be multiples of 8 elements");
  XMH3_REQUIRE(aligned16(x) && aligned16(out) && aligned16(freqs) && (!weight || aligned16(weight)),
               "rope: pointers must be 16-byte aligned");
  const int items = (split_half ? rot / 16 : rot / 8) + (int)(D - rot) / 8;
  int lph = 1;
  while (lph < items) lph <<= 1;
  XMH3_REQUIRE(lph <= 64 && D <= 512, "rope: head_dim must be at most 512");
  HeadArgs a{};
  a.x = x; a.out = out; a.B = B; a.S = S; a.H = H; a.D = D;
  a.sb = xstrides[0]; a.ss = xstrides[1]; a.sh = xstrides[2];
  a.ob = ostrides[0]; a.os = ostrides[1]; a.oh = ostrides[2];
  a.weight = weight; a.freqs = freqs; a.fb = fstrides[0]; a.fs = fstrides[1]; a.fh = fstrides[2];
  a.divS = FastDivU64::make((uint64_t)S); a.divH = FastDivU64::make((uint64_t)H);
  a.rot = rot; a.eps = eps;
  XMH3_REQUIRE(!norm || weight_dtype == dtype || weight_dtype == DT_F32,
               "rope: norm weight must have x's dtype or fp32");
#define XMH3_HS(TX, TF, SPLIT)                                                                \
  {                                                                                           \
    if (!norm) return launch_head<TX, TX, TF, false, SPLIT>(a, lph, st);                      \
    if (weight_dtype == DT_F32) return launch_head<TX, F32T, TF, true, SPLIT>(a, lph, st);     \
    return launch_head<TX, TX, TF, true, SPLIT>(a, lph, st);                                  \
  }
#define XMH3_HD(TX, TF)                     \
  {                                         \
    if (split_half) XMH3_HS(TX, TF, true)   \
    XMH3_HS(TX, TF, false)                  \
  }
  if (dtype == DT_BF16 && freqs_dtype == DT_F32) XMH3_HD(BF16T, F32T)
  if (dtype == DT_BF16 && freqs_dtype == DT_BF16) XMH3_HD(BF16T, BF16T)
  if (dtype == DT_F16 && freqs_dtype == DT_F32) XMH3_HD(F16T, F32T)
  if (dtype == DT_F16 && freqs_dtype == DT_F16) XMH3_HD(F16T, F16T)
  if (dtype == DT_F32 && freqs_dtype == DT_F32) XMH3_HD(F32T, F32T)
#undef XMH3_HD
#undef XMH3_HS
  return fail(XMH3_EUNSUPPORTED, "rope: dtype combination not supported");
}

}  // namespace xmh3

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
extern "C" int xmh3_norm_rope(const void* q_in, void* q_out, const void* k_in, void* k_out, int dtype,
                              int64_t tokens, int64_t width, int64_t ld_in, int64_t ld_out,
                              const void* scale, const void* shift, int mod_dtype, int64_t mod_ld,
                              int64_t mod_group, const void* freqs, int freqs_dtype,
                              int64_t freqs_token_stride, int head_dim, float eps,
                              hipStream_t stream) {
  return xmh3::norm_rope_rows(q_in, q_out, k_in, k_out, dtype, tokens, width, ld_in, ld_out, scale,
                              shift, mod_dtype, mod_ld, mod_group, freqs, freqs_dtype,
                              freqs_token_stride, head_dim, eps, stream);
}

extern "C" int xmh3_rms_adaln(const void* x, void* out, int dtype, int64_t rows, int64_t width,
                              int64_t ld_in, int64_t ld_out, const void* norm_weight,
                              const void* scale, const void* shift, int mod_dtype, int64_t mod_ld,
                              const int32_t* row_map, int64_t mod_group, float eps,
                              hipStream_t stream) {
  return xmh3::rms_adaln_rows(x, out, dtype, rows, width, ld_in, ld_out, norm_weight, scale, shift,
                              mod_dtype, mod_ld, row_map, mod_group, eps, stream);
}

// The reference's 46-argument launcher, same name and argument list, so a
// ctypes caller with pinned argtypes binds this library unchanged. It returns
// nothing, as the reference's does: an argument this build does not take
// (a non-contiguous last dimension, a strided weight or table pair layout)
// launches nothing and leaves the message in xmh3_last_error(). Both pair
// layouts (split_half true or false) run; size-1 table dimensions broadcast.
extern "C" void launch_rms_rope_kernel(
    const void* q, const void* k, const void* freqs, const void* q_scale, const void* k_scale, void* q_out,
    void* k_out, int64_t batch, int64_t dim1, int64_t dim2, int64_t head_dim, int64_t rot_dim,
    int64_t freqs_batch, int64_t freqs_dim1, int64_t freqs_dim2, int64_t q_s0, int64_t q_s1, int64_t q_s2,
    int64_t q_s3, int64_t k_s0, int64_t k_s1, int64_t k_s2, int64_t k_s3, int64_t qo_s0, int64_t qo_s1,
    int64_t qo_s2, int64_t qo_s3, int64_t ko_s0, int64_t ko_s1, int64_t ko_s2, int64_t ko_s3, int64_t f_s0,
    int64_t f_s1, int64_t f_s2, int64_t f_s3, int64_t f_s4, int64_t f_s5, int64_t qs_stride, int64_t ks_stride,
    float epsilon, int input_dtype_code, int freqs_dtype_code, int scale_dtype_code, bool has_k,
    bool split_half, hipStream_t stream) {
  using namespace xmh3;
  auto reject = [](const char* msg) { fail(XMH3_EUNSUPPORTED, msg); };
  if (q_s3 != 1 || qo_s3 != 1 || (has_k && (k_s3 != 1 || ko_s3 != 1)))
    return reject("launch_rms_rope_kernel: the head dimension must be contiguous");
  if (f_s5 != 1 || f_s4 != 2 || f_s3 != 4)
    return reject("launch_rms_rope_kernel: table pairs must be contiguous [rot/2, 2, 2]");
  if ((q_scale && qs_stride != 1) || (has_k && k_scale && ks_stride != 1))
    return reject("launch_rms_rope_kernel: the norm weights must be contiguous");
  if ((freqs_batch != 1 && freqs_batch != batch) || (freqs_dim1 != 1 && freqs_dim1 != dim1) ||
      (freqs_dim2 != 1 && freqs_dim2 != dim2))
    return reject("launch_rms_rope_kernel: table dimensions must be 1 or match the input");
  const int64_t fst[3] = {freqs_batch == 1 ? 0 : f_s0, freqs_dim1 == 1 ? 0 : f_s1, freqs_dim2 == 1 ? 0 : f_s2};
  const int norm = q_scale != nullptr;
  if (has_k && norm) {
    const int64_t xs[3] = {q_s0, q_s1, q_s2}, os[3] = {qo_s0, qo_s1, qo_s2};
    const int64_t ks[3] = {k_s0, k_s1, k_s2}, kos[3] = {ko_s0, ko_s1, ko_s2};
    rope_heads_qk(const_cast<void*>(q), q_out, const_cast<void*>(k), k_out, input_dtype_code, batch, dim1, dim2,
                  head_dim, xs, os, ks, kos, q_scale, k_scale ? k_scale : q_scale, scale_dtype_code, freqs,
                  freqs_dtype_code, fst, (int)rot_dim, epsilon, norm, split_half, stream);
    return;
  }
  {
    const int64_t xs[3] = {q_s0, q_s1, q_s2}, os[3] = {qo_s0, qo_s1, qo_s2};
    if (rope_heads(const_cast<void*>(q), q_out, input_dtype_code, batch, dim1, dim2, head_dim, xs, os, q_scale,
                   scale_dtype_code, freqs, freqs_dtype_code, fst, (int)rot_dim, epsilon, norm, split_half,
                   stream) != XMH3_OK)
      return;
  }
  if (has_k) {
    const int64_t xs[3] = {k_s0, k_s1, k_s2}, os[3] = {ko_s0, ko_s1, ko_s2};
    rope_heads(const_cast<void*>(k), k_out, input_dtype_code, batch, dim1, dim2, head_dim, xs, os,
               k_scale ? k_scale : q_scale, scale_dtype_code, freqs, freqs_dtype_code, fst, (int)rot_dim, epsilon,
               k_scale ? 1 : norm, split_half, stream);
  }
}

extern "C" int xmh3_rope_split_half(void* x, void* out, int dtype, int64_t B, int64_t S, int64_t H,
                                    int64_t head_dim, const int64_t* x_strides,
                                    const int64_t* out_strides, const void* norm_weight,
                                    int weight_dtype, const void* freqs, int freqs_dtype,
                                    const int64_t* freqs_strides, int rot_dim, float eps, int norm,
                                    hipStream_t stream) {
  return xmh3::rope_heads(x, out, dtype, B, S, H, head_dim, x_strides, out_strides, norm_weight,
                          weight_dtype, freqs, freqs_dtype, freqs_strides, rot_dim, eps, norm, 1,
                          stream);
}

extern "C" int xmh3_rope_heads_qk(void* q, void* q_out, void* k, void* k_out, int dtype, int64_t B, int64_t S,
                                  int64_t H, int64_t head_dim, const int64_t* q_strides,
                                  const int64_t* q_out_strides, const int64_t* k_strides,
                                  const int64_t* k_out_strides, const void* q_weight, const void* k_weight,
                                  int weight_dtype, const void* freqs, int freqs_dtype,
                                  const int64_t* freqs_strides, int rot_dim, float eps, int norm, int split_half,
                                  hipStream_t stream) {
  return xmh3::rope_heads_qk(q, q_out, k, k_out, dtype, B, S, H, head_dim, q_strides, q_out_strides, k_strides,
                             k_out_strides, q_weight, k_weight, weight_dtype, freqs, freqs_dtype, freqs_strides,
                             rot_dim, eps, norm, split_half, stream);
}

extern "C" int xmh3_rope_heads(void* x, void* out, int dtype, int64_t B, int64_t S, int64_t H, int64_t head_dim,
                               const int64_t* x_strides, const int64_t* out_strides, const void* norm_weight,
                               int weight_dtype, const void* freqs, int freqs_dtype, const int64_t* freqs_strides,
                               int rot_dim, float eps, int norm, int split_half, hipStream_t stream) {
  return xmh3::rope_heads(x, out, dtype, B, S, H, head_dim, x_strides, out_strides, norm_weight,
                          weight_dtype, freqs, freqs_dtype, freqs_strides, rot_dim, eps, norm, split_half,
                          stream);
}
