// Workgroup id -> output tile of the int8 GEMM. Host- and device-compilable
// (the host build is how the mapping is checked to be a bijection).
//
// Workgroups of one launch are dealt round-robin over the XCDs (workgroup
// pid runs on XCD pid % NUM_XCD), and each XCD has its own L2. The map gives
// each XCD a contiguous range of logical tiles (the first total % NUM_XCD
// XCDs one more), then walks the logical order in bands of GROUP_M row tiles,
// column-major inside a band, so concurrently running tiles of one XCD share
// A row panels and B column panels in that XCD's L2.
#pragma once

#if defined(__HIPCC__)
#define XMH3_HD __host__ __device__ __forceinline__
#else
#define XMH3_HD inline
#endif

#ifndef XMH3_GROUP_M
#define XMH3_GROUP_M 4
#endif
#ifndef XMH3_NUM_XCD
#define XMH3_NUM_XCD 8
#endif

namespace xmh3 {

constexpr int GROUP_M = XMH3_GROUP_M;   // M-tiles per swizzle band
constexpr int NUM_XCD = XMH3_NUM_XCD;   // XCDs workgroups are dealt over

XMH3_HD void tile_coords(int pid, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int total = tiles_m * tiles_n;
  const int q = total / NUM_XCD, r = total % NUM_XCD;
  const int x = pid % NUM_XCD, j = pid / NUM_XCD;
  const int logical = (x < r) ? x * (q + 1) + j : r * (q + 1) + (x - r) * q + j;
  const int in_group = GROUP_M * tiles_n;
  const int group = logical / in_group;
  const int first_m = group * GROUP_M;
  const int gsize = (tiles_m - first_m < GROUP_M) ? tiles_m - first_m : GROUP_M;
  const int rem = logical - group * in_group;
  tm = first_m + rem % gsize;
  tn = rem / gsize;
}

}  // namespace xmh3
