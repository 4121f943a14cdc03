// Shared device/host helpers for the sparseforge_amd HIP library (gfx950 / CDNA4).
//
// Everything here is header-only so that each translation unit of the library
// inlines it; the C-ABI entry points live in the sf_*.hip files.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "../../include/sparseforge_amd.h"

namespace sf {

// ---------------------------------------------------------------------------
// Error plumbing: every entry point returns an SF_* status; the message of the
// most recent failure on the calling host thread is kept for sf_last_error().
// ---------------------------------------------------------------------------
void set_error(const char* fmt, ...);

#define SF_CHECK_ARG(cond, ...)              \
  do {                                       \
    if (!(cond)) {                           \
      ::sf::set_error(__VA_ARGS__);          \
      return SF_ERR_INVALID;                 \
    }                                        \
  } while (0)

#define SF_CHECK_HIP(expr)                                                   \
  do {                                                                       \
    hipError_t _e = (expr);                                                  \
    if (_e != hipSuccess) {                                                  \
      ::sf::set_error("%s failed: %s", #expr, hipGetErrorString(_e));        \
      return SF_ERR_HIP;                                                     \
    }                                                                        \
  } while (0)

// Status of the most recent launch on this thread (launch-configuration errors).
inline int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return SF_ERR_HIP;
  }
  return SF_OK;
}

// ---------------------------------------------------------------------------
// bf16 <-> f32, round-to-nearest-even (the rounding torch uses for .to(bf16)).
// ---------------------------------------------------------------------------
__host__ __device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  uint32_t u = static_cast<uint32_t>(h) << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

__host__ __device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x0040u);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

// Round an f32 to the nearest bf16 and return it as f32.
__host__ __device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// Load/store one element of a tensor whose dtype is a runtime SF_DTYPE_* code.
__device__ __forceinline__ float load_as_f32(const void* p, int64_t i, int dtype) {
  return dtype == SF_DTYPE_F32 ? static_cast<const float*>(p)[i]
                               : bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
}
__device__ __forceinline__ void store_from_f32(void* p, int64_t i, int dtype, float v) {
  if (dtype == SF_DTYPE_F32)
    static_cast<float*>(p)[i] = v;
  else
    static_cast<uint16_t*>(p)[i] = f32_to_bf16(v);
}

// ---------------------------------------------------------------------------
// Total order used for top-N selection inside a group.  torch's CPU topk
// compares with NaN greater than every number and NaN == NaN, and -0 == +0.
// ordered_key maps a float to a uint32 with exactly that order.
// ---------------------------------------------------------------------------
__host__ __device__ __forceinline__ uint32_t ordered_key(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0xffffffffu;  // NaN: largest
  if ((u & 0x7fffffffu) == 0u) u = 0u;                      // -0 == +0
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// ---------------------------------------------------------------------------
// Tie table of torch.topk(k) over a group of 4 (CPU kernel of torch 2.10).
// Index: key = sum_i lt_i << 2i with lt_i = #{j : v_j < v_i}; value: bit i set
// when member i is kept.  The tables are data measured from torch.topk over
// all 75 weak orderings of four values; unreachable keys hold 0.
// ---------------------------------------------------------------------------
__constant__ static const uint8_t kTopkTies4[3][256] = {
    {4,0,0,1,0,0,0,0,0,0,2,1,2,0,2,0,0,0,0,0,0,2,0,1,0,0,2,1,0,2,2,0,0,0,1,1,0,0,1,1,2,2,0,0,2,2,0,0,4,0,4,0,0,4,4,0,4,4,0,0,0,0,0,0,
     0,0,0,0,0,2,0,1,0,0,2,1,0,2,2,0,0,4,0,1,4,0,0,0,0,0,0,0,2,0,0,0,0,0,1,1,0,0,0,0,2,0,0,0,2,0,0,0,0,4,4,0,4,0,0,0,4,0,0,0,0,0,0,0,
     0,0,8,1,0,0,1,1,2,2,0,0,2,2,0,0,0,0,8,1,0,0,0,0,2,0,0,0,2,0,0,0,4,4,0,0,4,0,0,0,0,0,0,0,0,0,0,0,4,4,0,0,4,0,0,0,0,0,0,0,0,0,0,0,
     8,0,8,0,0,8,8,0,8,8,0,0,0,0,0,0,0,8,8,0,8,0,0,0,8,0,0,0,0,0,0,0,8,8,0,0,8,0,0,0,0,0,0,0,0,0,0,0,0,0,0,0,0,0,0,0,0,0,0,0,0,0,0,0},
    {12,0,0,5,0,0,0,0,0,0,3,3,10,0,3,0,0,0,0,0,0,6,0,3,0,0,3,3,0,6,3,0,0,0,5,5,0,0,5,5,6,6,0,0,6,6,0,0,12,0,5,0,0,6,5,0,6,6,0,0,0,0,0,0,
     0,0,0,0,0,10,0,3,0,0,3,3,0,10,3,0,0,12,0,5,12,0,0,0,0,0,0,0,10,0,0,0,0,0,5,5,0,0,0,0,6,0,0,0,6,0,0,0,0,12,5,0,12,0,0,0,6,0,0,0,0,0,0,0,
     0,0,9,9,0,0,9,9,10,10,0,0,10,10,0,0,0,0,9,9,0,0,0,0,10,0,0,0,10,0,0,0,12,12,0,0,12,0,0,0,0,0,0,0,0,0,0,0,12,12,0,0,12,0,0,0,0,0,0,0,0,0,0,0,
     12,0,9,0,0,10,9,0,10,10,0,0,0,0,0,0,0,12,9,0,12,0,0,0,10,0,0,0,0,0,0,0,12,12,0,0,12,0,0,0,0,0,0,0,0,0,0,0,0,0,0,0,0,0,0,0,0,0,0,0,0,0,0,0},
    {13,0,0,13,0,0,0,0,0,0,11,11,11,0,11,0,0,0,0,0,0,7,0,7,0,0,7,7,0,7,7,0,0,0,13,13,0,0,7,7,7,7,0,0,7,7,0,0,13,0,13,0,0,7,7,0,7,7,0,0,0,0,0,0,
     0,0,0,0,0,11,0,11,0,0,11,11,0,11,11,0,0,13,0,13,14,0,0,0,0,0,0,0,14,0,0,0,0,0,13,13,0,0,0,0,14,0,0,0,14,0,0,0,0,13,13,0,14,0,0,0,14,0,0,0,0,0,0,0,
     0,0,13,13,0,0,11,11,14,11,0,0,14,11,0,0,0,0,13,13,0,0,0,0,14,0,0,0,14,0,0,0,13,13,0,0,14,0,0,0,0,0,0,0,0,0,0,0,14,13,0,0,14,0,0,0,0,0,0,0,0,0,0,0,
     13,0,13,0,0,11,11,0,14,11,0,0,0,0,0,0,0,13,13,0,14,0,0,0,14,0,0,0,0,0,0,0,13,13,0,0,14,0,0,0,0,0,0,0,0,0,0,0,0,0,0,0,0,0,0,0,0,0,0,0,0,0,0,0}};

// torch.topk(2) of a group of 4 in closed form, equal to the k = 2 table on all
// 75 weak orderings.  bij: member j ranks at or above member i (j > i, so j
// wins a tie), eij: members i and j are equal.  A member is kept unless two
// others outrank it, except when member 0 is the unique maximum: then the
// second kept member is the lowest index among the tied maxima of members
// 1..3, or member 2 when all three tie.  Pure boolean logic on comparison
// results (lane masks), no table gather.
__host__ __device__ __forceinline__ uint32_t topk2_keep_rel(bool b01, bool b02, bool b03, bool b12, bool b13,
                                                            bool b23, bool e12, bool e13, bool e23) {
  auto maj = [](bool x, bool y, bool z) { return (x && y) || (x && z) || (y && z); };
  bool k0 = !maj(b01, b02, b03), k1 = !maj(!b01, b12, b13), k2 = !maj(!b02, !b12, b23), k3 = !maj(!b03, !b13, !b23);
  const bool top0 = !b01 && !b02 && !b03;
  const bool ge1 = (!b12 || e12) && (!b13 || e13), ge2 = b12 && (!b23 || e23), ge3 = b13 && b23;
  const bool all3 = ge1 && ge2 && ge3;
  if (top0) {
    k1 = !all3 && ge1;
    k2 = all3 || (!ge1 && ge2);
    k3 = !all3 && !ge1 && !ge2;
  }
  return (k0 ? 1u : 0u) | (k1 ? 2u : 0u) | (k2 ? 4u : 0u) | (k3 ? 8u : 0u);
}

__host__ __device__ __forceinline__ uint32_t topk2_keep_keys(const uint32_t k[4]) {
  return topk2_keep_rel(k[1] >= k[0], k[2] >= k[0], k[3] >= k[0], k[2] >= k[1], k[3] >= k[1], k[3] >= k[2],
                        k[1] == k[2], k[1] == k[3], k[2] == k[3]);
}

// The same keep set as topk2_keep_rel for NaN-free values (-0 == +0), computed
// as integer arithmetic so that it runs as a few selects and adds per group
// rather than as lane-mask logic.  Member j outranks member i (i < j) when
// v_j >= v_i, otherwise i outranks j; each of the 6 pairs adds one to the
// rank of the member it does not favour, rank_i held in bits [2i, 2i + 2)
// (at most 3, so the fields never carry).  A member is kept when its rank is
// below 2, i.e. bit 2i + 1 is clear.  When member 0 outranks all three others
// the second kept member is the lowest index among the maxima of members
// 1..3, or member 2 when all three are equal.  Result: bit 2i + 1 set when
// member i is kept (the "spread" form, which flip counting uses directly).
__host__ __device__ __forceinline__ uint32_t topk2_spread_f(const float v[4]) {
  const bool c01 = v[1] >= v[0], c02 = v[2] >= v[0], c03 = v[3] >= v[0];
  const bool c12 = v[2] >= v[1], c13 = v[3] >= v[1], c23 = v[3] >= v[2];
  const uint32_t r = (c01 ? 1u : 4u) + (c02 ? 1u : 16u) + (c03 ? 1u : 64u) + (c12 ? 4u : 16u) +
                     (c13 ? 4u : 64u) + (c23 ? 16u : 64u);
  const uint32_t keep = ~r & 0xaau;
  const bool top0 = !(c01 || c02 || c03);
  const bool ge1 = v[1] >= v[2] && v[1] >= v[3], ge2 = c12 && v[2] >= v[3];
  const bool all3 = v[1] == v[2] && v[2] == v[3];
  const uint32_t second = all3 ? 0x20u : (ge1 ? 0x08u : (ge2 ? 0x20u : 0x80u));
  return top0 ? (0x02u | second) : keep;
}

// Spread form (bit 2i + 1) -> plain form (bit i).
__host__ __device__ __forceinline__ uint32_t unspread4(uint32_t s) {
  return ((s >> 1) & 1u) | ((s >> 2) & 2u) | ((s >> 3) & 4u) | ((s >> 4) & 8u);
}

// Without NaN the float comparisons give torch's order directly (-0 == +0).
__host__ __device__ __forceinline__ uint32_t topk2_keep_f(const float v[4]) { return unspread4(topk2_spread_f(v)); }

__device__ __forceinline__ bool any_nan4(const float v[4]) {
  return __builtin_isunordered(v[0], v[1]) || __builtin_isunordered(v[2], v[3]);
}

// Kept members (bitmask over 4) of torch.topk(k) on the group v[0..3].
__device__ __forceinline__ uint32_t topk4_keep(const float v[4], int k) {
  if (k == 2 && !any_nan4(v)) return topk2_keep_f(v);
  uint32_t key[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) key[i] = ordered_key(v[i]);
  if (k == 2) return topk2_keep_keys(key);
  uint32_t idx = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t lt = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) lt += key[j] < key[i] ? 1u : 0u;
    idx |= lt << (2 * i);
  }
  return kTopkTies4[k - 1][idx];
}

// k-th largest value of the group (topk(k).values[..., -1]); NaN is largest.
__device__ __forceinline__ float kth_largest4(const float v[4], int k) {
  // rank_i = #{j : v_j > v_i} + #{j < i : v_j == v_i}; the member with rank k-1 is it.
  uint32_t key[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) key[i] = ordered_key(v[i]);
  float out = v[0];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    int r = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) r += (key[j] > key[i]) || (j < i && key[j] == key[i]);
    if (r == k - 1) out = v[i];
  }
  return out;
}

__host__ __device__ __forceinline__ int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Group geometry: group g of the flattened [rows, ceil(cols/4)] grid.
struct Group {
  int64_t row, col, elem;  // first column / flat element of the group
  int n;                   // valid members (4, or the tail width)
  bool full;               // n == 4 (a complete N:M group)
};

// Grid-stride walk over the groups of a [rows, cols] matrix (gpr groups per
// row).  The row / group-column / element of the current group are advanced
// incrementally, so the loop does no 64-bit division (two per thread, once).
struct GroupWalk {
  int64_t gi, groups, stride;
  int64_t row, gc, elem;   // current group
  int64_t gpr, cols;
  int64_t sdiv, smod;      // stride = sdiv * gpr + smod
  int64_t estep, ewrap;    // element step per stride, correction when gc wraps
  __device__ __forceinline__ GroupWalk(int64_t groups_, int64_t cols_, int64_t gpr_)
      : GroupWalk(groups_, cols_, gpr_, blockIdx.x, gridDim.x) {}
  // The walk of workgroup `block` of a grid of `nblocks` (a multi-layer kernel
  // runs each layer's grid as a range of its own workgroups).
  __device__ __forceinline__ GroupWalk(int64_t groups_, int64_t cols_, int64_t gpr_, int64_t block, int64_t nblocks)
      : groups(groups_), gpr(gpr_), cols(cols_) {
    gi = block * (int64_t)blockDim.x + threadIdx.x;
    stride = nblocks * (int64_t)blockDim.x;
    row = gi / gpr;
    gc = gi - row * gpr;
    elem = row * cols + gc * 4;
    sdiv = stride / gpr;
    smod = stride - sdiv * gpr;
    estep = sdiv * cols + smod * 4;
    ewrap = cols - gpr * 4;
  }
  __device__ __forceinline__ bool live() const { return gi < groups; }
  __device__ __forceinline__ void next() {
    gi += stride;
    row += sdiv;
    gc += smod;
    elem += estep;
    if (gc >= gpr) {
      gc -= gpr;
      ++row;
      elem += ewrap;
    }
  }
  __device__ __forceinline__ Group group() const {
    Group G;
    G.row = row;
    G.col = gc * 4;
    G.elem = elem;
    const int64_t rem = cols - G.col;
    G.n = rem >= 4 ? 4 : static_cast<int>(rem);
    G.full = G.n == 4;
    return G;
  }
};

// Grid size for a grid-stride elementwise kernel: enough workgroups to fill
// all 256 CUs several times over, never more than the work needs.
inline int elementwise_grid(int64_t work_items, int block) {
  int64_t g = ceil_div(work_items, block);
  const int64_t cap = 256 * 16;
  if (g > cap) g = cap;
  if (g < 1) g = 1;
  return static_cast<int>(g);
}

}  // namespace sf
