// Mask construction on gfx950: hard N:M projection (K6), gate target (K7) and
// the fused periodic mask update (K8) of SparseLinear, plus the score
// statistics and the unstructured tau quantile they need.
//
// Work decomposition: one thread owns one 4-wide group along a row (the N:M
// group of the 2:4 path), so top-N selection, penalty targets and flip counts
// are register-local.  Rows with cols % 4 != 0 end in a partial "tail" group,
// which the reference treats elementwise (nm_2_4 keeps tail columns at 1).
// Grid-stride loops keep the launch at a fixed size; every kernel is
// memory-bound and reads each tensor once.
//
// Arithmetic follows the reference's op order: each PyTorch op rounds to the
// dtype of its result, reproduced with rnd(x, dtype); f32 division and sqrt
// are IEEE correctly rounded in HIP (the default), as on the CPU.

#include <initializer_list>
#include <utility>

#include <mutex>
#include <vector>

#include "sf_common.hpp"
#include "sf_rng.hpp"

namespace sf {
namespace {

constexpr int kBlock = 256;

__device__ __forceinline__ float rnd(float x, int dtype) { return dtype == SF_DTYPE_BF16 ? round_bf16(x) : x; }
__host__ __device__ __forceinline__ int promote(int a, int b) {
  return (a == SF_DTYPE_F32 || b == SF_DTYPE_F32) ? SF_DTYPE_F32 : SF_DTYPE_BF16;
}

// sigmoid(x) = 1 / (1 + exp(-x)) from the hardware base-2 exponential and
// reciprocal (v_exp_f32, v_rcp_f32, each within 1 ulp): within a few ulp of the
// f32 formula the reference evaluates (its own exp is not correctly rounded
// either); exactly 0.5 at x = 0, exactly 1 once exp(-x) < 2^-24, 0 at -inf.
__device__ __forceinline__ float sigmoidf_(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * 1.4426950408889634f));
}

typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// Load up to 4 consecutive elements [i, i + n) as f32; vector path when the
// group is full and aligned.  NT: a non-temporal load (the batched arena
// passes stream gigabytes that nothing re-reads before they are evicted).
template <int DT, bool NT = false>
__device__ __forceinline__ void load4(const void* base, int64_t i, int n, bool vec, float out[4]) {
  if (DT == SF_DTYPE_F32) {
    const float* p = static_cast<const float*>(base) + i;
    if (vec) {
      f32x4_t v;
      if constexpr (NT)
        v = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(p));
      else
        v = *reinterpret_cast<const f32x4_t*>(p);
      out[0] = v.x; out[1] = v.y; out[2] = v.z; out[3] = v.w;
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) out[j] = j < n ? p[j] : 0.0f;
    }
  } else {
    const uint16_t* p = static_cast<const uint16_t*>(base) + i;
    if (vec) {
      u32x2_t v;
      if constexpr (NT)
        v = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(p));
      else
        v = *reinterpret_cast<const u32x2_t*>(p);
      out[0] = bf16_to_f32(v.x & 0xffff); out[1] = bf16_to_f32(v.x >> 16);
      out[2] = bf16_to_f32(v.y & 0xffff); out[3] = bf16_to_f32(v.y >> 16);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) out[j] = j < n ? bf16_to_f32(p[j]) : 0.0f;
    }
  }
}

template <int DT, bool NT = false>
__device__ __forceinline__ void store4(void* base, int64_t i, int n, bool vec, const float v[4]) {
  if (DT == SF_DTYPE_F32) {
    float* p = static_cast<float*>(base) + i;
    if (vec) {
      const f32x4_t o{v[0], v[1], v[2], v[3]};
      if constexpr (NT)
        __builtin_nontemporal_store(o, reinterpret_cast<f32x4_t*>(p));
      else
        *reinterpret_cast<f32x4_t*>(p) = o;
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (j < n) p[j] = v[j];
    }
  } else {
    uint16_t* p = static_cast<uint16_t*>(base) + i;
    if (vec) {
      u32x2_t o;
      o.x = static_cast<uint32_t>(f32_to_bf16(v[0])) | (static_cast<uint32_t>(f32_to_bf16(v[1])) << 16);
      o.y = static_cast<uint32_t>(f32_to_bf16(v[2])) | (static_cast<uint32_t>(f32_to_bf16(v[3])) << 16);
      if constexpr (NT)
        __builtin_nontemporal_store(o, reinterpret_cast<u32x2_t*>(p));
      else
        *reinterpret_cast<u32x2_t*>(p) = o;
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (j < n) p[j] = f32_to_bf16(v[j]);
    }
  }
}

// Runtime-dtype variant used for the rarely-used operands (aux, frozen flags).
__device__ __forceinline__ void load4_any(const void* base, int dtype, int64_t i, int n, bool vec, float out[4]) {
  if (dtype == SF_DTYPE_F32)
    load4<SF_DTYPE_F32>(base, i, n, vec, out);
  else
    load4<SF_DTYPE_BF16>(base, i, n, vec, out);
}

// ---------------------------------------------------------------------------
// Score of one element (legacy/sparse_modeling.py:1041-1079).  w, h, a are the
// stored values (already widened to f32); each reference op rounds to its
// result dtype.
// ---------------------------------------------------------------------------
struct ScoreSpec {
  int metric, w_dtype, h_dtype, aux_dtype, score_dtype;
  float eps, movement_temp;
};

// Rounding to a compile-time dtype (the dtypes of W, H and the scores are
// template parameters of the hot kernels, so the f32 cases cost nothing).
template <int DT>
__device__ __forceinline__ float rndc(float x) {
  if constexpr (DT == SF_DTYPE_BF16)
    return round_bf16(x);
  else
    return x;
}

// RN(sqrt(x)).  For x in [2^-96, 2^127) the hardware square root (within
// 1 ulp) is corrected by the signs of its two neighbours' residuals x - y' y
// (exact with an FMA) -- the correctly rounded expansion the compiler emits,
// without its range scaling and special-value handling, which that range
// does not need; other x (zero, subnormal, huge, negative, inf, NaN) take
// sqrtf under a branch that is almost never taken.
__device__ __forceinline__ float sqrt_rn(float x) {
  const float y = __builtin_amdgcn_sqrtf(x);
  const float dn = __int_as_float(__float_as_int(y) - 1), up = __int_as_float(__float_as_int(y) + 1);
  float r = fmaf(-dn, y, x) <= 0.0f ? dn : y;
  r = fmaf(-up, y, x) > 0.0f ? up : r;
  float alt = 0.0f;
  const bool odd = !(x >= 0x1p-96f && x < 0x1p127f);
  if (__builtin_expect(odd, 0)) alt = sqrtf(x);
  return odd ? alt : r;
}

// sqrt_rn of the four values of a group with one range test and one branch: x is in [2^-96, 2^127)
// exactly when its bit pattern minus that of 2^-96 is below the width of the range (as unsigned: negative
// values, zeros, subnormals, inf and NaN all fall outside).  Both paths round correctly, so a group with
// one value outside the range may recompute all four with sqrtf and give the same results.
__device__ __forceinline__ void sqrt_rn4(const float x[4], float r[4]) {
  constexpr uint32_t lo = 0x0F800000u, width = 0x7F000000u - 0x0F800000u;  // 2^-96, 2^127
  uint32_t u = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t d = __float_as_uint(x[j]) - lo;
    u = d > u ? d : u;
    const float y = __builtin_amdgcn_sqrtf(x[j]);
    const float dn = __int_as_float(__float_as_int(y) - 1), up = __int_as_float(__float_as_int(y) + 1);
    float t = fmaf(-dn, y, x[j]) <= 0.0f ? dn : y;
    r[j] = fmaf(-up, y, x[j]) > 0.0f ? up : t;
  }
  if (__builtin_expect(u >= width, 0)) {
#pragma unroll
    for (int j = 0; j < 4; ++j) r[j] = sqrtf(x[j]);
  }
}

template <int WD, int HD>
__device__ __forceinline__ float score_of(const ScoreSpec& s, float w, float h, float a) {
  constexpr int PWH = (WD == SF_DTYPE_F32 || HD == SF_DTYPE_F32) ? SF_DTYPE_F32 : SF_DTYPE_BF16;
  switch (s.metric) {
    case SF_METRIC_HESSIAN_OBD: {  // (H + eps) * (W * W)
      float hp = rndc<HD>(h + s.eps);
      float ww = rndc<WD>(w * w);
      return rndc<PWH>(hp * ww);
    }
    case SF_METRIC_HESSIAN_RATIO: {  // |W| / sqrt(H + eps)
      float hp = rndc<HD>(h + s.eps);
      float sq = rndc<HD>(sqrt_rn(hp));
      return rndc<PWH>(fabsf(w) / sq);
    }
    case SF_METRIC_HESSIAN:
      return h;
    case SF_METRIC_WEIGHT_SQUARED:  // W * W (hessian_obd without a Hessian)
      return rndc<WD>(w * w);
    case SF_METRIC_WANDA: {  // |W| * sqrt(scaler + eps)
      float sp = rnd(a + s.eps, s.aux_dtype);
      float sq = rnd(sqrtf(sp), s.aux_dtype);
      return rnd(fabsf(w) * sq, promote(s.aux_dtype, WD));
    }
    case SF_METRIC_MOVEMENT: {  // |W * g| / max(temperature, eps)
      int pd = promote(WD, s.aux_dtype);
      float t = fabsf(rnd(w * a, pd));
      return rnd(t / s.movement_temp, pd);
    }
    default:  // magnitude
      return fabsf(w);
  }
}
// Run-time dtype variant (the sampled gather of the tau selection).
__device__ __forceinline__ float score_of_rt(const ScoreSpec& s, float w, float h, float a) {
  if (s.w_dtype == SF_DTYPE_F32)
    return s.h_dtype == SF_DTYPE_F32 ? score_of<SF_DTYPE_F32, SF_DTYPE_F32>(s, w, h, a)
                                     : score_of<SF_DTYPE_F32, SF_DTYPE_BF16>(s, w, h, a);
  return s.h_dtype == SF_DTYPE_F32 ? score_of<SF_DTYPE_BF16, SF_DTYPE_F32>(s, w, h, a)
                                   : score_of<SF_DTYPE_BF16, SF_DTYPE_BF16>(s, w, h, a);
}

// The score operands of one group (W, H, aux widened to f32).
struct GroupOps {
  float w[4], h[4], a[4];
};

template <int WD, int HD, bool NT = false>
__device__ __forceinline__ void load_group_ops(const ScoreSpec& s, const void* W, const void* H, const void* aux,
                                               const Group& g, bool vec, GroupOps& o) {
#pragma unroll
  for (int j = 0; j < 4; ++j) o.h[j] = o.a[j] = 0.0f;
  load4<WD, NT>(W, g.elem, g.n, vec, o.w);
  if (H) load4<HD, NT>(H, g.elem, g.n, vec, o.h);
  if (aux) {
    if (s.metric == SF_METRIC_WANDA)
      load4_any(aux, s.aux_dtype, g.col, g.n, vec, o.a);  // scaler_row [cols]
    else
      load4_any(aux, s.aux_dtype, g.elem, g.n, vec, o.a);  // grad_ema [rows, cols]
  }
}

// The 4 scores of a group from its operands.
template <int WD, int HD>
__device__ __forceinline__ void scores_of_ops(const ScoreSpec& s, const GroupOps& o, const Group& g, float sc[4]) {
  const float *w = o.w, *h = o.h, *a = o.a;
  if (s.metric == SF_METRIC_HESSIAN_RATIO && g.n == 4) {  // |W| / sqrt(H + eps), the sqrt range test per group
    constexpr int PWH = (WD == SF_DTYPE_F32 || HD == SF_DTYPE_F32) ? SF_DTYPE_F32 : SF_DTYPE_BF16;
    float hp[4], sq[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) hp[j] = rndc<HD>(h[j] + s.eps);
    sqrt_rn4(hp, sq);
#pragma unroll
    for (int j = 0; j < 4; ++j) sc[j] = rndc<PWH>(fabsf(w[j]) / rndc<HD>(sq[j]));
    return;
  }
  // one switch per group, the element loop inside each case
  switch (s.metric) {
#define SF_SCORES_CASE(M)                                                                            \
  case M: {                                                                                          \
    ScoreSpec sm = s;                                                                                \
    sm.metric = M;                                                                                   \
    _Pragma("unroll") for (int j = 0; j < 4; ++j) sc[j] = j < g.n ? score_of<WD, HD>(sm, w[j], h[j], a[j]) : 0.0f; \
    break;                                                                                           \
  }
    SF_SCORES_CASE(SF_METRIC_HESSIAN_RATIO)
    SF_SCORES_CASE(SF_METRIC_HESSIAN_OBD)
    SF_SCORES_CASE(SF_METRIC_HESSIAN)
    SF_SCORES_CASE(SF_METRIC_WANDA)
    SF_SCORES_CASE(SF_METRIC_MOVEMENT)
    SF_SCORES_CASE(SF_METRIC_WEIGHT_SQUARED)
#undef SF_SCORES_CASE
    default:
#pragma unroll
      for (int j = 0; j < 4; ++j) sc[j] = j < g.n ? fabsf(w[j]) : 0.0f;
  }
}

// Gather the operands of a group and compute the 4 scores.
template <int WD, int HD>
__device__ __forceinline__ void group_scores(const ScoreSpec& s, const void* W, const void* H, const void* aux,
                                             const Group& g, bool vec, int64_t cols, float sc[4]) {
  GroupOps o;
  load_group_ops<WD, HD>(s, W, H, aux, g, vec, o);
  scores_of_ops<WD, HD>(s, o, g, sc);
}

__device__ __forceinline__ float score_at(const ScoreSpec& s, const void* W, const void* H, const void* aux,
                                          int64_t e, int64_t cols) {
  float w = load_as_f32(W, e, s.w_dtype);
  float h = H ? load_as_f32(H, e, s.h_dtype) : 0.0f;
  float a = 0.0f;
  if (aux) a = load_as_f32(aux, s.metric == SF_METRIC_WANDA ? e % cols : e, s.aux_dtype);
  return score_of_rt(s, w, h, a);
}

ScoreSpec make_spec(const sf_mask_params* p, int w_dtype, int h_dtype, int aux_dtype) {
  ScoreSpec s;
  s.metric = p->metric;
  s.w_dtype = w_dtype;
  s.h_dtype = h_dtype;
  s.aux_dtype = aux_dtype;
  s.score_dtype = p->score_dtype;
  s.eps = p->eps_metric;
  s.movement_temp = p->movement_temp;
  return s;
}

// z-normalised score in the score dtype: ((s - mu) / sigma).to(score dtype)  (:1085-1088)
__device__ __forceinline__ float znorm(float s, float mu, float sigma, int score_dtype) {
  return rnd((s - mu) / sigma, score_dtype);
}
// a / b correctly rounded, given y = RN(1 / b): q = RN(a y), r = a - b q (exact
// with an FMA), RN(q + r y) is RN(a / b) when nothing under- or overflows
// (P. Markstein, IA-64 and Elementary Functions, 2000, thm. 8.10).  The rare
// operands where that can fail take the IEEE division instead.
__device__ __forceinline__ float div_by(float a, float b, float y) {
  const float q = a * y;
  const float r = fmaf(-b, q, a);
  float d = fmaf(r, y, q);
  // outside these ranges r = a - b q may be inexact (subnormal) or q may overflow;
  // zeros also go here so that the sign of a zero quotient is IEEE's.
  const bool slow = !(fabsf(a) > 0x1p-75f && fabsf(q) < 0x1p+100f && fabsf(y) > 0x1p-100f);
  float alt = 0.0f;
  if (__builtin_expect(slow, 0)) alt = a / b;
  return slow ? alt : d;
}
// d[j] = a[j] / b for a group (d must not alias a), with one fallback branch for the four quotients.
__device__ __forceinline__ void div4_by(const float a[4], float b, float y, float d[4]) {
  bool slow = !(fabsf(y) > 0x1p-100f);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float q = a[j] * y;
    const float r = fmaf(-b, q, a[j]);
    d[j] = fmaf(r, y, q);
    slow = slow || !(fabsf(a[j]) > 0x1p-75f && fabsf(q) < 0x1p+100f);
  }
  // The fallback goes to its own array and is selected afterwards: overwriting d[]
  // inside the branch was compiled into wrong results for some callers here.
  float alt[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (__builtin_expect(slow, 0)) {
#pragma unroll
    for (int j = 0; j < 4; ++j) alt[j] = a[j] / b;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) d[j] = slow ? alt[j] : d[j];
}

// ---------------------------------------------------------------------------
// K6: hard projection.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void hard_of_group(const float v[4], const Group& g, int kind, int n_keep, float out[4]) {
  if (kind == SF_HARD_NONE) {
#pragma unroll
    for (int j = 0; j < 4; ++j) out[j] = 1.0f;
  } else if (kind == SF_HARD_THRESHOLD) {
#pragma unroll
    for (int j = 0; j < 4; ++j) out[j] = v[j] > 0.5f ? 1.0f : 0.0f;
  } else {  // N:M over groups of 4; a tail group keeps every column
    uint32_t keep = g.full ? topk4_keep(v, n_keep) : 0xfu;
#pragma unroll
    for (int j = 0; j < 4; ++j) out[j] = ((keep >> j) & 1u) ? 1.0f : 0.0f;
  }
}

template <int SD, int OD>
__global__ void __launch_bounds__(kBlock) hard_mask_kernel(const void* __restrict__ soft, void* __restrict__ hard,
                                                           int64_t cols, int64_t groups, int64_t gpr, bool vec,
                                                           int kind, int n_keep) {
  for (GroupWalk w(groups, cols, gpr); w.live(); w.next()) {
    Group g = w.group();
    float v[4], o[4];
    load4<SD>(soft, g.elem, g.n, vec && g.full, v);
    hard_of_group(v, g, kind, n_keep, o);
    store4<OD>(hard, g.elem, g.n, vec && g.full, o);
  }
}

// Sum of an int64 across the workgroup, then one atomic per workgroup.
__device__ __forceinline__ void block_add_i64(int64_t v, int64_t* dst) {
  __shared__ int64_t red[kBlock / 64];
  for (int off = 32; off > 0; off >>= 1) v += __shfl_down(v, off, 64);
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  if (lane == 0) red[wv] = v;
  __syncthreads();
  if (threadIdx.x == 0) {
    int64_t t = 0;
    for (int i = 0; i < (int)(blockDim.x / 64); ++i) t += red[i];
    if (t) atomicAdd(reinterpret_cast<unsigned long long*>(dst), static_cast<unsigned long long>(t));
  }
}

template <int DT>
__global__ void __launch_bounds__(kBlock) flip_count_kernel(const void* __restrict__ prev, const void* __restrict__ now,
                                                            int64_t cols, int64_t groups, int64_t gpr, bool vec,
                                                            int kind, int n_keep, int64_t* flips) {
  int64_t cnt = 0;
  for (GroupWalk w(groups, cols, gpr); w.live(); w.next()) {
    Group g = w.group();
    float a[4], b[4], ha[4], hb[4];
    load4<DT>(prev, g.elem, g.n, vec && g.full, a);
    load4<DT>(now, g.elem, g.n, vec && g.full, b);
    hard_of_group(a, g, kind, n_keep, ha);
    hard_of_group(b, g, kind, n_keep, hb);
#pragma unroll
    for (int j = 0; j < 4; ++j) cnt += (j < g.n && ((ha[j] > 0.5f) != (hb[j] > 0.5f))) ? 1 : 0;
  }
  block_add_i64(cnt, flips);
}

// ---------------------------------------------------------------------------
// Score statistics: per-workgroup f64 partial sums, then one workgroup folds
// them in a fixed order (deterministic for a fixed grid).
// ---------------------------------------------------------------------------
constexpr int kStatsGrid = 4096;

__device__ __forceinline__ void block_sum2_f64(double a, double b, double* out_a, double* out_b) {
  __shared__ double ra[kBlock / 64], rb[kBlock / 64];
  for (int off = 32; off > 0; off >>= 1) {
    a += __shfl_down(a, off, 64);
    b += __shfl_down(b, off, 64);
  }
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  if (lane == 0) {
    ra[wv] = a;
    rb[wv] = b;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    double ta = 0, tb = 0;
    for (int i = 0; i < (int)(blockDim.x / 64); ++i) {
      ta += ra[i];
      tb += rb[i];
    }
    *out_a = ta;
    *out_b = tb;
  }
}

// Partial sums of workgroup `blk` of the kStatsGrid-workgroup grid over one
// layer.  VEC: every group full and vector-loadable (as in update_mask_kernel).
// RATIO: the metric is hessian_ratio (|W| / sqrt(H + eps), no aux operand), fixed at compile time.
// NT: W and H through non-temporal loads (the batched arena pass).
template <int WD, int HD, bool VEC, bool RATIO = false, bool NT = false>
__device__ __forceinline__ void stats_partial_block(const ScoreSpec& s_in, const void* __restrict__ W,
                                                    const void* __restrict__ H, const void* __restrict__ aux_in,
                                                    int64_t cols, int64_t groups, int64_t gpr, bool vec,
                                                    double* partial, int blk) {
  ScoreSpec s = s_in;
  const void* aux = aux_in;
  if constexpr (RATIO) {
    s.metric = SF_METRIC_HESSIAN_RATIO;
    aux = nullptr;
  }
  double sum = 0.0, sq = 0.0;
  auto add = [&](const Group& g, const GroupOps& o) {
    float sc[4];
    scores_of_ops<WD, HD>(s, o, g, sc);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (j < g.n) {
        double d = sc[j];
        sum += d;
        sq += d * d;
      }
  };
  GroupWalk w(groups, cols, gpr, blk, kStatsGrid);
  if constexpr (VEC) {
    // two groups per round, both loaded before either is used (the sums keep the walk's order)
    while (w.live()) {
      Group g0 = w.group();
      g0.n = 4;
      g0.full = true;
      w.next();
      const bool two = w.live();
      Group g1 = g0;
      if (two) {
        g1 = w.group();
        g1.n = 4;
        g1.full = true;
        w.next();
      }
      GroupOps o0, o1;
      load_group_ops<WD, HD, NT>(s, W, H, aux, g0, true, o0);
      if (two) load_group_ops<WD, HD, NT>(s, W, H, aux, g1, true, o1);
      add(g0, o0);
      if (two) add(g1, o1);
    }
  } else {
    for (; w.live(); w.next()) {
      const Group g = w.group();
      GroupOps o;
      load_group_ops<WD, HD>(s, W, H, aux, g, vec && g.full, o);
      add(g, o);
    }
  }
  block_sum2_f64(sum, sq, &partial[2 * blk], &partial[2 * blk + 1]);
}

template <int WD, int HD, bool VEC, bool RATIO>
__global__ void __launch_bounds__(kBlock) stats_partial_kernel(ScoreSpec s, const void* __restrict__ W,
                                                               const void* __restrict__ H, const void* __restrict__ aux,
                                                               int64_t cols, int64_t groups, int64_t gpr, bool vec,
                                                               double* partial) {
  stats_partial_block<WD, HD, VEC, RATIO>(s, W, H, aux, cols, groups, gpr, vec, partial, blockIdx.x);
}

// Fold of one layer's kStatsGrid partials by one workgroup, in a fixed order.
__device__ __forceinline__ void stats_final_block(const double* __restrict__ partial, int nparts, int64_t n,
                                                  float* stats) {
  // 8 partials per thread and round, their loads issued together: the partials
  // were just written by workgroups on every XCD, so each round costs a memory
  // latency, and a one-at-a-time loop paid it 16 times
  constexpr int kU = 8;
  double s8[kU], q8[kU];
#pragma unroll
  for (int u = 0; u < kU; ++u) s8[u] = q8[u] = 0.0;
  const int stride = blockDim.x;
  int i = threadIdx.x;
  for (; i + (kU - 1) * stride < nparts; i += kU * stride) {
    double a[kU], b[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      a[u] = partial[2 * (i + u * stride)];
      b[u] = partial[2 * (i + u * stride) + 1];
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      s8[u] += a[u];
      q8[u] += b[u];
    }
  }
  for (; i < nparts; i += stride) {
    s8[0] += partial[2 * i];
    q8[0] += partial[2 * i + 1];
  }
  double sum = 0.0, sq = 0.0;
#pragma unroll
  for (int u = 0; u < kU; ++u) {
    sum += s8[u];
    sq += q8[u];
  }
  __shared__ double tot[2];
  block_sum2_f64(sum, sq, &tot[0], &tot[1]);
  __syncthreads();
  if (threadIdx.x == 0) {
    double mean = tot[0] / (double)n;
    double var = tot[1] / (double)n - mean * mean;
    if (var < 0.0) var = 0.0;
    stats[0] = static_cast<float>(mean);
    stats[1] = static_cast<float>(sqrt(var)) + 1e-6f;  // std(unbiased=False) + 1e-6 in f32
  }
}

__global__ void __launch_bounds__(kBlock) stats_final_kernel(const double* __restrict__ partial, int nparts,
                                                             int64_t n, float* stats) {
  stats_final_block(partial, nparts, n, stats);
}

// ---------------------------------------------------------------------------
// tau quantile: the scores at the sample indices as order-preserving uint32
// keys (a wide gather kernel: the reads are random), then a 4 x 8-bit radix
// select of the two order statistics around rank q * (n - 1) over a few
// workgroups per pass, and torch.lerp between their z-scores.  The select
// runs on the raw scores: z = RN((s - mu) / sigma) in the score dtype is
// non-decreasing in s (sigma > 0; every op rounds monotonically), so the k-th
// smallest z is the z of the k-th smallest score, and the gather needs no
// statistics (a multi-layer update runs it beside the statistics pass).  NaN
// scores make z NaN as well, and NaN statistics make every z NaN: both give a
// NaN tau, as torch.quantile does.  Each pass histograms the current digit of
// the keys that match each statistic's prefix into per-wave LDS histograms
// (scores crowd into a few exponent bins, so per-wave copies keep atomic
// contention low); pass 0 also flags NaN (torch.quantile then takes the last
// rank).
// ---------------------------------------------------------------------------
__device__ __forceinline__ void tau_gather_block(const ScoreSpec& s, const void* __restrict__ W,
                                                 const void* __restrict__ H, const void* __restrict__ aux,
                                                 int64_t rows, int64_t cols, const int64_t* __restrict__ idx,
                                                 int64_t m, uint32_t* __restrict__ keys, int64_t blk, int64_t nblk) {
  const int64_t n = cols * rows;
  for (int64_t i = blk * (int64_t)blockDim.x + threadIdx.x; i < m; i += nblk * blockDim.x) {
    int64_t e = idx ? idx[i] : i;
    e = e < 0 ? 0 : (e >= n ? n - 1 : e);  // indices outside the layer are clamped, never dereferenced
    keys[i] = ordered_key(score_at(s, W, H, aux, e, cols));
  }
}

__global__ void __launch_bounds__(kBlock) tau_gather_kernel(ScoreSpec s, const void* __restrict__ W,
                                                            const void* __restrict__ H, const void* __restrict__ aux,
                                                            int64_t rows, int64_t cols,
                                                            const int64_t* __restrict__ idx, int64_t m,
                                                            uint32_t* __restrict__ keys) {
  tau_gather_block(s, W, H, aux, rows, cols, idx, m, keys, blockIdx.x, gridDim.x);
}

__device__ __forceinline__ float key_to_float(uint32_t k) {
  uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  if (k == 0xffffffffu) u = 0x7fc00000u;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

constexpr int kSelGrid = 32;             // workgroups of a radix pass
constexpr int kSelStride = 2 * 256 + 1;  // partial histogram words per workgroup (+ NaN flag)

// Select state after fixing the digits of passes 0..p.
struct SelState {
  uint32_t prefix[2];  // digits fixed so far of the lo / hi order statistic
  int64_t krem[2];     // rank still to skip inside the current prefix
  float wgt;           // lerp weight
  int any_nan;
};

// Fix the digit of pass `pass` in `st` from that pass's partial histograms
// (run by a whole workgroup; `st` is in LDS).  Pass 0 also derives the
// ranks: rank = q * (n - 1) in f32 as torch.quantile does, the last rank
// when any key is NaN.
__device__ void advance_state(SelState& st, const uint32_t* __restrict__ partial, int nparts, int pass, int64_t m,
                              float q) {
  __shared__ uint32_t tot[2][256];
  __shared__ int nan_any;
  const int t = threadIdx.x;
  if (t == 0) nan_any = 0;
  __syncthreads();
  for (int i = t; i < 2 * 256; i += blockDim.x) {
    uint32_t c = 0;
#pragma unroll 8
    for (int p = 0; p < nparts; ++p) c += partial[(int64_t)p * kSelStride + i];
    (&tot[0][0])[i] = c;
  }
  if (pass == 0 && t < nparts && partial[(int64_t)t * kSelStride + 2 * 256]) atomicOr(&nan_any, 1);
  __syncthreads();
  if (t == 0 && pass == 0) {
    const int64_t last = m - 1;
    float rank = q * static_cast<float>(last);
    if (nan_any) rank = static_cast<float>(last);
    const int64_t lo = static_cast<int64_t>(rank);
    st.krem[0] = lo;
    st.krem[1] = static_cast<int64_t>(ceilf(rank));
    st.wgt = rank - static_cast<float>(lo);
    st.any_nan = nan_any;
    st.prefix[0] = st.prefix[1] = 0u;
  }
  __syncthreads();
  // inclusive prefix sums of both histograms (Hillis-Steele over 256 bins;
  // pass 0 histograms every key once, in tot[0], for both statistics)
  __shared__ uint32_t inc[2][256];
  const int b = t;  // blockDim.x == 256: one bin per thread, both statistics
  const uint32_t h0 = tot[0][b], h1 = pass == 0 ? tot[0][b] : tot[1][b];
  uint32_t v0 = h0, v1 = h1;
  for (int off = 1; off < 256; off <<= 1) {
    inc[0][b] = v0;
    inc[1][b] = v1;
    __syncthreads();
    if (b >= off) {
      v0 += inc[0][b - off];
      v1 += inc[1][b - off];
    }
    __syncthreads();
  }
  // the digit of statistic k is the one bin whose [exclusive, inclusive)
  // prefix range holds its remaining rank (the last bin if the rank is past
  // the total, which a consistent histogram never produces)
  const int shift = 24 - 8 * pass;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const uint32_t incl = k == 0 ? v0 : v1;
    const uint32_t excl = incl - (k == 0 ? h0 : h1);
    const int64_t r = st.krem[k];
    if ((r >= (int64_t)excl && r < (int64_t)incl) || (b == 255 && r >= (int64_t)incl)) {
      inc[k][0] = static_cast<uint32_t>(b);
      inc[k][1] = static_cast<uint32_t>(r - (int64_t)excl);
    }
  }
  __syncthreads();
  if (t < 2) {
    st.prefix[t] |= inc[t][0] << shift;
    st.krem[t] = inc[t][1];
  }
  __syncthreads();
}

// Radix pass `pass` over kSelGrid workgroups.  Every workgroup first brings
// the state up to date with the previous pass (redundantly, so no workgroup
// waits for another), then histograms the current digit of the keys that
// match each statistic's prefix into per-wave LDS histograms and publishes
// the sum.  Workgroup 0 publishes the state the next pass starts from.
// Workgroup `blk` of the pass over a grid of `nblk` workgroups.
__device__ __forceinline__ void tau_pass_block(const uint32_t* __restrict__ keys, int64_t m, int pass, float q,
                                               const SelState* __restrict__ state_in, SelState* __restrict__ state_out,
                                               const uint32_t* __restrict__ partial_in,
                                               uint32_t* __restrict__ partial_out, int blk, int nblk) {
  constexpr int kWaves = kBlock / 64;
  __shared__ uint32_t hist[kWaves][2][256];
  __shared__ SelState st;
  __shared__ int nan;
  const int t = threadIdx.x;
  if (pass >= 2 && t == 0) st = *state_in;
  if (t == 0) nan = 0;
  __syncthreads();
  if (pass >= 1) advance_state(st, partial_in, nblk, pass - 1, m, q);
  if (pass >= 1 && blk == 0 && t == 0) *state_out = st;
  for (int i = t; i < kWaves * 2 * 256; i += kBlock) (&hist[0][0][0])[i] = 0u;
  __syncthreads();
  const int wv = t >> 6;
  const int shift = 24 - 8 * pass;
  const uint32_t pmask = pass == 0 ? 0u : ~0u << (shift + 8);
  const uint32_t p0 = pass == 0 ? 0u : st.prefix[0], p1 = pass == 0 ? 0u : st.prefix[1];
  int local_nan = 0;
  auto count = [&](uint32_t k) {
    const uint32_t d = (k >> shift) & 0xffu;
    local_nan |= k == 0xffffffffu;
    if ((k & pmask) == p0) atomicAdd(&hist[wv][0][d], 1u);
    if (pass > 0 && (k & pmask) == p1) atomicAdd(&hist[wv][1][d], 1u);
  };
  // 8 keys per thread and round, loaded before any is counted (one memory
  // latency per round rather than per key)
  constexpr int kU = 8;
  const int64_t stride = (int64_t)nblk * blockDim.x;
  int64_t i = blk * (int64_t)blockDim.x + t;
  for (; i + (kU - 1) * stride < m; i += kU * stride) {
    uint32_t k8[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) k8[u] = keys[i + u * stride];
#pragma unroll
    for (int u = 0; u < kU; ++u) count(k8[u]);
  }
  for (; i < m; i += stride) count(keys[i]);
  if (local_nan) atomicOr(&nan, 1);
  __syncthreads();
  uint32_t* out = partial_out + (int64_t)blk * kSelStride;
  for (int i = t; i < 2 * 256; i += kBlock) {
    uint32_t c = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) c += (&hist[w][0][0])[i];
    out[i] = c;
  }
  if (t == 0) out[2 * 256] = nan;
}

__global__ void __launch_bounds__(kBlock) tau_pass_kernel(const uint32_t* __restrict__ keys, int64_t m, int pass, float q,
                                                          const SelState* __restrict__ state_in,
                                                          SelState* __restrict__ state_out,
                                                          const uint32_t* __restrict__ partial_in,
                                                          uint32_t* __restrict__ partial_out) {
  tau_pass_block(keys, m, pass, q, state_in, state_out, partial_in, partial_out, blockIdx.x, gridDim.x);
}

// After pass 3: fix its digit, z-normalise the two order statistics and lerp
// them (torch.lerp: small weight -> a + w (b - a), else b - (b - a)(1 - w),
// each op rounded).
__device__ __forceinline__ void tau_final_block(int64_t m, float q, int nparts, const SelState* __restrict__ state_in,
                                                const uint32_t* __restrict__ partial_in,
                                                const float* __restrict__ stats, int score_dtype,
                                                float* __restrict__ tau) {
  __shared__ SelState st;
  if (threadIdx.x == 0) st = *state_in;
  __syncthreads();
  advance_state(st, partial_in, nparts, 3, m, q);
  if (threadIdx.x == 0) {
    const float mu = stats[0], sigma = stats[1];
    const float lo = znorm(key_to_float(st.prefix[0]), mu, sigma, score_dtype);
    const float hi = znorm(key_to_float(st.prefix[1]), mu, sigma, score_dtype);
    const float w = st.wgt;
    const float dlt = __fsub_rn(hi, lo);
    *tau = fabsf(w) < 0.5f ? __fadd_rn(lo, __fmul_rn(w, dlt)) : __fsub_rn(hi, __fmul_rn(dlt, __fsub_rn(1.0f, w)));
  }
}

__global__ void __launch_bounds__(kBlock) tau_final_kernel(int64_t m, float q, int nparts,
                                                           const SelState* __restrict__ state_in,
                                                           const uint32_t* __restrict__ partial_in,
                                                           const float* __restrict__ stats, int score_dtype,
                                                           float* __restrict__ tau) {
  tau_final_block(m, q, nparts, state_in, partial_in, stats, score_dtype, tau);
}

__global__ void __launch_bounds__(kBlock) sample_indices_kernel(int64_t* idx, int64_t m, uint64_t n, uint64_t seed) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < m; i += (int64_t)gridDim.x * blockDim.x)
    idx[i] = static_cast<int64_t>(uniform_below(counter_hash(seed, static_cast<uint64_t>(i)), n));
}

// ---------------------------------------------------------------------------
// Sorted tau samples: m indices distributed as m independent uniform draws
// from [0, n) (torch.randint's law), delivered in non-decreasing order.  With
// E_0..E_m independent Exp(1) and S_k = E_0 + ... + E_k, the vector
// (S_0 / S_m, ..., S_(m-1) / S_m) has the law of the order statistics of m
// independent U(0, 1) (L. Devroye, "Non-Uniform Random Variate Generation",
// 1986, ch. V.2), and floor(U n) maps U(0, 1) to the uniform integers of
// [0, n).  E_j = -log(U_j), U_j = (r_j + 1) 2^-53 from the top 53 bits of
// counter_hash(seed, j); each E_j is held as the integer round(E_j 2^32), so
// every partial sum is exact whatever the summation order (the chunks and the
// workgroup scan below) and S_k is non-decreasing in k; the index is
// floor(double(S_k) / double(S_m) n), a composition of non-decreasing
// roundings, so the list is sorted by construction.
// Pass 1 writes round(E_j 2^32) over the index list (j < m) and each chunk's
// sum to the workspace; pass 2 turns the list into indices in place.
// ---------------------------------------------------------------------------
constexpr int kSortedPer = 16;                        // positions per thread
constexpr int kSortedChunk = kBlock * kSortedPer;     // positions per workgroup
constexpr int kSortedLists = 64;                      // lists per launch (kernel-argument table)

struct SortedSampleArgs {
  int64_t* idx;  // lists of m indices, list c at idx + c m
  int64_t m;
  int64_t chunks;  // workgroups per list: ceil((m + 1) / kSortedChunk)
  uint64_t seed[kSortedLists];
  int64_t n[kSortedLists];
};

__device__ __forceinline__ uint64_t exp_fixed(uint64_t seed, uint64_t j) {
  const uint64_t r = counter_hash(seed, j) >> 11;
  const double u = static_cast<double>(r + 1) * 0x1p-53;  // (0, 1]
  const double e = -log(u);                              // [0, 36.8]
  return static_cast<uint64_t>(e * 0x1p32 + 0.5);
}

// Exact sum of one value per thread (uint64, so any order gives the same total).
__device__ __forceinline__ uint64_t block_sum_u64(uint64_t v) {
  __shared__ uint64_t part[kBlock / 64];
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = v;
  __syncthreads();
  uint64_t t = 0;
#pragma unroll
  for (int w = 0; w < kBlock / 64; ++w) t += part[w];
  __syncthreads();
  return t;
}

__global__ void __launch_bounds__(kBlock) sorted_sample_exp_kernel(SortedSampleArgs a, uint64_t* chunk_sums) {
  const int c = blockIdx.y;
  const int64_t j0 = (int64_t)blockIdx.x * kSortedChunk + (int64_t)threadIdx.x * kSortedPer;
  uint64_t* out = reinterpret_cast<uint64_t*>(a.idx + c * a.m);
  uint64_t s = 0;
#pragma unroll
  for (int k = 0; k < kSortedPer; ++k) {
    const int64_t j = j0 + k;
    if (j <= a.m) {
      const uint64_t e = exp_fixed(a.seed[c], static_cast<uint64_t>(j));
      s += e;
      if (j < a.m) out[j] = e;
    }
  }
  const uint64_t tot = block_sum_u64(s);
  if (threadIdx.x == 0) chunk_sums[c * a.chunks + blockIdx.x] = tot;
}

__global__ void __launch_bounds__(kBlock) sorted_sample_idx_kernel(SortedSampleArgs a, const uint64_t* chunk_sums) {
  const int c = blockIdx.y;
  const uint64_t* cs = chunk_sums + c * a.chunks;
  // sum of the chunks before this one, and of all (S_m)
  uint64_t before = 0, all = 0;
  for (int64_t h = threadIdx.x; h < a.chunks; h += kBlock) {
    const uint64_t v = cs[h];
    all += v;
    if (h < (int64_t)blockIdx.x) before += v;
  }
  before = block_sum_u64(before);
  all = block_sum_u64(all);
  // this thread's positions, their sum, and the exclusive scan of the thread sums
  const int64_t j0 = (int64_t)blockIdx.x * kSortedChunk + (int64_t)threadIdx.x * kSortedPer;
  uint64_t* e = reinterpret_cast<uint64_t*>(a.idx + c * a.m);
  uint64_t v[kSortedPer];
  uint64_t s = 0;
#pragma unroll
  for (int k = 0; k < kSortedPer; ++k) {
    v[k] = j0 + k < a.m ? e[j0 + k] : 0;
    s += v[k];
  }
  __shared__ uint64_t scan[kBlock];
  scan[threadIdx.x] = s;
  __syncthreads();
  for (int o = 1; o < kBlock; o <<= 1) {  // inclusive Hillis-Steele scan (exact: integers)
    const uint64_t add = threadIdx.x >= o ? scan[threadIdx.x - o] : 0;
    __syncthreads();
    scan[threadIdx.x] += add;
    __syncthreads();
  }
  uint64_t run = before + scan[threadIdx.x] - s;
  const double total = static_cast<double>(all);
  const int64_t n = a.n[c];
  const double dn = static_cast<double>(n);
#pragma unroll
  for (int k = 0; k < kSortedPer; ++k) {
    if (j0 + k < a.m) {
      run += v[k];
      int64_t i = static_cast<int64_t>(static_cast<double>(run) / total * dn);
      a.idx[c * a.m + j0 + k] = i < n ? i : n - 1;
    }
  }
}

// ---------------------------------------------------------------------------
// K7 / K8: gate target of one group, and the fused update.
// ---------------------------------------------------------------------------
struct GateSpec {
  ScoreSpec s;
  int gate, n_keep;
  int has_frozen;
  int mask_dtype, frozen_dtype;
  float denom;        // T + 1e-8 in f32
  float rdenom;       // RN(1 / denom)
  float beta_struct;  // 0 disables the mix
  float one_minus_beta;
};

// G of one group (compute_gate_target, :1083-1229).  mprev / frz: current mask
// and frozen flags of the group (frz only read when has_frozen).
// rsigma = RN(1 / sigma) (computed once per thread); gs.rdenom = RN(1 / denom).
template <int SD>
__device__ __forceinline__ void gate_of_group(const GateSpec& gs, const float sc[4], const Group& g, float mu,
                                              float sigma, float rsigma, float tau, const float mprev[4],
                                              const float frz[4], float G[4]) {
  float z[4], t[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) t[j] = sc[j] - mu;
  div4_by(t, sigma, rsigma, z);
#pragma unroll
  for (int j = 0; j < 4; ++j) z[j] = rndc<SD>(z[j]);
  if (gs.gate == SF_GATE_UNSTRUCTURED || gs.gate == SF_GATE_STRUCTURED) {
    const float th = gs.gate == SF_GATE_UNSTRUCTURED ? tau : kth_largest4(z, gs.n_keep);
    float x[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) t[j] = z[j] - th;
    div4_by(t, gs.denom, gs.rdenom, x);
#pragma unroll
    for (int j = 0; j < 4; ++j) G[j] = rndc<SD>(sigmoidf_(x[j]));
  } else if (gs.gate == SF_GATE_STRUCTURED_EXACT) {
    uint32_t keep = topk4_keep(z, gs.n_keep);
#pragma unroll
    for (int j = 0; j < 4; ++j) G[j] = ((keep >> j) & 1u) ? 1.0f : 0.0f;
  } else {  // SF_GATE_ZSCORE: z itself, pooled per block by the block_sparse gate
#pragma unroll
    for (int j = 0; j < 4; ++j) G[j] = z[j];
  }
  if (gs.beta_struct > 0.0f) {  // (:1199-1225): target = topN(z) on full groups, G itself on the tail
    uint32_t keep = g.full ? topk4_keep(z, gs.n_keep) : 0u;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float t = g.full ? (((keep >> j) & 1u) ? 1.0f : 0.0f) : G[j];
      G[j] = rndc<SD>(gs.one_minus_beta * G[j] + gs.beta_struct * t);
    }
  }
  if (gs.has_frozen) {  // G[frozen] = mask[frozen]  (:1227-1229)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (frz[j] != 0.0f) G[j] = rndc<SD>(mprev[j]);
  }
}

template <int WD, int HD, int SD>
__global__ void __launch_bounds__(kBlock) gate_target_kernel(GateSpec gs, const void* __restrict__ W,
                                                             const void* __restrict__ H, const void* __restrict__ aux,
                                                             const void* __restrict__ mask,
                                                             const void* __restrict__ frozen,
                                                             const float* __restrict__ stats,
                                                             const float* __restrict__ tau_p, void* __restrict__ Gout,
                                                             int g_dtype, int64_t cols, int64_t groups, int64_t gpr,
                                                             bool vec) {
  const float mu = stats[0], sigma = stats[1], rsigma = 1.0f / sigma;
  const float tau = tau_p ? *tau_p : 0.0f;
  for (GroupWalk w(groups, cols, gpr); w.live(); w.next()) {
    Group g = w.group();
    const bool v = vec && g.full;
    float sc[4], mp[4] = {0, 0, 0, 0}, fz[4] = {0, 0, 0, 0}, G[4];
    group_scores<WD, HD>(gs.s, W, H, aux, g, v, cols, sc);
    if (gs.has_frozen) {
      load4_any(frozen, gs.frozen_dtype, g.elem, g.n, v, fz);
      load4_any(mask, gs.mask_dtype, g.elem, g.n, v, mp);
    }
    gate_of_group<SD>(gs, sc, g, mu, sigma, rsigma, tau, mp, fz, G);
    if (g_dtype == SF_DTYPE_F32)
      store4<SF_DTYPE_F32>(Gout, g.elem, g.n, v, G);
    else
      store4<SF_DTYPE_BF16>(Gout, g.elem, g.n, v, G);
  }
}

struct UpdateSpec {
  GateSpec gs;
  int penalty, pen_n;
  float pen_coef;
  float bin_lo, bin_hi;  // (1 - d), (1 + d) in f32; d == 0 disables
  int binarize;
  float keep_a, a;  // (1 - a), a
  int apply_freeze, snap_high;
  float freeze_low, freeze_high;
  int hard_kind, hard_n;
};

// Penalty pull toward a target, then clamp (:1291-1573), and the
// multiplicative binarisation push (:1576-1590).  mp: the mask the penalty
// compares against; sd: dtype of G.
// tg: the explicit target of SF_PENALTY_TARGET (block16 / block_sparse modes).
template <int MD, int SD>
__device__ __forceinline__ void pull_and_push(const UpdateSpec& us, const Group& g, const float mp[4], float G[4],
                                              const float* tg = nullptr) {
  if (us.penalty != SF_PENALTY_NONE) {
    if (us.penalty == SF_PENALTY_TARGET) {  // G -= c * (mask.to(G.dtype) - target)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float delta = rndc<SD>(rndc<SD>(mp[j]) - tg[j]);
        G[j] = rndc<SD>(G[j] - rndc<SD>(us.pen_coef * delta));
      }
    } else if (us.penalty == SF_PENALTY_MID) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float pg = rndc<SD>(rndc<MD>(1.0f - 2.0f * mp[j]));
        G[j] = rndc<SD>(G[j] - rndc<SD>(us.pen_coef * pg));
      }
    } else {  // nm_2_4 / structured_topn: target = topN(G) on full groups, 1 on the tail
      uint32_t keep = g.full ? topk4_keep(G, us.pen_n) : 0xfu;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float t = ((keep >> j) & 1u) ? 1.0f : 0.0f;
        float delta = rndc<SD>(rndc<SD>(mp[j]) - t);
        G[j] = rndc<SD>(G[j] - rndc<SD>(us.pen_coef * delta));
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) G[j] = G[j] != G[j] ? G[j] : fminf(fmaxf(G[j], 0.0f), 1.0f);  // clamp keeps NaN
  }
  if (us.binarize) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (G[j] < 0.5f)
        G[j] = rndc<SD>(G[j] * us.bin_lo);
      else if (G[j] > 0.5f)
        G[j] = rndc<SD>(G[j] * us.bin_hi);
    }
  }
}

// EMA: mask.mul_(1 - a).add_(G, alpha=a).clamp_(0, 1)  (:1593)
template <int MD>
__device__ __forceinline__ void ema_of(const UpdateSpec& us, const float mp[4], const float G[4], float mn[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float m1 = rnd(mp[j] * us.keep_a, MD);
    float m2 = rnd(fmaf(G[j], us.a, m1), MD);
    mn[j] = m2 != m2 ? m2 : fminf(fmaxf(m2, 0.0f), 1.0f);  // clamp_ keeps NaN
  }
}

// Freeze snaps of the new mask and the frozen flags (:1621-1642).  fz: current flags.
__device__ __forceinline__ void freeze_group(const UpdateSpec& us, const Group& g, bool v, float mn[4],
                                             const float fz[4], void* frozen) {
  float fl[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    bool f0 = mn[j] <= us.freeze_low;
    bool f1 = mn[j] >= us.freeze_high;
    bool applied = f0;
    if (f0) mn[j] = 0.0f;
    if (us.snap_high) {
      if (f1) mn[j] = 1.0f;
      applied = applied || f1;
    }
    fl[j] = fmaxf(fz[j], applied ? 1.0f : 0.0f);
  }
  if (us.gs.has_frozen) {
    if (us.gs.frozen_dtype == SF_DTYPE_F32)
      store4<SF_DTYPE_F32>(frozen, g.elem, g.n, v, fl);
    else
      store4<SF_DTYPE_BF16>(frozen, g.elem, g.n, v, fl);
  }
}

// Kept members (bit j = member j) of the hard projection of one group.
__device__ __forceinline__ uint32_t hard_bits(const float v[4], const Group& g, int kind, int n_keep) {
  if (kind == SF_HARD_NONE) return 0xfu;
  if (kind == SF_HARD_THRESHOLD) {
    uint32_t b = 0u;
#pragma unroll
    for (int j = 0; j < 4; ++j) b |= (v[j] > 0.5f ? 1u : 0u) << j;
    return b;
  }
  return g.full ? topk4_keep(v, n_keep) : 0xfu;  // a tail group keeps every column
}

// Positions of a group where the hard views of a and b differ (:1659-1661).
__device__ __forceinline__ int flips_of(const float a[4], const float b[4], const Group& g, int kind, int n) {
  // 2:4 on a full NaN-free group (the common case): compare the spread keep sets directly
  if (kind >= SF_HARD_NM_TAIL_KEEP && n == 2 && g.full && !any_nan4(a) && !any_nan4(b))
    return __popc(topk2_spread_f(a) ^ topk2_spread_f(b));
  return __popc((hard_bits(a, g, kind, n) ^ hard_bits(b, g, kind, n)) & ((1u << g.n) - 1u));
}

// Specialisations of the fused update for the configurations training runs
// spend their time in: kFastPlain = hessian_ratio scores, unstructured gate,
// no penalty, binarisation, frozen flags, freezing or structural mix, 2:4 flip
// count; kFastNm24 = the same with the nm_2_4 penalty.  The spec's fields are
// fixed to those values, so the compiler drops every other branch (the
// arithmetic is the generic path's, operation for operation).
constexpr int kFastNone = 0, kFastPlain = 1, kFastNm24 = 2;

template <int FAST>
__device__ __forceinline__ UpdateSpec fast_spec(const UpdateSpec& in) {
  UpdateSpec us = in;
  if constexpr (FAST != kFastNone) {
    us.gs.s.metric = SF_METRIC_HESSIAN_RATIO;
    us.gs.gate = SF_GATE_UNSTRUCTURED;
    us.gs.beta_struct = 0.0f;
    us.gs.has_frozen = 0;
    us.apply_freeze = 0;
    us.binarize = 0;
    us.penalty = FAST == kFastNm24 ? SF_PENALTY_NM_2_4 : SF_PENALTY_NONE;
    us.pen_n = 2;
    us.hard_kind = SF_HARD_NM_TAIL_KEEP;
    us.hard_n = 2;
  }
  return us;
}

// Workgroups of an update grid: 8 groups per thread (each workgroup's set-up --
// the statistics and tau loads, 1 / sigma -- and its flip-count reduction
// amortised over 8 rounds; measured faster than the capped elementwise grid).
int update_grid(int64_t groups) {
  const int64_t g = ceil_div(groups, 8 * kBlock);
  return static_cast<int>(g < 1 ? 1 : g);
}

// The specialisation a spec qualifies for (kFastNone: the generic kernel).
int fast_kind(const UpdateSpec& us) {
  const GateSpec& gs = us.gs;
  if (gs.s.metric != SF_METRIC_HESSIAN_RATIO || gs.gate != SF_GATE_UNSTRUCTURED || gs.beta_struct != 0.0f ||
      gs.has_frozen || us.apply_freeze || us.binarize || us.hard_kind != SF_HARD_NM_TAIL_KEEP || us.hard_n != 2)
    return kFastNone;
  if (us.penalty == SF_PENALTY_NONE) return kFastPlain;
  if (us.penalty == SF_PENALTY_NM_2_4 && us.pen_n == 2) return kFastNm24;
  return kFastNone;
}

// VEC: cols % 4 == 0 and every operand 16-byte aligned, so every group is a
// full, vector-loadable group of 4 (known at compile time: no tail branches).
// Workgroup `blk` of a grid of `nblk` over one layer.
// NT: W, H and the mask through non-temporal loads and stores (the batched arena pass).
template <int WD, int HD, int MD, int SD, bool VEC, int FAST = kFastNone, bool NT = false>
__device__ __forceinline__ void update_mask_block(const UpdateSpec& us_in, const void* __restrict__ W,
                                                  const void* __restrict__ H, const void* __restrict__ aux,
                                                  void* __restrict__ mask, void* __restrict__ frozen,
                                                  const float* __restrict__ stats, const float* __restrict__ tau_p,
                                                  int64_t cols, int64_t groups, int64_t gpr, bool vec, int64_t* flips,
                                                  int64_t blk, int64_t nblk) {
  const UpdateSpec us = fast_spec<FAST>(us_in);
  const GateSpec& gs = us.gs;
  const float mu = stats[0], sigma = stats[1], rsigma = 1.0f / sigma;
  const float tau = tau_p ? *tau_p : 0.0f;
  int64_t cnt = 0;
  auto load = [&](const Group& g, bool v, GroupOps& o, float mp[4], float fz[4]) {
    load_group_ops<WD, HD, NT>(gs.s, W, H, aux, g, v, o);
    load4<MD, NT>(mask, g.elem, g.n, v, mp);
#pragma unroll
    for (int j = 0; j < 4; ++j) fz[j] = 0.0f;
    if (gs.has_frozen) load4_any(frozen, gs.frozen_dtype, g.elem, g.n, v, fz);
  };
  auto finish = [&](const Group& g, bool v, const GroupOps& o, const float mp[4], const float fz[4]) {
    float sc[4], G[4], mn[4];
    scores_of_ops<WD, HD>(gs.s, o, g, sc);
    gate_of_group<SD>(gs, sc, g, mu, sigma, rsigma, tau, mp, fz, G);
    pull_and_push<MD, SD>(us, g, mp, G);
    ema_of<MD>(us, mp, G, mn);
    if (us.apply_freeze) freeze_group(us, g, v, mn, fz, frozen);
    store4<MD, NT>(mask, g.elem, g.n, v, mn);
    if (flips) cnt += flips_of(mp, mn, g, us.hard_kind, us.hard_n);
  };
  GroupWalk w(groups, cols, gpr, blk, nblk);
  if constexpr (VEC) {
    // two groups per round, every load of both issued before either is used: one memory
    // latency per two groups
    while (w.live()) {
      Group g0 = w.group();
      g0.n = 4;
      g0.full = true;
      w.next();
      const bool two = w.live();
      Group g1 = g0;
      if (two) {
        g1 = w.group();
        g1.n = 4;
        g1.full = true;
        w.next();
      }
      GroupOps o0, o1;
      float m0[4], m1[4], f0[4], f1[4];
      load(g0, true, o0, m0, f0);
      if (two) load(g1, true, o1, m1, f1);
      finish(g0, true, o0, m0, f0);
      if (two) finish(g1, true, o1, m1, f1);
    }
  } else {
    for (; w.live(); w.next()) {
      const Group g = w.group();
      const bool v = vec && g.full;
      GroupOps o;
      float mp[4], fz[4];
      load(g, v, o, mp, fz);
      finish(g, v, o, mp, fz);
    }
  }
  if (flips) block_add_i64(cnt, flips);
}

template <int WD, int HD, int MD, int SD, bool VEC, int FAST>
__global__ void __launch_bounds__(kBlock) update_mask_kernel(UpdateSpec us, const void* __restrict__ W,
                                                             const void* __restrict__ H, const void* __restrict__ aux,
                                                             void* __restrict__ mask, void* __restrict__ frozen,
                                                             const float* __restrict__ stats,
                                                             const float* __restrict__ tau_p, int64_t cols,
                                                             int64_t groups, int64_t gpr, bool vec, int64_t* flips) {
  update_mask_block<WD, HD, MD, SD, VEC, FAST>(us, W, H, aux, mask, frozen, stats, tau_p, cols, groups, gpr, vec,
                                               flips, blockIdx.x, gridDim.x);
}

// ---------------------------------------------------------------------------
// Multi-layer mask update: the score statistics, tau selection and fused
// update of up to kMultiLayers layers that share every parameter but their
// shape, as a handful of launches.  Each layer runs exactly the workgroup
// grid its single-layer launch would (the statistics' kStatsGrid partials
// fold in the same order, the update walks the same groups), laid end to end
// in one grid, so every output equals the single-layer entry points' bit for
// bit.  The layer table travels in the kernel arguments.
// ---------------------------------------------------------------------------
constexpr int kMultiLayers = 28;

struct MultiLayer {
  const void* W;
  const void* H;
  const void* aux;
  void* mask;
  void* frozen;
  float* stats;
  float* tau;
  int64_t* flips;
  const int64_t* idx;  // tau sample indices (null: every element)
  int64_t rows, cols;
  int64_t m;           // tau sample size
  int64_t keys_off;    // first key of the layer's sample in the keys buffer
  int32_t nblk;        // workgroups of the layer's update grid
  int32_t vec;         // vector-loadable groups
  int32_t nsel;        // workgroups of the layer's radix passes
  int32_t win_off;     // first window start of the layer in the window-start buffer (statistics fold)
};

struct MultiArgs {
  UpdateSpec us;
  int32_t count;
  int32_t first[kMultiLayers + 1];  // update grid: layer l owns workgroups [first[l], first[l + 1])
  MultiLayer l[kMultiLayers];
};
static_assert(sizeof(MultiArgs) <= 4000, "multi-layer table exceeds the kernel argument budget");

// Layer of workgroup b of the update grid (first[0] == 0, first[count] == grid).
__device__ __forceinline__ int multi_layer_of(const MultiArgs& a, int b) {
  int l = 0;
#pragma unroll
  for (int i = 1; i < kMultiLayers; ++i) l += (i < a.count && a.first[i] <= b) ? 1 : 0;
  return l;
}

// Statistics partials: kStatsGrid workgroups per layer, layer = blockIdx.x / kStatsGrid.
// The first n * gather workgroups gather the layers' tau samples (gather per
// layer; 0 when the tau stage runs on its own), the rest are the statistics
// grids.  The gather's random reads go first and overlap the statistics pass,
// whose cost is its arithmetic.
template <int WD, int HD, bool VEC, bool RATIO>
__global__ void __launch_bounds__(kBlock) stats_partial_multi_kernel(MultiArgs a, double* partial, int gather,
                                                                     uint32_t* keys) {
  int b = blockIdx.x;
  if (b < a.count * gather) {
    const MultiLayer& L = a.l[b / gather];
    tau_gather_block(a.us.gs.s, L.W, L.H, L.aux, L.rows, L.cols, L.idx, L.m, keys + L.keys_off, b % gather, gather);
    return;
  }
  b -= a.count * gather;
  const int l = b / kStatsGrid, blk = b - l * kStatsGrid;
  const MultiLayer& L = a.l[l];
  const int64_t gpr = ceil_div(L.cols, 4);
  stats_partial_block<WD, HD, VEC, RATIO, true>(a.us.gs.s, L.W, L.H, L.aux, L.cols, L.rows * gpr, gpr, L.vec != 0,
                                          partial + (int64_t)l * 2 * kStatsGrid, blk);
}

// ---------------------------------------------------------------------------
// Statistics with the tau sample folded in (batched update, every layer's
// groups vector-loadable).  Round r of statistics workgroup b covers the
// 1024 elements [1024 (b + r kStatsGrid), +1024), each wave a 256-element
// sub-window of them (64 lanes x one group), so every element is scored
// exactly once per pass.  When a layer's sample is in non-decreasing index
// order, the samples that fall in sub-window v are the positions
// [wstart[v], wstart[v + 1]) of the list: the wave stages its sub-window's
// scores in LDS and those samples take their keys from there, instead of a
// separate gather reading W and H at random positions (at a 262 144 sample
// over a 4096 x 4096 layer that gather touches about 63 % of W's 128-byte
// lines and 39 % of H's).  Each wave works alone (no workgroup barrier: LDS
// accesses of one wave are performed in order), a round's samples are
// resolved one iteration later, so their index loads have a whole iteration
// to arrive, and only sampled scores are turned into keys: the pass is
// bound by its score arithmetic, and every instruction added per element
// shows.  The keys land where the gather puts them (key i for sample i), so
// the selection and tau are unchanged.  A layer whose sample is not sorted
// gets empty sub-window ranges and is gathered at random by
// sample_windows_multi_kernel instead.
// ---------------------------------------------------------------------------
constexpr int kWinShift = 8;  // log2 of a sub-window: one wave's 64 groups of 4
constexpr int kWinGrid = 64;  // workgroups per layer of the order check: one flag per lane of a wave

__device__ __forceinline__ int64_t clamp_index(int64_t e, int64_t n) { return e < 0 ? 0 : (e >= n ? n - 1 : e); }

// ok[l][b] = 1 when the (clamped) sample indices workgroup b checked are in non-decreasing order.
__global__ void __launch_bounds__(kBlock) sample_order_multi_kernel(MultiArgs a, int32_t* ok) {
  const int l = blockIdx.y;
  const MultiLayer& L = a.l[l];
  if (!L.idx) return;  // uniform: the whole workgroup
  const int64_t n = L.rows * L.cols;
  const int64_t tid = (int64_t)blockIdx.x * kBlock + threadIdx.x, nth = (int64_t)kWinGrid * kBlock;
  bool bad = false;
  for (int64_t i = tid + 1; i < L.m; i += nth) bad = bad || clamp_index(L.idx[i - 1], n) > clamp_index(L.idx[i], n);
  const int any = __syncthreads_or(bad ? 1 : 0);
  if (threadIdx.x == 0) ok[l * kWinGrid + blockIdx.x] = any ? 0 : 1;
}

// Sub-window starts: wstart[v] = the first sample position whose (clamped) index is at least 256 v,
// v = 0..nsub (nsub = the layer's sub-windows; wstart[nsub] = m), written by the samples that open them
// (sample i writes the sub-windows after its predecessor's, up to its own: nsub + 1 writes in all).  A
// layer whose sample is not sorted gets wstart = 0 everywhere (empty ranges), and its sample's keys are
// gathered here at random positions instead.
__global__ void __launch_bounds__(kBlock) sample_windows_multi_kernel(MultiArgs a, const int32_t* ok,
                                                                      int32_t* wstart, uint32_t* keys) {
  const int l = blockIdx.y;
  const MultiLayer& L = a.l[l];
  if (!L.idx) return;
  const int64_t n = L.rows * L.cols, m = L.m;
  const int64_t nsub = (n + (1 << kWinShift) - 1) >> kWinShift;
  int32_t* ws = wstart + L.win_off;
  const int64_t tid = (int64_t)blockIdx.x * kBlock + threadIdx.x, nth = (int64_t)gridDim.x * kBlock;
  const bool sorted = __all(ok[l * kWinGrid + (threadIdx.x & 63)] != 0);
  if (!sorted) {  // empty ranges for the statistics pass; the sample is gathered here, at random
    for (int64_t v = tid; v <= nsub; v += nth) ws[v] = 0;
    tau_gather_block(a.us.gs.s, L.W, L.H, L.aux, L.rows, L.cols, L.idx, m, keys + L.keys_off, blockIdx.x,
                     gridDim.x);
    return;
  }
  for (int64_t i = tid; i < m; i += nth) {
    const int64_t v = clamp_index(L.idx[i], n) >> kWinShift;
    const int64_t from = i == 0 ? 0 : (clamp_index(L.idx[i - 1], n) >> kWinShift) + 1;
    for (int64_t u = from; u <= v; ++u) ws[u] = static_cast<int32_t>(i);
    if (i == m - 1)
      for (int64_t u = v + 1; u <= nsub; ++u) ws[u] = static_cast<int32_t>(m);
  }
}

// The statistics of one workgroup with the sample's keys folded in; hessian_ratio scores (|W| / sqrt(H + eps),
// no aux operand: the paper's metric), so the walk is a plain group index (element = 4 x group).
template <int WD, int HD>
__device__ __forceinline__ void stats_fold_block(const ScoreSpec& s_in, const MultiLayer& L,
                                                 const int32_t* __restrict__ wstart, uint32_t* __restrict__ keys,
                                                 double* partial, int blk) {
  ScoreSpec s = s_in;
  s.metric = SF_METRIC_HESSIAN_RATIO;
  const int64_t groups = L.rows * (L.cols >> 2), n = L.rows * L.cols;
  const int64_t* idx = L.idx;
  uint32_t* kout = keys + L.keys_off;
  const int32_t* ws = wstart + L.win_off;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // raw scores of the wave's two sub-windows of an iteration, double-buffered: [wave][parity][round][element]
  __shared__ __align__(16) float win[kBlock / 64][2][2][256];
  float(*mine)[2][256] = win[wave];
  const int64_t stride = (int64_t)kStatsGrid * kBlock;
  double sum = 0.0, sq = 0.0;
  // The previous iteration's samples, resolved in one pass: lane l serves sample (l % 32) of sub-window
  // l / 32 (rounds 0 and 1), so its range, element base and first index are this lane's.
  const int h = lane >> 5, j = lane & 31;
  int32_t ps = 0, pe = 0;  // the lane's sub-window: sample positions [ps, pe)
  int64_t pb = 0;          // its first element
  int64_t pv = 0;          // index of sample ps + j
  int par = 0;
  auto resolve = [&](int pp) {
    for (int32_t i = ps + j; i < pe; i += 32) {
      const int64_t e = i == ps + j ? pv : idx[i];
      int64_t off = e - pb;  // clamp_index(e, n) - pb: the clamped ends lie in the first / last sub-window
      off = off < 0 ? 0 : off;
      off = off > n - 1 - pb ? n - 1 - pb : off;
      kout[i] = ordered_key(mine[pp][h][off]);
    }
  };
  auto load_group = [&](int64_t g, GroupOps& o) {
    Group G;
    G.row = 0;
    G.col = 0;
    G.elem = 4 * g;
    G.n = 4;
    G.full = true;
    load_group_ops<WD, HD, true>(s, L.W, L.H, nullptr, G, true, o);
  };
  auto score_ops = [&](const GroupOps& o, float sc[4]) {
    Group G;
    G.n = 4;
    scores_of_ops<WD, HD>(s, o, G, sc);
  };
  // two rounds per iteration, both loaded before either is used (a lane past the layer loads group 0 and
  // discards it, so the loads are unconditional); the loop bound is wave-uniform and each thread adds its
  // groups in the order of stats_partial_block
  for (int64_t base = (int64_t)blk * kBlock + 64 * wave; base < groups; base += 2 * stride, par ^= 1) {
    const bool two = base + stride < groups;
    const int64_t g0 = base + lane, g1 = base + stride + lane;
    const bool live0 = g0 < groups, live1 = g1 < groups;
    GroupOps o0, o1;
    load_group(live0 ? g0 : 0, o0);
    load_group(live1 ? g1 : 0, o1);
    const int64_t v0 = base >> (kWinShift - 2), v1 = (base + stride) >> (kWinShift - 2);
    int32_t s0 = 0, e0 = 0, s1 = 0, e1 = 0;
    if (idx) {
      s0 = ws[v0];
      e0 = ws[v0 + 1];
      if (two) {
        s1 = ws[v1];
        e1 = ws[v1 + 1];
      }
      resolve(par ^ 1);  // the previous iteration's samples, from the other buffer
    }
    float sc0[4], sc1[4];
    score_ops(o0, sc0);
    score_ops(o1, sc1);
    if (live0) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const double d = sc0[k];
        sum += d;
        sq += d * d;
      }
    }
    if (live1) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const double d = sc1[k];
        sum += d;
        sq += d * d;
      }
    }
    if (!idx) {  // the sample is every element, in element order (4-byte stores: keys_off may be odd)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        if (live0) kout[4 * g0 + k] = ordered_key(sc0[k]);
        if (live1) kout[4 * g1 + k] = ordered_key(sc1[k]);
      }
      continue;
    }
    if (e0 > s0 && live0) *reinterpret_cast<float4*>(&mine[par][0][4 * lane]) = make_float4(sc0[0], sc0[1], sc0[2], sc0[3]);
    if (e1 > s1 && live1) *reinterpret_cast<float4*>(&mine[par][1][4 * lane]) = make_float4(sc1[0], sc1[1], sc1[2], sc1[3]);
    // this iteration's samples: the lane's first index loads now, the rest after the next iteration's loads
    ps = h ? s1 : s0;
    pe = h ? e1 : e0;
    pb = (h ? v1 : v0) << kWinShift;
    pv = ps + j < pe ? idx[ps + j] : 0;
  }
  if (idx) resolve(par ^ 1);
  block_sum2_f64(sum, sq, &partial[2 * blk], &partial[2 * blk + 1]);
}

template <int WD, int HD>
__global__ void __launch_bounds__(kBlock) stats_fold_multi_kernel(MultiArgs a, double* partial, uint32_t* keys,
                                                                  const int32_t* wstart) {
  const int l = blockIdx.x / kStatsGrid, blk = blockIdx.x - l * kStatsGrid;
  stats_fold_block<WD, HD>(a.us.gs.s, a.l[l], wstart, keys, partial + (int64_t)l * 2 * kStatsGrid, blk);
}

__global__ void __launch_bounds__(kBlock) stats_final_multi_kernel(MultiArgs a, const double* partial) {
  const int l = blockIdx.x;
  stats_final_block(partial + (int64_t)l * 2 * kStatsGrid, kStatsGrid, a.l[l].rows * a.l[l].cols, a.l[l].stats);
}

// tau: grid (x, layer); each layer's gather strides over gridDim.x workgroups,
// its radix passes use its own nsel of them.
__global__ void __launch_bounds__(kBlock) tau_gather_multi_kernel(MultiArgs a, uint32_t* keys) {
  const MultiLayer& L = a.l[blockIdx.y];
  tau_gather_block(a.us.gs.s, L.W, L.H, L.aux, L.rows, L.cols, L.idx, L.m, keys + L.keys_off, blockIdx.x,
                   gridDim.x);
}

__global__ void __launch_bounds__(kBlock) tau_pass_multi_kernel(MultiArgs a, const uint32_t* keys, int pass, float q,
                                                                SelState* states, uint32_t* parts0, uint32_t* parts1) {
  const int l = blockIdx.y;
  const MultiLayer& L = a.l[l];
  if ((int)blockIdx.x >= L.nsel) return;  // the whole workgroup: no barrier is skipped
  // pass p reads state p-2 (slot p & 1) and partials p-1, writes state p-1 (slot (p + 1) & 1) and partials p
  SelState* st = states + 2 * l;
  const int64_t pstride = (int64_t)kSelStride * kSelGrid;
  uint32_t* part[2] = {parts0 + l * pstride, parts1 + l * pstride};
  tau_pass_block(keys + L.keys_off, L.m, pass, q, &st[pass & 1], &st[(pass + 1) & 1], part[(pass + 1) & 1],
                 part[pass & 1], blockIdx.x, L.nsel);
}

__global__ void __launch_bounds__(kBlock) tau_final_multi_kernel(MultiArgs a, float q, const SelState* states,
                                                                 const uint32_t* parts1) {
  const int l = blockIdx.x;
  const MultiLayer& L = a.l[l];
  tau_final_block(L.m, q, L.nsel, &states[2 * l], parts1 + l * (int64_t)kSelStride * kSelGrid, L.stats,
                  a.us.gs.s.score_dtype, L.tau);
}

template <int WD, int HD, int MD, int SD, bool VEC, int FAST>
__global__ void __launch_bounds__(kBlock) update_mask_multi_kernel(MultiArgs a) {
  const int l = multi_layer_of(a, blockIdx.x);
  const MultiLayer& L = a.l[l];
  const int64_t gpr = ceil_div(L.cols, 4);
  update_mask_block<WD, HD, MD, SD, VEC, FAST, true>(a.us, L.W, L.H, L.aux, L.mask, L.frozen, L.stats, L.tau, L.cols,
                                               L.rows * gpr, gpr, L.vec != 0, L.flips, blockIdx.x - a.first[l],
                                               L.nblk);
}

// ---------------------------------------------------------------------------
// GLU gate/up joint update (legacy/utils.py:363-643).  The joint score
// S = score(gate) + score(up) is written once (its statistics, tau sample and
// the update all read it), then one pass computes G from S with the gate
// layer's mask and frozen flags and applies the same G to both masks.
// ---------------------------------------------------------------------------
template <int WD, int HD>
__global__ void __launch_bounds__(kBlock) joint_scores_kernel(ScoreSpec sg, const void* __restrict__ Wg,
                                                              const void* __restrict__ Hg, const void* __restrict__ ag,
                                                              ScoreSpec su, const void* __restrict__ Wu,
                                                              const void* __restrict__ Hu, const void* __restrict__ au,
                                                              void* __restrict__ S, int s_dtype, int64_t cols,
                                                              int64_t groups, int64_t gpr, bool vec) {
  for (GroupWalk w(groups, cols, gpr); w.live(); w.next()) {
    Group g = w.group();
    const bool v = vec && g.full;
    float a[4], b[4], o[4];
    group_scores<WD, HD>(sg, Wg, Hg, ag, g, v, cols, a);
    group_scores<WD, HD>(su, Wu, Hu, au, g, v, cols, b);
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = rnd(a[j] + b[j], s_dtype);
    if (s_dtype == SF_DTYPE_F32)
      store4<SF_DTYPE_F32>(S, g.elem, g.n, v, o);
    else
      store4<SF_DTYPE_BF16>(S, g.elem, g.n, v, o);
  }
}

// One layer's importance scores, rounded to s_dtype (_compute_importance_scores).
template <int WD, int HD>
__global__ void __launch_bounds__(kBlock) importance_scores_kernel(ScoreSpec sp, const void* __restrict__ W,
                                                                   const void* __restrict__ H,
                                                                   const void* __restrict__ aux, void* __restrict__ S,
                                                                   int s_dtype, int64_t cols, int64_t groups,
                                                                   int64_t gpr, bool vec) {
  for (GroupWalk w(groups, cols, gpr); w.live(); w.next()) {
    Group g = w.group();
    const bool v = vec && g.full;
    float a[4], o[4];
    group_scores<WD, HD>(sp, W, H, aux, g, v, cols, a);
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = rnd(a[j], s_dtype);
    if (s_dtype == SF_DTYPE_F32)
      store4<SF_DTYPE_F32>(S, g.elem, g.n, v, o);
    else
      store4<SF_DTYPE_BF16>(S, g.elem, g.n, v, o);
  }
}

template <int SD, int MD>
__global__ void __launch_bounds__(kBlock) glu_update_kernel(UpdateSpec us, const void* __restrict__ S,
                                                            void* __restrict__ mask_g, void* __restrict__ mask_u,
                                                            const void* __restrict__ frozen_g,
                                                            const float* __restrict__ stats,
                                                            const float* __restrict__ tau_p, int up_kind, int up_n,
                                                            int64_t cols, int64_t groups, int64_t gpr, bool vec,
                                                            int64_t* flips_g, int64_t* flips_u) {
  const GateSpec& gs = us.gs;  // z and G live in the mask dtype (:541-545)
  const float mu = stats[0], sigma = stats[1], rsigma = 1.0f / sigma;
  const float tau = tau_p ? *tau_p : 0.0f;
  int64_t cg = 0, cu = 0;
  for (GroupWalk w(groups, cols, gpr); w.live(); w.next()) {
    Group g = w.group();
    const bool v = vec && g.full;
    float sc[4], pg[4], pu[4], fz[4] = {0, 0, 0, 0}, G[4], ng[4], nu[4];
    load4<SD>(S, g.elem, g.n, v, sc);
    load4<MD>(mask_g, g.elem, g.n, v, pg);
    load4<MD>(mask_u, g.elem, g.n, v, pu);
    if (gs.has_frozen) load4_any(frozen_g, gs.frozen_dtype, g.elem, g.n, v, fz);
    gate_of_group<MD>(gs, sc, g, mu, sigma, rsigma, tau, pg, fz, G);
    pull_and_push<MD, MD>(us, g, pg, G);  // the penalty compares against the gate mask (:615-641)
    ema_of<MD>(us, pg, G, ng);
    ema_of<MD>(us, pu, G, nu);
    store4<MD>(mask_g, g.elem, g.n, v, ng);
    store4<MD>(mask_u, g.elem, g.n, v, nu);
    if (flips_g) cg += flips_of(pg, ng, g, us.hard_kind, us.hard_n);
    if (flips_u) cu += flips_of(pu, nu, g, up_kind, up_n);
  }
  if (flips_g) block_add_i64(cg, flips_g);
  __syncthreads();  // both sums share the workgroup's reduction array
  if (flips_u) block_add_i64(cu, flips_u);
}

// ---------------------------------------------------------------------------
// host-side helpers
// ---------------------------------------------------------------------------
bool aligned(const void* p, int bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) == 0; }
bool dtype_ok(int d) { return d == SF_DTYPE_F32 || d == SF_DTYPE_BF16; }
int esize(int d) { return d == SF_DTYPE_F32 ? 4 : 2; }

// vector loads need cols % 4 == 0 and 4-element alignment of every operand
bool vec_ok(int64_t cols, std::initializer_list<std::pair<const void*, int>> ops) {
  if (cols % 4 != 0) return false;
  for (auto& o : ops)
    if (o.first && !aligned(o.first, 4 * esize(o.second))) return false;
  return true;
}

int check_common(const sf_mask_params* p) {
  SF_CHECK_ARG(p != nullptr, "null sf_mask_params");
  SF_CHECK_ARG(p->rows >= 0 && p->cols >= 0, "negative shape [%lld, %lld]", (long long)p->rows, (long long)p->cols);
  SF_CHECK_ARG(p->metric >= SF_METRIC_MAGNITUDE && p->metric <= SF_METRIC_WEIGHT_SQUARED, "bad metric %d",
               p->metric);
  SF_CHECK_ARG(dtype_ok(p->score_dtype), "bad score dtype %d", p->score_dtype);
  return SF_OK;
}

int check_metric_operands(const sf_mask_params* p, const void* H, const void* aux) {
  const int m = p->metric;
  if (m == SF_METRIC_HESSIAN_OBD || m == SF_METRIC_HESSIAN_RATIO || m == SF_METRIC_HESSIAN)
    SF_CHECK_ARG(H != nullptr, "metric %d needs hessian_diag", m);
  if (m == SF_METRIC_WANDA || m == SF_METRIC_MOVEMENT) SF_CHECK_ARG(aux != nullptr, "metric %d needs aux tensor", m);
  return SF_OK;
}

#define SF_DISPATCH_WH(wd, hd, ...)                                              \
  do {                                                                           \
    if ((wd) == SF_DTYPE_F32 && (hd) == SF_DTYPE_F32) {                          \
      constexpr int WD_ = SF_DTYPE_F32, HD_ = SF_DTYPE_F32;                      \
      __VA_ARGS__;                                                               \
    } else if ((wd) == SF_DTYPE_F32) {                                           \
      constexpr int WD_ = SF_DTYPE_F32, HD_ = SF_DTYPE_BF16;                     \
      __VA_ARGS__;                                                               \
    } else if ((hd) == SF_DTYPE_F32) {                                           \
      constexpr int WD_ = SF_DTYPE_BF16, HD_ = SF_DTYPE_F32;                     \
      __VA_ARGS__;                                                               \
    } else {                                                                     \
      constexpr int WD_ = SF_DTYPE_BF16, HD_ = SF_DTYPE_BF16;                    \
      __VA_ARGS__;                                                               \
    }                                                                            \
  } while (0)

}  // namespace
}  // namespace sf

using namespace sf;

extern "C" int sf_hard_mask(const void* soft, int soft_dtype, void* hard, int hard_dtype, int64_t rows, int64_t cols,
                            int kind, int n_keep, int m_group, void* stream) {
  SF_CHECK_ARG(rows >= 0 && cols >= 0, "negative shape");
  SF_CHECK_ARG(dtype_ok(soft_dtype) && dtype_ok(hard_dtype), "bad dtype");
  SF_CHECK_ARG(kind >= SF_HARD_NONE && kind <= SF_HARD_NM_STRICT, "bad hard kind %d", kind);
  if (rows == 0 || cols == 0) return SF_OK;
  SF_CHECK_ARG(soft && hard, "null tensor");
  if (kind == SF_HARD_NM_TAIL_KEEP || kind == SF_HARD_NM_STRICT) {
    if (m_group != 4 || n_keep < 1 || n_keep > 3) {
      set_error("N:M hard mask with N=%d M=%d: only M=4, 1<=N<=3 is built on device", n_keep, m_group);
      return SF_ERR_UNSUPPORTED;
    }
    SF_CHECK_ARG(kind != SF_HARD_NM_STRICT || cols % m_group == 0,
                 "in_features (%lld) must be divisible by M (%d).", (long long)cols, m_group);
  }
  const int64_t gpr = ceil_div(cols, 4), groups = rows * gpr;
  const bool vec = vec_ok(cols, {{soft, soft_dtype}, {hard, hard_dtype}});
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int grid = elementwise_grid(groups, kBlock);
#define SF_LAUNCH_HARD(SDT, ODT) \
  hard_mask_kernel<SDT, ODT><<<grid, kBlock, 0, st>>>(soft, hard, cols, groups, gpr, vec, kind, n_keep)
  if (soft_dtype == SF_DTYPE_F32 && hard_dtype == SF_DTYPE_F32) SF_LAUNCH_HARD(SF_DTYPE_F32, SF_DTYPE_F32);
  else if (soft_dtype == SF_DTYPE_F32) SF_LAUNCH_HARD(SF_DTYPE_F32, SF_DTYPE_BF16);
  else if (hard_dtype == SF_DTYPE_F32) SF_LAUNCH_HARD(SF_DTYPE_BF16, SF_DTYPE_F32);
  else SF_LAUNCH_HARD(SF_DTYPE_BF16, SF_DTYPE_BF16);
#undef SF_LAUNCH_HARD
  return launch_status("sf_hard_mask");
}

extern "C" int sf_hard_flip_count(const void* prev, const void* now, int dtype, int64_t rows, int64_t cols, int kind,
                                  int n_keep, int m_group, int64_t* flips, void* stream) {
  SF_CHECK_ARG(rows >= 0 && cols >= 0 && dtype_ok(dtype), "bad shape or dtype");
  SF_CHECK_ARG(flips != nullptr, "null flips counter");
  SF_CHECK_ARG(kind >= SF_HARD_NONE && kind <= SF_HARD_NM_STRICT, "bad hard kind %d", kind);
  if (rows == 0 || cols == 0) return SF_OK;
  SF_CHECK_ARG(prev && now, "null tensor");
  if (kind >= SF_HARD_NM_TAIL_KEEP && (m_group != 4 || n_keep < 1 || n_keep > 3)) {
    set_error("N:M flip count with N=%d M=%d: only M=4 is built on device", n_keep, m_group);
    return SF_ERR_UNSUPPORTED;
  }
  const int64_t gpr = ceil_div(cols, 4), groups = rows * gpr;
  const bool vec = vec_ok(cols, {{prev, dtype}, {now, dtype}});
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int grid = elementwise_grid(groups, kBlock);
  if (dtype == SF_DTYPE_F32)
    flip_count_kernel<SF_DTYPE_F32><<<grid, kBlock, 0, st>>>(prev, now, cols, groups, gpr, vec, kind, n_keep, flips);
  else
    flip_count_kernel<SF_DTYPE_BF16><<<grid, kBlock, 0, st>>>(prev, now, cols, groups, gpr, vec, kind, n_keep, flips);
  return launch_status("sf_hard_flip_count");
}

namespace sf {
namespace {
// Workspace layout: [stats partials | 2 select states | 2 x partial histograms | keys], 256-byte aligned parts.
size_t align256(size_t b) { return (b + 255) / 256 * 256; }
size_t ws_stats_bytes() { return align256(sizeof(double) * 2 * kStatsGrid); }
size_t ws_state_off() { return ws_stats_bytes(); }
size_t ws_partial_off() { return ws_state_off() + align256(2 * sizeof(SelState)); }
size_t ws_partial_bytes() { return align256(sizeof(uint32_t) * kSelStride * kSelGrid); }
size_t ws_keys_off() { return ws_partial_off() + 2 * ws_partial_bytes(); }
}  // namespace
}  // namespace sf

extern "C" size_t sf_mask_workspace_size(int64_t rows, int64_t cols, int64_t sample_size) {
  (void)rows;
  (void)cols;
  if (sample_size <= 0) return ws_stats_bytes();
  return ws_keys_off() + sizeof(uint32_t) * static_cast<size_t>(sample_size);
}

extern "C" int sf_score_stats(const sf_mask_params* p, const void* W, int w_dtype, const void* H, int h_dtype,
                              const void* aux, int aux_dtype, float* stats_out, void* workspace,
                              size_t workspace_bytes, void* stream) {
  if (int rc = check_common(p)) return rc;
  if (int rc = check_metric_operands(p, H, aux)) return rc;
  SF_CHECK_ARG(dtype_ok(w_dtype) && (!H || dtype_ok(h_dtype)) && (!aux || dtype_ok(aux_dtype)), "bad dtype");
  SF_CHECK_ARG(W && stats_out, "null tensor");
  SF_CHECK_ARG(workspace && workspace_bytes >= sizeof(double) * 2 * kStatsGrid, "workspace too small");
  const int64_t n = p->rows * p->cols;
  SF_CHECK_ARG(n > 0, "empty score tensor");
  if (!H) h_dtype = SF_DTYPE_F32;
  ScoreSpec s = make_spec(p, w_dtype, h_dtype, aux_dtype);
  const int64_t gpr = ceil_div(p->cols, 4), groups = p->rows * gpr;
  const bool vec = vec_ok(p->cols, {{W, w_dtype}, {H, h_dtype}}) &&
                   (!aux || p->metric != SF_METRIC_MOVEMENT || aligned(aux, 4 * esize(aux_dtype))) &&
                   (!aux || p->metric != SF_METRIC_WANDA || aligned(aux, 4 * esize(aux_dtype)));
  double* partial = static_cast<double*>(workspace);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (vec && p->metric == SF_METRIC_HESSIAN_RATIO)
    SF_DISPATCH_WH(w_dtype, h_dtype,
                   stats_partial_kernel<WD_, HD_, true, true><<<kStatsGrid, kBlock, 0, st>>>(
                       s, W, H, aux, p->cols, groups, gpr, vec, partial));
  else if (vec)
    SF_DISPATCH_WH(w_dtype, h_dtype,
                   stats_partial_kernel<WD_, HD_, true, false><<<kStatsGrid, kBlock, 0, st>>>(
                       s, W, H, aux, p->cols, groups, gpr, vec, partial));
  else
    SF_DISPATCH_WH(w_dtype, h_dtype,
                   stats_partial_kernel<WD_, HD_, false, false><<<kStatsGrid, kBlock, 0, st>>>(
                       s, W, H, aux, p->cols, groups, gpr, vec, partial));
  stats_final_kernel<<<1, kBlock, 0, st>>>(partial, kStatsGrid, n, stats_out);
  return launch_status("sf_score_stats");
}

extern "C" int sf_sample_indices(int64_t* idx, int64_t sample_size, int64_t n, uint64_t seed, void* stream) {
  SF_CHECK_ARG(sample_size >= 0 && n > 0, "bad sample size %lld / n %lld", (long long)sample_size, (long long)n);
  if (sample_size == 0) return SF_OK;
  SF_CHECK_ARG(idx != nullptr, "null index tensor");
  hipStream_t st = static_cast<hipStream_t>(stream);
  sample_indices_kernel<<<elementwise_grid(sample_size, kBlock), kBlock, 0, st>>>(idx, sample_size,
                                                                                   static_cast<uint64_t>(n), seed);
  return launch_status("sf_sample_indices");
}

extern "C" size_t sf_sample_indices_sorted_workspace_size(int64_t sample_size, int count) {
  if (sample_size < 0 || count <= 0) return 0;
  return sizeof(uint64_t) * static_cast<size_t>(count) * static_cast<size_t>(ceil_div(sample_size + 1, kSortedChunk));
}

extern "C" int sf_sample_indices_sorted(int64_t* idx, int64_t sample_size, const int64_t* n, const uint64_t* seeds,
                                        int count, void* workspace, size_t workspace_bytes, void* stream) {
  SF_CHECK_ARG(sample_size >= 0 && count >= 0, "bad sample size %lld / count %d", (long long)sample_size, count);
  // below 2^28: the fixed-point sums stay far below 2^64 (S_m is about (m + 1) 2^32, one term at most
  // 37 2^32), and a list has at most 2^16 chunks, whose sums every workgroup of the index pass reads
  SF_CHECK_ARG(sample_size < (int64_t(1) << 28), "sample size %lld not below 2^28", (long long)sample_size);
  if (sample_size == 0 || count == 0) return SF_OK;
  SF_CHECK_ARG(idx && n && seeds, "null argument");
  for (int c = 0; c < count; ++c) SF_CHECK_ARG(n[c] > 0, "list %d: n = %lld", c, (long long)n[c]);
  SF_CHECK_ARG(workspace && workspace_bytes >= sf_sample_indices_sorted_workspace_size(sample_size, count),
               "workspace too small");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t chunks = ceil_div(sample_size + 1, kSortedChunk);
  uint64_t* sums = static_cast<uint64_t*>(workspace);
  for (int c0 = 0; c0 < count; c0 += kSortedLists) {
    const int k = count - c0 < kSortedLists ? count - c0 : kSortedLists;
    SortedSampleArgs a;
    memset(&a, 0, sizeof(a));
    a.idx = idx + static_cast<int64_t>(c0) * sample_size;
    a.m = sample_size;
    a.chunks = chunks;
    for (int c = 0; c < k; ++c) {
      a.seed[c] = seeds[c0 + c];
      a.n[c] = n[c0 + c];
    }
    const dim3 grid(static_cast<unsigned>(chunks), static_cast<unsigned>(k));
    sorted_sample_exp_kernel<<<grid, kBlock, 0, st>>>(a, sums + static_cast<int64_t>(c0) * chunks);
    sorted_sample_idx_kernel<<<grid, kBlock, 0, st>>>(a, sums + static_cast<int64_t>(c0) * chunks);
  }
  return launch_status("sf_sample_indices_sorted");
}

namespace sf {
namespace {
// Argument checks and launches of the tau selection, over a scratch region `ws`
// laid out as sf_mask_workspace_size describes (the caller's workspace, or the
// library's static scratch for sf_tau_quantile_noalloc).  Every scratch word a
// kernel reads was written earlier in the same call: nothing needs clearing.
int tau_quantile_checks(const sf_mask_params* p, const void* W, const void* H, const void* aux, const float* stats,
                        const int64_t* sample_idx, int64_t sample_size, float* tau_out) {
  if (int rc = check_common(p)) return rc;
  if (int rc = check_metric_operands(p, H, aux)) return rc;
  SF_CHECK_ARG(W && stats && tau_out, "null tensor");
  SF_CHECK_ARG(sample_size > 0, "empty tau sample");
  SF_CHECK_ARG(sample_idx || sample_size == p->rows * p->cols, "sample_size must equal numel without indices");
  return SF_OK;
}

int tau_quantile_launch(const sf_mask_params* p, const void* W, int w_dtype, const void* H, int h_dtype,
                        const void* aux, int aux_dtype, const float* stats, const int64_t* sample_idx,
                        int64_t sample_size, float q, float* tau_out, char* ws, hipStream_t st) {
  if (!H) h_dtype = SF_DTYPE_F32;
  ScoreSpec s = make_spec(p, w_dtype, h_dtype, aux_dtype);
  uint32_t* keys = reinterpret_cast<uint32_t*>(ws + ws_keys_off());
  SelState* states = reinterpret_cast<SelState*>(ws + ws_state_off());
  uint32_t* parts[2] = {reinterpret_cast<uint32_t*>(ws + ws_partial_off()),
                        reinterpret_cast<uint32_t*>(ws + ws_partial_off() + ws_partial_bytes())};
  tau_gather_kernel<<<elementwise_grid(sample_size, kBlock), kBlock, 0, st>>>(s, W, H, aux, p->rows, p->cols,
                                                                               sample_idx, sample_size, keys);
  // pass p reads state p-2 (slot p & 1) and partials p-1, writes state p-1 (slot (p + 1) & 1) and partials p
  const int grid = static_cast<int>(ceil_div(sample_size, kBlock) < kSelGrid ? ceil_div(sample_size, kBlock) : kSelGrid);
  for (int pass = 0; pass < 4; ++pass)
    tau_pass_kernel<<<grid, kBlock, 0, st>>>(keys, sample_size, pass, q, &states[pass & 1], &states[(pass + 1) & 1],
                                             parts[(pass + 1) & 1], parts[pass & 1]);
  tau_final_kernel<<<1, kBlock, 0, st>>>(sample_size, q, grid, &states[0], parts[1], stats, s.score_dtype, tau_out);
  return SF_OK;
}

// ---- static scratch of sf_tau_quantile_noalloc -------------------------------
// One copy per GPU, held until the process ends.  Host code never passes the
// array's name to a kernel: it is a host-side stand-in, and the device address
// of each GPU's copy comes from hipGetSymbolAddress with that GPU current.
// Same layout as a caller's workspace (sf_mask_workspace_size) at the largest sample it accepts.
constexpr size_t up256(size_t b) { return (b + 255) / 256 * 256; }
constexpr size_t kNoallocScratchBytes = up256(sizeof(double) * 2 * kStatsGrid) + up256(2 * sizeof(SelState)) +
                                        2 * up256(sizeof(uint32_t) * kSelStride * kSelGrid) +
                                        sizeof(uint32_t) * static_cast<size_t>(SF_TAU_NOALLOC_MAX_SAMPLE);
static __device__ __align__(256) unsigned char scratch[kNoallocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_lock;
char* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on `device` (resolved once per device, with that device current).
int scratch_on(int device, char** out) {
  SF_CHECK_ARG(device >= 0 && device < kMaxDevices, "device ordinal %d out of range", device);
  std::lock_guard<std::mutex> guard(g_scratch_lock);
  if (!g_scratch_ptr[device]) {
    int prev = -1;
    SF_CHECK_HIP(hipGetDevice(&prev));
    if (prev != device) SF_CHECK_HIP(hipSetDevice(device));
    void* addr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
    if (prev != device) SF_CHECK_HIP(hipSetDevice(prev));
    if (e != hipSuccess || !addr) {
      set_error("hipGetSymbolAddress(scratch) on device %d failed: %s", device, hipGetErrorString(e));
      return SF_ERR_HIP;
    }
    g_scratch_ptr[device] = static_cast<char*>(addr);
  }
  *out = g_scratch_ptr[device];
  return SF_OK;
}
}  // namespace
}  // namespace sf

extern "C" int sf_tau_quantile(const sf_mask_params* p, const void* W, int w_dtype, const void* H, int h_dtype,
                               const void* aux, int aux_dtype, const float* stats, const int64_t* sample_idx,
                               int64_t sample_size, float q, float* tau_out, void* workspace, size_t workspace_bytes,
                               void* stream) {
  if (int rc = tau_quantile_checks(p, W, H, aux, stats, sample_idx, sample_size, tau_out)) return rc;
  SF_CHECK_ARG(workspace && workspace_bytes >= sf_mask_workspace_size(p->rows, p->cols, sample_size),
               "workspace too small");
  tau_quantile_launch(p, W, w_dtype, H, h_dtype, aux, aux_dtype, stats, sample_idx, sample_size, q, tau_out,
                      static_cast<char*>(workspace), static_cast<hipStream_t>(stream));
  return launch_status("sf_tau_quantile");
}

extern "C" int sf_tau_quantile_noalloc(const sf_mask_params* p, const void* W, int w_dtype, const void* H,
                                       int h_dtype, const void* aux, int aux_dtype, const float* stats,
                                       const int64_t* sample_idx, int64_t sample_size, float q, float* tau_out,
                                       void* stream) {
  if (int rc = tau_quantile_checks(p, W, H, aux, stats, sample_idx, sample_size, tau_out)) return rc;
  SF_CHECK_ARG(sample_size <= SF_TAU_NOALLOC_MAX_SAMPLE,
               "sf_tau_quantile_noalloc: tau sample of %lld elements exceeds the static scratch maximum of %d "
               "(use sf_tau_quantile with a workspace)",
               (long long)sample_size, SF_TAU_NOALLOC_MAX_SAMPLE);
  hipStream_t st = static_cast<hipStream_t>(stream);
  int device = -1;
  if (st) {
    SF_CHECK_HIP(hipStreamGetDevice(st, &device));
  } else {
    SF_CHECK_HIP(hipGetDevice(&device));
  }
  char* ws = nullptr;
  if (int rc = scratch_on(device, &ws)) return rc;
  if (sf_mask_workspace_size(p->rows, p->cols, sample_size) > kNoallocScratchBytes) {
    set_error("sf_tau_quantile_noalloc: scratch layout exceeds the static array");
    return SF_ERR_INVALID;
  }
  tau_quantile_launch(p, W, w_dtype, H, h_dtype, aux, aux_dtype, stats, sample_idx, sample_size, q, tau_out, ws, st);
  return launch_status("sf_tau_quantile_noalloc");
}

namespace sf {
namespace {
int make_gate_spec(const sf_mask_params* p, int w_dtype, int h_dtype, int aux_dtype, int mask_dtype, int frozen_dtype,
                   GateSpec* gs) {
  SF_CHECK_ARG(p->gate >= SF_GATE_UNSTRUCTURED && p->gate <= SF_GATE_ZSCORE, "bad gate %d", p->gate);
  SF_CHECK_ARG(p->gate != SF_GATE_ZSCORE || (p->beta_struct == 0.0f && !p->has_frozen),
               "the z-score output takes no beta mix and no frozen override");
  if ((p->gate != SF_GATE_UNSTRUCTURED && p->gate != SF_GATE_ZSCORE) || p->beta_struct > 0.0f) {
    if (p->m_group != 4 || p->n_keep < 1 || p->n_keep > 3) {
      set_error("structured gate with N=%d M=%d: only M=4 is built on device", p->n_keep, p->m_group);
      return SF_ERR_UNSUPPORTED;
    }
  }
  if (p->gate == SF_GATE_STRUCTURED || p->gate == SF_GATE_STRUCTURED_EXACT)
    SF_CHECK_ARG(p->cols % p->m_group == 0, "in_features (%lld) must be divisible by M (%d).", (long long)p->cols,
                 p->m_group);
  gs->s = make_spec(p, w_dtype, h_dtype, aux_dtype);
  gs->gate = p->gate;
  gs->n_keep = p->n_keep;
  gs->has_frozen = p->has_frozen;
  gs->mask_dtype = mask_dtype;
  gs->frozen_dtype = frozen_dtype;
  gs->denom = p->temperature + 1e-8f;
  gs->rdenom = 1.0f / gs->denom;  // IEEE f32 division on the host: correctly rounded
  gs->beta_struct = p->beta_struct;
  gs->one_minus_beta = static_cast<float>(1.0 - static_cast<double>(p->beta_struct));
  return SF_OK;
}
// Scalars of the fused update (penalty, binarisation, EMA, freeze, flip view) from the host params.
int make_update_spec(const sf_mask_params* p, int w_dtype, int h_dtype, int aux_dtype, int mask_dtype,
                     int frozen_dtype, bool want_flips, UpdateSpec* us) {
  if (int rc = make_gate_spec(p, w_dtype, h_dtype, aux_dtype, mask_dtype, frozen_dtype, &us->gs)) return rc;
  us->penalty = p->penalty_coef != 0.0f ? p->penalty : SF_PENALTY_NONE;
  us->pen_n = p->n_keep;
  if (us->penalty == SF_PENALTY_NM_2_4) us->pen_n = 2;
  if (us->penalty == SF_PENALTY_NM_2_4 || us->penalty == SF_PENALTY_STRUCTURED_TOPN) {
    if (us->penalty == SF_PENALTY_STRUCTURED_TOPN && (p->m_group != 4 || p->n_keep < 1 || p->n_keep > 3)) {
      set_error("structured_topn penalty with N=%d M=%d: only M=4 is built on device", p->n_keep, p->m_group);
      return SF_ERR_UNSUPPORTED;
    }
    SF_CHECK_ARG(us->penalty != SF_PENALTY_STRUCTURED_TOPN || p->cols % 4 == 0,
                 "structured_topn penalty needs cols % M == 0 (the caller falls back to mid)");
  }
  us->pen_coef = p->penalty_coef;
  us->binarize = p->binarize != 0.0f;
  us->bin_lo = static_cast<float>(1.0 - static_cast<double>(p->binarize));
  us->bin_hi = static_cast<float>(1.0 + static_cast<double>(p->binarize));
  us->keep_a = static_cast<float>(1.0 - static_cast<double>(p->mask_lr));
  // torch converts add_'s alpha to the op's dtype: bf16 when mask and G are both bf16
  us->a = (mask_dtype == SF_DTYPE_BF16 && p->score_dtype == SF_DTYPE_BF16) ? round_bf16(p->mask_lr) : p->mask_lr;
  us->apply_freeze = p->apply_freeze;
  us->snap_high = p->snap_high;
  us->freeze_low = p->freeze_low;
  us->freeze_high = p->freeze_high;
  us->hard_kind = p->hard_kind;
  us->hard_n = p->hard_n;
  if (p->hard_kind >= SF_HARD_NM_TAIL_KEEP && want_flips) {
    if (p->hard_m != 4 || p->hard_n < 1 || p->hard_n > 3) {
      set_error("flip count with N=%d M=%d: only M=4 is built on device", p->hard_n, p->hard_m);
      return SF_ERR_UNSUPPORTED;
    }
    SF_CHECK_ARG(p->hard_kind != SF_HARD_NM_STRICT || p->cols % 4 == 0,
                 "in_features (%lld) must be divisible by M (%d).", (long long)p->cols, p->hard_m);
  }
  return SF_OK;
}
}  // namespace
}  // namespace sf

extern "C" int sf_gate_target(const sf_mask_params* p, const void* W, int w_dtype, const void* H, int h_dtype,
                              const void* aux, int aux_dtype, const void* mask, int mask_dtype, const void* frozen,
                              int frozen_dtype, const float* stats, const float* tau, void* G, int g_dtype,
                              void* stream) {
  if (int rc = check_common(p)) return rc;
  if (int rc = check_metric_operands(p, H, aux)) return rc;
  SF_CHECK_ARG(W && stats && G, "null tensor");
  SF_CHECK_ARG(dtype_ok(w_dtype) && dtype_ok(g_dtype), "bad dtype");
  SF_CHECK_ARG(p->gate != SF_GATE_UNSTRUCTURED || tau != nullptr, "unstructured gate needs tau");
  SF_CHECK_ARG(!p->has_frozen || (frozen && mask), "frozen override needs mask and frozen flags");
  if (!H) h_dtype = SF_DTYPE_F32;
  GateSpec gs;
  if (int rc = make_gate_spec(p, w_dtype, h_dtype, aux_dtype, mask_dtype, frozen_dtype, &gs)) return rc;
  if (p->rows == 0 || p->cols == 0) return SF_OK;
  const int64_t gpr = ceil_div(p->cols, 4), groups = p->rows * gpr;
  const bool vec = vec_ok(p->cols, {{W, w_dtype}, {H, h_dtype}, {G, g_dtype}, {mask, mask_dtype},
                                    {p->has_frozen ? frozen : nullptr, frozen_dtype}}) &&
                   (!aux || aligned(aux, 4 * esize(aux_dtype)));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int grid = elementwise_grid(groups, kBlock);
  if (p->score_dtype == SF_DTYPE_F32)
    SF_DISPATCH_WH(w_dtype, h_dtype,
                   gate_target_kernel<WD_, HD_, SF_DTYPE_F32><<<grid, kBlock, 0, st>>>(
                       gs, W, H, aux, mask, frozen, stats, tau, G, g_dtype, p->cols, groups, gpr, vec));
  else
    SF_DISPATCH_WH(w_dtype, h_dtype,
                   gate_target_kernel<WD_, HD_, SF_DTYPE_BF16><<<grid, kBlock, 0, st>>>(
                       gs, W, H, aux, mask, frozen, stats, tau, G, g_dtype, p->cols, groups, gpr, vec));
  return launch_status("sf_gate_target");
}

extern "C" int sf_update_mask(const sf_mask_params* p, const void* W, int w_dtype, const void* H, int h_dtype,
                              const void* aux, int aux_dtype, void* mask, int mask_dtype, void* frozen,
                              int frozen_dtype, const float* stats, const float* tau, int64_t* flips, void* stream) {
  if (int rc = check_common(p)) return rc;
  if (int rc = check_metric_operands(p, H, aux)) return rc;
  SF_CHECK_ARG(W && stats && mask, "null tensor");
  SF_CHECK_ARG(dtype_ok(w_dtype) && dtype_ok(mask_dtype), "bad dtype");
  SF_CHECK_ARG(p->gate != SF_GATE_UNSTRUCTURED || tau != nullptr, "unstructured gate needs tau");
  SF_CHECK_ARG(!p->has_frozen || frozen, "has_frozen without frozen flags");
  SF_CHECK_ARG(p->penalty >= SF_PENALTY_NONE && p->penalty <= SF_PENALTY_STRUCTURED_TOPN, "bad penalty %d", p->penalty);
  SF_CHECK_ARG(p->hard_kind >= SF_HARD_NONE && p->hard_kind <= SF_HARD_NM_STRICT, "bad hard kind %d", p->hard_kind);
  SF_CHECK_ARG(p->gate != SF_GATE_ZSCORE, "the z-score gate form is an output of sf_gate_target only");
  if (!H) h_dtype = SF_DTYPE_F32;
  UpdateSpec us;
  if (int rc = make_update_spec(p, w_dtype, h_dtype, aux_dtype, mask_dtype, frozen_dtype, flips != nullptr, &us))
    return rc;
  if (p->rows == 0 || p->cols == 0) return SF_OK;
  const int64_t gpr = ceil_div(p->cols, 4), groups = p->rows * gpr;
  const bool vec = vec_ok(p->cols, {{W, w_dtype}, {H, h_dtype}, {mask, mask_dtype},
                                    {p->has_frozen ? frozen : nullptr, frozen_dtype}}) &&
                   (!aux || aligned(aux, 4 * esize(aux_dtype)));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int grid = update_grid(groups);
#define SF_LAUNCH_UPD_V(MDT, SDT, VEC, FAST)                                                                \
  SF_DISPATCH_WH(w_dtype, h_dtype,                                                                          \
                 update_mask_kernel<WD_, HD_, MDT, SDT, VEC, FAST><<<grid, kBlock, 0, st>>>(                \
                     us, W, H, aux, mask, frozen, stats, tau, p->cols, groups, gpr, vec, flips))
#define SF_LAUNCH_UPD(MDT, SDT)                                                                             \
  do {                                                                                                      \
    if (vec)                                                                                                \
      SF_LAUNCH_UPD_V(MDT, SDT, true, kFastNone);                                                           \
    else                                                                                                    \
      SF_LAUNCH_UPD_V(MDT, SDT, false, kFastNone);                                                          \
  } while (0)
  const bool sf32 = p->score_dtype == SF_DTYPE_F32;
  const int fk = vec ? fast_kind(us) : kFastNone;
  if (mask_dtype == SF_DTYPE_F32) {
    if (sf32 && fk == kFastPlain)
      SF_LAUNCH_UPD_V(SF_DTYPE_F32, SF_DTYPE_F32, true, kFastPlain);
    else if (sf32 && fk == kFastNm24)
      SF_LAUNCH_UPD_V(SF_DTYPE_F32, SF_DTYPE_F32, true, kFastNm24);
    else if (sf32)
      SF_LAUNCH_UPD(SF_DTYPE_F32, SF_DTYPE_F32);
    else
      SF_LAUNCH_UPD(SF_DTYPE_F32, SF_DTYPE_BF16);
  } else {
    if (sf32)
      SF_LAUNCH_UPD(SF_DTYPE_BF16, SF_DTYPE_F32);
    else
      SF_LAUNCH_UPD(SF_DTYPE_BF16, SF_DTYPE_BF16);
  }
#undef SF_LAUNCH_UPD
#undef SF_LAUNCH_UPD_V
  return launch_status("sf_update_mask");
}

namespace sf {
namespace {
// Multi-layer workspace: [stats partials | select states | 2 x partial histograms | keys], per batch of
// kMultiLayers layers (the batches run one after another on the stream and reuse it).
size_t multi_partial_bytes() { return align256(sizeof(double) * 2 * kStatsGrid * kMultiLayers); }
size_t multi_states_bytes() { return align256(sizeof(SelState) * 2 * kMultiLayers); }
size_t multi_hist_bytes() { return align256(sizeof(uint32_t) * kSelStride * kSelGrid * kMultiLayers); }
size_t multi_keys_off() { return multi_partial_bytes() + multi_states_bytes() + 2 * multi_hist_bytes(); }
size_t multi_ok_bytes() { return align256(sizeof(int32_t) * kWinGrid * kMultiLayers); }
// window starts of a layer's sample for the statistics fold (windows + 1 entries)
int64_t layer_window_starts(const sf_mask_layer& l) {
  return ((l.rows * l.cols + (1 << kWinShift) - 1) >> kWinShift) + 1;
}

bool layer_empty(const sf_mask_layer& l) { return l.rows == 0 || l.cols == 0; }

// Calls f(first, end, keys) for each batch: up to kMultiLayers non-empty layers of [first, end), and the
// keys their tau samples need.
template <typename F>
void for_each_batch(const sf_mask_layer* layers, int count, F&& f) {
  int i = 0;
  while (i < count) {
    while (i < count && layer_empty(layers[i])) ++i;
    if (i == count) break;
    const int first = i;
    int taken = 0;
    int64_t keys = 0;
    while (i < count && taken < kMultiLayers) {
      if (!layer_empty(layers[i])) {
        keys += layers[i].sample_size;
        ++taken;
      }
      ++i;
    }
    f(first, i, keys);
  }
}

// Workspace of sf_update_mask_multi.  Serial layout: [stats partials | select states | radix partials x 2 |
// keys | sample window starts | sample order flags].  The pipelined schedule (below) appends a second
// stats-partials region and a second keys region,
// so that batch b + 1's statistics and tau gather never write what batch b's selection still reads.  It is
// offered only while a batch's sample keys stay below kOverlapMaxKeys (a tau sample over every element of
// large layers would double a workspace of gigabytes).
constexpr int64_t kOverlapMaxKeys = int64_t(1) << 25;
struct MultiSizes {
  int64_t keys = 0;  // largest batch's sample keys
  int64_t wins = 0;  // largest batch's window starts (layers with sample indices)
  int batches = 0;
  size_t serial_bytes = 0, overlap_bytes = 0, keys1_off = 0, partial1_off = 0, wins_off = 0, ok_off = 0;
};
MultiSizes multi_sizes(const sf_mask_layer* layers, int count) {
  MultiSizes z;
  if (layers && count > 0)
    for_each_batch(layers, count, [&](int first, int end, int64_t k) {
      z.keys = k > z.keys ? k : z.keys;
      int64_t wn = 0;
      for (int i = first; i < end; ++i)
        if (!layer_empty(layers[i]) && layers[i].sample_idx) wn += layer_window_starts(layers[i]);
      z.wins = wn > z.wins ? wn : z.wins;
      ++z.batches;
    });
  const size_t kb = sizeof(uint32_t) * static_cast<size_t>(z.keys);
  z.wins_off = align256(multi_keys_off() + kb);
  z.ok_off = z.wins_off + align256(sizeof(int32_t) * static_cast<size_t>(z.wins));
  z.serial_bytes = z.ok_off + multi_ok_bytes();
  z.partial1_off = align256(z.serial_bytes);
  z.keys1_off = z.partial1_off + multi_partial_bytes();
  z.overlap_bytes = z.keys1_off + kb;
  return z;
}

// Second stream of the pipelined multi-layer update, one per GPU, and its events (two per batch), created
// on first use with that GPU current and held until the process ends.  The lock is held while a call
// enqueues its work, so calls from several host threads never share an event in flight.
struct SideStream {
  hipStream_t stream = nullptr;
  std::vector<hipEvent_t> ev;
};
std::mutex g_side_lock;
SideStream g_side[64];

int side_stream(int device, size_t events, SideStream** out) {
  SF_CHECK_ARG(device >= 0 && device < 64, "device ordinal %d out of range", device);
  SideStream& ss = g_side[device];
  if (!ss.stream) SF_CHECK_HIP(hipStreamCreateWithFlags(&ss.stream, hipStreamNonBlocking));
  while (ss.ev.size() < events) {
    hipEvent_t e;
    SF_CHECK_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    ss.ev.push_back(e);
  }
  *out = &ss;
  return SF_OK;
}
}  // namespace
}  // namespace sf

extern "C" size_t sf_update_mask_multi_workspace_size(const sf_mask_layer* layers, int count) {
  const MultiSizes z = multi_sizes(layers, count);
  return z.batches > 1 && z.keys <= kOverlapMaxKeys ? z.overlap_bytes : z.serial_bytes;
}

extern "C" int sf_update_mask_multi(const sf_mask_params* p, float q, const sf_mask_layer* layers, int count,
                                    int stages, int w_dtype, int h_dtype, int aux_dtype, int mask_dtype,
                                    int frozen_dtype, void* workspace, size_t workspace_bytes, void* stream) {
  if (int rc = check_common(p)) return rc;
  SF_CHECK_ARG(count >= 0 && (count == 0 || layers), "bad layer table (count %d)", count);
  SF_CHECK_ARG(stages > 0 && (stages & ~SF_MULTI_ALL) == 0, "bad stage mask %d", stages);
  SF_CHECK_ARG(dtype_ok(w_dtype) && dtype_ok(mask_dtype), "bad dtype");
  SF_CHECK_ARG(p->penalty >= SF_PENALTY_NONE && p->penalty <= SF_PENALTY_STRUCTURED_TOPN, "bad penalty %d", p->penalty);
  SF_CHECK_ARG(p->hard_kind >= SF_HARD_NONE && p->hard_kind <= SF_HARD_NM_STRICT, "bad hard kind %d", p->hard_kind);
  SF_CHECK_ARG(p->gate != SF_GATE_ZSCORE, "the z-score gate form is an output of sf_gate_target only");
  const bool unstructured = p->gate == SF_GATE_UNSTRUCTURED;
  bool any_h = false, any_aux = false, any_flips = false;
  for (int i = 0; i < count; ++i) {
    const sf_mask_layer& l = layers[i];
    SF_CHECK_ARG(l.rows >= 0 && l.cols >= 0, "layer %d: negative shape", i);
    if (layer_empty(l)) continue;
    if (int rc = check_metric_operands(p, l.H, l.aux)) return rc;
    SF_CHECK_ARG(l.W && l.mask && l.stats, "layer %d: null tensor", i);
    SF_CHECK_ARG(!unstructured || l.tau, "layer %d: unstructured gate needs tau", i);
    SF_CHECK_ARG(!p->has_frozen || l.frozen, "layer %d: has_frozen without frozen flags", i);
    if (unstructured) {
      SF_CHECK_ARG(l.sample_size > 0, "layer %d: empty tau sample", i);
      SF_CHECK_ARG(l.sample_idx || l.sample_size == l.rows * l.cols,
                   "layer %d: sample_size must equal numel without indices", i);
    }
    any_h = any_h || l.H;
    any_aux = any_aux || l.aux;
    any_flips = any_flips || l.flips;
  }
  SF_CHECK_ARG(!any_h || dtype_ok(h_dtype), "bad hessian dtype");
  SF_CHECK_ARG(!any_aux || dtype_ok(aux_dtype), "bad aux dtype");
  if (!any_h) h_dtype = SF_DTYPE_F32;
  // every layer's shape passes the single-layer checks; the spec itself does not depend on the shape
  UpdateSpec us;
  bool have_spec = false;
  for (int i = 0; i < count; ++i) {
    if (layer_empty(layers[i])) continue;
    sf_mask_params pl = *p;
    pl.rows = layers[i].rows;
    pl.cols = layers[i].cols;
    if (int rc = make_update_spec(&pl, w_dtype, h_dtype, aux_dtype, mask_dtype, frozen_dtype, any_flips, &us))
      return rc;
    have_spec = true;
  }
  if (!have_spec) return SF_OK;
  const MultiSizes z = multi_sizes(layers, count);
  SF_CHECK_ARG(workspace && workspace_bytes >= z.serial_bytes, "workspace too small");
  char* ws = static_cast<char*>(workspace);
  SelState* states = reinterpret_cast<SelState*>(ws + multi_partial_bytes());
  uint32_t* parts0 = reinterpret_cast<uint32_t*>(ws + multi_partial_bytes() + multi_states_bytes());
  uint32_t* parts1 = reinterpret_cast<uint32_t*>(ws + multi_partial_bytes() + multi_states_bytes() + multi_hist_bytes());
  // statistics partials and tau keys: region 0, and region 1 for odd batches of the pipelined schedule
  double* partial_r[2] = {reinterpret_cast<double*>(ws), reinterpret_cast<double*>(ws + z.partial1_off)};
  uint32_t* keys_r[2] = {reinterpret_cast<uint32_t*>(ws + multi_keys_off()),
                         reinterpret_cast<uint32_t*>(ws + z.keys1_off)};
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool sf32 = p->score_dtype == SF_DTYPE_F32;

  // the batches' layer tables and launch shapes
  struct Batch {
    MultiArgs a;
    int n, total, gather_grid;
    bool all_vec, any_idx, fold;
  };
  std::vector<Batch> batches;
  batches.reserve(static_cast<size_t>(z.batches));
  for_each_batch(layers, count, [&](int first, int end, int64_t) {
    batches.emplace_back();
    Batch& bt = batches.back();
    MultiArgs& a = bt.a;
    memset(&a, 0, sizeof(a));
    a.us = us;
    int n = 0, gather_grid = 1;
    bool all_vec = true, any_idx = false, fold_ok = true;
    int64_t koff = 0, woff = 0;
    a.first[0] = 0;
    for (int i = first; i < end; ++i) {
      const sf_mask_layer& l = layers[i];
      if (layer_empty(l)) continue;
      MultiLayer& L = a.l[n];
      L.W = l.W;
      L.H = l.H;
      L.aux = l.aux;
      L.mask = l.mask;
      L.frozen = l.frozen;
      L.stats = l.stats;
      L.tau = l.tau;
      L.flips = l.flips;
      L.idx = l.sample_idx;
      L.rows = l.rows;
      L.cols = l.cols;
      const int64_t groups = l.rows * ceil_div(l.cols, 4);
      L.nblk = update_grid(groups);
      // the single-layer update's vector test (it implies the statistics' one)
      L.vec = vec_ok(l.cols, {{l.W, w_dtype}, {l.H, h_dtype}, {l.mask, mask_dtype},
                              {p->has_frozen ? l.frozen : nullptr, frozen_dtype}}) &&
              (!l.aux || aligned(l.aux, 4 * esize(aux_dtype)));
      all_vec = all_vec && L.vec;
      if (unstructured) {
        L.m = l.sample_size;
        L.nsel = static_cast<int32_t>(ceil_div(l.sample_size, kBlock) < kSelGrid ? ceil_div(l.sample_size, kBlock)
                                                                                   : kSelGrid);
        L.keys_off = koff;
        koff += l.sample_size;
        const int gg = elementwise_grid(l.sample_size, kBlock);
        gather_grid = gg > gather_grid ? gg : gather_grid;
        // the fold keeps sample positions and window starts in int32
        fold_ok = fold_ok && l.sample_size <= INT32_MAX;
        if (l.sample_idx) {
          any_idx = true;
          L.win_off = static_cast<int32_t>(woff);
          woff += layer_window_starts(l);
        }
      }
      a.first[n + 1] = a.first[n] + L.nblk;
      ++n;
    }
    a.count = n;
    bt.n = n;
    bt.total = a.first[n];
    bt.gather_grid = gather_grid;
    bt.all_vec = all_vec;
    bt.any_idx = any_idx;
    bt.fold = all_vec && fold_ok && woff <= INT32_MAX && p->metric == SF_METRIC_HESSIAN_RATIO;
  });

  const bool want_tau = unstructured && (stages & SF_MULTI_TAU);
  // the tau gather rides in the statistics launch when both stages run
  const bool fused_gather = want_tau && (stages & SF_MULTI_STATS);
  int32_t* wins = reinterpret_cast<int32_t*>(ws + z.wins_off);
  int32_t* okf = reinterpret_cast<int32_t*>(ws + z.ok_off);
  auto launch_stats = [&](const Batch& bt, double* partial, uint32_t* keys) {
    const MultiArgs& a = bt.a;
    if (fused_gather && bt.fold) {
      // the tau sample's keys from the statistics pass itself (sorted samples; others gathered beside it)
      if (bt.any_idx) {
        sample_order_multi_kernel<<<dim3(kWinGrid, bt.n), kBlock, 0, st>>>(a, okf);
        sample_windows_multi_kernel<<<dim3(kWinGrid, bt.n), kBlock, 0, st>>>(a, okf, wins, keys);
      }
      SF_DISPATCH_WH(w_dtype, h_dtype,
                     stats_fold_multi_kernel<WD_, HD_><<<bt.n * kStatsGrid, kBlock, 0, st>>>(a, partial, keys, wins));
      return;
    }
    const int g = fused_gather ? bt.gather_grid : 0;
    const int grid = bt.n * g + bt.n * kStatsGrid;
    if (bt.all_vec && p->metric == SF_METRIC_HESSIAN_RATIO)
      SF_DISPATCH_WH(w_dtype, h_dtype,
                     stats_partial_multi_kernel<WD_, HD_, true, true><<<grid, kBlock, 0, st>>>(a, partial, g, keys));
    else if (bt.all_vec)
      SF_DISPATCH_WH(w_dtype, h_dtype,
                     stats_partial_multi_kernel<WD_, HD_, true, false><<<grid, kBlock, 0, st>>>(a, partial, g, keys));
    else
      SF_DISPATCH_WH(w_dtype, h_dtype,
                     stats_partial_multi_kernel<WD_, HD_, false, false><<<grid, kBlock, 0, st>>>(a, partial, g,
                                                                                                 keys));
  };
  auto launch_tau = [&](const Batch& bt, uint32_t* keys, hipStream_t s) {
    const MultiArgs& a = bt.a;
    if (!fused_gather) tau_gather_multi_kernel<<<dim3(bt.gather_grid, bt.n), kBlock, 0, s>>>(a, keys);
    for (int pass = 0; pass < 4; ++pass)
      tau_pass_multi_kernel<<<dim3(kSelGrid, bt.n), kBlock, 0, s>>>(a, keys, pass, q, states, parts0, parts1);
    tau_final_multi_kernel<<<bt.n, kBlock, 0, s>>>(a, q, states, parts1);
  };
  auto launch_update = [&](const Batch& bt) {
    const MultiArgs& a = bt.a;
    const int total = bt.total;
    const bool all_vec = bt.all_vec;
#define SF_LAUNCH_UPDM_V(MDT, SDT, VEC, FAST) \
  SF_DISPATCH_WH(w_dtype, h_dtype, update_mask_multi_kernel<WD_, HD_, MDT, SDT, VEC, FAST><<<total, kBlock, 0, st>>>(a))
#define SF_LAUNCH_UPDM(MDT, SDT)                            \
  do {                                                      \
    if (all_vec)                                            \
      SF_LAUNCH_UPDM_V(MDT, SDT, true, kFastNone);          \
    else                                                    \
      SF_LAUNCH_UPDM_V(MDT, SDT, false, kFastNone);         \
  } while (0)
    const int fk = all_vec ? fast_kind(us) : kFastNone;
    if (mask_dtype == SF_DTYPE_F32) {
      if (sf32 && fk == kFastPlain)
        SF_LAUNCH_UPDM_V(SF_DTYPE_F32, SF_DTYPE_F32, true, kFastPlain);
      else if (sf32 && fk == kFastNm24)
        SF_LAUNCH_UPDM_V(SF_DTYPE_F32, SF_DTYPE_F32, true, kFastNm24);
      else if (sf32)
        SF_LAUNCH_UPDM(SF_DTYPE_F32, SF_DTYPE_F32);
      else
        SF_LAUNCH_UPDM(SF_DTYPE_F32, SF_DTYPE_BF16);
    } else {
      if (sf32)
        SF_LAUNCH_UPDM(SF_DTYPE_BF16, SF_DTYPE_F32);
      else
        SF_LAUNCH_UPDM(SF_DTYPE_BF16, SF_DTYPE_BF16);
    }
#undef SF_LAUNCH_UPDM
#undef SF_LAUNCH_UPDM_V
  };
  auto launched = [&]() {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
      set_error("sf_update_mask_multi: launch failed: %s", hipGetErrorString(e));
      return SF_ERR_HIP;
    }
    return SF_OK;
  };

  const int nb = static_cast<int>(batches.size());
  const bool pipelined = stages == SF_MULTI_ALL && unstructured && nb > 1 && z.keys <= kOverlapMaxKeys &&
                         workspace_bytes >= z.overlap_bytes;
  if (!pipelined) {
    // serial: each batch's statistics, tau selection and update in turn, on the caller's stream
    for (const Batch& bt : batches) {
      if (stages & SF_MULTI_STATS) {
        launch_stats(bt, partial_r[0], keys_r[0]);
        stats_final_multi_kernel<<<bt.n, kBlock, 0, st>>>(bt.a, partial_r[0]);
      }
      if (want_tau) launch_tau(bt, keys_r[0], st);
      if (stages & SF_MULTI_UPDATE) launch_update(bt);
      if (int rc = launched()) return rc;
    }
    return launch_status("sf_update_mask_multi");
  }

  // Pipelined: the statistics (with the tau gather) and the updates run in order on the caller's stream,
  // S0 S1 U0 S2 U1 ... S(n-1) U(n-2) U(n-1); batch b's statistics fold and radix selection (a few small
  // launches) run on the side stream once S(b) is done, beside S(b + 1), and U(b) waits for them.
  // S(b + 2) reuses batch b's regions only after U(b), hence after batch b's selection.  The same
  // kernels as the serial schedule, on the same data, so every output is identical.
  int device = -1;
  SF_CHECK_HIP(hipGetDevice(&device));
  std::lock_guard<std::mutex> guard(g_side_lock);
  SideStream* side = nullptr;
  if (int rc = side_stream(device, 2 * static_cast<size_t>(nb), &side)) return rc;
  hipStream_t ss = side->stream;
  for (int b = 0; b <= nb; ++b) {
    if (b < nb) {
      const Batch& bt = batches[b];
      double* partial = partial_r[b & 1];
      uint32_t* keys = keys_r[b & 1];
      launch_stats(bt, partial, keys);
      SF_CHECK_HIP(hipEventRecord(side->ev[2 * b], st));
      SF_CHECK_HIP(hipStreamWaitEvent(ss, side->ev[2 * b], 0));
      stats_final_multi_kernel<<<bt.n, kBlock, 0, ss>>>(bt.a, partial);
      launch_tau(bt, keys, ss);
      SF_CHECK_HIP(hipEventRecord(side->ev[2 * b + 1], ss));
    }
    if (b >= 1) {
      SF_CHECK_HIP(hipStreamWaitEvent(st, side->ev[2 * (b - 1) + 1], 0));
      launch_update(batches[b - 1]);
    }
    if (int rc = launched()) return rc;
  }
  return launch_status("sf_update_mask_multi");
}

extern "C" int sf_importance_scores(const sf_mask_params* p, const void* W, int w_dtype, const void* H, int h_dtype,
                                    const void* aux, int aux_dtype, void* S, int s_dtype, void* stream) {
  if (int rc = check_common(p)) return rc;
  if (int rc = check_metric_operands(p, H, aux)) return rc;
  SF_CHECK_ARG(dtype_ok(w_dtype) && dtype_ok(s_dtype), "bad dtype");
  SF_CHECK_ARG(!H || dtype_ok(h_dtype), "bad hessian dtype");
  SF_CHECK_ARG(!aux || dtype_ok(aux_dtype), "bad aux dtype");
  if (p->rows == 0 || p->cols == 0) return SF_OK;
  SF_CHECK_ARG(W && S, "null tensor");
  if (!H) h_dtype = SF_DTYPE_F32;
  const ScoreSpec sp = make_spec(p, w_dtype, h_dtype, aux_dtype);
  const int64_t cols = p->cols, gpr = ceil_div(cols, 4), groups = p->rows * gpr;
  const bool vec = vec_ok(cols, {{W, w_dtype}, {H, h_dtype}, {aux, aux_dtype}, {S, s_dtype}});
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int grid = elementwise_grid(groups, kBlock);
  SF_DISPATCH_WH(w_dtype, h_dtype,
                 importance_scores_kernel<WD_, HD_><<<grid, kBlock, 0, st>>>(sp, W, H, aux, S, s_dtype, cols, groups,
                                                                             gpr, vec));
  return launch_status("sf_importance_scores");
}

extern "C" int sf_joint_scores(const sf_mask_params* gate_p, const void* gate_W, const void* gate_H,
                               const void* gate_aux, const sf_mask_params* up_p, const void* up_W, const void* up_H,
                               const void* up_aux, int w_dtype, int h_dtype, int aux_dtype, void* S, int s_dtype,
                               void* stream) {
  if (int rc = check_common(gate_p)) return rc;
  if (int rc = check_common(up_p)) return rc;
  if (int rc = check_metric_operands(gate_p, gate_H, gate_aux)) return rc;
  if (int rc = check_metric_operands(up_p, up_H, up_aux)) return rc;
  SF_CHECK_ARG(gate_p->rows == up_p->rows && gate_p->cols == up_p->cols, "gate and up shapes differ");
  SF_CHECK_ARG(dtype_ok(w_dtype) && dtype_ok(s_dtype), "bad dtype");
  SF_CHECK_ARG((!gate_H && !up_H) || dtype_ok(h_dtype), "bad hessian dtype");
  SF_CHECK_ARG((!gate_aux && !up_aux) || dtype_ok(aux_dtype), "bad aux dtype");
  if (gate_p->rows == 0 || gate_p->cols == 0) return SF_OK;
  SF_CHECK_ARG(gate_W && up_W && S, "null tensor");
  if (!gate_H && !up_H) h_dtype = SF_DTYPE_F32;
  const ScoreSpec sg = make_spec(gate_p, w_dtype, h_dtype, aux_dtype);
  const ScoreSpec su = make_spec(up_p, w_dtype, h_dtype, aux_dtype);
  const int64_t cols = gate_p->cols, gpr = ceil_div(cols, 4), groups = gate_p->rows * gpr;
  const bool vec = vec_ok(cols, {{gate_W, w_dtype}, {up_W, w_dtype}, {gate_H, h_dtype}, {up_H, h_dtype},
                                 {gate_aux, aux_dtype}, {up_aux, aux_dtype}, {S, s_dtype}});
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int grid = elementwise_grid(groups, kBlock);
  SF_DISPATCH_WH(w_dtype, h_dtype,
                 joint_scores_kernel<WD_, HD_><<<grid, kBlock, 0, st>>>(sg, gate_W, gate_H, gate_aux, su, up_W, up_H,
                                                                       up_aux, S, s_dtype, cols, groups, gpr, vec));
  return launch_status("sf_joint_scores");
}

extern "C" int sf_glu_update_masks(const sf_mask_params* p, const void* S, int s_dtype, void* gate_mask,
                                   void* up_mask, int mask_dtype, const void* gate_frozen, int frozen_dtype,
                                   const float* stats, const float* tau, int up_hard_kind, int up_hard_n,
                                   int64_t* gate_flips, int64_t* up_flips, void* stream) {
  if (int rc = check_common(p)) return rc;
  SF_CHECK_ARG(S && stats && gate_mask && up_mask, "null tensor");
  SF_CHECK_ARG(dtype_ok(s_dtype) && dtype_ok(mask_dtype), "bad dtype");
  SF_CHECK_ARG(p->score_dtype == mask_dtype, "the joint target lives in the mask dtype (score_dtype must equal it)");
  SF_CHECK_ARG(p->gate != SF_GATE_UNSTRUCTURED || tau != nullptr, "unstructured gate needs tau");
  SF_CHECK_ARG(!p->has_frozen || (gate_frozen && dtype_ok(frozen_dtype)), "has_frozen without frozen flags");
  SF_CHECK_ARG(p->penalty >= SF_PENALTY_NONE && p->penalty <= SF_PENALTY_STRUCTURED_TOPN && p->penalty != SF_PENALTY_NM_2_4,
               "the joint update pulls with the mid or structured_topn penalty only (got %d)", p->penalty);
  SF_CHECK_ARG(p->hard_kind >= SF_HARD_NONE && p->hard_kind <= SF_HARD_NM_STRICT, "bad hard kind %d", p->hard_kind);
  SF_CHECK_ARG(p->gate != SF_GATE_ZSCORE, "the z-score gate form is an output of sf_gate_target only");
  SF_CHECK_ARG(up_hard_kind >= SF_HARD_NONE && up_hard_kind <= SF_HARD_NM_STRICT, "bad hard kind %d", up_hard_kind);
  if (up_hard_kind >= SF_HARD_NM_TAIL_KEEP && up_flips) {
    if (up_hard_n < 1 || up_hard_n > 3) {
      set_error("flip count with N=%d: only M=4, 1<=N<=3 is built on device", up_hard_n);
      return SF_ERR_UNSUPPORTED;
    }
    SF_CHECK_ARG(up_hard_kind != SF_HARD_NM_STRICT || p->cols % 4 == 0, "in_features (%lld) must be divisible by M.",
                 (long long)p->cols);
  }
  UpdateSpec us;
  if (int rc = make_update_spec(p, s_dtype, s_dtype, SF_DTYPE_F32, mask_dtype, frozen_dtype, gate_flips != nullptr, &us))
    return rc;
  us.apply_freeze = 0;  // the joint update has no freeze step (:446-479)
  if (p->rows == 0 || p->cols == 0) return SF_OK;
  const int64_t gpr = ceil_div(p->cols, 4), groups = p->rows * gpr;
  const bool vec = vec_ok(p->cols, {{S, s_dtype}, {gate_mask, mask_dtype}, {up_mask, mask_dtype},
                                    {p->has_frozen ? gate_frozen : nullptr, frozen_dtype}});
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int grid = elementwise_grid(groups, kBlock);
#define SF_LAUNCH_GLU(SDT, MDT)                                                                                  \
  glu_update_kernel<SDT, MDT><<<grid, kBlock, 0, st>>>(us, S, gate_mask, up_mask, gate_frozen, stats, tau,       \
                                                       up_hard_kind, up_hard_n, p->cols, groups, gpr, vec,       \
                                                       gate_flips, up_flips)
  if (s_dtype == SF_DTYPE_F32 && mask_dtype == SF_DTYPE_F32)
    SF_LAUNCH_GLU(SF_DTYPE_F32, SF_DTYPE_F32);
  else if (s_dtype == SF_DTYPE_F32)
    SF_LAUNCH_GLU(SF_DTYPE_F32, SF_DTYPE_BF16);
  else if (mask_dtype == SF_DTYPE_F32)
    SF_LAUNCH_GLU(SF_DTYPE_BF16, SF_DTYPE_F32);
  else
    SF_LAUNCH_GLU(SF_DTYPE_BF16, SF_DTYPE_BF16);
#undef SF_LAUNCH_GLU
  return launch_status("sf_glu_update_masks");
}

// ---------------------------------------------------------------------------
// Effective mask of a forward call (SparseLinear.forward, :759-771 and
// FusedMaskedLinearSTE.forward, :72-73): E = mask.to(weight dtype), or with
// hardening E = (hx * mask + (1 - hx) * hard(mask)).to(weight dtype), each
// product and the sum rounded in the mask dtype.
// ---------------------------------------------------------------------------
namespace sf {
namespace {
// hsrc: a precomputed hard mask (hdt) used in place of the group projection (the block types).
template <int MD, int ED>
__global__ void __launch_bounds__(kBlock) effective_mask_kernel(const void* __restrict__ mask, void* __restrict__ eff,
                                                                int64_t cols, int64_t groups, int64_t gpr, bool vec,
                                                                int mix, float hx, float one_minus_hx, int kind,
                                                                int n_keep, const void* __restrict__ hsrc, int hdt) {
  for (GroupWalk w(groups, cols, gpr); w.live(); w.next()) {
    Group g = w.group();
    const bool v = vec && g.full;
    float m[4], e[4];
    load4<MD>(mask, g.elem, g.n, v, m);
    if (mix) {
      float h[4];
      if (hsrc)
        load4_any(hsrc, hdt, g.elem, g.n, v, h);
      else
        hard_of_group(m, g, kind, n_keep, h);
#pragma unroll
      for (int j = 0; j < 4; ++j) e[j] = rnd(rnd(hx * m[j], MD) + rnd(one_minus_hx * h[j], MD), MD);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) e[j] = m[j];
    }
    store4<ED>(eff, g.elem, g.n, v, e);
  }
}
// Hard projection as a byte and-mask: 0xFF where the element is kept, 0x00 where it is pruned.
template <int MD>
__global__ void __launch_bounds__(kBlock) hard_bytes_kernel(const void* __restrict__ mask, uint8_t* __restrict__ out,
                                                            int64_t cols, int64_t groups, int64_t gpr, bool vec,
                                                            int kind, int n_keep, const void* __restrict__ hsrc,
                                                            int hdt) {
  for (GroupWalk w(groups, cols, gpr); w.live(); w.next()) {
    Group g = w.group();
    const bool v = vec && g.full;
    float m[4], h[4];
    if (hsrc) {
      load4_any(hsrc, hdt, g.elem, g.n, v, h);
    } else {
      load4<MD>(mask, g.elem, g.n, v, m);
      hard_of_group(m, g, kind, n_keep, h);
    }
    if (v) {
      uint32_t w = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) w |= (h[j] > 0.5f ? 0xffu : 0u) << (8 * j);
      *reinterpret_cast<uint32_t*>(out + g.elem) = w;
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (j < g.n) out[g.elem + j] = h[j] > 0.5f ? 0xff : 0;
    }
  }
}
}  // namespace
}  // namespace sf

namespace sf {
namespace {
int effective_mask_impl(const void* mask, int mask_dtype, const void* hsrc, int hdt, void* eff, int eff_dtype,
                        int64_t rows, int64_t cols, int mode, float hx, int hard_kind, int hard_n, int hard_m,
                        void* stream);
}  // namespace
}  // namespace sf

extern "C" int sf_effective_mask(const void* mask, int mask_dtype, void* eff, int eff_dtype, int64_t rows,
                                 int64_t cols, int mode, float hx, int hard_kind, int hard_n, int hard_m,
                                 void* stream) {
  return effective_mask_impl(mask, mask_dtype, nullptr, SF_DTYPE_F32, eff, eff_dtype, rows, cols, mode, hx, hard_kind,
                             hard_n, hard_m, stream);
}

extern "C" int sf_effective_mask_given(const void* mask, int mask_dtype, const void* hard, int hard_dtype, void* eff,
                                       int eff_dtype, int64_t rows, int64_t cols, int mode, float hx, void* stream) {
  SF_CHECK_ARG(dtype_ok(hard_dtype), "bad hard-mask dtype");
  SF_CHECK_ARG(rows == 0 || cols == 0 || hard != nullptr, "null hard mask");
  return effective_mask_impl(mask, mask_dtype, hard, hard_dtype, eff, eff_dtype, rows, cols, mode, hx,
                             SF_HARD_THRESHOLD, 2, 4, stream);
}

namespace sf {
namespace {
int effective_mask_impl(const void* mask, int mask_dtype, const void* hsrc, int hdt, void* eff, int eff_dtype,
                        int64_t rows, int64_t cols, int mode, float hx, int hard_kind, int hard_n, int hard_m,
                        void* stream) {
  SF_CHECK_ARG(rows >= 0 && cols >= 0, "negative shape");
  SF_CHECK_ARG(mode == SF_EFF_SOFT || mode == SF_EFF_MIX || mode == SF_EFF_HARD, "bad effective-mask mode %d", mode);
  SF_CHECK_ARG(dtype_ok(mask_dtype) && (dtype_ok(eff_dtype) || (mode == SF_EFF_HARD && eff_dtype == SF_DTYPE_U8)),
               "bad dtype");
  if (mode == SF_EFF_HARD) {  // hx = 0: E = hard(mask)
    mode = SF_EFF_MIX;
    hx = 0.0f;
  }
  SF_CHECK_ARG(hard_kind >= SF_HARD_NONE && hard_kind <= SF_HARD_NM_STRICT, "bad hard kind %d", hard_kind);
  if (rows == 0 || cols == 0) return SF_OK;
  SF_CHECK_ARG(mask && eff, "null tensor");
  if (mode == SF_EFF_MIX && hard_kind >= SF_HARD_NM_TAIL_KEEP) {
    if (hard_m != 4 || hard_n < 1 || hard_n > 3) {
      set_error("N:M hard mask with N=%d M=%d: only M=4 is built on device", hard_n, hard_m);
      return SF_ERR_UNSUPPORTED;
    }
    SF_CHECK_ARG(hard_kind != SF_HARD_NM_STRICT || cols % 4 == 0, "in_features (%lld) must be divisible by M (%d).",
                 (long long)cols, hard_m);
  }
  const int64_t gpr = ceil_div(cols, 4), groups = rows * gpr;
  if (eff_dtype == SF_DTYPE_U8) {
    const bool vb = vec_ok(cols, {{mask, mask_dtype}, {hsrc, hdt}}) && aligned(eff, 4);
    hipStream_t sb = static_cast<hipStream_t>(stream);
    const int gb = elementwise_grid(groups, kBlock);
    if (mask_dtype == SF_DTYPE_F32)
      hard_bytes_kernel<SF_DTYPE_F32><<<gb, kBlock, 0, sb>>>(mask, static_cast<uint8_t*>(eff), cols, groups, gpr, vb,
                                                             hard_kind, hard_n, hsrc, hdt);
    else
      hard_bytes_kernel<SF_DTYPE_BF16><<<gb, kBlock, 0, sb>>>(mask, static_cast<uint8_t*>(eff), cols, groups, gpr, vb,
                                                              hard_kind, hard_n, hsrc, hdt);
    return launch_status("sf_effective_mask");
  }
  const bool vec = vec_ok(cols, {{mask, mask_dtype}, {eff, eff_dtype}, {hsrc, hdt}});
  // (1 - hx) computed in double as in Python, then the f32 scalar of the op
  const float omh = static_cast<float>(1.0 - static_cast<double>(hx));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int grid = elementwise_grid(groups, kBlock);
  const int mix = mode == SF_EFF_MIX;
#define SF_LAUNCH_EFF(MDT, EDT)                                                                              \
  effective_mask_kernel<MDT, EDT><<<grid, kBlock, 0, st>>>(mask, eff, cols, groups, gpr, vec, mix, hx, omh, \
                                                           hard_kind, hard_n, hsrc, hdt)
  if (mask_dtype == SF_DTYPE_F32 && eff_dtype == SF_DTYPE_F32) SF_LAUNCH_EFF(SF_DTYPE_F32, SF_DTYPE_F32);
  else if (mask_dtype == SF_DTYPE_F32) SF_LAUNCH_EFF(SF_DTYPE_F32, SF_DTYPE_BF16);
  else if (eff_dtype == SF_DTYPE_F32) SF_LAUNCH_EFF(SF_DTYPE_BF16, SF_DTYPE_F32);
  else SF_LAUNCH_EFF(SF_DTYPE_BF16, SF_DTYPE_BF16);
#undef SF_LAUNCH_EFF
  return launch_status("sf_effective_mask");
}
}  // namespace
}  // namespace sf

// ---------------------------------------------------------------------------
// Transpose of a byte mask ([rows, cols] -> [cols, rows]): the K-major byte
// mask of the input-gradient GEMM (dx = dy (W.E), whose B operand is W read
// along its columns).  64 x 64 byte tiles through LDS, 4-byte words in and out.
// ---------------------------------------------------------------------------
namespace sf {
namespace {
__global__ void __launch_bounds__(256) transpose_u8_kernel(const uint8_t* __restrict__ src, int64_t rows, int64_t cols,
                                                           uint8_t* __restrict__ dst, bool vec) {
  __shared__ uint32_t tile[64][17];
  const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
  const int t = threadIdx.x;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = t / 16 + 16 * j, w = t % 16;
    const int64_t gr = r0 + r, gc = c0 + 4 * w;
    uint32_t v = 0;
    if (gr < rows) {
      if (vec && gc + 4 <= cols) {
        v = *reinterpret_cast<const uint32_t*>(src + gr * cols + gc);
      } else {
        for (int b = 0; b < 4; ++b)
          if (gc + b < cols) v |= static_cast<uint32_t>(src[gr * cols + gc + b]) << (8 * b);
      }
    }
    tile[r][w] = v;
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = t / 16 + 16 * j, w = t % 16;  // output row c0 + c, output bytes of input rows 4w .. 4w + 3
    const int64_t orow = c0 + c, ocol = r0 + 4 * w;
    if (orow >= cols) continue;
    uint32_t v = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) v |= ((tile[4 * w + b][c >> 2] >> (8 * (c & 3))) & 0xffu) << (8 * b);
    if (vec && ocol + 4 <= rows) {
      *reinterpret_cast<uint32_t*>(dst + orow * rows + ocol) = v;
    } else {
      for (int b = 0; b < 4; ++b)
        if (ocol + b < rows) dst[orow * rows + ocol + b] = static_cast<uint8_t>(v >> (8 * b));
    }
  }
}
}  // namespace
}  // namespace sf

extern "C" int sf_transpose_u8(const uint8_t* src, int64_t rows, int64_t cols, uint8_t* dst, void* stream) {
  SF_CHECK_ARG(rows >= 0 && cols >= 0, "negative shape");
  if (rows == 0 || cols == 0) return SF_OK;
  SF_CHECK_ARG(src && dst, "null tensor");
  SF_CHECK_ARG(ceil_div(cols, 64) < (1ll << 31) && ceil_div(rows, 64) < 65536, "transpose grid too large");
  const bool vec = rows % 4 == 0 && cols % 4 == 0 && aligned(src, 4) && aligned(dst, 4);
  dim3 grid(static_cast<unsigned>(ceil_div(cols, 64)), static_cast<unsigned>(ceil_div(rows, 64)));
  transpose_u8_kernel<<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(src, rows, cols, dst, vec);
  return launch_status("sf_transpose_u8");
}

// ---------------------------------------------------------------------------
// Block hard types and block_sparse soft masks (legacy/sparse_modeling.py:
// _blockify_tensor :460-507, block16 / block_sparse16 / block_sparse32 hard
// projections :537-718, block-level gate :1100-1158, G blockify :1237, block
// penalties :1298-1529, mask blockify :1598-1601).  Blocks are the bs x bs
// tiles of the fully covered core [:rows/bs*bs, :cols/bs*bs]; block (br, bc)
// is entry br * ib + bc of a block vector.  Elements outside the core keep
// their value (blockify) or take a fixed one (hard masks, targets, G).
// ---------------------------------------------------------------------------
namespace sf {
namespace {

__device__ __forceinline__ float load1_any(const void* base, int dtype, int64_t i) {
  return dtype == SF_DTYPE_F32 ? static_cast<const float*>(base)[i]
                               : bf16_to_f32(static_cast<const uint16_t*>(base)[i]);
}

// One wave per block: mean of x (stat 0) or sqrt(mean(x * x)) (stat 1, the square in f32).
// The sum runs in f64 in a fixed tree order and is rounded to f32 once.
__global__ void __launch_bounds__(kBlock) block_stat_kernel(const void* __restrict__ x, int x_dtype, int64_t cols,
                                                            int bs, int64_t ib, int64_t nb, int rms,
                                                            float* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t waves = ((int64_t)gridDim.x * blockDim.x) >> 6;
  const int lg = bs == 16 ? 4 : 5;
  for (int64_t b = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6; b < nb; b += waves) {
    const int64_t br = b / ib, bc = b - br * ib;
    const int64_t base = br * bs * cols + bc * bs;
    double acc = 0.0;
    for (int e = lane; e < bs * bs; e += 64) {
      float v = load1_any(x, x_dtype, base + (int64_t)(e >> lg) * cols + (e & (bs - 1)));
      if (rms) v = v * v;
      acc += static_cast<double>(v);
    }
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if (lane == 0) {
      const float m = static_cast<float>(acc / static_cast<double>(bs * bs));
      out[b] = rms ? sqrtf(m) : m;
    }
  }
}

// ---------------------------------------------------------------------------
// torch.topk's CPU selection, which fixes which of several equal values are
// kept.  torch (ATen native/TopKImpl.h, topk_impl_loop) compares (value, index)
// pairs by value only -- ordered_key: NaN largest, -0 == +0 -- and runs
// std::partial_sort(first, first + k, last) when k * 64 <= n, else
// std::nth_element(first, first + k - 1, last); the first k pairs are kept.
// Both are GCC libstdc++'s algorithms (bits/stl_algo.h __introselect with a
// median-of-three pivot, __unguarded_partition and __insertion_sort below four
// elements; bits/stl_heap.h __heap_select / __make_heap / __adjust_heap /
// __push_heap for partial_sort and when the depth limit 2 lg n runs out),
// restated here on pairs packed as (key << 32) | index; `a before b` is
// key(a) > key(b).
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t pair_key(uint64_t v) { return static_cast<uint32_t>(v >> 32); }

// Pairs in global memory (one array of keys, one of indices).
struct SelGlobal {
  uint32_t* K;
  int32_t* I;
  __device__ uint32_t key(int64_t a) const { return K[a]; }
  __device__ uint64_t get(int64_t a) const { return (static_cast<uint64_t>(K[a]) << 32) | static_cast<uint32_t>(I[a]); }
  __device__ void put(int64_t a, uint64_t v) const {
    K[a] = pair_key(v);
    I[a] = static_cast<int32_t>(static_cast<uint32_t>(v));
  }
  __device__ void swap(int64_t a, int64_t b) const {
    const uint64_t t = get(a);
    put(a, get(b));
    put(b, t);
  }
};

// One thread's pairs in LDS, element a at a * kSelTileThreads (indices fit a byte).
constexpr int kSelTileThreads = 32;
struct SelTile {
  uint32_t* K;
  uint8_t* I;
  __device__ uint32_t key(int64_t a) const { return K[a * kSelTileThreads]; }
  __device__ uint64_t get(int64_t a) const {
    return (static_cast<uint64_t>(K[a * kSelTileThreads]) << 32) | I[a * kSelTileThreads];
  }
  __device__ void put(int64_t a, uint64_t v) const {
    K[a * kSelTileThreads] = pair_key(v);
    I[a * kSelTileThreads] = static_cast<uint8_t>(v);
  }
  __device__ void swap(int64_t a, int64_t b) const {
    const uint64_t t = get(a);
    put(a, get(b));
    put(b, t);
  }
};

template <class A>
__device__ void sel_move_median_to_first(const A& s, int64_t result, int64_t a, int64_t b, int64_t c) {
  const uint32_t ka = s.key(a), kb = s.key(b), kc = s.key(c);
  if (ka > kb) {
    if (kb > kc) s.swap(result, b);
    else if (ka > kc) s.swap(result, c);
    else s.swap(result, a);
  } else if (ka > kc) {
    s.swap(result, a);
  } else if (kb > kc) {
    s.swap(result, c);
  } else {
    s.swap(result, b);
  }
}

// __unguarded_partition(first, last, pivot): the median-of-three leaves an
// element on each side that stops the scans.
// The range checks never fire under that invariant; they only keep every scan inside
// [pivot, last) whatever the data.
template <class A>
__device__ int64_t sel_unguarded_partition(const A& s, int64_t first, int64_t last, int64_t pivot) {
  const uint32_t kp = s.key(pivot);
  const int64_t hi = last - 1;
  while (true) {
    while (first < hi && s.key(first) > kp) ++first;
    --last;
    while (last > pivot && kp > s.key(last)) --last;
    if (!(first < last)) return first;
    s.swap(first, last);
    ++first;
  }
}

template <class A>
__device__ void sel_insertion_sort(const A& s, int64_t first, int64_t last) {
  if (first == last) return;
  for (int64_t i = first + 1; i < last; ++i) {
    const uint64_t val = s.get(i);
    if (pair_key(val) > s.key(first)) {
      for (int64_t j = i; j > first; --j) s.put(j, s.get(j - 1));
      s.put(first, val);
    } else {
      int64_t j = i, nxt = i - 1;
      while (nxt >= first && pair_key(val) > s.key(nxt)) {
        s.put(j, s.get(nxt));
        j = nxt;
        --nxt;
      }
      s.put(j, val);
    }
  }
}

template <class A>
__device__ void sel_adjust_heap(const A& s, int64_t first, int64_t hole, int64_t len, uint64_t value) {
  const int64_t top = hole;
  int64_t second = hole;
  while (second < (len - 1) / 2) {
    second = 2 * (second + 1);
    if (s.key(first + second) > s.key(first + second - 1)) --second;
    s.put(first + hole, s.get(first + second));
    hole = second;
  }
  if ((len & 1) == 0 && second == (len - 2) / 2) {
    second = 2 * (second + 1);
    s.put(first + hole, s.get(first + second - 1));
    hole = second - 1;
  }
  int64_t parent = (hole - 1) / 2;  // __push_heap
  while (hole > top && s.key(first + parent) > pair_key(value)) {
    s.put(first + hole, s.get(first + parent));
    hole = parent;
    parent = (hole - 1) / 2;
  }
  s.put(first + hole, value);
}

template <class A>
__device__ void sel_heap_select(const A& s, int64_t first, int64_t middle, int64_t last) {
  const int64_t len = middle - first;
  if (len >= 2) {  // __make_heap
    for (int64_t parent = (len - 2) / 2;; --parent) {
      sel_adjust_heap(s, first, parent, len, s.get(first + parent));
      if (parent == 0) break;
    }
  }
  for (int64_t i = middle; i < last; ++i) {
    if (s.key(i) > s.key(first)) {  // __pop_heap(first, middle, i)
      const uint64_t value = s.get(i);
      s.put(i, s.get(first));
      sel_adjust_heap(s, first, 0, len, value);
    }
  }
}

__device__ __forceinline__ int floor_log2(int64_t n) { return 63 - __clzll(static_cast<unsigned long long>(n)); }

// The first k pairs of [0, n) become torch's kept set (sequential; 1 <= k < n).
template <class A>
__device__ void sel_topk_seq(const A& s, int64_t n, int64_t k) {
  if (k * 64 <= n) {
    sel_heap_select(s, 0, k, n);
    return;
  }
  const int64_t nth = k - 1;
  int64_t first = 0, last = n;
  int depth = 2 * floor_log2(n);
  while (last - first > 3) {
    if (depth == 0) {
      sel_heap_select(s, first, nth + 1, last);
      s.swap(first, nth);
      return;
    }
    --depth;
    sel_move_median_to_first(s, first, first + 1, first + (last - first) / 2, last - 1);
    const int64_t cut = sel_unguarded_partition(s, first + 1, last, first);
    if (cut <= nth) first = cut;
    else last = cut;
  }
  sel_insertion_sort(s, first, last);
}

// keep[i] = 1 for the entries torch.topk(v, k) keeps, else 0.  One workgroup;
// the partition of each introselect step runs data-parallel: the left scan
// stops at keys <= the pivot's, the right scan at keys >= it; the i-th left
// stop (ascending) swaps with the i-th right stop (descending) while it lies
// before it (m pairs), and the scans end at min(left stop m + 1, right stop m).
// That is the permutation the sequential scans make (they pass only untouched
// positions and stop at swapped ones).  Median-of-three, the final insertion
// sort and the heap selections run on thread 0.  Workspace: keys, indices and
// the two stop lists, n entries each.
constexpr int kTopkBlock = 1024;
__global__ void __launch_bounds__(kTopkBlock) topk_keep_kernel(const float* __restrict__ v, int64_t n, int64_t k,
                                                               float* __restrict__ keep, uint32_t* __restrict__ K,
                                                               int32_t* __restrict__ I, int32_t* __restrict__ PL,
                                                               int32_t* __restrict__ PR, int* __restrict__ status) {
  __shared__ int64_t s_first, s_last, s_cut;
  __shared__ int s_depth;
  __shared__ int s_scl[kTopkBlock / 64], s_scr[kTopkBlock / 64];
  __shared__ int s_tot[2];
  const int tid = threadIdx.x;
  if (k <= 0 || k >= n) {
    for (int64_t i = tid; i < n; i += blockDim.x) keep[i] = k > 0 ? 1.0f : 0.0f;
    return;
  }
  for (int64_t i = tid; i < n; i += blockDim.x) {
    K[i] = ordered_key(v[i]);
    I[i] = static_cast<int32_t>(i);
  }
  __syncthreads();
  const SelGlobal sg{K, I};
  if (k * 64 <= n) {
    if (tid == 0) sel_heap_select(sg, 0, k, n);
  } else {
    const int64_t nth = k - 1;
    if (tid == 0) {
      s_first = 0;
      s_last = n;
      s_depth = 2 * floor_log2(n);
    }
    __syncthreads();
    while (true) {
      const int64_t first = s_first, last = s_last;
      const int depth = s_depth;
      __syncthreads();  // every thread has read the state before thread 0 changes it
      if (last - first <= 3) {
        if (tid == 0) sel_insertion_sort(sg, first, last);
        break;
      }
      if (depth == 0) {
        if (tid == 0) {
          sel_heap_select(sg, first, nth + 1, last);
          sg.swap(first, nth);
        }
        break;
      }
      if (tid == 0) {
        s_depth = depth - 1;
        sel_move_median_to_first(sg, first, first + 1, first + (last - first) / 2, last - 1);
      }
      __syncthreads();
      const uint32_t piv = K[first];
      const int64_t len = last - first, chunk = (len + kTopkBlock - 1) / kTopkBlock;
      const int64_t c0 = first + tid * chunk < last ? first + tid * chunk : last;
      const int64_t c1 = c0 + chunk < last ? c0 + chunk : last;
      int cl = 0, cr = 0;
      for (int64_t p = c0; p < c1; ++p) {
        const uint32_t kp = K[p];
        cl += (p > first && kp <= piv) ? 1 : 0;
        cr += kp >= piv ? 1 : 0;
      }
      // exclusive scans of cl and cr over the threads: inside each wave by shuffles, then over
      // the 16 wave totals
      const int lane = tid & 63, wv = tid >> 6;
      int il = cl, ir = cr;
      for (int off = 1; off < 64; off <<= 1) {
        const int tl = __shfl_up(il, off, 64), tr = __shfl_up(ir, off, 64);
        if (lane >= off) {
          il += tl;
          ir += tr;
        }
      }
      if (lane == 63) {
        s_scl[wv] = il;
        s_scr[wv] = ir;
      }
      __syncthreads();
      int bl = 0, br = 0, nl = 0, nr = 0;
      for (int w2 = 0; w2 < kTopkBlock / 64; ++w2) {
        if (w2 < wv) {
          bl += s_scl[w2];
          br += s_scr[w2];
        }
        nl += s_scl[w2];
        nr += s_scr[w2];
      }
      int rl = bl + il - cl, rr = br + ir - cr;
      for (int64_t p = c0; p < c1; ++p) {
        const uint32_t kp = K[p];
        if (p > first && kp <= piv) PL[rl++] = static_cast<int32_t>(p);
        if (kp >= piv) PR[nr - 1 - rr++] = static_cast<int32_t>(p);
      }
      if (tid == 0) {
        s_tot[0] = 0;
      }
      __syncthreads();
      const int nmin = nl < nr ? nl : nr;
      int cnt = 0;
      for (int i = tid; i < nmin; i += kTopkBlock) cnt += PL[i] < PR[i] ? 1 : 0;
      if (cnt) atomicAdd(&s_tot[0], cnt);
      __syncthreads();
      const int m = s_tot[0];  // the pairs that are swapped form a prefix: PL rises, PR falls
      if (tid == 0) {
        int64_t cut = m < nl ? PL[m] : last;
        if (m >= 1 && PR[m - 1] < cut) cut = PR[m - 1];
        if (!(cut > first && cut < last)) {  // not reachable for a median-of-three pivot
          *status = 1;
          cut = -1;
        }
        s_cut = cut;
      }
      __syncthreads();
      const int64_t cut = s_cut;
      if (cut < 0) break;
      for (int i = tid; i < m; i += kTopkBlock) sg.swap(PL[i], PR[i]);
      __syncthreads();
      if (tid == 0) {
        if (cut <= nth) s_first = cut;
        else s_last = cut;
      }
      __syncthreads();
    }
  }
  __syncthreads();
  for (int64_t p = tid; p < n; p += blockDim.x) keep[I[p]] = p < k ? 1.0f : 0.0f;
}

// block16: torch.topk(k) of each 16 x 16 tile (row-major positions), one
// thread per tile running the selection above on its 256 pairs in LDS.
template <int XD, int OD>
__global__ void __launch_bounds__(kSelTileThreads) tile_topk_kernel(const void* __restrict__ x, int64_t cols,
                                                                    int64_t ib, int64_t nb, int k, bool vec,
                                                                    void* __restrict__ out) {
  __shared__ uint32_t keys[256 * kSelTileThreads];
  __shared__ uint8_t idx[256 * kSelTileThreads];
  const int t = threadIdx.x;
  const SelTile st{keys + t, idx + t};
  for (int64_t b = (int64_t)blockIdx.x * kSelTileThreads + t; b < nb; b += (int64_t)gridDim.x * kSelTileThreads) {
    const int64_t br = b / ib, bc = b - br * ib;
    const int64_t e0 = br * 16 * cols + bc * 16;
    for (int r = 0; r < 16; ++r)
      for (int q = 0; q < 4; ++q) {
        float xv[4];
        load4<XD>(x, e0 + r * cols + 4 * q, 4, vec, xv);
#pragma unroll
        for (int j = 0; j < 4; ++j) st.put(r * 16 + 4 * q + j, (static_cast<uint64_t>(ordered_key(xv[j])) << 32) |
                                                                    static_cast<uint32_t>(r * 16 + 4 * q + j));
      }
    uint32_t kept[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
    if (k >= 256) {
      for (int w = 0; w < 8; ++w) kept[w] = 0xffffffffu;
    } else if (k > 0) {
      sel_topk_seq(st, 256, k);
      for (int p = 0; p < k; ++p) {
        const int e = static_cast<uint8_t>(st.get(p));
        kept[e >> 5] |= 1u << (e & 31);
      }
    }
    for (int r = 0; r < 16; ++r)
      for (int q = 0; q < 4; ++q) {
        float o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int e = r * 16 + 4 * q + j;
          o[j] = ((kept[e >> 5] >> (e & 31)) & 1u) ? 1.0f : 0.0f;
        }
        store4<OD>(out, e0 + r * cols + 4 * q, 4, vec, o);
      }
  }
}

// out = val on the elements outside the core (rows >= of, or cols >= inf).
template <int OD>
__global__ void __launch_bounds__(kBlock) edge_fill_kernel(void* __restrict__ out, int64_t rows, int64_t cols,
                                                           int64_t of, int64_t inf, float val) {
  const int64_t n1 = (rows - of) * cols, w2 = cols - inf, n = n1 + of * w2;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    int64_t e;
    if (i < n1) {
      e = of * cols + i;
    } else {
      const int64_t j = i - n1, r = j / w2;
      e = r * cols + inf + (j - r * w2);
    }
    if (OD == SF_DTYPE_F32)
      static_cast<float*>(out)[e] = val;
    else
      static_cast<uint16_t*>(out)[e] = f32_to_bf16(val);
  }
}

// Expand per-block values over the core: out = rnd(f(bvals[block])), f the
// identity or, with tau, sigmoid((b - tau) / denom) in f32.  Outside the core
// the element keeps its value (edge_write 0) or becomes edge_val.  Where
// ov_flags != 0 the element takes rnd(ov_src) instead (frozen override).
struct FillSpec {
  int64_t of, inf, ib;
  int lg;  // log2(bs)
  int edge_write;
  float edge_val;
  float denom, rdenom;
  int ov_src_dt, ov_flags_dt;
};

template <int OD>
__global__ void __launch_bounds__(kBlock) block_fill_kernel(FillSpec f, const float* __restrict__ bvals,
                                                            const float* __restrict__ tau_p, void* __restrict__ out,
                                                            const void* __restrict__ ov_src,
                                                            const void* __restrict__ ov_flags, int64_t cols,
                                                            int64_t groups, int64_t gpr, bool vec) {
  const float tau = tau_p ? *tau_p : 0.0f;
  for (GroupWalk w(groups, cols, gpr); w.live(); w.next()) {
    Group g = w.group();
    const bool v = vec && g.full;
    float o[4], fz[4] = {0, 0, 0, 0}, src[4];
    const bool row_in = g.row < f.of;
    if (!f.edge_write) load4<OD>(out, g.elem, g.n, v, o);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t c = g.col + j;
      if (row_in && c < f.inf) {
        float b = bvals[(g.row >> f.lg) * f.ib + (c >> f.lg)];
        if (tau_p) b = sigmoidf_(div_by(b - tau, f.denom, f.rdenom));
        o[j] = rndc<OD>(b);
      } else if (f.edge_write) {
        o[j] = rndc<OD>(f.edge_val);
      }
    }
    if (ov_flags) {
      load4_any(ov_flags, f.ov_flags_dt, g.elem, g.n, v, fz);
      load4_any(ov_src, f.ov_src_dt, g.elem, g.n, v, src);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (fz[j] != 0.0f) o[j] = rndc<OD>(src[j]);
    }
    store4<OD>(out, g.elem, g.n, v, o);
  }
}

// A gate target G already in memory (the staged block path): penalty pull
// (explicit target or the in-group modes), clamp, binarisation push, EMA and,
// with do_freeze, the freeze snaps and flags.
template <int MD, int SD>
__global__ void __launch_bounds__(kBlock) apply_gate_kernel(UpdateSpec us, const void* __restrict__ G,
                                                            const void* __restrict__ target, int target_dt,
                                                            void* __restrict__ mask, void* __restrict__ frozen,
                                                            int do_freeze, int64_t cols, int64_t groups, int64_t gpr,
                                                            bool vec) {
  for (GroupWalk w(groups, cols, gpr); w.live(); w.next()) {
    Group g = w.group();
    const bool v = vec && g.full;
    float gv[4], mp[4], tg[4] = {0, 0, 0, 0}, mn[4], fz[4] = {0, 0, 0, 0};
    load4<SD>(G, g.elem, g.n, v, gv);
    load4<MD>(mask, g.elem, g.n, v, mp);
    if (target) load4_any(target, target_dt, g.elem, g.n, v, tg);
    pull_and_push<MD, SD>(us, g, mp, gv, tg);
    ema_of<MD>(us, mp, gv, mn);
    if (do_freeze) {
      if (us.gs.has_frozen) load4_any(frozen, us.gs.frozen_dtype, g.elem, g.n, v, fz);
      freeze_group(us, g, v, mn, fz, frozen);
    }
    store4<MD>(mask, g.elem, g.n, v, mn);
  }
}

template <int MD>
__global__ void __launch_bounds__(kBlock) freeze_kernel(UpdateSpec us, void* __restrict__ mask,
                                                        void* __restrict__ frozen, int64_t cols, int64_t groups,
                                                        int64_t gpr, bool vec) {
  for (GroupWalk w(groups, cols, gpr); w.live(); w.next()) {
    Group g = w.group();
    const bool v = vec && g.full;
    float mn[4], fz[4] = {0, 0, 0, 0};
    load4<MD>(mask, g.elem, g.n, v, mn);
    if (us.gs.has_frozen) load4_any(frozen, us.gs.frozen_dtype, g.elem, g.n, v, fz);
    freeze_group(us, g, v, mn, fz, frozen);
    store4<MD>(mask, g.elem, g.n, v, mn);
  }
}

int check_block(int64_t rows, int64_t cols, int bs) {
  SF_CHECK_ARG(rows >= 0 && cols >= 0, "negative shape");
  SF_CHECK_ARG(bs == 16 || bs == 32, "block size %d: only 16 and 32 exist", bs);
  return SF_OK;
}
}  // namespace
}  // namespace sf

extern "C" int sf_block_stat(const void* x, int x_dtype, int64_t rows, int64_t cols, int bs, int stat, float* out,
                             void* stream) {
  if (int rc = check_block(rows, cols, bs)) return rc;
  SF_CHECK_ARG(dtype_ok(x_dtype), "bad dtype");
  SF_CHECK_ARG(stat == SF_BLOCK_MEAN || stat == SF_BLOCK_RMS, "bad block statistic %d", stat);
  const int64_t ob = rows / bs, ib = cols / bs, nb = ob * ib;
  if (nb == 0) return SF_OK;
  SF_CHECK_ARG(x && out, "null tensor");
  block_stat_kernel<<<elementwise_grid(nb * 64, kBlock), kBlock, 0, static_cast<hipStream_t>(stream)>>>(
      x, x_dtype, cols, bs, ib, nb, stat == SF_BLOCK_RMS, out);
  return launch_status("sf_block_stat");
}

extern "C" size_t sf_topk_keep_workspace_size(int64_t n) {
  return n <= 0 ? 0 : static_cast<size_t>(n) * 16 + 256;
}

extern "C" int sf_topk_keep(const float* v, int64_t n, int64_t k, float* keep, void* workspace,
                            size_t workspace_bytes, void* stream) {
  SF_CHECK_ARG(n >= 0, "negative length");
  if (n == 0) return SF_OK;
  SF_CHECK_ARG(v && keep, "null tensor");
  SF_CHECK_ARG(n < (1ll << 31), "top-k over more than 2^31 entries");
  SF_CHECK_ARG(workspace && workspace_bytes >= sf_topk_keep_workspace_size(n) &&
                   (reinterpret_cast<uintptr_t>(workspace) & 15) == 0,
               "top-k needs a 16-byte aligned workspace of sf_topk_keep_workspace_size(n) bytes");
  unsigned char* w = static_cast<unsigned char*>(workspace);
  uint32_t* K = reinterpret_cast<uint32_t*>(w);
  int32_t* I = reinterpret_cast<int32_t*>(w + 4 * n);
  int32_t* PL = reinterpret_cast<int32_t*>(w + 8 * n);
  int32_t* PR = reinterpret_cast<int32_t*>(w + 12 * n);
  int* status = reinterpret_cast<int*>(w + 16 * n);
  hipStream_t st = static_cast<hipStream_t>(stream);
  topk_keep_kernel<<<1, kTopkBlock, 0, st>>>(v, n, k, keep, K, I, PL, PR, status);
  return launch_status("sf_topk_keep");
}

extern "C" int sf_tile_topk(const void* x, int x_dtype, int64_t rows, int64_t cols, int bs, int64_t k, void* out,
                            int out_dtype, void* stream) {
  if (int rc = check_block(rows, cols, bs)) return rc;
  SF_CHECK_ARG(dtype_ok(x_dtype) && dtype_ok(out_dtype), "bad dtype");
  if (bs != 16) {
    set_error("per-tile top-k is built for 16 x 16 tiles (block16) only");
    return SF_ERR_UNSUPPORTED;
  }
  if (rows == 0 || cols == 0) return SF_OK;
  SF_CHECK_ARG(x && out, "null tensor");
  const int64_t of = rows / 16 * 16, inf = cols / 16 * 16, ib = inf / 16, nb = (of / 16) * ib;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool vec = vec_ok(cols, {{x, x_dtype}, {out, out_dtype}});
  if (nb > 0) {
    const int kk = static_cast<int>(k <= 0 ? 0 : (k >= 256 ? 256 : k));
#define SF_LAUNCH_TILE(XD, OD) \
  tile_topk_kernel<XD, OD><<<static_cast<unsigned>(ceil_div(nb, kSelTileThreads) < 65536 ? ceil_div(nb, kSelTileThreads) : 65536), kSelTileThreads, 0, st>>>(x, cols, ib, nb, kk, vec, out)
    if (x_dtype == SF_DTYPE_F32 && out_dtype == SF_DTYPE_F32) SF_LAUNCH_TILE(SF_DTYPE_F32, SF_DTYPE_F32);
    else if (x_dtype == SF_DTYPE_F32) SF_LAUNCH_TILE(SF_DTYPE_F32, SF_DTYPE_BF16);
    else if (out_dtype == SF_DTYPE_F32) SF_LAUNCH_TILE(SF_DTYPE_BF16, SF_DTYPE_F32);
    else SF_LAUNCH_TILE(SF_DTYPE_BF16, SF_DTYPE_BF16);
#undef SF_LAUNCH_TILE
  }
  if (of < rows || inf < cols) {
    const int64_t ne = (rows - of) * cols + of * (cols - inf);
    if (out_dtype == SF_DTYPE_F32)
      edge_fill_kernel<SF_DTYPE_F32><<<elementwise_grid(ne, kBlock), kBlock, 0, st>>>(out, rows, cols, of, inf, 1.0f);
    else
      edge_fill_kernel<SF_DTYPE_BF16><<<elementwise_grid(ne, kBlock), kBlock, 0, st>>>(out, rows, cols, of, inf, 1.0f);
  }
  return launch_status("sf_tile_topk");
}

extern "C" int sf_block_fill(const float* bvals, int64_t rows, int64_t cols, int bs, const float* tau, float temperature,
                             void* out, int out_dtype, int edge_write, float edge_val, const void* ov_src,
                             int ov_src_dtype, const void* ov_flags, int ov_flags_dtype, void* stream) {
  if (int rc = check_block(rows, cols, bs)) return rc;
  SF_CHECK_ARG(dtype_ok(out_dtype), "bad dtype");
  SF_CHECK_ARG(!ov_flags || (ov_src && dtype_ok(ov_src_dtype) && dtype_ok(ov_flags_dtype)), "bad override operands");
  if (rows == 0 || cols == 0) return SF_OK;
  SF_CHECK_ARG(out, "null tensor");
  FillSpec f;
  f.of = rows / bs * bs;
  f.inf = cols / bs * bs;
  f.ib = f.inf / bs;
  SF_CHECK_ARG(bvals || f.of == 0 || f.inf == 0, "null block values");
  f.lg = bs == 16 ? 4 : 5;
  f.edge_write = edge_write;
  f.edge_val = edge_val;
  f.denom = temperature + 1e-8f;
  f.rdenom = 1.0f / f.denom;
  f.ov_src_dt = ov_src_dtype;
  f.ov_flags_dt = ov_flags_dtype;
  const int64_t gpr = ceil_div(cols, 4), groups = rows * gpr;
  const bool vec = vec_ok(cols, {{out, out_dtype}, {ov_flags ? ov_src : nullptr, ov_src_dtype},
                                 {ov_flags, ov_flags_dtype}});
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int grid = elementwise_grid(groups, kBlock);
  if (out_dtype == SF_DTYPE_F32)
    block_fill_kernel<SF_DTYPE_F32><<<grid, kBlock, 0, st>>>(f, bvals, tau, out, ov_src, ov_flags, cols, groups, gpr,
                                                             vec);
  else
    block_fill_kernel<SF_DTYPE_BF16><<<grid, kBlock, 0, st>>>(f, bvals, tau, out, ov_src, ov_flags, cols, groups, gpr,
                                                              vec);
  return launch_status("sf_block_fill");
}

extern "C" int sf_apply_gate(const sf_mask_params* p, const void* G, const void* target, int target_dtype, void* mask,
                             int mask_dtype, void* frozen, int frozen_dtype, int do_freeze, void* stream) {
  if (int rc = check_common(p)) return rc;
  SF_CHECK_ARG(dtype_ok(mask_dtype) && (!target || dtype_ok(target_dtype)), "bad dtype");
  SF_CHECK_ARG(p->penalty >= SF_PENALTY_NONE && p->penalty <= SF_PENALTY_TARGET, "bad penalty %d", p->penalty);
  SF_CHECK_ARG(p->penalty != SF_PENALTY_TARGET || p->penalty_coef == 0.0f || target, "target penalty needs a target");
  SF_CHECK_ARG(!do_freeze || !p->has_frozen || frozen, "has_frozen without frozen flags");
  UpdateSpec us;
  sf_mask_params q = *p;
  q.gate = SF_GATE_UNSTRUCTURED;  // the gate form is not used here
  q.beta_struct = 0.0f;
  if (int rc = make_update_spec(&q, SF_DTYPE_F32, SF_DTYPE_F32, SF_DTYPE_F32, mask_dtype, frozen_dtype, false, &us))
    return rc;
  us.apply_freeze = do_freeze && p->apply_freeze;
  if (p->rows == 0 || p->cols == 0) return SF_OK;
  SF_CHECK_ARG(G && mask, "null tensor");
  const int64_t gpr = ceil_div(p->cols, 4), groups = p->rows * gpr;
  const bool vec = vec_ok(p->cols, {{G, p->score_dtype}, {mask, mask_dtype}, {target, target_dtype},
                                    {us.apply_freeze && p->has_frozen ? frozen : nullptr, frozen_dtype}});
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int grid = elementwise_grid(groups, kBlock);
  const int fr = us.apply_freeze;
#define SF_LAUNCH_APPLY(MDT, SDT)                                                                             \
  apply_gate_kernel<MDT, SDT><<<grid, kBlock, 0, st>>>(us, G, target, target_dtype, mask, frozen, fr, p->cols, \
                                                       groups, gpr, vec)
  const bool sf32 = p->score_dtype == SF_DTYPE_F32;
  if (mask_dtype == SF_DTYPE_F32) {
    if (sf32) SF_LAUNCH_APPLY(SF_DTYPE_F32, SF_DTYPE_F32);
    else SF_LAUNCH_APPLY(SF_DTYPE_F32, SF_DTYPE_BF16);
  } else {
    if (sf32) SF_LAUNCH_APPLY(SF_DTYPE_BF16, SF_DTYPE_F32);
    else SF_LAUNCH_APPLY(SF_DTYPE_BF16, SF_DTYPE_BF16);
  }
#undef SF_LAUNCH_APPLY
  return launch_status("sf_apply_gate");
}

extern "C" int sf_freeze_mask(const sf_mask_params* p, void* mask, int mask_dtype, void* frozen, int frozen_dtype,
                              void* stream) {
  if (int rc = check_common(p)) return rc;
  SF_CHECK_ARG(dtype_ok(mask_dtype), "bad dtype");
  SF_CHECK_ARG(!p->has_frozen || frozen, "has_frozen without frozen flags");
  UpdateSpec us;
  sf_mask_params q = *p;
  q.gate = SF_GATE_UNSTRUCTURED;
  q.beta_struct = 0.0f;
  q.penalty = SF_PENALTY_NONE;
  if (int rc = make_update_spec(&q, SF_DTYPE_F32, SF_DTYPE_F32, SF_DTYPE_F32, mask_dtype, frozen_dtype, false, &us))
    return rc;
  if (p->rows == 0 || p->cols == 0 || !p->apply_freeze) return SF_OK;
  SF_CHECK_ARG(mask, "null tensor");
  const int64_t gpr = ceil_div(p->cols, 4), groups = p->rows * gpr;
  const bool vec = vec_ok(p->cols, {{mask, mask_dtype}, {p->has_frozen ? frozen : nullptr, frozen_dtype}});
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int grid = elementwise_grid(groups, kBlock);
  if (mask_dtype == SF_DTYPE_F32)
    freeze_kernel<SF_DTYPE_F32><<<grid, kBlock, 0, st>>>(us, mask, frozen, p->cols, groups, gpr, vec);
  else
    freeze_kernel<SF_DTYPE_BF16><<<grid, kBlock, 0, st>>>(us, mask, frozen, p->cols, groups, gpr, vec);
  return launch_status("sf_freeze_mask");
}

// ---------------------------------------------------------------------------
// Masked weight of FusedMaskedLinearSTE: out = round(W * E), then round(out * s)
// when s != 1 (legacy/sparse_modeling.py:72-81; the backward's W . E at :113-115
// is the s = 1 case).  E is a byte and-mask or values in W's dtype.  8
// consecutive elements per thread per step (16-byte loads for bf16 W).
// ---------------------------------------------------------------------------
namespace sf {
namespace {
template <int WD, int ED>
__global__ void __launch_bounds__(kBlock) apply_mask_kernel(const void* __restrict__ W, const void* __restrict__ E,
                                                            float scale, int has_scale, void* __restrict__ out,
                                                            int64_t n, bool vec) {
  const int64_t n8 = (n + 7) / 8;
  for (int64_t i8 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i8 < n8; i8 += (int64_t)gridDim.x * blockDim.x) {
    const int64_t e0 = i8 * 8;
    const int m = n - e0 >= 8 ? 8 : static_cast<int>(n - e0);
    const bool v = vec && m == 8;
    float w[8], e[8], o[8];
    load4<WD>(W, e0, m, v, w);
    load4<WD>(W, e0 + 4, m - 4, v, w + 4);
    if (ED == SF_DTYPE_U8) {
      const uint8_t* eb = static_cast<const uint8_t*>(E) + e0;
      uint32_t lo = 0, hi = 0;
      if (v) {
        const uint2 q = *reinterpret_cast<const uint2*>(eb);
        lo = q.x;
        hi = q.y;
      } else {
        for (int j = 0; j < m; ++j) (j < 4 ? lo : hi) |= static_cast<uint32_t>(eb[j]) << (8 * (j & 3));
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) e[j] = (((j < 4 ? lo : hi) >> (8 * (j & 3))) & 0xffu) ? 1.0f : 0.0f;
    } else {
      load4<ED>(E, e0, m, v, e);
      load4<ED>(E, e0 + 4, m - 4, v, e + 4);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float x = rndc<WD>(w[j] * e[j]);
      if (has_scale) x = rndc<WD>(x * scale);
      o[j] = x;
    }
    store4<WD>(out, e0, m, v, o);
    store4<WD>(out, e0 + 4, m - 4, v, o + 4);
  }
}
}  // namespace
}  // namespace sf

extern "C" int sf_apply_mask(const void* W, int w_dtype, const void* E, int e_dtype, float scale, void* out,
                             int64_t rows, int64_t cols, void* stream) {
  SF_CHECK_ARG(rows >= 0 && cols >= 0, "negative shape");
  SF_CHECK_ARG(dtype_ok(w_dtype), "bad weight dtype");
  SF_CHECK_ARG(e_dtype == SF_DTYPE_U8 || e_dtype == w_dtype, "the mask must be a byte mask or in the weight dtype");
  const int64_t n = rows * cols;
  if (n == 0) return SF_OK;
  SF_CHECK_ARG(W && E && out, "null tensor");
  const bool vec = aligned(W, 16) && aligned(out, 16) &&
                   (e_dtype == SF_DTYPE_U8 ? aligned(E, 8) : aligned(E, 16));
  const int has_scale = scale != 1.0f;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int grid = elementwise_grid((n + 7) / 8, kBlock);
#define SF_LAUNCH_APPLY_MASK(WDT, EDT) \
  apply_mask_kernel<WDT, EDT><<<grid, kBlock, 0, st>>>(W, E, scale, has_scale, out, n, vec)
  if (w_dtype == SF_DTYPE_BF16) {
    if (e_dtype == SF_DTYPE_U8) SF_LAUNCH_APPLY_MASK(SF_DTYPE_BF16, SF_DTYPE_U8);
    else SF_LAUNCH_APPLY_MASK(SF_DTYPE_BF16, SF_DTYPE_BF16);
  } else {
    if (e_dtype == SF_DTYPE_U8) SF_LAUNCH_APPLY_MASK(SF_DTYPE_F32, SF_DTYPE_U8);
    else SF_LAUNCH_APPLY_MASK(SF_DTYPE_F32, SF_DTYPE_F32);
  }
#undef SF_LAUNCH_APPLY_MASK
  return launch_status("sf_apply_mask");
}
