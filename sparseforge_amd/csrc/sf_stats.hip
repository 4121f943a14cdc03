// Mask statistics and penalties (legacy/utils.py mid_penalty :876-938,
// sparsity_penalty :942-1025, nm_2_4_tile_stats :1029-1234, mask_stats
// :2069-2280).
//
// The reference walks every SparseLinear with a dozen separate torch
// reductions per layer (sum, sum of squares, entropy, six threshold counts, two
// conditional sums, m * (1 - m), a NaN scan, a sort of every group of 4) and a
// host sync per scalar.  Here one HBM pass per mask produces all of them:
// each thread walks groups of 4 along a row (16-byte loads for f32, 8-byte for
// bf16, the next group's load issued before this one's arithmetic) and keeps
// the sums in f64 registers (the entropy terms in f32); the eight counts are
// wave ballots added on the scalar unit.  The workgroup folds the sums, and a
// one-workgroup pass adds the per-workgroup partials in a fixed order.  With
// sixteen statistics per element the pass is bound by VALU issue (about 58
// instructions per element), not by HBM.  The
// number of workgroups depends only on the shape, so results are bitwise
// reproducible.  The host composes mid_penalty / sparsity_penalty /
// nm_2_4_tile_stats / mask_stats from the rows of all layers after one copy.
#include "sf_common.hpp"

namespace sf {
namespace {

constexpr int kBlock = 256;
constexpr int kParts = 1024;  // most workgroups of the partial pass
constexpr int kSlots = SF_MSTAT_COUNT;
constexpr double kLn2 = 0.69314718055994530942;
constexpr float kInvLn2 = 1.44269504088896340736f;

struct StatSpec {
  int64_t cols, groups, gpr, tail_col;
  float lo, hi;                // entropy clamp bounds: f32 values of eps and 1 - eps
  float t01, t001, t90, t99;   // 0.1, 0.01, 0.9, 0.99 as the mask dtype holds them
  bool vec;                    // every group full and vector-aligned
};

// Round to the mask dtype: v_cvt_pk_bf16_f32 rounds to nearest even, as torch does.
template <int DT>
__device__ __forceinline__ float rnd(float x) {
  if constexpr (DT == SF_DTYPE_BF16)
    return static_cast<float>(static_cast<__bf16>(x));
  else
    return x;
}

template <int DT>
__device__ __forceinline__ void load_group(const void* p, int64_t i, int n, bool vec, float v[4]) {
  if (vec) {
    if constexpr (DT == SF_DTYPE_F32) {
      const float4 q = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + i);
      v[0] = q.x;
      v[1] = q.y;
      v[2] = q.z;
      v[3] = q.w;
    } else {
      const uint2 q = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p) + i);
      v[0] = bf16_to_f32(static_cast<uint16_t>(q.x & 0xffffu));
      v[1] = bf16_to_f32(static_cast<uint16_t>(q.x >> 16));
      v[2] = bf16_to_f32(static_cast<uint16_t>(q.y & 0xffffu));
      v[3] = bf16_to_f32(static_cast<uint16_t>(q.y >> 16));
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = j < n ? load_as_f32(p, i + j, DT) : 0.0f;
  }
}

// Per-thread accumulators: f64 sums (f32 inputs add exactly), u32 counts.
struct Acc {
  double s[kSlots];
  uint32_t n[kSlots];
};

// The summed terms of one element (every f64 slot but TOP2 / BOT2).  The
// entropy term -(c ln c) - (1 - c) ln(1 - c) is evaluated in f32 and summed in
// f64, in log2 units (ln 2 multiplies each workgroup's sum once).  The
// reference takes both logs in f64, where 1 - c is exact; here 1 - c = u + t
// exactly with u = fl(1 - c) and t its rounding error (Fast2Sum: 1 >= c), so
// (1 - c) log2(1 - c) = u log2 u + t (log2 u + 1 / ln 2) to within t^2 / u.
// v_log_f32 is within 1 ulp of log2 over the clamped range [eps, 1] (u is 0
// or at least 2^-24, never denormal), so every term is within a few f32 ulp
// of the f64 one; log1pf would cost three times the memory pass.  c == 1
// gives 0 * -inf = NaN, as in f64.
template <int DT>
__device__ __forceinline__ void add_sums(const StatSpec& s, float x, Acc& a) {
  const double d = static_cast<double>(x);
  a.s[SF_MSTAT_SUM] += d;
  a.s[SF_MSTAT_SUM2] += d * d;
  // m.clamp(eps, 1 - eps) in the mask dtype (NaN passes through)
  float c = x < s.lo ? s.lo : (x > s.hi ? s.hi : x);
  c = rnd<DT>(c);
  const float u = 1.0f - c;
  const float t = -c - (u - 1.0f);
  const float lu = __builtin_amdgcn_logf(u);
  const float ent2 = -(c * __builtin_amdgcn_logf(c)) - (u * lu + t * (lu + kInvLn2));
  a.s[SF_MSTAT_ENTROPY] += static_cast<double>(ent2);
  a.s[SF_MSTAT_SUM_LT05] += x < 0.5f ? d : 0.0;
  a.s[SF_MSTAT_SUM_GT05] += x > 0.5f ? d : 0.0;
  // m * (1 - m): both operations rounded to the mask dtype, as torch evaluates them
  const float om = rnd<DT>(1.0f - x);
  a.s[SF_MSTAT_MID] += static_cast<double>(rnd<DT>(x * om));
}

// The counted tests of one element, in the order of kCountSlot.
constexpr int kNCount = 8;
constexpr int kCountSlot[kNCount] = {SF_MSTAT_LT05, SF_MSTAT_LT01, SF_MSTAT_LT001,     SF_MSTAT_GT90,
                                     SF_MSTAT_GT99, SF_MSTAT_GT05, SF_MSTAT_NONFINITE, SF_MSTAT_TAIL_LT05};
__device__ __forceinline__ void count_tests(const StatSpec& s, float x, bool tail, bool (&b)[kNCount]) {
  b[0] = x < 0.5f;
  b[1] = x < s.t01;
  b[2] = x < s.t001;
  b[3] = x > s.t90;
  b[4] = x > s.t99;
  b[5] = x > 0.5f;
  b[6] = !isfinite(x);
  b[7] = tail && b[0];
}

// TOP2 / BOT2 of a full group: members ranked by the descending sort order
// (ordered keys: NaN largest, -0 == +0; equal keys by position).  Only which
// values land in each pair matters for the two sums, so a group without NaN
// takes them from a min / max network (the two pair sums are exact in f64);
// a group holding NaN ranks its members by key.
__device__ __forceinline__ void add_tile(const float v[4], Acc& a) {
  float top[2], bot[2];
  if (!(isnan(v[0]) || isnan(v[1]) || isnan(v[2]) || isnan(v[3]))) {
    const float h0 = fmaxf(v[0], v[1]), l0 = fminf(v[0], v[1]);
    const float h1 = fmaxf(v[2], v[3]), l1 = fminf(v[2], v[3]);
    top[0] = fmaxf(h0, h1);
    bot[0] = fminf(l0, l1);
    const float mh = fminf(h0, h1), ml = fmaxf(l0, l1);  // the middle two
    top[1] = fmaxf(mh, ml);
    bot[1] = fminf(mh, ml);
  } else {
    uint32_t key[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) key[i] = ordered_key(v[i]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      int r = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) r += (key[j] > key[i]) || (j < i && key[j] == key[i]);
      if (r == 0) top[0] = v[i];
      if (r == 1) top[1] = v[i];
      if (r == 2) bot[0] = v[i];
      if (r == 3) bot[1] = v[i];
    }
  }
  a.s[SF_MSTAT_TOP2] += static_cast<double>(top[0]) + static_cast<double>(top[1]);
  a.s[SF_MSTAT_BOT2] += static_cast<double>(bot[0]) + static_cast<double>(bot[1]);
}

// Sum of each slot over the workgroup in a fixed tree order; thread t < kSlots
// of the workgroup gets slot t.
__device__ __forceinline__ double block_fold(double (&a)[kSlots]) {
  __shared__ double red[kBlock / 64][kSlots];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
#pragma unroll
  for (int k = 0; k < kSlots; ++k) {
    double v = a[k];
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    a[k] = v;
  }
  if (lane == 0) {
#pragma unroll
    for (int k = 0; k < kSlots; ++k) red[wv][k] = a[k];
  }
  __syncthreads();
  double t = 0.0;
  if (threadIdx.x < kSlots)
    for (int w = 0; w < kBlock / 64; ++w) t += red[w][threadIdx.x];
  return t;
}

// One group of the walk: its sums into `a`; its counts into the wave-uniform
// `wc` through ballots when every lane of the wave is live (WAVE), else into
// each lane's own counts.
template <int DT, bool VEC, bool WAVE>
__device__ __forceinline__ void stats_values(const StatSpec& s, const float (&v)[4], const Group& g, Acc& a,
                                             uint32_t (&wc)[kNCount]) {
  const int n = VEC ? 4 : g.n;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (VEC || j < n) add_sums<DT>(s, v[j], a);
    bool b[kNCount];
    count_tests(s, v[j], g.col + j >= s.tail_col, b);
#pragma unroll
    for (int k = 0; k < kNCount; ++k) {
      const bool hit = (VEC || j < n) && b[k];
      if constexpr (WAVE)
        wc[k] += static_cast<uint32_t>(__popcll(__ballot(hit)));
      else
        a.n[kCountSlot[k]] += hit;
    }
  }
  if (VEC || n == 4) add_tile(v, a);
}

template <int DT, bool VEC, bool WAVE>
__device__ __forceinline__ void stats_group(const StatSpec& s, const void* __restrict__ mask, const Group& g, Acc& a,
                                            uint32_t (&wc)[kNCount]) {
  float v[4];
  load_group<DT>(mask, g.elem, g.n, VEC || (s.vec && g.full), v);
  stats_values<DT, VEC, WAVE>(s, v, g, a, wc);
}

template <int DT, bool VEC>
__global__ void __launch_bounds__(kBlock) mask_stats_partial_kernel(StatSpec s, const void* __restrict__ mask,
                                                                    double* __restrict__ partial) {
  Acc a;
#pragma unroll
  for (int k = 0; k < kSlots; ++k) {
    a.s[k] = 0.0;
    a.n[k] = 0u;
  }
  uint32_t wc[kNCount];
#pragma unroll
  for (int k = 0; k < kNCount; ++k) wc[k] = 0u;
  GroupWalk w(s.groups, s.cols, s.gpr);
  // Walk steps in which every lane of the wave is live (the wave's last lane
  // has its largest group index): the step count is wave-uniform.  The stride
  // is at least one workgroup, so at most one step with some lanes past the
  // end remains.
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
  int64_t wave_last = static_cast<int64_t>(blockIdx.x) * kBlock +
                      static_cast<int64_t>(__builtin_amdgcn_readfirstlane(threadIdx.x) | 63u);
  if constexpr (VEC) {
    // software-pipelined: the next step's 16 bytes are requested before this
    // step's arithmetic (lanes past the end re-read their current group, so the
    // load stays unconditional and its wait counted)
    if (wave_last < s.groups) {
      Group g = w.group();
      float v[4];
      load_group<DT>(mask, g.elem, 4, true, v);
      for (;;) {
        w.next();
        wave_last += stride;
        const Group gn = w.group();
        float nv[4];
        load_group<DT>(mask, w.live() ? gn.elem : g.elem, 4, true, nv);
        stats_values<DT, VEC, true>(s, v, g, a, wc);
        g = gn;
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = nv[j];
        if (wave_last >= s.groups) break;
      }
      if (w.live()) stats_values<DT, VEC, false>(s, v, g, a, wc);
    } else if (w.live()) {
      stats_group<DT, VEC, false>(s, mask, w.group(), a, wc);
    }
  } else {
    for (; wave_last < s.groups; wave_last += stride, w.next()) stats_group<DT, VEC, true>(s, mask, w.group(), a, wc);
    if (w.live()) stats_group<DT, VEC, false>(s, mask, w.group(), a, wc);
  }
  // lane 0 is live whenever any lane of its wave is: it carries the wave's counts
  if ((threadIdx.x & 63) == 0) {
#pragma unroll
    for (int k = 0; k < kNCount; ++k) a.n[kCountSlot[k]] += wc[k];
  }
  double t[kSlots];
#pragma unroll
  for (int k = 0; k < kSlots; ++k) t[k] = a.s[k] + static_cast<double>(a.n[k]);  // each slot is a sum or a count
  double tot = block_fold(t);
  if (threadIdx.x == SF_MSTAT_ENTROPY) tot *= kLn2;  // the entropy was summed in log2 units
  if (threadIdx.x < kSlots) partial[blockIdx.x * (int64_t)kSlots + threadIdx.x] = tot;
}

// out[k] = sum over the parts.  Thread t reads slot t % 16 of parts t / 16,
// t / 16 + 16, ... (consecutive threads read consecutive doubles), then the
// 16 partial sums of each slot are added in a fixed order (deterministic).
static_assert(kSlots == 16 && kBlock == 256, "the final fold maps 16 slots x 16 part strides onto the workgroup");
__global__ void __launch_bounds__(kBlock) mask_stats_final_kernel(const double* __restrict__ partial, int nparts,
                                                                  double* __restrict__ out) {
  __shared__ double red[kBlock];
  const int k = threadIdx.x & 15, p0 = threadIdx.x >> 4;
  double t0 = 0.0, t1 = 0.0, t2 = 0.0, t3 = 0.0;  // four chains: the loads are not serialised by the adds
  int p = p0;
  for (; p + 48 < nparts; p += 64) {
    t0 += partial[p * (int64_t)kSlots + k];
    t1 += partial[(p + 16) * (int64_t)kSlots + k];
    t2 += partial[(p + 32) * (int64_t)kSlots + k];
    t3 += partial[(p + 48) * (int64_t)kSlots + k];
  }
  for (; p < nparts; p += 16) t0 += partial[p * (int64_t)kSlots + k];
  red[threadIdx.x] = (t0 + t1) + (t2 + t3);
  __syncthreads();
  if (threadIdx.x < kSlots) {
    double tot = 0.0;
#pragma unroll
    for (int j = 0; j < 16; ++j) tot += red[j * 16 + threadIdx.x];
    out[threadIdx.x] = tot;
  }
}

__global__ void __launch_bounds__(kBlock) mask_hist_kernel(const void* __restrict__ mask, int dtype, int64_t n,
                                                           const int64_t* __restrict__ idx, int64_t take, int bins,
                                                           float lo, float hi, unsigned long long* __restrict__ hist) {
  const float span = hi - lo, fb = static_cast<float>(bins);
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < take; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t j = idx[i];
    if (j < 0 || j >= n) continue;
    const float x = load_as_f32(mask, j, dtype);
    if (!(x >= lo && x <= hi)) continue;
    int b = static_cast<int>((x - lo) * fb / span);
    if (b >= bins) b = bins - 1;
    atomicAdd(&hist[b], 1ull);
  }
}

__global__ void __launch_bounds__(kBlock) keep_split_sum_kernel(const float* __restrict__ v,
                                                                const float* __restrict__ keep, int64_t n,
                                                                double* __restrict__ out) {
  double up = 0.0, lo = 0.0;
  for (int64_t i = threadIdx.x; i < n; i += kBlock) {
    const double x = static_cast<double>(v[i]);
    if (keep[i] != 0.0f)
      up += x;
    else
      lo += x;
  }
  __shared__ double red[2][kBlock];
  red[0][threadIdx.x] = up;
  red[1][threadIdx.x] = lo;
  __syncthreads();
  for (int h = kBlock / 2; h > 0; h >>= 1) {
    if (threadIdx.x < h) {
      red[0][threadIdx.x] += red[0][threadIdx.x + h];
      red[1][threadIdx.x] += red[1][threadIdx.x + h];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    out[0] = red[0][0];
    out[1] = red[1][0];
  }
}

}  // namespace
}  // namespace sf

using namespace sf;

extern "C" size_t sf_mask_stats_workspace_size(void) { return sizeof(double) * kParts * kSlots; }

extern "C" int sf_mask_stats(const void* mask, int dtype, int64_t rows, int64_t cols, int64_t tail_col, float eps,
                             double* out, void* workspace, size_t workspace_bytes, void* stream) {
  SF_CHECK_ARG(dtype == SF_DTYPE_F32 || dtype == SF_DTYPE_BF16, "bad mask dtype %d", dtype);
  SF_CHECK_ARG(rows >= 0 && cols >= 0, "negative shape");
  SF_CHECK_ARG(out, "null output");
  SF_CHECK_ARG(rows * cols == 0 || mask, "null mask");
  SF_CHECK_ARG(workspace && workspace_bytes >= sf_mask_stats_workspace_size(), "workspace too small");
  StatSpec s;
  s.cols = cols;
  s.gpr = ceil_div(cols, 4);
  s.groups = rows * s.gpr;
  s.tail_col = tail_col < 0 ? 0 : tail_col;
  s.lo = eps;
  s.hi = static_cast<float>(1.0 - static_cast<double>(eps));
  auto in_dtype = [&](float t) { return dtype == SF_DTYPE_BF16 ? round_bf16(t) : t; };
  s.t01 = in_dtype(0.1f);
  s.t001 = in_dtype(0.01f);
  s.t90 = in_dtype(0.9f);
  s.t99 = in_dtype(0.99f);
  const int64_t align = dtype == SF_DTYPE_F32 ? 16 : 8;
  s.vec = cols % 4 == 0 && (reinterpret_cast<uintptr_t>(mask) % align) == 0;
  hipStream_t st = static_cast<hipStream_t>(stream);
  double* partial = static_cast<double*>(workspace);
  int nparts = 0;
  if (s.groups > 0) {
    nparts = static_cast<int>(ceil_div(s.groups, kBlock) < kParts ? ceil_div(s.groups, kBlock) : kParts);
    if (dtype == SF_DTYPE_F32) {
      if (s.vec)
        mask_stats_partial_kernel<SF_DTYPE_F32, true><<<nparts, kBlock, 0, st>>>(s, mask, partial);
      else
        mask_stats_partial_kernel<SF_DTYPE_F32, false><<<nparts, kBlock, 0, st>>>(s, mask, partial);
    } else {
      if (s.vec)
        mask_stats_partial_kernel<SF_DTYPE_BF16, true><<<nparts, kBlock, 0, st>>>(s, mask, partial);
      else
        mask_stats_partial_kernel<SF_DTYPE_BF16, false><<<nparts, kBlock, 0, st>>>(s, mask, partial);
    }
    if (int rc = launch_status("sf_mask_stats")) return rc;
  }
  mask_stats_final_kernel<<<1, kBlock, 0, st>>>(partial, nparts, out);
  return launch_status("sf_mask_stats (final)");
}

extern "C" int sf_mask_hist(const void* mask, int dtype, int64_t n, const int64_t* idx, int64_t take, int bins,
                            float lo, float hi, unsigned long long* hist, void* stream) {
  SF_CHECK_ARG(dtype == SF_DTYPE_F32 || dtype == SF_DTYPE_BF16, "bad mask dtype %d", dtype);
  SF_CHECK_ARG(n >= 0 && take >= 0, "negative size");
  SF_CHECK_ARG(bins > 0, "bins must be positive");
  SF_CHECK_ARG(hi > lo, "histogram range: hi (%g) must exceed lo (%g)", (double)hi, (double)lo);
  SF_CHECK_ARG(hist, "null histogram");
  if (take == 0 || n == 0) return SF_OK;
  SF_CHECK_ARG(mask && idx, "null tensor");
  hipStream_t st = static_cast<hipStream_t>(stream);
  mask_hist_kernel<<<elementwise_grid(take, kBlock), kBlock, 0, st>>>(mask, dtype, n, idx, take, bins, lo, hi, hist);
  return launch_status("sf_mask_hist");
}

extern "C" int sf_keep_split_sum(const float* v, const float* keep, int64_t n, double* out, void* stream) {
  SF_CHECK_ARG(n >= 0, "negative size");
  SF_CHECK_ARG(out, "null output");
  SF_CHECK_ARG(n == 0 || (v && keep), "null tensor");
  hipStream_t st = static_cast<hipStream_t>(stream);
  keep_split_sum_kernel<<<1, kBlock, 0, st>>>(v, keep, n, out);
  return launch_status("sf_keep_split_sum");
}
