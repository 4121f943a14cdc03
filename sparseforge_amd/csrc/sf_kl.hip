// Distillation KL of Distill_Model.kl_loss (legacy/sparse_modeling.py:1749-1828)
// on gfx950: KL(P_teacher || Q_student) at temperature T over the vocabulary,
// logits clamped to +-100, summed per chunk of tokens; a chunk whose
// log-probabilities hold a NaN (a NaN logit) is skipped, a non-finite chunk sum
// is dropped, and the total is scaled by T^2 / tokens.
//
// One workgroup per token row streams both logit rows once (HBM-bound: 2
// elements read per vocabulary entry).  With a = clamp(s) / T, b = clamp(t) / T
// and running maxima ms, mt:
//   Zs = sum exp(a - ms), Zt = sum exp(b - mt), A = sum exp(b - mt) (b - a)
//   KL_row = sum p (log p - log q) = A / Zt - (mt + log Zt) + (ms + log Zs)
// Each thread keeps (ms, Zs, mt, Zt, A) over 8-element slices, rescaling when a
// slice raises a maximum; the workgroup merges them, and the row's KL is formed
// in f64.  A single-workgroup pass then sums rows per chunk in f64 in a fixed
// order, applies the chunk skips, and writes the loss and the per-row gradient
// scale (0 for skipped chunks).  The backward pass re-reads both rows:
//   dL/ds = g (T / tokens) (q - p) [-100 <= s <= 100].

#include <initializer_list>

#include "sf_common.hpp"

namespace sf {
namespace {

constexpr int kKlBlock = 256;
constexpr int kKlFinalBlock = 1024;
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kKlU = 4;  // slices of a row a thread loads before using them (forward)
constexpr int kKlBwdU = 4;  // the same for the backward

__device__ __forceinline__ float exp_f(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }

typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// 8 consecutive logits as f32.  The vector paths load non-temporally: the logits (gigabytes) stream
// through once per pass, and nothing re-reads them before they are evicted.
template <int DT>
__device__ __forceinline__ void load8(const void* base, int64_t i, int n, bool vec, float v[8]) {
  if (DT == SF_DTYPE_F32) {
    const float* p = static_cast<const float*>(base) + i;
    if (vec) {
      const f32x4_t x = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(p));
      const f32x4_t y = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(p + 4));
      v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w; v[4] = y.x; v[5] = y.y; v[6] = y.z; v[7] = y.w;
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] = k < n ? p[k] : 0.0f;
    }
  } else {
    const uint16_t* p = static_cast<const uint16_t*>(base) + i;
    if (vec) {
      const u32x4_t x = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
      const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        v[2 * k] = bf16_to_f32(static_cast<uint16_t>(w[k] & 0xffffu));
        v[2 * k + 1] = bf16_to_f32(static_cast<uint16_t>(w[k] >> 16));
      }
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] = k < n ? bf16_to_f32(p[k]) : 0.0f;
    }
  }
}

// Round to nearest even bf16 with the hardware conversion (a NaN stays a NaN: only a
// non-finite upstream gradient can bring one here).
__device__ __forceinline__ uint16_t bf16_rne(float x) { return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x)); }

template <int DT>
__device__ __forceinline__ void store8(void* base, int64_t i, int n, bool vec, const float v[8]) {
  if (DT == SF_DTYPE_F32) {
    float* p = static_cast<float*>(base) + i;
    if (vec) {
      __builtin_nontemporal_store(f32x4_t{v[0], v[1], v[2], v[3]}, reinterpret_cast<f32x4_t*>(p));
      __builtin_nontemporal_store(f32x4_t{v[4], v[5], v[6], v[7]}, reinterpret_cast<f32x4_t*>(p + 4));
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (k < n) p[k] = v[k];
    }
  } else {
    uint16_t* p = static_cast<uint16_t*>(base) + i;
    if (vec) {
      uint32_t w[4];
#pragma unroll
      for (int k = 0; k < 4; ++k)
        w[k] = static_cast<uint32_t>(bf16_rne(v[2 * k])) | (static_cast<uint32_t>(bf16_rne(v[2 * k + 1])) << 16);
      __builtin_nontemporal_store(u32x4_t{w[0], w[1], w[2], w[3]}, reinterpret_cast<u32x4_t*>(p));
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (k < n) p[k] = bf16_rne(v[k]);
    }
  }
}

// clamp(x, -100, 100) / T as the reference's clamp_ then mul_(1 / T), the clamp as
// one v_med3 (equal to min(max(x, -100), 100) for every x but NaN).  A NaN logit's
// value here does not matter: the row's NaN flag drops its chunk from the loss and
// zeroes the chunk's gradient.
__device__ __forceinline__ float scaled(float x, float inv_t) {
  return __builtin_amdgcn_fmed3f(x, -100.0f, 100.0f) * inv_t;
}

struct KlAcc {
  float ms, zs, mt, zt, a;
};

__device__ __forceinline__ KlAcc kl_merge(KlAcc x, KlAcc y) {
  KlAcc r;
  if (y.ms == -INFINITY) {
    r.ms = x.ms; r.zs = x.zs;
  } else if (x.ms == -INFINITY) {
    r.ms = y.ms; r.zs = y.zs;
  } else {
    r.ms = fmaxf(x.ms, y.ms);
    r.zs = x.zs * exp_f(x.ms - r.ms) + y.zs * exp_f(y.ms - r.ms);
  }
  if (y.mt == -INFINITY) {
    r.mt = x.mt; r.zt = x.zt; r.a = x.a;
  } else if (x.mt == -INFINITY) {
    r.mt = y.mt; r.zt = y.zt; r.a = y.a;
  } else {
    r.mt = fmaxf(x.mt, y.mt);
    const float ex = exp_f(x.mt - r.mt), ey = exp_f(y.mt - r.mt);
    r.zt = x.zt * ex + y.zt * ey;
    r.a = x.a * ex + y.a * ey;
  }
  return r;
}

__device__ __forceinline__ KlAcc kl_shfl_xor(const KlAcc& x, int off) {
  KlAcc y;
  y.ms = __shfl_xor(x.ms, off, 64);
  y.zs = __shfl_xor(x.zs, off, 64);
  y.mt = __shfl_xor(x.mt, off, 64);
  y.zt = __shfl_xor(x.zt, off, 64);
  y.a = __shfl_xor(x.a, off, 64);
  return y;
}

// One 8-element slice of a row into a thread's accumulators: the slice maxima,
// a rescale only when a maximum rises, then the exp sums (n < 8: a partial
// slice, whose missing elements do not count).
__device__ __forceinline__ void kl_slice(KlAcc& acc, bool& bad, float (&a)[8], float (&b)[8], int n, float inv_t) {
  float cs = -INFINITY, ct = -INFINITY;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    if (k < n) {
      bad |= __builtin_isunordered(a[k], b[k]);
      a[k] = scaled(a[k], inv_t);
      b[k] = scaled(b[k], inv_t);
      cs = fmaxf(cs, a[k]);
      ct = fmaxf(ct, b[k]);
    }
  }
  if (cs > acc.ms) {
    acc.zs *= exp_f(acc.ms - cs);
    acc.ms = cs;
  }
  if (ct > acc.mt) {
    const float sc = exp_f(acc.mt - ct);
    acc.zt *= sc;
    acc.a *= sc;
    acc.mt = ct;
  }
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    if (k < n) {
      acc.zs += exp_f(a[k] - acc.ms);
      const float e = exp_f(b[k] - acc.mt);
      acc.zt += e;
      acc.a = fmaf(e, b[k] - a[k], acc.a);
    }
  }
}

// One workgroup per token row; thread t takes slices t, t + 256, ... in order.
// VEC (vocab % 8 == 0, 16-byte aligned rows): every slice is whole and a
// thread's next two slices of both rows are loaded before either is used.
template <int DT, bool VEC>
__global__ void __launch_bounds__(kKlBlock) kl_rows_kernel(const void* __restrict__ s, const void* __restrict__ t,
                                                           int64_t vocab, float inv_t, double* __restrict__ lse,
                                                           double* __restrict__ row_kl, int* __restrict__ row_nan) {
  const int64_t r = blockIdx.x, base = r * vocab;
  KlAcc acc{-INFINITY, 0.0f, -INFINITY, 0.0f, 0.0f};
  bool bad = false;
  if constexpr (VEC) {
    const int64_t slices = vocab / 8, step = blockDim.x;
    int64_t c = threadIdx.x;
    for (; c + (kKlU - 1) * step < slices; c += kKlU * step) {
      float a[kKlU][8], b[kKlU][8];
#pragma unroll
      for (int u = 0; u < kKlU; ++u) {
        load8<DT>(s, base + 8 * (c + u * step), 8, true, a[u]);
        load8<DT>(t, base + 8 * (c + u * step), 8, true, b[u]);
      }
#pragma unroll
      for (int u = 0; u < kKlU; ++u) kl_slice(acc, bad, a[u], b[u], 8, inv_t);
    }
    for (; c < slices; c += step) {
      float a0[8], b0[8];
      load8<DT>(s, base + 8 * c, 8, true, a0);
      load8<DT>(t, base + 8 * c, 8, true, b0);
      kl_slice(acc, bad, a0, b0, 8, inv_t);
    }
  } else {
    for (int64_t j0 = threadIdx.x * 8; j0 < vocab; j0 += 8 * (int64_t)blockDim.x) {
      const int n = vocab - j0 >= 8 ? 8 : static_cast<int>(vocab - j0);
      float a[8], b[8];
      load8<DT>(s, base + j0, n, false, a);
      load8<DT>(t, base + j0, n, false, b);
      kl_slice(acc, bad, a, b, n, inv_t);
    }
  }
  int nan = bad;
  for (int off = 32; off > 0; off >>= 1) acc = kl_merge(acc, kl_shfl_xor(acc, off));
  for (int off = 32; off > 0; off >>= 1) nan |= __shfl_xor(nan, off, 64);
  __shared__ KlAcc part[kKlBlock / 64];
  __shared__ int pnan[kKlBlock / 64];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  if (lane == 0) {
    part[wv] = acc;
    pnan[wv] = nan;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    KlAcc x = part[0];
    int nn = pnan[0];
    for (int w = 1; w < (int)(blockDim.x / 64); ++w) {
      x = kl_merge(x, part[w]);
      nn |= pnan[w];
    }
    const double ls = static_cast<double>(x.ms) + log(static_cast<double>(x.zs));
    const double lt = static_cast<double>(x.mt) + log(static_cast<double>(x.zt));
    lse[2 * r] = ls;
    lse[2 * r + 1] = lt;
    row_kl[r] = static_cast<double>(x.a) / static_cast<double>(x.zt) - lt + ls;
    row_nan[r] = nn;
  }
}

// Sum rows per chunk in a fixed order; skip chunks with a NaN row or a non-finite
// sum; loss = (f32(total) * T^2) / tokens in f32, cast to out_dtype, 0 if not
// finite; row_scale = T / tokens for kept rows, 0 for skipped ones (and for all
// rows when the loss is replaced by 0, which then carries no gradient).
__global__ void __launch_bounds__(kKlFinalBlock) kl_final_kernel(const double* __restrict__ row_kl,
                                                                 const int* __restrict__ row_nan, int64_t rows,
                                                                 int64_t chunk, float temperature, float t_sq,
                                                                 float* __restrict__ row_scale, void* out,
                                                                 int out_dtype) {
  __shared__ double ssum[kKlFinalBlock / 64];
  __shared__ int snan[kKlFinalBlock / 64];
  __shared__ int s_ok;
  __shared__ double s_total;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, nw = blockDim.x / 64;
  const float grad_scale = static_cast<float>(static_cast<double>(temperature) / static_cast<double>(rows));
  if (tid == 0) s_total = 0.0;
  for (int64_t c0 = 0; c0 < rows; c0 += chunk) {
    const int64_t c1 = c0 + chunk < rows ? c0 + chunk : rows;
    double sum = 0.0;
    int nan = 0;
    for (int64_t i = c0 + tid; i < c1; i += blockDim.x) {
      sum += row_kl[i];
      nan |= row_nan[i];
    }
    for (int off = 32; off > 0; off >>= 1) {
      sum += __shfl_xor(sum, off, 64);
      nan |= __shfl_xor(nan, off, 64);
    }
    if (lane == 0) {
      ssum[wv] = sum;
      snan[wv] = nan;
    }
    __syncthreads();
    if (tid == 0) {
      double cs = 0.0;
      int cn = 0;
      for (int w = 0; w < nw; ++w) {
        cs += ssum[w];
        cn |= snan[w];
      }
      const int ok = !cn && isfinite(cs);
      if (ok) s_total += cs;
      s_ok = ok;
    }
    __syncthreads();
    const float sc = s_ok ? grad_scale : 0.0f;
    for (int64_t i = c0 + tid; i < c1; i += blockDim.x) row_scale[i] = sc;
    __syncthreads();
  }
  if (tid == 0) {
    float kl = static_cast<float>(s_total) * t_sq;
    kl = kl / static_cast<float>(rows);
    const float stored = out_dtype == SF_DTYPE_BF16 ? round_bf16(kl) : kl;
    const int ok = isfinite(stored);
    store_from_f32(out, 0, out_dtype, ok ? stored : 0.0f);
    s_ok = ok;
  }
  __syncthreads();
  if (!s_ok)
    for (int64_t i = tid; i < rows; i += blockDim.x) row_scale[i] = 0.0f;
}

// d loss / d student logit: factor (q - p) inside the clamp range, 0 outside it.
__device__ __forceinline__ float kl_grad1(float a, float b, float inv_t, double ls, double lt, float factor) {
  const bool in_range = a >= -100.0f && a <= 100.0f;  // clamp passes the gradient inside [min, max]
  const float q = exp_f(static_cast<float>(static_cast<double>(scaled(a, inv_t)) - ls));
  const float p = exp_f(static_cast<float>(static_cast<double>(scaled(b, inv_t)) - lt));
  return in_range ? factor * (q - p) : 0.0f;
}

// One workgroup per token row, slices as in kl_rows_kernel (VEC: kKlBwdU
// slices' loads in flight per thread); rows whose chunk was dropped get zeros.
template <int DT, bool VEC>
__global__ void __launch_bounds__(kKlBlock) kl_backward_kernel(const void* __restrict__ s, const void* __restrict__ t,
                                                               int64_t vocab, float inv_t,
                                                               const double* __restrict__ lse,
                                                               const float* __restrict__ row_scale,
                                                               const void* __restrict__ gout, int gout_dtype,
                                                               void* __restrict__ gs) {
  const int64_t r = blockIdx.x, base = r * vocab;
  const float factor = row_scale[r] * load_as_f32(gout, 0, gout_dtype);
  const double ls = lse[2 * r], lt = lse[2 * r + 1];
  if constexpr (VEC) {
    const int64_t slices = vocab / 8, step = blockDim.x;
    if (factor == 0.0f) {
      const float z[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
      for (int64_t c = threadIdx.x; c < slices; c += step) store8<DT>(gs, base + 8 * c, 8, true, z);
      return;
    }
    int64_t c = threadIdx.x;
    for (; c + (kKlBwdU - 1) * step < slices; c += kKlBwdU * step) {
      float a[kKlBwdU][8], b[kKlBwdU][8];
#pragma unroll
      for (int u = 0; u < kKlBwdU; ++u) {
        load8<DT>(s, base + 8 * (c + u * step), 8, true, a[u]);
        load8<DT>(t, base + 8 * (c + u * step), 8, true, b[u]);
      }
#pragma unroll
      for (int u = 0; u < kKlBwdU; ++u) {
#pragma unroll
        for (int k = 0; k < 8; ++k) a[u][k] = kl_grad1(a[u][k], b[u][k], inv_t, ls, lt, factor);
        store8<DT>(gs, base + 8 * (c + u * step), 8, true, a[u]);
      }
    }
    for (; c < slices; c += step) {
      float a0[8], b0[8];
      load8<DT>(s, base + 8 * c, 8, true, a0);
      load8<DT>(t, base + 8 * c, 8, true, b0);
#pragma unroll
      for (int k = 0; k < 8; ++k) a0[k] = kl_grad1(a0[k], b0[k], inv_t, ls, lt, factor);
      store8<DT>(gs, base + 8 * c, 8, true, a0);
    }
  } else {
    for (int64_t j0 = threadIdx.x * 8; j0 < vocab; j0 += 8 * (int64_t)blockDim.x) {
      const int n = vocab - j0 >= 8 ? 8 : static_cast<int>(vocab - j0);
      float a[8], b[8], g[8];
      load8<DT>(s, base + j0, n, false, a);
      if (factor != 0.0f) load8<DT>(t, base + j0, n, false, b);
#pragma unroll
      for (int k = 0; k < 8; ++k) g[k] = factor == 0.0f ? 0.0f : kl_grad1(a[k], b[k], inv_t, ls, lt, factor);
      store8<DT>(gs, base + j0, n, false, g);
    }
  }
}

bool kl_dtype_ok(int d) { return d == SF_DTYPE_F32 || d == SF_DTYPE_BF16; }
bool kl_vec_ok(int64_t vocab, int dtype, std::initializer_list<const void*> ptrs) {
  if (vocab % 8 != 0) return false;
  for (const void* p : ptrs)
    if (reinterpret_cast<uintptr_t>(p) % 16 != 0) return false;
  (void)dtype;
  return true;
}
size_t a256(size_t b) { return (b + 255) / 256 * 256; }
}  // namespace
}  // namespace sf

using namespace sf;

extern "C" int64_t sf_kl_chunk_rows(int64_t vocab) { return vocab > 100000 ? 128 : (vocab > 50000 ? 512 : 2048); }

extern "C" size_t sf_kl_workspace_size(int64_t rows) {
  if (rows <= 0) return 0;
  const size_t r = static_cast<size_t>(rows);
  return a256(r * sizeof(double)) + a256(r * sizeof(int));
}

extern "C" int sf_kl_forward(const void* student, const void* teacher, int dtype, int64_t rows, int64_t vocab,
                             float temperature, int64_t chunk_rows, void* out, int out_dtype, double* row_lse,
                             float* row_scale, void* workspace, size_t workspace_bytes, void* stream) {
  SF_CHECK_ARG(rows > 0 && vocab > 0, "empty logits [%lld, %lld]", (long long)rows, (long long)vocab);
  SF_CHECK_ARG(kl_dtype_ok(dtype) && kl_dtype_ok(out_dtype), "bad dtype");
  SF_CHECK_ARG(student && teacher && out && row_lse && row_scale, "null tensor");
  SF_CHECK_ARG(temperature > 0.0f, "temperature must be positive");
  SF_CHECK_ARG(chunk_rows > 0, "chunk_rows must be positive");
  SF_CHECK_ARG(rows < (1ll << 31), "more than 2^31 token rows");
  SF_CHECK_ARG(workspace && workspace_bytes >= sf_kl_workspace_size(rows), "workspace too small");
  double* row_kl = static_cast<double*>(workspace);
  int* row_nan = reinterpret_cast<int*>(static_cast<char*>(workspace) + a256(static_cast<size_t>(rows) * 8));
  const float inv_t = static_cast<float>(1.0 / static_cast<double>(temperature));
  const bool vec = kl_vec_ok(vocab, dtype, {student, teacher});
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(rows));
#define SF_KL_ROWS(DT, V) kl_rows_kernel<DT, V><<<grid, kKlBlock, 0, st>>>(student, teacher, vocab, inv_t, row_lse, \
                                                                          row_kl, row_nan)
  if (dtype == SF_DTYPE_F32) {
    if (vec)
      SF_KL_ROWS(SF_DTYPE_F32, true);
    else
      SF_KL_ROWS(SF_DTYPE_F32, false);
  } else {
    if (vec)
      SF_KL_ROWS(SF_DTYPE_BF16, true);
    else
      SF_KL_ROWS(SF_DTYPE_BF16, false);
  }
#undef SF_KL_ROWS
  const float t_sq = static_cast<float>(static_cast<double>(temperature) * static_cast<double>(temperature));
  kl_final_kernel<<<1, kKlFinalBlock, 0, st>>>(row_kl, row_nan, rows, chunk_rows, temperature, t_sq, row_scale, out,
                                               out_dtype);
  return launch_status("sf_kl_forward");
}

extern "C" int sf_kl_backward(const void* student, const void* teacher, int dtype, int64_t rows, int64_t vocab,
                              float temperature, const double* row_lse, const float* row_scale, const void* grad_out,
                              int grad_out_dtype, void* grad_student, void* stream) {
  SF_CHECK_ARG(rows > 0 && vocab > 0, "empty logits");
  SF_CHECK_ARG(kl_dtype_ok(dtype) && kl_dtype_ok(grad_out_dtype), "bad dtype");
  SF_CHECK_ARG(student && teacher && row_lse && row_scale && grad_out && grad_student, "null tensor");
  SF_CHECK_ARG(temperature > 0.0f, "temperature must be positive");
  SF_CHECK_ARG(rows < (1ll << 31), "more than 2^31 token rows");
  const float inv_t = static_cast<float>(1.0 / static_cast<double>(temperature));
  const bool vec = kl_vec_ok(vocab, dtype, {student, teacher, grad_student});
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(rows));
#define SF_KL_BWD(DT, V)                                                                                    \
  kl_backward_kernel<DT, V><<<grid, kKlBlock, 0, st>>>(student, teacher, vocab, inv_t, row_lse, row_scale, grad_out, \
                                                       grad_out_dtype, grad_student)
  if (dtype == SF_DTYPE_F32) {
    if (vec)
      SF_KL_BWD(SF_DTYPE_F32, true);
    else
      SF_KL_BWD(SF_DTYPE_F32, false);
  } else {
    if (vec)
      SF_KL_BWD(SF_DTYPE_BF16, true);
    else
      SF_KL_BWD(SF_DTYPE_BF16, false);
  }
#undef SF_KL_BWD
  return launch_status("sf_kl_backward");
}
