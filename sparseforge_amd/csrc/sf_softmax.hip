// Attention softmax of the retraining student and teacher (the eager attention
// the reference retrains with, legacy/model_llama.py:39-55: p =
// softmax(scores, dim=-1, dtype=float32).to(scores.dtype)), with its backward
// and the double backward of that backward (the Hutchinson HVP differentiates
// the backward once more, legacy/utils.py:714-869), each fused into one pass.
//
// Rows are the last dimension of [batches, S, S] scores; with `causal`, row i
// of each S x S block keeps columns 0..i and its masked tail (scores -inf)
// has probability exactly 0, so the kernels read only the kept columns and
// write zeros past them.  One wave per row holds the row in registers (lane l:
// the 8-column chunks l, l + 64, ...).  Every pass recomputes y = softmax(x)
// in f32 from the scores it is given, bit for bit the forward's y, so the
// autograd keeps the scores (x's dtype) instead of an f32 copy of y.
//
//   forward          p   = DT(y)
//   backward         gx  = DT(y (g - c)),                     c = sum y g,   g = f32(gp)
//   double backward  ggp = DT(y (h - d)),                     d = sum y h,   h = f32(ggx)
//                    u   = g h - c h - d g                    (the gradient reaching y)
//                    gx2 = DT(y (u - e)),                     e = sum y u
// (torch's _softmax_backward_data, softmax_double_backward and the softmax
// backward that carries u to the scores; the cast to x's dtype rounds to
// nearest even as .to() does.)
#include <initializer_list>
#include <type_traits>

#include "sf_common.hpp"

namespace sf {
namespace {

constexpr int kSmWaves = 4;  // rows per workgroup, one wave each

__device__ __forceinline__ float wave_max(float v) {
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ uint16_t to_bf16_rne(float x) { return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x)); }

typedef float f32x4_nt __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_nt __attribute__((ext_vector_type(4)));

// 8 elements of a row from column e0 (VEC: one 16- or 32-byte load; else
// element by element, columns at or past n read as `fill`).
template <int DT, bool VEC>
__device__ __forceinline__ void ld8(const void* row, int64_t e0, int64_t n, float fill, float (&v)[8]) {
  if constexpr (VEC) {
    if constexpr (DT == SF_DTYPE_F32) {
      const f32x4_nt a = __builtin_nontemporal_load(reinterpret_cast<const f32x4_nt*>(static_cast<const float*>(row) + e0));
      const f32x4_nt b =
          __builtin_nontemporal_load(reinterpret_cast<const f32x4_nt*>(static_cast<const float*>(row) + e0 + 4));
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
      const u32x4_nt q = __builtin_nontemporal_load(reinterpret_cast<const u32x4_nt*>(static_cast<const uint16_t*>(row) + e0));
      const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        v[2 * k] = __uint_as_float(w[k] << 16);
        v[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
      }
    }
  } else {
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = e0 + k < n ? load_as_f32(row, e0 + k, DT) : fill;
  }
}

template <int DT, bool VEC>
__device__ __forceinline__ void st8(void* row, int64_t e0, int64_t n, const float (&v)[8]) {
  if constexpr (VEC) {
    if constexpr (DT == SF_DTYPE_F32) {
      __builtin_nontemporal_store(f32x4_nt{v[0], v[1], v[2], v[3]}, reinterpret_cast<f32x4_nt*>(static_cast<float*>(row) + e0));
      __builtin_nontemporal_store(f32x4_nt{v[4], v[5], v[6], v[7]},
                                  reinterpret_cast<f32x4_nt*>(static_cast<float*>(row) + e0 + 4));
    } else {
      uint32_t w[4];
#pragma unroll
      for (int k = 0; k < 4; ++k)
        w[k] = static_cast<uint32_t>(to_bf16_rne(v[2 * k])) | (static_cast<uint32_t>(to_bf16_rne(v[2 * k + 1])) << 16);
      __builtin_nontemporal_store(u32x4_nt{w[0], w[1], w[2], w[3]}, reinterpret_cast<u32x4_nt*>(static_cast<uint16_t*>(row) + e0));
    }
  } else {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if (e0 + k < n) {
        if constexpr (DT == SF_DTYPE_F32)
          static_cast<float*>(row)[e0 + k] = v[k];
        else
          static_cast<uint16_t*>(row)[e0 + k] = to_bf16_rne(v[k]);
      }
    }
  }
}

struct SmRow {
  int64_t r, L;  // row, kept columns
};

__device__ __forceinline__ bool sm_row(int64_t rows, int64_t S, int causal, SmRow& w) {
  w.r = static_cast<int64_t>(blockIdx.x) * kSmWaves + (threadIdx.x >> 6);
  if (w.r >= rows) return false;  // the whole wave: the kernels use no workgroup barrier
  w.L = causal ? w.r % S + 1 : S;
  return true;
}

// y = softmax of the row's kept columns (chunk j of the lane: columns 8 (lane + 64 j) ..), 0 past them.
template <int DT, bool VEC, int NJ>
__device__ __forceinline__ void row_softmax(const void* xrow, int64_t L, float (&y)[NJ][8]) {
  const int lane = threadIdx.x & 63;
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int64_t e0 = 8 * (lane + 64 * j);
    if (e0 < L) {
      ld8<DT, VEC>(xrow, e0, L, -INFINITY, y[j]);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        if (e0 + k >= L) y[j][k] = -INFINITY;
        m = fmaxf(m, y[j][k]);
      }
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k) y[j][k] = -INFINITY;
    }
  }
  m = wave_max(m);
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      y[j][k] = expf(y[j][k] - m);
      s += y[j][k];
    }
  s = wave_sum(s);
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int k = 0; k < 8; ++k) y[j][k] = y[j][k] / s;
}

// Load the kept part of another row of the same shape (0 past L).
template <int DT, bool VEC, int NJ>
__device__ __forceinline__ void row_load(const void* row, int64_t L, float (&v)[NJ][8]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int64_t e0 = 8 * (lane + 64 * j);
    if (e0 < L) {
      ld8<DT, VEC>(row, e0, L, 0.0f, v[j]);
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (e0 + k >= L) v[j][k] = 0.0f;
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k) v[j][k] = 0.0f;
    }
  }
}

// Store a whole row (S columns): the values' chunks, zeros for chunks wholly past L.
template <int DT, bool VEC, int NJ>
__device__ __forceinline__ void row_store(void* row, int64_t S, int64_t L, const float (&v)[NJ][8]) {
  const int lane = threadIdx.x & 63;
  const float zero[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int64_t e0 = 8 * (lane + 64 * j);
    if (e0 < S) st8<DT, VEC>(row, e0, S, e0 < L ? v[j] : zero);
  }
}

template <int DT, bool VEC, int NJ>
__global__ void __launch_bounds__(64 * kSmWaves) softmax_fwd_kernel(const void* __restrict__ x, void* __restrict__ p,
                                                                   int64_t rows, int64_t S, int causal) {
  SmRow w;
  if (!sm_row(rows, S, causal, w)) return;
  const size_t es = DT == SF_DTYPE_F32 ? 4 : 2;
  float y[NJ][8];
  row_softmax<DT, VEC, NJ>(static_cast<const char*>(x) + w.r * S * es, w.L, y);
  row_store<DT, VEC, NJ>(static_cast<char*>(p) + w.r * S * es, S, w.L, y);
}

template <int DT, bool VEC, int NJ>
__global__ void __launch_bounds__(64 * kSmWaves) softmax_bwd_kernel(const void* __restrict__ x,
                                                                   const void* __restrict__ gp, void* __restrict__ gx,
                                                                   int64_t rows, int64_t S, int causal) {
  SmRow w;
  if (!sm_row(rows, S, causal, w)) return;
  const size_t es = DT == SF_DTYPE_F32 ? 4 : 2;
  const int64_t off = w.r * S * es;
  float y[NJ][8], g[NJ][8];
  row_load<DT, VEC, NJ>(static_cast<const char*>(gp) + off, w.L, g);
  row_softmax<DT, VEC, NJ>(static_cast<const char*>(x) + off, w.L, y);
  float c = 0.0f;
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int k = 0; k < 8; ++k) c += g[j][k] * y[j][k];
  c = wave_sum(c);
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int k = 0; k < 8; ++k) g[j][k] = y[j][k] * (g[j][k] - c);
  row_store<DT, VEC, NJ>(static_cast<char*>(gx) + off, S, w.L, g);
}

template <int DT, bool VEC, int NJ>
__global__ void __launch_bounds__(64 * kSmWaves) softmax_dbwd_kernel(const void* __restrict__ x,
                                                                    const void* __restrict__ gp,
                                                                    const void* __restrict__ ggx,
                                                                    void* __restrict__ ggp, void* __restrict__ gx2,
                                                                    int64_t rows, int64_t S, int causal) {
  SmRow w;
  if (!sm_row(rows, S, causal, w)) return;
  const size_t es = DT == SF_DTYPE_F32 ? 4 : 2;
  const int64_t off = w.r * S * es;
  float y[NJ][8], g[NJ][8], h[NJ][8];
  row_load<DT, VEC, NJ>(static_cast<const char*>(gp) + off, w.L, g);
  row_load<DT, VEC, NJ>(static_cast<const char*>(ggx) + off, w.L, h);
  row_softmax<DT, VEC, NJ>(static_cast<const char*>(x) + off, w.L, y);
  float c = 0.0f, d = 0.0f;
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      c += g[j][k] * y[j][k];
      d += h[j][k] * y[j][k];
    }
  c = wave_sum(c);
  d = wave_sum(d);
  // u (the gradient reaching y) into g, ggp into h
  float e = 0.0f;
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float u = g[j][k] * h[j][k] - c * h[j][k] - d * g[j][k];
      h[j][k] = y[j][k] * (h[j][k] - d);
      g[j][k] = u;
      e += u * y[j][k];
    }
  e = wave_sum(e);
  row_store<DT, VEC, NJ>(static_cast<char*>(ggp) + off, S, w.L, h);
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int k = 0; k < 8; ++k) g[j][k] = y[j][k] * (g[j][k] - e);
  row_store<DT, VEC, NJ>(static_cast<char*>(gx2) + off, S, w.L, g);
}

constexpr int64_t kSmMaxCols = 64 * 8 * 8;  // NJ <= 8: 4096 columns held in registers

int sm_checks(int dtype, int64_t rows, int64_t S, std::initializer_list<const void*> ptrs) {
  SF_CHECK_ARG(dtype == SF_DTYPE_F32 || dtype == SF_DTYPE_BF16, "bad dtype %d", dtype);
  SF_CHECK_ARG(rows >= 0 && S > 0, "bad shape [%lld, %lld]", (long long)rows, (long long)S);
  SF_CHECK_ARG(S <= kSmMaxCols, "rows of %lld columns exceed the %lld the row softmax holds in registers",
               (long long)S, (long long)kSmMaxCols);
  for (const void* p : ptrs) SF_CHECK_ARG(rows == 0 || p, "null tensor");
  return SF_OK;
}

bool sm_vec(int64_t S, std::initializer_list<const void*> ptrs) {
  if (S % 8) return false;
  for (const void* p : ptrs)
    if (reinterpret_cast<uintptr_t>(p) % 16) return false;
  return true;
}

// NJ = chunks per lane: the smallest power of two with 512 NJ >= S.
template <template <int, bool, int> class K, typename F>
void sm_dispatch(int dtype, bool vec, int64_t S, F&& launch) {
  const int nj = S <= 512 ? 1 : S <= 1024 ? 2 : S <= 2048 ? 4 : 8;
  auto go = [&](auto dt_c, auto vec_c) {
    constexpr int DT = decltype(dt_c)::value;
    constexpr bool V = decltype(vec_c)::value;
    switch (nj) {
      case 1: launch(K<DT, V, 1>{}); break;
      case 2: launch(K<DT, V, 2>{}); break;
      case 4: launch(K<DT, V, 4>{}); break;
      default: launch(K<DT, V, 8>{}); break;
    }
  };
  using F32 = std::integral_constant<int, SF_DTYPE_F32>;
  using B16 = std::integral_constant<int, SF_DTYPE_BF16>;
  using T = std::true_type;
  using Fa = std::false_type;
  if (dtype == SF_DTYPE_F32)
    vec ? go(F32{}, T{}) : go(F32{}, Fa{});
  else
    vec ? go(B16{}, T{}) : go(B16{}, Fa{});
}

// Kernel tags: each names one instantiation for sm_dispatch.
template <int DT, bool V, int NJ>
struct FwdK {
  static constexpr auto fn = softmax_fwd_kernel<DT, V, NJ>;
};
template <int DT, bool V, int NJ>
struct BwdK {
  static constexpr auto fn = softmax_bwd_kernel<DT, V, NJ>;
};
template <int DT, bool V, int NJ>
struct DbwdK {
  static constexpr auto fn = softmax_dbwd_kernel<DT, V, NJ>;
};

unsigned sm_grid(int64_t rows) { return static_cast<unsigned>(ceil_div(rows, kSmWaves)); }

}  // namespace
}  // namespace sf

using namespace sf;

extern "C" int sf_softmax_rows(const void* x, int dtype, int64_t rows, int64_t cols, int causal, void* p,
                               void* stream) {
  if (int rc = sm_checks(dtype, rows, cols, {x, p})) return rc;
  if (rows == 0) return SF_OK;
  SF_CHECK_ARG(ceil_div(rows, kSmWaves) < (1ll << 31), "too many rows");
  hipStream_t st = static_cast<hipStream_t>(stream);
  sm_dispatch<FwdK>(dtype, sm_vec(cols, {x, p}), cols, [&](auto k) {
    hipLaunchKernelGGL(decltype(k)::fn, dim3(sm_grid(rows)), dim3(64 * kSmWaves), 0, st, x, p, rows, cols, causal);
  });
  return launch_status("sf_softmax_rows");
}

extern "C" int sf_softmax_rows_backward(const void* x, const void* grad_p, int dtype, int64_t rows, int64_t cols,
                                        int causal, void* grad_x, void* stream) {
  if (int rc = sm_checks(dtype, rows, cols, {x, grad_p, grad_x})) return rc;
  if (rows == 0) return SF_OK;
  SF_CHECK_ARG(ceil_div(rows, kSmWaves) < (1ll << 31), "too many rows");
  hipStream_t st = static_cast<hipStream_t>(stream);
  sm_dispatch<BwdK>(dtype, sm_vec(cols, {x, grad_p, grad_x}), cols, [&](auto k) {
    hipLaunchKernelGGL(decltype(k)::fn, dim3(sm_grid(rows)), dim3(64 * kSmWaves), 0, st, x, grad_p, grad_x, rows,
                       cols, causal);
  });
  return launch_status("sf_softmax_rows_backward");
}

extern "C" int sf_softmax_rows_double_backward(const void* x, const void* grad_p, const void* grad_grad_x,
                                               int dtype, int64_t rows, int64_t cols, int causal, void* grad_grad_p,
                                               void* grad2_x, void* stream) {
  if (int rc = sm_checks(dtype, rows, cols, {x, grad_p, grad_grad_x, grad_grad_p, grad2_x})) return rc;
  if (rows == 0) return SF_OK;
  SF_CHECK_ARG(ceil_div(rows, kSmWaves) < (1ll << 31), "too many rows");
  hipStream_t st = static_cast<hipStream_t>(stream);
  sm_dispatch<DbwdK>(dtype, sm_vec(cols, {x, grad_p, grad_grad_x, grad_grad_p, grad2_x}), cols, [&](auto k) {
    hipLaunchKernelGGL(decltype(k)::fn, dim3(sm_grid(rows)), dim3(64 * kSmWaves), 0, st, x, grad_p, grad_grad_x,
                       grad_grad_p, grad2_x, rows, cols, causal);
  });
  return launch_status("sf_softmax_rows_double_backward");
}
