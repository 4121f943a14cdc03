// RMSNorm of the retraining student and teacher.  The reference retrains
// HuggingFace's LlamaForCausalLM (legacy/model_llama.py:18-57), whose
// LlamaRMSNorm (transformers 5.15, models/llama/modeling_llama.py) is
//   y = w * (x32 * rsqrt(mean(x32^2, -1) + eps)).to(x dtype),  x32 = x.float(),
// and the Hutchinson probe (legacy/utils.py:714-869) differentiates its
// backward once more.  Each of the three passes is one kernel over the rows:
//
//   forward          r = 1 / sqrt(sum(x^2) / D + eps) per row (kept for the
//                    backward passes), n = DT(x r), y = DT(w n)
//   backward         g = f32(DT(gy w)), A = sum g x,
//                    gx = DT(g r + ((-0.5 A) r^3 / D) (2 x)),   gw = sum over rows of DT(gy n)
//   double backward  with a = gy w, A = sum a x, G = sum ggx x, B = sum ggx a,
//                    C = sum ggw gy x (all per row) and c = r^3 / D:
//                    ggy = DT(r ggx w - c G w x + r ggw x)
//                    gx2 = DT(-c (B + C) x + 3 r^5 / D^2 A G x - c (a G + A ggx) + r ggw gy)
//                    gw2 = sum over rows of (r ggx gy - c G gy x)
//
// The forward and the backward evaluate torch's op sequence (the f32 products
// and the casts to the activations' dtype DT where torch rounds); the row sums
// run in another order than torch's reductions, so results agree to within f32
// rounding, not bit for bit.  The double backward is the closed form of the
// backward's derivatives in f32 (torch's autograd of the same ops rounds its
// intermediates to DT).  One wave per row holds it in registers (lane l: the
// 8-column chunks l, l + 64, ...).  The weight gradients are column sums over
// the rows: each workgroup folds its rows' terms per column and its four waves
// in a fixed order into one partial row, and a column pass adds the partial
// rows in a fixed order (the number of workgroups depends only on the shape, so
// the sums are reproducible).
#include <initializer_list>
#include <type_traits>

#include "sf_common.hpp"

namespace sf {
namespace {

constexpr int kNrWaves = 4;        // rows in flight per workgroup, one wave each
constexpr int kNrMaxCols = 4096;   // row length bound: 8 chunks of 8 per lane
constexpr int kNrColGroups = 1024;  // most workgroups of the passes with weight gradients (a row per wave
                                    // up to 4096 rows)

__device__ __forceinline__ float nr_wave_sum(float v) {
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// round to the activations' dtype (bf16: nearest even, as .to() does)
template <int DT>
__device__ __forceinline__ float dt_round(float x) {
  if constexpr (DT == SF_DTYPE_BF16)
    return static_cast<float>(static_cast<__bf16>(x));
  else
    return x;
}

template <int DT>
__device__ __forceinline__ void nr_ld8(const void* p, int64_t e0, float (&v)[8]) {
  if constexpr (DT == SF_DTYPE_F32) {
    const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + e0);
    const float4 b = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + e0 + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    const uint4 q = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p) + e0);
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[2 * k] = __uint_as_float(w[k] << 16);
      v[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
    }
  }
}

template <int DT>
__device__ __forceinline__ void nr_st8(void* p, int64_t e0, const float (&v)[8]) {
  if constexpr (DT == SF_DTYPE_F32) {
    *reinterpret_cast<float4*>(static_cast<float*>(p) + e0) = make_float4(v[0], v[1], v[2], v[3]);
    *reinterpret_cast<float4*>(static_cast<float*>(p) + e0 + 4) = make_float4(v[4], v[5], v[6], v[7]);
  } else {
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t lo = __builtin_bit_cast(uint16_t, static_cast<__bf16>(v[2 * k]));
      const uint32_t hi = __builtin_bit_cast(uint16_t, static_cast<__bf16>(v[2 * k + 1]));
      w[k] = lo | (hi << 16);
    }
    *reinterpret_cast<uint4*>(static_cast<uint16_t*>(p) + e0) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

struct NormArgs {
  const void* x;    // [rows, D]
  const void* w;    // [D]
  const void* gy;   // [rows, D] (backward passes)
  const void* ggx;  // [rows, D] (double backward)
  const void* ggw;  // [D] or null (double backward)
  float* rstd;      // [rows]: written by the forward, read by the backward passes
  void* out0;       // y / gx / ggy
  void* out1;       // gx2 (double backward)
  float* part;      // [gridDim.x, D] weight-gradient partial rows
  int64_t rows, D;
  float eps, inv_d, fd;  // 1 / D and D as f32
};

// The workgroup's per-lane column terms acc (lane's chunks) folded over its four waves
// in wave order into partial row blockIdx.x.
template <int NJ>
__device__ __forceinline__ void fold_columns(const NormArgs& a, const float (&acc)[NJ][8]) {
  extern __shared__ float red[];  // [kNrWaves][D]
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int64_t e0 = 8 * (lane + 64 * j);
    if (e0 < a.D) {
#pragma unroll
      for (int k = 0; k < 8; ++k) red[wv * a.D + e0 + k] = acc[j][k];
    }
  }
  __syncthreads();
  for (int64_t c = threadIdx.x; c < a.D; c += blockDim.x) {
    float t = red[c];
#pragma unroll
    for (int q = 1; q < kNrWaves; ++q) t += red[q * a.D + c];
    a.part[static_cast<int64_t>(blockIdx.x) * a.D + c] = t;
  }
}

template <int DT, int NJ>
__global__ void __launch_bounds__(64 * kNrWaves) rms_fwd_kernel(NormArgs a) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kNrWaves + (threadIdx.x >> 6);
  if (row >= a.rows) return;  // the whole wave: no workgroup barrier in this kernel
  const int lane = threadIdx.x & 63;
  const void* xr = static_cast<const char*>(a.x) + row * a.D * (DT == SF_DTYPE_F32 ? 4 : 2);
  float v[NJ][8];
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int64_t e0 = 8 * (lane + 64 * j);
    if (e0 < a.D) {
      nr_ld8<DT>(xr, e0, v[j]);
#pragma unroll
      for (int k = 0; k < 8; ++k) s += v[j][k] * v[j][k];
    }
  }
  s = nr_wave_sum(s);
  const float r = 1.0f / sqrtf(s * a.inv_d + a.eps);
  if (lane == 0) a.rstd[row] = r;
  void* yr = static_cast<char*>(a.out0) + row * a.D * (DT == SF_DTYPE_F32 ? 4 : 2);
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int64_t e0 = 8 * (lane + 64 * j);
    if (e0 < a.D) {
      float wv[8], o[8];
      nr_ld8<DT>(a.w, e0, wv);
#pragma unroll
      for (int k = 0; k < 8; ++k) o[k] = wv[k] * dt_round<DT>(v[j][k] * r);
      nr_st8<DT>(yr, e0, o);
    }
  }
}

template <int DT, int NJ>
__global__ void __launch_bounds__(64 * kNrWaves) rms_bwd_kernel(NormArgs a) {
  const int lane = threadIdx.x & 63;
  const size_t esz = DT == SF_DTYPE_F32 ? 4 : 2;
  float wv[NJ][8], acc[NJ][8];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int64_t e0 = 8 * (lane + 64 * j);
#pragma unroll
    for (int k = 0; k < 8; ++k) acc[j][k] = 0.0f;
    if (e0 < a.D) nr_ld8<DT>(a.w, e0, wv[j]);
  }
  // rows of this wave: a wave-uniform count, so every wave reaches the fold's barrier
  for (int64_t row = static_cast<int64_t>(blockIdx.x) * kNrWaves + (threadIdx.x >> 6); row < a.rows;
       row += static_cast<int64_t>(gridDim.x) * kNrWaves) {
    const float r = a.rstd[row];
    const void* xr = static_cast<const char*>(a.x) + row * a.D * esz;
    const void* gr = static_cast<const char*>(a.gy) + row * a.D * esz;
    float xv[NJ][8], gv[NJ][8], dn[NJ][8];
    float sa = 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int64_t e0 = 8 * (lane + 64 * j);
      if (e0 < a.D) {
        nr_ld8<DT>(xr, e0, xv[j]);
        nr_ld8<DT>(gr, e0, gv[j]);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          dn[j][k] = dt_round<DT>(gv[j][k] * wv[j][k]);
          sa += dn[j][k] * xv[j][k];
        }
      }
    }
    sa = nr_wave_sum(sa);
    const float gp = ((-0.5f * sa) * (r * r * r)) / a.fd;  // rsqrt's then mean's backward
    void* outr = static_cast<char*>(a.out0) + row * a.D * esz;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int64_t e0 = 8 * (lane + 64 * j);
      if (e0 < a.D) {
        float o[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          o[k] = dn[j][k] * r + gp * (2.0f * xv[j][k]);
          acc[j][k] += dt_round<DT>(gv[j][k] * dt_round<DT>(xv[j][k] * r));
        }
        nr_st8<DT>(outr, e0, o);
      }
    }
  }
  fold_columns<NJ>(a, acc);
}

template <int DT, int NJ, bool GGW>
__global__ void __launch_bounds__(64 * kNrWaves) rms_dbwd_kernel(NormArgs a) {
  const int lane = threadIdx.x & 63;
  const size_t esz = DT == SF_DTYPE_F32 ? 4 : 2;
  float wv[NJ][8], qv[NJ][8], acc[NJ][8];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int64_t e0 = 8 * (lane + 64 * j);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      acc[j][k] = 0.0f;
      qv[j][k] = 0.0f;
    }
    if (e0 < a.D) {
      nr_ld8<DT>(a.w, e0, wv[j]);
      if constexpr (GGW) nr_ld8<DT>(a.ggw, e0, qv[j]);
    }
  }
  for (int64_t row = static_cast<int64_t>(blockIdx.x) * kNrWaves + (threadIdx.x >> 6); row < a.rows;
       row += static_cast<int64_t>(gridDim.x) * kNrWaves) {
    const float r = a.rstd[row];
    const void* xr = static_cast<const char*>(a.x) + row * a.D * esz;
    const void* gr = static_cast<const char*>(a.gy) + row * a.D * esz;
    const void* hr = static_cast<const char*>(a.ggx) + row * a.D * esz;
    float xv[NJ][8], gv[NJ][8], hv[NJ][8];
    float sA = 0.0f, sG = 0.0f, sB = 0.0f, sC = 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int64_t e0 = 8 * (lane + 64 * j);
      if (e0 < a.D) {
        nr_ld8<DT>(xr, e0, xv[j]);
        nr_ld8<DT>(gr, e0, gv[j]);
        nr_ld8<DT>(hr, e0, hv[j]);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const float av = gv[j][k] * wv[j][k];
          sA += av * xv[j][k];
          sG += hv[j][k] * xv[j][k];
          sB += hv[j][k] * av;
          if constexpr (GGW) sC += qv[j][k] * gv[j][k] * xv[j][k];
        }
      }
    }
    sA = nr_wave_sum(sA);
    sG = nr_wave_sum(sG);
    sB = nr_wave_sum(sB);
    if constexpr (GGW) sC = nr_wave_sum(sC);
    const float r3 = r * r * r;
    const float c = r3 / a.fd;
    const float cx = -c * (sB + sC) + (3.0f * r3 * r * r / (a.fd * a.fd)) * sA * sG;  // coefficient of x in gx2
    void* o0 = static_cast<char*>(a.out0) + row * a.D * esz;
    void* o1 = static_cast<char*>(a.out1) + row * a.D * esz;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int64_t e0 = 8 * (lane + 64 * j);
      if (e0 < a.D) {
        float ggy[8], gx2[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const float x = xv[j][k], g = gv[j][k], h = hv[j][k], w = wv[j][k], q = qv[j][k];
          const float av = g * w;
          ggy[k] = r * h * w - c * sG * w * x + r * q * x;
          gx2[k] = cx * x - c * (av * sG + sA * h) + r * q * g;
          acc[j][k] += r * h * g - c * sG * g * x;
        }
        nr_st8<DT>(o0, e0, ggy);
        nr_st8<DT>(o1, e0, gx2);
      }
    }
  }
  fold_columns<NJ>(a, acc);
}

// out[c] = sum over the partial rows of part[p][c], cast to the weight's dtype: a workgroup takes 64
// columns, its thread group q (0..3) the rows p = q, q + 4, ... in increasing order (16 loads in
// flight per thread), and the four group sums are added in q order (a fixed order: reproducible).
__global__ void __launch_bounds__(256) rms_colsum_kernel(const float* __restrict__ part, int64_t nparts, int64_t D,
                                                         void* out, int dt) {
  __shared__ float red[4][64];
  const int l = threadIdx.x & 63, q = threadIdx.x >> 6;
  const int64_t c = static_cast<int64_t>(blockIdx.x) * 64 + l;
  float acc = 0.0f;
  if (c < D) {
    int64_t p = q;
    for (; p + 4 * 15 < nparts; p += 4 * 16) {
      float v[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) v[j] = part[(p + 4 * j) * D + c];
#pragma unroll
      for (int j = 0; j < 16; ++j) acc += v[j];
    }
    for (; p < nparts; p += 4) acc += part[p * D + c];
  }
  red[q][l] = acc;
  __syncthreads();
  if (q == 0 && c < D) store_from_f32(out, c, dt, ((red[0][l] + red[1][l]) + red[2][l]) + red[3][l]);
}

int nr_chunks(int64_t D) {  // 8-column chunks per lane
  const int64_t per = ceil_div(D, 512);
  return per <= 1 ? 1 : per <= 2 ? 2 : per <= 4 ? 4 : 8;
}

int nr_checks(int dtype, int64_t rows, int64_t D, std::initializer_list<const void*> ptrs) {
  SF_CHECK_ARG(dtype == SF_DTYPE_BF16 || dtype == SF_DTYPE_F32, "dtype %d (bf16 or f32)", dtype);
  SF_CHECK_ARG(rows >= 0 && D > 0 && D % 8 == 0 && D <= kNrMaxCols,
               "rows %lld x %lld: the row length must be a multiple of 8 and at most %d", (long long)rows,
               (long long)D, kNrMaxCols);
  for (const void* p : ptrs) {
    SF_CHECK_ARG(p != nullptr, "null tensor");
    SF_CHECK_ARG((reinterpret_cast<uintptr_t>(p) & 15u) == 0, "tensors must be 16-byte aligned");
  }
  return SF_OK;
}

NormArgs nr_args(const void* x, const void* w, int64_t rows, int64_t D, float eps) {
  NormArgs a{};
  a.x = x;
  a.w = w;
  a.rows = rows;
  a.D = D;
  a.eps = eps;
  a.inv_d = 1.0f / static_cast<float>(D);
  a.fd = static_cast<float>(D);
  return a;
}

// workgroups of a pass with weight gradients: one per four rows up to kNrColGroups
unsigned nr_col_grid(int64_t rows) {
  const int64_t g = ceil_div(rows, kNrWaves);
  return static_cast<unsigned>(g < kNrColGroups ? (g > 0 ? g : 1) : kNrColGroups);
}

template <template <int, int> class K, typename F>
void nr_dispatch(int dtype, int nj, F&& f) {
  auto go = [&](auto dt) {
    constexpr int DT = decltype(dt)::value;
    switch (nj) {
      case 1: f(K<DT, 1>{}); break;
      case 2: f(K<DT, 2>{}); break;
      case 4: f(K<DT, 4>{}); break;
      default: f(K<DT, 8>{}); break;
    }
  };
  if (dtype == SF_DTYPE_F32)
    go(std::integral_constant<int, SF_DTYPE_F32>{});
  else
    go(std::integral_constant<int, SF_DTYPE_BF16>{});
}

template <int DT, int NJ>
struct FwdN {
  static constexpr auto fn = rms_fwd_kernel<DT, NJ>;
};
template <int DT, int NJ>
struct BwdN {
  static constexpr auto fn = rms_bwd_kernel<DT, NJ>;
};
template <int DT, int NJ>
struct DbwdN {
  static constexpr auto fn = rms_dbwd_kernel<DT, NJ, false>;
};
template <int DT, int NJ>
struct DbwdNQ {
  static constexpr auto fn = rms_dbwd_kernel<DT, NJ, true>;
};

int nr_colsum(const float* part, unsigned nparts, int64_t D, void* out, int dt, hipStream_t st) {
  hipLaunchKernelGGL(rms_colsum_kernel, dim3(static_cast<unsigned>(ceil_div(D, 64))), dim3(256), 0, st, part,
                     static_cast<int64_t>(nparts), D, out, dt);
  return launch_status("sf_rmsnorm (weight-gradient column sums)");
}

}  // namespace
}  // namespace sf

using namespace sf;

extern "C" size_t sf_rmsnorm_workspace_size(int64_t rows, int64_t cols) {
  if (rows < 0 || cols <= 0) return 0;
  return sizeof(float) * static_cast<size_t>(nr_col_grid(rows)) * static_cast<size_t>(cols);
}

extern "C" int sf_rmsnorm_forward(const void* x, const void* weight, int dtype, int64_t rows, int64_t cols, float eps,
                                  void* y, float* rstd, void* stream) {
  if (int rc = nr_checks(dtype, rows, cols, {x, weight, y, rstd})) return rc;
  if (rows == 0) return SF_OK;
  SF_CHECK_ARG(ceil_div(rows, kNrWaves) < (1ll << 31), "too many rows");
  NormArgs a = nr_args(x, weight, rows, cols, eps);
  a.out0 = y;
  a.rstd = rstd;
  hipStream_t st = static_cast<hipStream_t>(stream);
  nr_dispatch<FwdN>(dtype, nr_chunks(cols), [&](auto k) {
    hipLaunchKernelGGL(decltype(k)::fn, dim3(static_cast<unsigned>(ceil_div(rows, kNrWaves))), dim3(64 * kNrWaves),
                       0, st, a);
  });
  return launch_status("sf_rmsnorm_forward");
}

extern "C" int sf_rmsnorm_backward(const void* x, const void* weight, const void* grad_y, const float* rstd, int dtype,
                                   int64_t rows, int64_t cols, void* grad_x, void* grad_weight, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  if (int rc = nr_checks(dtype, rows, cols, {x, weight, grad_y, rstd, grad_x, grad_weight, workspace})) return rc;
  SF_CHECK_ARG(workspace_bytes >= sf_rmsnorm_workspace_size(rows, cols), "workspace too small");
  hipStream_t st = static_cast<hipStream_t>(stream);
  NormArgs a = nr_args(x, weight, rows, cols, 0.0f);
  a.gy = grad_y;
  a.rstd = const_cast<float*>(rstd);
  a.out0 = grad_x;
  a.part = static_cast<float*>(workspace);
  const unsigned grid = nr_col_grid(rows);
  const size_t smem = sizeof(float) * kNrWaves * static_cast<size_t>(cols);
  nr_dispatch<BwdN>(dtype, nr_chunks(cols), [&](auto k) {
    hipLaunchKernelGGL(decltype(k)::fn, dim3(grid), dim3(64 * kNrWaves), smem, st, a);
  });
  if (int rc = launch_status("sf_rmsnorm_backward")) return rc;
  return nr_colsum(a.part, grid, cols, grad_weight, dtype, st);
}

extern "C" int sf_rmsnorm_double_backward(const void* x, const void* weight, const void* grad_y, const float* rstd,
                                          const void* grad_grad_x, const void* grad_grad_weight, int dtype,
                                          int64_t rows, int64_t cols, void* grad_grad_y, void* grad2_x,
                                          void* grad2_weight, void* workspace, size_t workspace_bytes, void* stream) {
  if (int rc = nr_checks(dtype, rows, cols,
                         {x, weight, grad_y, rstd, grad_grad_x, grad_grad_y, grad2_x, grad2_weight, workspace}))
    return rc;
  if (grad_grad_weight)
    SF_CHECK_ARG((reinterpret_cast<uintptr_t>(grad_grad_weight) & 15u) == 0, "tensors must be 16-byte aligned");
  SF_CHECK_ARG(workspace_bytes >= sf_rmsnorm_workspace_size(rows, cols), "workspace too small");
  hipStream_t st = static_cast<hipStream_t>(stream);
  NormArgs a = nr_args(x, weight, rows, cols, 0.0f);
  a.gy = grad_y;
  a.ggx = grad_grad_x;
  a.ggw = grad_grad_weight;
  a.rstd = const_cast<float*>(rstd);
  a.out0 = grad_grad_y;
  a.out1 = grad2_x;
  a.part = static_cast<float*>(workspace);
  const unsigned grid = nr_col_grid(rows);
  const size_t smem = sizeof(float) * kNrWaves * static_cast<size_t>(cols);
  auto launch = [&](auto k) { hipLaunchKernelGGL(decltype(k)::fn, dim3(grid), dim3(64 * kNrWaves), smem, st, a); };
  if (grad_grad_weight)
    nr_dispatch<DbwdNQ>(dtype, nr_chunks(cols), launch);
  else
    nr_dispatch<DbwdN>(dtype, nr_chunks(cols), launch);
  if (int rc = launch_status("sf_rmsnorm_double_backward")) return rc;
  return nr_colsum(a.part, grid, cols, grad2_weight, dtype, st);
}
