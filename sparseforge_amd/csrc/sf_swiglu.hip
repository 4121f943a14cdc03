// The gated MLP product of the retraining student and teacher: HuggingFace's
// LlamaMLP (the LlamaForCausalLM the reference retrains, legacy/model_llama.py:18-57)
// computes down(silu(gate(x)) * up(x)); here y = silu(g) * u with g, u the two
// projections, and the Hutchinson probe (legacy/utils.py:714-869) differentiates
// its backward once more.  Each pass is one elementwise kernel (8 elements per
// thread), in f32 with the activations' dtype DT where torch rounds:
//
//   forward          s = DT(g / (1 + exp(-g))),  y = DT(s u)
//   backward         gg = DT(DT(gy u) sig (1 + g (1 - sig))),  gu = DT(gy s),  sig = 1 / (1 + exp(-g))
//   double backward  with s1 = sig (1 + g (1 - sig)) and s2 = sig (1 - sig) (2 + g (1 - 2 sig)) (the first
//                    and second derivatives of silu), given ggg, ggu (the gradients of gg, gu):
//                    dgy = DT(ggg u s1 + ggu s),  du = DT(ggg gy s1),  dg = DT(ggg gy u s2 + ggu gy s1)
//
// The forward and backward follow torch's silu / mul kernels and their autograd
// (silu_backward: dy sig (1 + x (1 - sig))); the double backward is the closed
// form in f32 (torch's autograd of the same ops rounds its intermediates to DT).
#include <initializer_list>
#include <type_traits>

#include "sf_common.hpp"

namespace sf {
namespace {

constexpr int kSgBlock = 256;

template <int DT>
__device__ __forceinline__ float sg_round(float x) {
  if constexpr (DT == SF_DTYPE_BF16)
    return static_cast<float>(static_cast<__bf16>(x));
  else
    return x;
}

template <int DT>
__device__ __forceinline__ void sg_ld8(const void* p, int64_t e0, float (&v)[8]) {
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
__device__ __forceinline__ void sg_st8(void* p, int64_t e0, const float (&v)[8]) {
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

struct SgArgs {
  const void* g;
  const void* u;
  const void* gy;
  const void* ggg;  // null: zero
  const void* ggu;  // null: zero
  void* o0;         // y / gg / dgy
  void* o1;         // gu / du
  void* o2;         // dg
  int64_t n;        // elements, a multiple of 8
};

template <int DT>
__global__ void __launch_bounds__(kSgBlock) swiglu_fwd_kernel(SgArgs a) {
  for (int64_t e0 = 8 * (static_cast<int64_t>(blockIdx.x) * kSgBlock + threadIdx.x); e0 < a.n;
       e0 += 8 * static_cast<int64_t>(gridDim.x) * kSgBlock) {
    float g[8], u[8], y[8];
    sg_ld8<DT>(a.g, e0, g);
    sg_ld8<DT>(a.u, e0, u);
#pragma unroll
    for (int k = 0; k < 8; ++k) y[k] = sg_round<DT>(g[k] / (1.0f + expf(-g[k]))) * u[k];
    sg_st8<DT>(a.o0, e0, y);
  }
}

template <int DT>
__global__ void __launch_bounds__(kSgBlock) swiglu_bwd_kernel(SgArgs a) {
  for (int64_t e0 = 8 * (static_cast<int64_t>(blockIdx.x) * kSgBlock + threadIdx.x); e0 < a.n;
       e0 += 8 * static_cast<int64_t>(gridDim.x) * kSgBlock) {
    float g[8], u[8], gy[8], gg[8], gu[8];
    sg_ld8<DT>(a.g, e0, g);
    sg_ld8<DT>(a.u, e0, u);
    sg_ld8<DT>(a.gy, e0, gy);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float ex = expf(-g[k]);
      const float sig = 1.0f / (1.0f + ex);
      gg[k] = (sg_round<DT>(gy[k] * u[k]) * sig) * (1.0f + g[k] * (1.0f - sig));
      gu[k] = gy[k] * sg_round<DT>(g[k] / (1.0f + ex));
    }
    sg_st8<DT>(a.o0, e0, gg);
    sg_st8<DT>(a.o1, e0, gu);
  }
}

template <int DT, bool HG, bool HU>
__global__ void __launch_bounds__(kSgBlock) swiglu_dbwd_kernel(SgArgs a) {
  for (int64_t e0 = 8 * (static_cast<int64_t>(blockIdx.x) * kSgBlock + threadIdx.x); e0 < a.n;
       e0 += 8 * static_cast<int64_t>(gridDim.x) * kSgBlock) {
    float g[8], u[8], gy[8], hg[8], hu[8], dgy[8], du[8], dg[8];
    sg_ld8<DT>(a.g, e0, g);
    sg_ld8<DT>(a.u, e0, u);
    sg_ld8<DT>(a.gy, e0, gy);
#pragma unroll
    for (int k = 0; k < 8; ++k) hg[k] = hu[k] = 0.0f;
    if constexpr (HG) sg_ld8<DT>(a.ggg, e0, hg);
    if constexpr (HU) sg_ld8<DT>(a.ggu, e0, hu);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float x = g[k], ex = expf(-x), sig = 1.0f / (1.0f + ex);
      const float s0 = sg_round<DT>(x / (1.0f + ex));  // the rounded silu the backward multiplied by
      const float s1 = sig * (1.0f + x * (1.0f - sig));
      const float s2 = sig * (1.0f - sig) * (2.0f + x * (1.0f - 2.0f * sig));
      dgy[k] = hg[k] * u[k] * s1 + hu[k] * s0;
      du[k] = hg[k] * gy[k] * s1;
      dg[k] = hg[k] * gy[k] * u[k] * s2 + hu[k] * gy[k] * s1;
    }
    sg_st8<DT>(a.o0, e0, dgy);
    sg_st8<DT>(a.o1, e0, du);
    sg_st8<DT>(a.o2, e0, dg);
  }
}

int sg_checks(int dtype, int64_t n, std::initializer_list<const void*> ptrs) {
  SF_CHECK_ARG(dtype == SF_DTYPE_BF16 || dtype == SF_DTYPE_F32, "dtype %d (bf16 or f32)", dtype);
  SF_CHECK_ARG(n >= 0 && n % 8 == 0, "element count %lld: a multiple of 8", (long long)n);
  for (const void* p : ptrs) {
    SF_CHECK_ARG(p != nullptr, "null tensor");
    SF_CHECK_ARG((reinterpret_cast<uintptr_t>(p) & 15u) == 0, "tensors must be 16-byte aligned");
  }
  return SF_OK;
}

unsigned sg_grid(int64_t n) { return elementwise_grid(ceil_div(n, 8), kSgBlock); }

}  // namespace
}  // namespace sf

using namespace sf;

extern "C" int sf_swiglu_forward(const void* g, const void* u, int dtype, int64_t n, void* y, void* stream) {
  if (int rc = sg_checks(dtype, n, {g, u, y})) return rc;
  if (n == 0) return SF_OK;
  SgArgs a{};
  a.g = g;
  a.u = u;
  a.o0 = y;
  a.n = n;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == SF_DTYPE_F32)
    hipLaunchKernelGGL(swiglu_fwd_kernel<SF_DTYPE_F32>, dim3(sg_grid(n)), dim3(kSgBlock), 0, st, a);
  else
    hipLaunchKernelGGL(swiglu_fwd_kernel<SF_DTYPE_BF16>, dim3(sg_grid(n)), dim3(kSgBlock), 0, st, a);
  return launch_status("sf_swiglu_forward");
}

extern "C" int sf_swiglu_backward(const void* g, const void* u, const void* grad_y, int dtype, int64_t n,
                                  void* grad_g, void* grad_u, void* stream) {
  if (int rc = sg_checks(dtype, n, {g, u, grad_y, grad_g, grad_u})) return rc;
  if (n == 0) return SF_OK;
  SgArgs a{};
  a.g = g;
  a.u = u;
  a.gy = grad_y;
  a.o0 = grad_g;
  a.o1 = grad_u;
  a.n = n;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == SF_DTYPE_F32)
    hipLaunchKernelGGL(swiglu_bwd_kernel<SF_DTYPE_F32>, dim3(sg_grid(n)), dim3(kSgBlock), 0, st, a);
  else
    hipLaunchKernelGGL(swiglu_bwd_kernel<SF_DTYPE_BF16>, dim3(sg_grid(n)), dim3(kSgBlock), 0, st, a);
  return launch_status("sf_swiglu_backward");
}

extern "C" int sf_swiglu_double_backward(const void* g, const void* u, const void* grad_y, const void* grad_grad_g,
                                         const void* grad_grad_u, int dtype, int64_t n, void* grad_grad_y,
                                         void* grad2_g, void* grad2_u, void* stream) {
  if (int rc = sg_checks(dtype, n, {g, u, grad_y, grad_grad_y, grad2_g, grad2_u})) return rc;
  for (const void* p : {grad_grad_g, grad_grad_u})
    SF_CHECK_ARG((reinterpret_cast<uintptr_t>(p) & 15u) == 0, "tensors must be 16-byte aligned");
  if (n == 0) return SF_OK;
  SgArgs a{};
  a.g = g;
  a.u = u;
  a.gy = grad_y;
  a.ggg = grad_grad_g;
  a.ggu = grad_grad_u;
  a.o0 = grad_grad_y;
  a.o1 = grad2_u;
  a.o2 = grad2_g;
  a.n = n;
  hipStream_t st = static_cast<hipStream_t>(stream);
  auto go = [&](auto dt) {
    constexpr int DT = decltype(dt)::value;
    const dim3 gd(sg_grid(n)), bd(kSgBlock);
    if (grad_grad_g && grad_grad_u)
      hipLaunchKernelGGL((swiglu_dbwd_kernel<DT, true, true>), gd, bd, 0, st, a);
    else if (grad_grad_g)
      hipLaunchKernelGGL((swiglu_dbwd_kernel<DT, true, false>), gd, bd, 0, st, a);
    else if (grad_grad_u)
      hipLaunchKernelGGL((swiglu_dbwd_kernel<DT, false, true>), gd, bd, 0, st, a);
    else
      hipLaunchKernelGGL((swiglu_dbwd_kernel<DT, false, false>), gd, bd, 0, st, a);
  };
  if (dtype == SF_DTYPE_F32)
    go(std::integral_constant<int, SF_DTYPE_F32>{});
  else
    go(std::integral_constant<int, SF_DTYPE_BF16>{});
  return launch_status("sf_swiglu_double_backward");
}
