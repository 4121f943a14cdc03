// Hutchinson Hessian-diagonal estimation (K9) on gfx950.
//
// update_hessian_hutchinson (legacy/utils.py:714-869) draws a Rademacher
// probe v per SparseLinear weight, forms dot = sum_W sum(g_W * v_W) from the
// first-order gradients (create_graph=True), takes hvp = d dot / d W through
// the double backward, and folds est = clamp(hvp * v, 0) into the layer's
// hessian_diag by an EMA.  Here:
//
//   sf_rademacher          v materialised (the backward of the dot needs it)
//   sf_rademacher_dot      sum(g * v) with v regenerated on the fly
//   sf_hutchinson_update   H <- beta H + (1 - beta) clamp(hvp * v, 0): one pass,
//                          v regenerated from (seed, index) -- 0 bytes of HBM --
//                          or read from an explicit tensor (parity tests feed
//                          the reference's own probes).
//
// v(seed, i) = +1 / -1 from bit i % 64 of SplitMix64 output i / 64 of the
// stream seeded with `seed` (sf_rng.hpp): a pure function of (seed, i), so
// the dot, the backward and the update agree on v without storing it.

#include "sf_common.hpp"
#include "sf_rng.hpp"

namespace sf {
namespace {

constexpr int kBlock = 256;
constexpr int kDotGrid = 1024;

__device__ __forceinline__ float rnd(float x, int dtype) { return dtype == SF_DTYPE_BF16 ? round_bf16(x) : x; }

__device__ __forceinline__ float probe(const void* v, int v_dtype, uint64_t seed, int64_t i) {
  return v ? load_as_f32(v, i, v_dtype) : rademacher(seed, static_cast<uint64_t>(i));
}

__global__ void __launch_bounds__(kBlock) rademacher_kernel(void* v, int dtype, int64_t n, uint64_t seed) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    store_from_f32(v, i, dtype, rademacher(seed, static_cast<uint64_t>(i)));
}

// Per-workgroup f64 partial sums of g * v (fixed grid: deterministic), then one
// workgroup folds them in index order.
__global__ void __launch_bounds__(kBlock) rademacher_dot_partial(const void* __restrict__ g, int g_dtype,
                                                                 const void* __restrict__ v, int v_dtype, int64_t n,
                                                                 uint64_t seed, double* __restrict__ partial) {
  double s = 0.0;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    s += static_cast<double>(load_as_f32(g, i, g_dtype)) * probe(v, v_dtype, seed, i);
  __shared__ double red[kBlock / 64];
  for (int off = 32; off > 0; off >>= 1) s += __shfl_down(s, off, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    double t = 0.0;
    for (int w = 0; w < kBlock / 64; ++w) t += red[w];
    partial[blockIdx.x] = t;
  }
}

__global__ void __launch_bounds__(kBlock) rademacher_dot_final(const double* __restrict__ partial, int nparts,
                                                               float* __restrict__ out) {
  __shared__ double red[kBlock];
  double s = 0.0;
  for (int i = threadIdx.x; i < nparts; i += kBlock) s += partial[i];
  red[threadIdx.x] = s;
  __syncthreads();
  for (int off = kBlock / 2; off > 0; off >>= 1) {
    if (threadIdx.x < off) red[threadIdx.x] += red[threadIdx.x + off];
    __syncthreads();
  }
  if (threadIdx.x == 0) *out = static_cast<float>(red[0]);
}

// H <- H * beta + (1 - beta) * clamp(hvp * v, 0), in the reference's op order:
// est = (hvp * v) in the promoted dtype, clamp_min(0), H.mul_(beta) then
// add_(est, alpha=1 - beta) (a fused multiply-add in torch's CPU kernel).
template <int HD>
__global__ void __launch_bounds__(kBlock) hutch_update_kernel(void* __restrict__ H, const void* __restrict__ hvp,
                                                              int hvp_dtype, const void* __restrict__ v, int v_dtype,
                                                              int est_dtype, int64_t n, uint64_t seed, float beta,
                                                              float omb) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    float est = rnd(load_as_f32(hvp, i, hvp_dtype) * probe(v, v_dtype, seed, i), est_dtype);
    est = est < 0.0f ? 0.0f : est;  // clamp(min=0); NaN passes through as in torch.clamp
    const float h = rnd(load_as_f32(H, i, HD) * beta, HD);
    store_from_f32(H, i, HD, rnd(fmaf(est, omb, h), HD));
  }
}

// The same update, 4 consecutive elements per thread and 2 such vectors in flight per iteration
// (16-byte H accesses, 8- or 16-byte hvp accesses); the 4 elements share one 64-bit hash word, so
// one hash serves the vector.  Needs n % 4 == 0 and 16-byte aligned H / hvp (8-byte for bf16).
template <typename T>
__device__ __forceinline__ void ld4v(const void* p, int64_t i, int dt, float o[4]) {
  if (dt == SF_DTYPE_F32) {
    const float4 x = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + i);
    o[0] = x.x; o[1] = x.y; o[2] = x.z; o[3] = x.w;
  } else {
    const uint2 x = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p) + i);
    o[0] = bf16_to_f32(x.x & 0xffffu); o[1] = bf16_to_f32(x.x >> 16);
    o[2] = bf16_to_f32(x.y & 0xffffu); o[3] = bf16_to_f32(x.y >> 16);
  }
}

// ld4v / the 4-element store as non-temporal accesses (the multi-tensor update streams the whole
// accumulator arena once; nothing re-reads it before it is evicted).
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void ld4v_nt(const void* p, int64_t i, int dt, float o[4]) {
  if (dt == SF_DTYPE_F32) {
    const f32x4_t x = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(static_cast<const float*>(p) + i));
    o[0] = x.x; o[1] = x.y; o[2] = x.z; o[3] = x.w;
  } else {
    const u32x2_t x = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(static_cast<const uint16_t*>(p) + i));
    o[0] = bf16_to_f32(x.x & 0xffffu); o[1] = bf16_to_f32(x.x >> 16);
    o[2] = bf16_to_f32(x.y & 0xffffu); o[3] = bf16_to_f32(x.y >> 16);
  }
}
template <int HD>
__device__ __forceinline__ void st4v_nt(void* p, int64_t i, const float v[4]) {
  if (HD == SF_DTYPE_F32) {
    __builtin_nontemporal_store(f32x4_t{v[0], v[1], v[2], v[3]}, reinterpret_cast<f32x4_t*>(static_cast<float*>(p) + i));
  } else {
    u32x2_t o;
    o.x = static_cast<uint32_t>(f32_to_bf16(v[0])) | (static_cast<uint32_t>(f32_to_bf16(v[1])) << 16);
    o.y = static_cast<uint32_t>(f32_to_bf16(v[2])) | (static_cast<uint32_t>(f32_to_bf16(v[3])) << 16);
    __builtin_nontemporal_store(o, reinterpret_cast<u32x2_t*>(static_cast<uint16_t*>(p) + i));
  }
}

template <int HD>
__global__ void __launch_bounds__(kBlock) hutch_update_vec_kernel(void* __restrict__ H, const void* __restrict__ hvp,
                                                                  int hvp_dtype, int est_dtype, int64_t n4,
                                                                  uint64_t seed, float beta, float omb) {
  constexpr int kU = 2;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t j = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; j < n4; j += kU * stride) {
    float h[kU][4], e[kU][4];
    bool live[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int64_t jj = j + u * stride;
      live[u] = jj < n4;
      if (live[u]) {
        ld4v<float>(H, 4 * jj, HD, h[u]);
        ld4v<float>(hvp, 4 * jj, hvp_dtype, e[u]);
      }
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      if (!live[u]) continue;
      const int64_t i0 = 4 * (j + u * stride);
      const uint64_t word = counter_hash(seed, static_cast<uint64_t>(i0) >> 6);
      float out[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float v = ((word >> ((i0 + q) & 63)) & 1ull) ? 1.0f : -1.0f;
        float est = rnd(e[u][q] * v, est_dtype);
        est = est < 0.0f ? 0.0f : est;
        const float hb = rnd(h[u][q] * beta, HD);
        out[q] = rnd(fmaf(est, omb, hb), HD);
      }
      if (HD == SF_DTYPE_F32) {
        *reinterpret_cast<float4*>(static_cast<float*>(H) + i0) = make_float4(out[0], out[1], out[2], out[3]);
      } else {
        uint2 x;
        x.x = static_cast<uint32_t>(f32_to_bf16(out[0])) | (static_cast<uint32_t>(f32_to_bf16(out[1])) << 16);
        x.y = static_cast<uint32_t>(f32_to_bf16(out[2])) | (static_cast<uint32_t>(f32_to_bf16(out[3])) << 16);
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(H) + i0) = x;
      }
    }
  }
}

// Multi-tensor accumulator update: one launch covers up to kHutchMulti
// tensors (table in the kernel arguments).  Tensor i owns workgroups
// [first[i], first[i + 1]), grid-striding over its float4s like the single
// kernel with its own workgroup count, so every element gets the single
// kernel's value (the probe bit depends only on (seed, element index)).
constexpr int kHutchMulti = 48;
struct HutchEntry {
  void* H;
  const void* hvp;
  int64_t n4;
  uint64_t seed;
  float beta, omb;
};
struct HutchArgs {
  int count, h_dtype, hvp_dtype, est_dtype;
  int32_t first[kHutchMulti + 1];
  HutchEntry t[kHutchMulti];
};
static_assert(sizeof(HutchArgs) <= 4000, "Hutchinson table exceeds the kernel argument budget");

template <int HD>
__global__ void __launch_bounds__(kBlock) hutch_update_multi_kernel(HutchArgs a) {
  const int b = blockIdx.x;
  int i = 0;
#pragma unroll
  for (int k = 1; k < kHutchMulti; ++k) i += (k < a.count && a.first[k] <= b) ? 1 : 0;
  const HutchEntry& e = a.t[i];
  const int64_t nblk = a.first[i + 1] - a.first[i];
  const int64_t stride = nblk * kBlock;
  // two vectors per iteration, both loaded before either is used
  constexpr int kU = 2;
  for (int64_t j = (b - a.first[i]) * (int64_t)kBlock + threadIdx.x; j < e.n4; j += kU * stride) {
    float h[kU][4], x[kU][4];
    bool live[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int64_t jj = j + u * stride;
      live[u] = jj < e.n4;
      if (live[u]) {
        ld4v_nt(e.H, 4 * jj, HD, h[u]);
        ld4v_nt(e.hvp, 4 * jj, a.hvp_dtype, x[u]);
      }
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      if (!live[u]) continue;
      const int64_t i0 = 4 * (j + u * stride);
      const uint64_t word = counter_hash(e.seed, static_cast<uint64_t>(i0) >> 6);
      float out[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float v = ((word >> ((i0 + q) & 63)) & 1ull) ? 1.0f : -1.0f;
        float est = rnd(x[u][q] * v, a.est_dtype);
        est = est < 0.0f ? 0.0f : est;
        const float hb = rnd(h[u][q] * e.beta, HD);
        out[q] = rnd(fmaf(est, e.omb, hb), HD);
      }
      st4v_nt<HD>(e.H, i0, out);
    }
  }
}

bool dt_ok(int d) { return d == SF_DTYPE_F32 || d == SF_DTYPE_BF16; }

}  // namespace
}  // namespace sf

using namespace sf;

extern "C" int sf_rademacher(void* v, int dtype, int64_t n, uint64_t seed, void* stream) {
  SF_CHECK_ARG(n >= 0 && dt_ok(dtype), "bad size or dtype");
  if (n == 0) return SF_OK;
  SF_CHECK_ARG(v, "null tensor");
  rademacher_kernel<<<elementwise_grid(n, kBlock), kBlock, 0, static_cast<hipStream_t>(stream)>>>(v, dtype, n, seed);
  return launch_status("sf_rademacher");
}

extern "C" size_t sf_rademacher_dot_workspace_size(void) { return sizeof(double) * kDotGrid; }

extern "C" int sf_rademacher_dot(const void* g, int g_dtype, const void* v, int v_dtype, int64_t n, uint64_t seed,
                                 float* out, void* workspace, size_t workspace_bytes, void* stream) {
  SF_CHECK_ARG(n >= 0 && dt_ok(g_dtype) && (!v || dt_ok(v_dtype)), "bad size or dtype");
  SF_CHECK_ARG(out && (n == 0 || g), "null tensor");
  SF_CHECK_ARG(workspace && workspace_bytes >= sf_rademacher_dot_workspace_size(), "workspace too small");
  hipStream_t st = static_cast<hipStream_t>(stream);
  double* partial = static_cast<double*>(workspace);
  rademacher_dot_partial<<<kDotGrid, kBlock, 0, st>>>(g, g_dtype, v, v_dtype, n, seed, partial);
  rademacher_dot_final<<<1, kBlock, 0, st>>>(partial, kDotGrid, out);
  return launch_status("sf_rademacher_dot");
}

extern "C" int sf_hutchinson_update(void* H, int h_dtype, const void* hvp, int hvp_dtype, const void* v, int v_dtype,
                                    int64_t n, uint64_t seed, double beta, void* stream) {
  SF_CHECK_ARG(n >= 0 && dt_ok(h_dtype) && dt_ok(hvp_dtype) && (!v || dt_ok(v_dtype)), "bad size or dtype");
  if (n == 0) return SF_OK;
  SF_CHECK_ARG(H && hvp, "null tensor");
  // (hvp * v) takes the promoted dtype of the two (v is in the weight dtype in the reference)
  const int est_dtype = (hvp_dtype == SF_DTYPE_F32 || (v && v_dtype == SF_DTYPE_F32)) ? SF_DTYPE_F32 : SF_DTYPE_BF16;
  const float b = static_cast<float>(beta), omb = static_cast<float>(1.0 - beta);
  hipStream_t st = static_cast<hipStream_t>(stream);
  auto al = [](const void* q, int dt) { return (reinterpret_cast<uintptr_t>(q) % (dt == SF_DTYPE_F32 ? 16 : 8)) == 0; };
  if (!v && n % 4 == 0 && al(H, h_dtype) && al(hvp, hvp_dtype)) {
    const int gridv = elementwise_grid((n / 4 + 1) / 2, kBlock);
    if (h_dtype == SF_DTYPE_F32)
      hutch_update_vec_kernel<SF_DTYPE_F32><<<gridv, kBlock, 0, st>>>(H, hvp, hvp_dtype, est_dtype, n / 4, seed, b, omb);
    else
      hutch_update_vec_kernel<SF_DTYPE_BF16><<<gridv, kBlock, 0, st>>>(H, hvp, hvp_dtype, est_dtype, n / 4, seed, b,
                                                                       omb);
    return launch_status("sf_hutchinson_update");
  }
  const int grid = elementwise_grid(n, kBlock);
  if (h_dtype == SF_DTYPE_F32)
    hutch_update_kernel<SF_DTYPE_F32><<<grid, kBlock, 0, st>>>(H, hvp, hvp_dtype, v, v_dtype, est_dtype, n, seed, b, omb);
  else
    hutch_update_kernel<SF_DTYPE_BF16><<<grid, kBlock, 0, st>>>(H, hvp, hvp_dtype, v, v_dtype, est_dtype, n, seed, b,
                                                                omb);
  return launch_status("sf_hutchinson_update");
}

extern "C" int sf_hutchinson_update_multi(const sf_hutch_tensor* tensors, int count, int h_dtype, int hvp_dtype,
                                          void* stream) {
  SF_CHECK_ARG(count >= 0 && (count == 0 || tensors), "bad tensor table (count %d)", count);
  SF_CHECK_ARG(dt_ok(h_dtype) && dt_ok(hvp_dtype), "bad dtype");
  auto al = [](const void* q, int dt) { return (reinterpret_cast<uintptr_t>(q) % (dt == SF_DTYPE_F32 ? 16 : 8)) == 0; };
  for (int i = 0; i < count; ++i) {
    const sf_hutch_tensor& t = tensors[i];
    SF_CHECK_ARG(t.n >= 0 && t.n % 4 == 0, "tensor %d: n = %lld is not a multiple of 4", i, (long long)t.n);
    if (t.n == 0) continue;
    SF_CHECK_ARG(t.H && t.hvp, "tensor %d: null tensor", i);
    SF_CHECK_ARG(al(t.H, h_dtype) && al(t.hvp, hvp_dtype), "tensor %d: operands not 4-element aligned", i);
  }
  const int est_dtype = hvp_dtype == SF_DTYPE_F32 ? SF_DTYPE_F32 : SF_DTYPE_BF16;
  hipStream_t st = static_cast<hipStream_t>(stream);
  HutchArgs a;
  int i = 0;
  while (i < count) {
    memset(&a, 0, sizeof(a));
    a.h_dtype = h_dtype;
    a.hvp_dtype = hvp_dtype;
    a.est_dtype = est_dtype;
    int n = 0;
    int64_t blocks = 0;
    for (; i < count && n < kHutchMulti; ++i) {
      const sf_hutch_tensor& t = tensors[i];
      if (t.n == 0) continue;
      HutchEntry& e = a.t[n];
      e.H = t.H;
      e.hvp = t.hvp;
      e.n4 = t.n / 4;
      e.seed = t.seed;
      e.beta = static_cast<float>(t.beta);
      e.omb = static_cast<float>(1.0 - t.beta);
      a.first[n] = static_cast<int32_t>(blocks);
      // the single kernel's grid for this tensor (its workgroups stride over it the same way)
      blocks += elementwise_grid((e.n4 + 1) / 2, kBlock);
      ++n;
    }
    if (n == 0) break;
    a.count = n;
    a.first[n] = static_cast<int32_t>(blocks);
    if (h_dtype == SF_DTYPE_F32)
      hutch_update_multi_kernel<SF_DTYPE_F32><<<static_cast<int>(blocks), kBlock, 0, st>>>(a);
    else
      hutch_update_multi_kernel<SF_DTYPE_BF16><<<static_cast<int>(blocks), kBlock, 0, st>>>(a);
    if (int rc = launch_status("sf_hutchinson_update_multi")) return rc;
  }
  return SF_OK;
}
