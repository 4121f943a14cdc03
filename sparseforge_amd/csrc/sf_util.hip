// Library-wide entry points: error string and version.
#include <stdarg.h>

#include "sf_common.hpp"

namespace sf {

static thread_local char g_last_error[1024] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

}  // namespace sf

extern "C" const char* sf_last_error(void) { return sf::g_last_error; }

// Major * 10000 + minor * 100 + patch.
extern "C" int sf_version(void) { return 100; }

// ---------------------------------------------------------------------------
// Sustained MFMA rate probe (a measurement aid for bench.py, no counterpart in
// the reference).  Every wave keeps 16 independent 32x32 accumulators busy
// with v_mfma_f32_32x32x16_bf16 on register operands distributed like a
// GEMM's (activations ~N(0, 1), weights ~N(0, 0.02)): the MFMA pipe's power,
// and with it the clock it sustains, depends on the operand bits (zeros or
// constant exponents overstate the rate).
// No memory traffic inside the loop: what one GPU can sustain on MFMA alone,
// the practical ceiling under the published dense peak.
// ---------------------------------------------------------------------------
namespace sf {
namespace {
typedef __bf16 bf16x8_p __attribute__((ext_vector_type(8)));
typedef float f32x16_p __attribute__((ext_vector_type(16)));

__device__ __forceinline__ uint32_t mix32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

__global__ void __launch_bounds__(256, 1) mfma_probe_kernel(int iters, float* __restrict__ out) {
  const uint32_t t = blockIdx.x * 256u + threadIdx.x;
  bf16x8_p a[4], b[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      // roughly normal values (a sum of three uniforms) like a GEMM's activations (scale 1)
      // and weights (scale 0.02): exponents and mantissas vary as they do there
      const uint32_t r0 = mix32(t * 64u + i * 8u + e), r1 = mix32(r0 ^ 0x9e3779b9u), r2 = mix32(r1 + 0x85ebca6bu);
      const float u = ((r0 >> 8) + (r1 >> 8) + (r2 >> 8)) * (1.0f / 16777216.0f) - 1.5f;
      const float v = ((r0 & 0xffffu) + (r1 & 0xffffu) + (r2 & 0xffffu)) * (1.0f / 65536.0f) - 1.5f;
      a[i][e] = (__bf16)(2.0f * u);
      b[i][e] = (__bf16)(0.04f * v);
    }
  f32x16_p acc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = f32x16_p{};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        acc[j * 4 + i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[j * 4 + i], 0, 0, 0);
  }
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) s += acc[i][e];
  out[t] = s;
}
}  // namespace
// Streaming patterns of the HBM probe (n elements, vector of 4 per thread and round):
//   0: the fused mask update's traffic: read W (bf16), H (f32), M (f32), write M (14 B / element)
//   1: the score statistics' traffic: read W (bf16), H (f32) (6 B / element), one f32 per thread to M
//   2: a copy: read H (f32), write M (f32) (8 B / element)
// The arithmetic is a token FMA per element, so only the memory system limits it.
__global__ void __launch_bounds__(256) hbm_probe_kernel(int pattern, const uint2* __restrict__ W,
                                                        const float4* __restrict__ H, float4* __restrict__ M,
                                                        int64_t n4) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  float acc = 0.0f;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n4; i += stride) {
    const float4 h = H[i];
    if (pattern == 2) {
      M[i] = h;
      continue;
    }
    const uint2 w = W[i];
    const float a = __uint_as_float(w.x << 16), b = __uint_as_float(w.x & 0xffff0000u);
    const float c = __uint_as_float(w.y << 16), d = __uint_as_float(w.y & 0xffff0000u);
    if (pattern == 1) {
      acc += a * h.x + b * h.y + c * h.z + d * h.w;
      continue;
    }
    float4 m = M[i];
    m.x = fmaf(a, h.x, m.x * 0.9f);
    m.y = fmaf(b, h.y, m.y * 0.9f);
    m.z = fmaf(c, h.z, m.z * 0.9f);
    m.w = fmaf(d, h.w, m.w * 0.9f);
    M[i] = m;
  }
  if (pattern == 1) reinterpret_cast<float*>(M)[blockIdx.x * (int64_t)blockDim.x + threadIdx.x] = acc;
}
}  // namespace sf

extern "C" int sf_hbm_probe(int pattern, const void* W, const void* H, void* M, int64_t n, int blocks, void* stream) {
  SF_CHECK_ARG(pattern >= 0 && pattern <= 2, "bad probe pattern %d", pattern);
  SF_CHECK_ARG(n > 0 && n % 4 == 0 && blocks > 0, "bad probe size (n %lld, blocks %d)", (long long)n, blocks);
  SF_CHECK_ARG((pattern == 2 || W) && H && M, "null tensor");
  SF_CHECK_ARG(pattern != 1 || (int64_t)blocks * 256 <= n, "pattern 1 writes one float per thread to M");
  sf::hbm_probe_kernel<<<blocks, 256, 0, static_cast<hipStream_t>(stream)>>>(
      pattern, static_cast<const uint2*>(W), static_cast<const float4*>(H), static_cast<float4*>(M), n / 4);
  return sf::launch_status("sf_hbm_probe");
}

// out: device float[blocks * 256] (checksums).  FLOPs = blocks * 4 * iters * 16 * 32768.
extern "C" int sf_mfma_probe(int iters, int blocks, float* out, void* stream) {
  SF_CHECK_ARG(iters > 0 && blocks > 0 && out, "bad probe arguments");
  sf::mfma_probe_kernel<<<blocks, 256, 0, static_cast<hipStream_t>(stream)>>>(iters, out);
  return sf::launch_status("sf_mfma_probe");
}
