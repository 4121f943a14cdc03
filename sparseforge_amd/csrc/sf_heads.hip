// Attention head layout of the retraining model (cfg5): the rotary embedding
// and the change between the projections' token-major rows and the per-head
// operands of the attention products, in one pass each way.
//
// HuggingFace's eager LlamaAttention (the reference retrains it,
// legacy/model_llama.py:39-55) views q, k, v [B, S, H * D] as [B, H, S, D],
// rotates q and k (x cos + rotate_half(x) sin, in the activations' dtype),
// and multiplies per head.  With torch ops that is a transposed view, five
// strided elementwise passes for the rotation and a copy per operand to make
// the batched products' operands contiguous, and as many again in each
// backward pass.  Here:
//   to_heads    y = scale * rot(x)  (or scale * x), x [B, S, H * D] ->
//               y [B * H, S, D] (TR = 0) or [B * H, D, S] (TR = 1, the
//               key operand of q k^T, transposed per head)
//   from_heads  its adjoint, g [B * H, S, D] or [B * H, D, S] ->
//               x_bar [B, S, H * D] = rot^T(scale * g)
// rot(x)[d] = x[d] c[d] + x[d^] ss[d] with d^ = (d + D/2) mod D, c = cos, ss =
// (-sin on the first half, sin on the second), both rounded to the dtype, each
// product rounded to the dtype and then their sum (torch's bf16 / f32 ops in
// that order).  rot^T(g)[e] = g[e] c[e] + g[e^] ss[e^], with the same
// roundings: it is what autograd computes for the torch form, and the
// adjoint of the adjoint is the forward map, so the pair is differentiable
// any number of times (the Hutchinson product differentiates it twice).
// scale is 1 or a power of two (exact).
//
// One workgroup per (64 positions, head, batch): the 64 x D tile is read
// with 16-byte row loads into LDS, then every output row (of D along d, or
// of 64 along s for TR = 1) is written with 16-byte stores.

#include "sf_common.hpp"

namespace sf {
namespace {

constexpr int kHdThreads = 256;
constexpr int kHdRows = 64;    // positions per workgroup
constexpr int kHdMaxD = 128;   // head dimension bound (LDS tile 64 x 128 x 4 B)

template <int DT>
__device__ __forceinline__ float rnd_dt(float x) {
  if constexpr (DT == SF_DTYPE_BF16)
    return round_bf16(x);
  else
    return x;
}

template <int DT>
__device__ __forceinline__ float ld(const void* p, int64_t i) {
  if constexpr (DT == SF_DTYPE_BF16)
    return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
  else
    return static_cast<const float*>(p)[i];
}

// 8 consecutive elements at p + i (i a multiple of 8, 16-byte aligned rows for bf16; two 16-byte loads for f32)
template <int DT>
__device__ __forceinline__ void ld8(const void* p, int64_t i, float v[8]) {
  if constexpr (DT == SF_DTYPE_BF16) {
    const uint4 q = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p) + i);
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[2 * k] = bf16_to_f32(static_cast<uint16_t>(w[k] & 0xffffu));
      v[2 * k + 1] = bf16_to_f32(static_cast<uint16_t>(w[k] >> 16));
    }
  } else {
    const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + i);
    const float4 b = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + i + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
}

template <int DT>
__device__ __forceinline__ void st8(void* p, int64_t i, const float v[8]) {
  if constexpr (DT == SF_DTYPE_BF16) {
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      w[k] = static_cast<uint32_t>(f32_to_bf16(v[2 * k])) | (static_cast<uint32_t>(f32_to_bf16(v[2 * k + 1])) << 16);
    *reinterpret_cast<uint4*>(static_cast<uint16_t*>(p) + i) = make_uint4(w[0], w[1], w[2], w[3]);
  } else {
    *reinterpret_cast<float4*>(static_cast<float*>(p) + i) = make_float4(v[0], v[1], v[2], v[3]);
    *reinterpret_cast<float4*>(static_cast<float*>(p) + i + 4) = make_float4(v[4], v[5], v[6], v[7]);
  }
}

struct HeadsArgs {
  const void* in;
  void* out;
  const float* cos;  // [S, D] f32 tables (ROT)
  const float* sin;
  int64_t B, S;
  int H, D;
  float scale;
};

// ADJ = 0: to_heads (in token-major, out head-major); ADJ = 1: from_heads (in head-major, out token-major).
template <int DT, bool ROT, bool TR, bool ADJ>
__global__ void __launch_bounds__(kHdThreads) heads_kernel(HeadsArgs a) {
  __shared__ float tile[kHdRows][kHdMaxD + 1];  // [position][d], the input tile (scaled when ADJ)
  const int64_t s0 = (int64_t)blockIdx.x * kHdRows;
  const int h = blockIdx.y, D = a.D, half = D / 2;
  const int64_t b = blockIdx.z, S = a.S, HD = (int64_t)a.H * D;
  const int rows = S - s0 < kHdRows ? static_cast<int>(S - s0) : kHdRows;
  const int t = threadIdx.x;
  const int64_t bh = b * a.H + h;
  // phase 1: the input tile into LDS as [position][d]
  if (!ADJ || !TR) {
    // rows of D along d: token-major x[b, s, h D + d] or head-major g[bh, s, d]
    const int per_row = D / 8;
    for (int i = t; i < rows * per_row; i += kHdThreads) {
      const int r = i / per_row, c = (i - r * per_row) * 8;
      const int64_t src = ADJ ? (bh * S + s0 + r) * D + c : (b * S + s0 + r) * HD + (int64_t)h * D + c;
      float v[8];
      ld8<DT>(a.in, src, v);
#pragma unroll
      for (int k = 0; k < 8; ++k) tile[r][c + k] = ADJ ? rnd_dt<DT>(v[k] * a.scale) : v[k];
    }
  } else {
    // head-major transposed g[bh, d, s]: rows of positions along s (a partial tile reads element by element)
    const int per_row = kHdRows / 8;
    for (int i = t; i < D * per_row; i += kHdThreads) {
      const int d = i / per_row, c = (i - d * per_row) * 8;
      const int64_t src = (bh * D + d) * S + s0 + c;
      float v[8];
      if (rows == kHdRows && (S % 8) == 0) {
        ld8<DT>(a.in, src, v);
      } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = c + k < rows ? ld<DT>(a.in, src + k) : 0.0f;
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) tile[c + k][d] = rnd_dt<DT>(v[k] * a.scale);
    }
  }
  __syncthreads();
  // phase 2: output rows.  rot_row: the 8 outputs (position r, dims c .. c + 7), c a multiple of 8, so the
  // 8 dims lie in one half and their partners c^ .. c^ + 7 too (D / 2 is a multiple of 8).
  auto rot_row = [&](int r, int c, float v[8]) {
    const int ce = c < half ? c + half : c - half;  // c^
    if constexpr (!ROT) {
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] = ADJ ? tile[r][c + k] : rnd_dt<DT>(tile[r][c + k] * a.scale);
    } else {
      const int64_t srow = (s0 + r) * D;
      float cs[8], sn[8];
      ld8<SF_DTYPE_F32>(a.cos, srow + c, cs);
      // forward: ss[d] at d = c + k; adjoint: ss[e] at e = c^ + k
      const int sc = ADJ ? ce : c;
      ld8<SF_DTYPE_F32>(a.sin, srow + sc, sn);
      const bool neg = sc < half;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float cc = rnd_dt<DT>(cs[k]);
        const float ss = rnd_dt<DT>(neg ? -sn[k] : sn[k]);
        const float y = rnd_dt<DT>(rnd_dt<DT>(tile[r][c + k] * cc) + rnd_dt<DT>(tile[r][ce + k] * ss));
        v[k] = ADJ ? y : rnd_dt<DT>(y * a.scale);
      }
    }
  };
  if (ADJ || !TR) {
    // rows of D along d: head-major y[bh, s, d] or token-major x_bar[b, s, h D + d]
    const int per_row = D / 8;
    for (int i = t; i < rows * per_row; i += kHdThreads) {
      const int r = i / per_row, c = (i - r * per_row) * 8;
      float v[8];
      rot_row(r, c, v);
      const int64_t dst = ADJ ? (b * S + s0 + r) * HD + (int64_t)h * D + c : (bh * S + s0 + r) * D + c;
      st8<DT>(a.out, dst, v);
    }
  } else {
    // head-major transposed y[bh, d, s] (forward only): rows of positions along s
    const int per_row = kHdRows / 8;
    for (int i = t; i < D * per_row; i += kHdThreads) {
      const int d = i / per_row, c = (i - d * per_row) * 8;
      const int e = d < half ? d + half : d - half;
      const int64_t dst = (bh * D + d) * S + s0 + c;
      float v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        v[k] = 0.0f;
        if (c + k < rows) {
          if constexpr (ROT) {
            const int64_t sd = (s0 + c + k) * D;
            const float cc = rnd_dt<DT>(a.cos[sd + d]);
            const float ss = rnd_dt<DT>(d < half ? -a.sin[sd + d] : a.sin[sd + d]);
            const float y = rnd_dt<DT>(rnd_dt<DT>(tile[c + k][d] * cc) + rnd_dt<DT>(tile[c + k][e] * ss));
            v[k] = rnd_dt<DT>(y * a.scale);
          } else {
            v[k] = rnd_dt<DT>(tile[c + k][d] * a.scale);
          }
        }
      }
      if (rows == kHdRows && (S % 8) == 0) {
        st8<DT>(a.out, dst, v);
      } else {
        for (int k = 0; k < 8 && c + k < rows; ++k) {
          if constexpr (DT == SF_DTYPE_BF16)
            static_cast<uint16_t*>(a.out)[dst + k] = f32_to_bf16(v[k]);
          else
            static_cast<float*>(a.out)[dst + k] = v[k];
        }
      }
    }
  }
}

template <bool ROT, bool TR, bool ADJ>
int launch_heads(int dtype, const HeadsArgs& a, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>(ceil_div(a.S, kHdRows)), static_cast<unsigned>(a.H),
                  static_cast<unsigned>(a.B));
  if (dtype == SF_DTYPE_BF16)
    heads_kernel<SF_DTYPE_BF16, ROT, TR, ADJ><<<grid, kHdThreads, 0, st>>>(a);
  else
    heads_kernel<SF_DTYPE_F32, ROT, TR, ADJ><<<grid, kHdThreads, 0, st>>>(a);
  return SF_OK;
}

int heads_call(const char* what, bool adj, const void* in, int dtype, int64_t B, int64_t S, int64_t H, int64_t D,
               const float* cos, const float* sin, int rotate, int transposed, float scale, void* out,
               void* stream) {
  SF_CHECK_ARG(dtype == SF_DTYPE_BF16 || dtype == SF_DTYPE_F32, "%s: bad dtype %d", what, dtype);
  SF_CHECK_ARG(B >= 0 && S >= 0 && H >= 0, "%s: negative shape", what);
  SF_CHECK_ARG(D >= 8 && D <= kHdMaxD && D % 16 == 0, "%s: head dim %lld not in [16, 128] step 16", what,
               (long long)D);
  SF_CHECK_ARG(H < 65536 && B < 65536, "%s: too many heads / batches", what);
  SF_CHECK_ARG(!rotate || (cos && sin), "%s: rotation without tables", what);
  if (B == 0 || S == 0 || H == 0) return SF_OK;
  SF_CHECK_ARG(in && out, "%s: null tensor", what);
  SF_CHECK_ARG((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(out)) % 16 == 0,
               "%s: tensors must be 16-byte aligned", what);
  SF_CHECK_ARG(!rotate || (reinterpret_cast<uintptr_t>(cos) | reinterpret_cast<uintptr_t>(sin)) % 16 == 0,
               "%s: rotary tables must be 16-byte aligned", what);
  HeadsArgs a{in, out, cos, sin, B, S, static_cast<int>(H), static_cast<int>(D), scale};
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool r = rotate != 0, tr = transposed != 0;
  if (!adj) {
    if (r)
      tr ? launch_heads<true, true, false>(dtype, a, st) : launch_heads<true, false, false>(dtype, a, st);
    else
      tr ? launch_heads<false, true, false>(dtype, a, st) : launch_heads<false, false, false>(dtype, a, st);
  } else {
    if (r)
      tr ? launch_heads<true, true, true>(dtype, a, st) : launch_heads<true, false, true>(dtype, a, st);
    else
      tr ? launch_heads<false, true, true>(dtype, a, st) : launch_heads<false, false, true>(dtype, a, st);
  }
  return launch_status(what);
}

// dst[b][c][r] = src[b][r][c] for [batch, rows, cols] matrices of 2- or 4-byte elements: one workgroup
// per 64 x 64 tile, read as rows of 16-byte chunks into LDS, written as rows of the transpose.
template <typename E>
__global__ void __launch_bounds__(kHdThreads) transpose_batched_kernel(const E* __restrict__ src, E* __restrict__ dst,
                                                                      int64_t rows, int64_t cols) {
  constexpr int kV = 16 / sizeof(E);  // elements per 16-byte chunk
  __shared__ E tile[64][64 + kV];
  const int64_t b = blockIdx.z, r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
  const E* s = src + b * rows * cols;
  E* d = dst + b * rows * cols;
  const int t = threadIdx.x;
  const bool vec = (cols % kV) == 0 && (rows % kV) == 0 && r0 + 64 <= rows && c0 + 64 <= cols;
  constexpr int per_row = 64 / kV;
  for (int i = t; i < 64 * per_row; i += kHdThreads) {
    const int r = i / per_row, c = (i - r * per_row) * kV;
    if (vec) {
      const uint4 q = *reinterpret_cast<const uint4*>(s + (r0 + r) * cols + c0 + c);
      const E* e = reinterpret_cast<const E*>(&q);
#pragma unroll
      for (int k = 0; k < kV; ++k) tile[r][c + k] = e[k];
    } else {
#pragma unroll
      for (int k = 0; k < kV; ++k)
        if (r0 + r < rows && c0 + c + k < cols) tile[r][c + k] = s[(r0 + r) * cols + c0 + c + k];
    }
  }
  __syncthreads();
  for (int i = t; i < 64 * per_row; i += kHdThreads) {
    const int c = i / per_row, r = (i - c * per_row) * kV;  // output row c (a source column), positions r ..
    if (vec) {
      uint4 q;
      E* e = reinterpret_cast<E*>(&q);
#pragma unroll
      for (int k = 0; k < kV; ++k) e[k] = tile[r + k][c];
      *reinterpret_cast<uint4*>(d + (c0 + c) * rows + r0 + r) = q;
    } else {
#pragma unroll
      for (int k = 0; k < kV; ++k)
        if (c0 + c < cols && r0 + r + k < rows) d[(c0 + c) * rows + r0 + r + k] = tile[r + k][c];
    }
  }
}

}  // namespace
}  // namespace sf

using namespace sf;

extern "C" int sf_transpose_batched(const void* src, int elem_bytes, int64_t batch, int64_t rows, int64_t cols,
                                    void* dst, void* stream) {
  SF_CHECK_ARG(elem_bytes == 2 || elem_bytes == 4, "sf_transpose_batched: element size %d", elem_bytes);
  SF_CHECK_ARG(batch >= 0 && rows >= 0 && cols >= 0, "sf_transpose_batched: negative shape");
  if (batch == 0 || rows == 0 || cols == 0) return SF_OK;
  SF_CHECK_ARG(src && dst && src != dst, "sf_transpose_batched: null or aliased tensors");
  SF_CHECK_ARG((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) % 16 == 0,
               "sf_transpose_batched: tensors must be 16-byte aligned");
  SF_CHECK_ARG(batch < 65536 && ceil_div(rows, 64) < 65536, "sf_transpose_batched: grid too large");
  const dim3 grid(static_cast<unsigned>(ceil_div(cols, 64)), static_cast<unsigned>(ceil_div(rows, 64)),
                  static_cast<unsigned>(batch));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (elem_bytes == 2)
    transpose_batched_kernel<uint16_t><<<grid, kHdThreads, 0, st>>>(static_cast<const uint16_t*>(src),
                                                                    static_cast<uint16_t*>(dst), rows, cols);
  else
    transpose_batched_kernel<uint32_t><<<grid, kHdThreads, 0, st>>>(static_cast<const uint32_t*>(src),
                                                                    static_cast<uint32_t*>(dst), rows, cols);
  return launch_status("sf_transpose_batched");
}

extern "C" int sf_to_heads(const void* x, int dtype, int64_t B, int64_t S, int64_t H, int64_t D, const float* cos,
                           const float* sin, int rotate, int transposed, float scale, void* y, void* stream) {
  return heads_call("sf_to_heads", false, x, dtype, B, S, H, D, cos, sin, rotate, transposed, scale, y, stream);
}

extern "C" int sf_from_heads(const void* g, int dtype, int64_t B, int64_t S, int64_t H, int64_t D, const float* cos,
                             const float* sin, int rotate, int transposed, float scale, void* x_grad, void* stream) {
  return heads_call("sf_from_heads", true, g, dtype, B, S, H, D, cos, sin, rotate, transposed, scale, x_grad,
                    stream);
}
