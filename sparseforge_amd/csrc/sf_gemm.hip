// Dense MFMA GEMM engine of the SparseLinear path (K1-K5) on gfx950.
//
//   C[M, N] = sum_k A(m, k) * B'(n, k)  (+ segment 2: sum_k A2(m, k) * B2(n, k))
//   B'(n, k) = B(n, k) * E(n, k) * s    (E: effective mask, optional)
//
// A is stored K-contiguous (A[m * lda + k]) or M-contiguous (A[k * lda + m]);
// B is stored K-contiguous (B[n * ldb + k]) or N-contiguous (B[k * ldb + n]).
// The three products of a masked linear map onto it as
//   forward   y  = x (W.E)^T   : A K-contig (x [T, in]),   B K-contig (W [out, in])
//   input grad dx = dy (W.E)   : A K-contig (dy [T, out]), B N-contig (W [out, in])
//   weight grad dW = dy^T x    : A M-contig (dy [T, out]), B N-contig (x [T, in])
// The second K segment concatenates the SLoRB low-rank term into the same
// accumulators ([x | z] . [W.E | S]^T) instead of a separate GEMM + add.
//
// Tiling: 256 threads = 4 waves in a 2 x 2 grid; a workgroup owns a 256 x 256
// tile of C, each wave 128 x 128 as 4 x 4 MFMA 32x32 blocks.  A and B tiles of
// BK k-values are staged through double-buffered LDS with k contiguous per
// row, so an MFMA operand fragment is one 16-byte LDS read per lane.
// M/N-contiguous operands are transposed in registers (8 x 8 blocks) on their
// way into LDS.  The mask multiply happens in registers between the global
// load and the LDS store: no masked copy of W is ever written to memory.
// Global loads of step k+1 are issued before the MFMAs of step k.

#include "sf_common.hpp"

namespace sf {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int kTileM = 256;
constexpr int kTileN = 256;
constexpr int kWaveM = 128;
constexpr int kWaveN = 128;
constexpr int kFragM = kWaveM / 32;  // 4
constexpr int kFragN = kWaveN / 32;  // 4

struct GemmArgs {
  int64_t M, N, K1, K2;
  const void* A1;
  int64_t lda1;
  const void* A2;
  int64_t lda2;
  const void* B1;
  int64_t ldb1;
  const void* B2;
  int64_t ldb2;
  const void* bmask;  // effective mask of B1 (element dtype, B1's layout and ld)
  float bscale;       // 1: none
  int has_scale;
  void* C;
  int64_t ldc;
  int c_dtype;
  const void* bias;  // [N], element dtype or f32
  int bias_dtype;
  const void* emask;  // [M, N] row-major with ld = ldc: C *= emask
  const void* dw;     // [M, N]: C += decay * dw * (emask < 0.5)
  float decay;
  int accumulate;  // C += result
  int64_t tiles_n;
};

// Element traits.  bf16 uses v_mfma_f32_32x32x16_bf16 (8 k-values per lane),
// f32 uses v_mfma_f32_32x32x2_f32 (1 k-value per lane).
template <typename T>
struct Tr;

template <>
struct Tr<uint16_t> {
  static constexpr int VEC = 8;      // elements per 16-byte vector
  static constexpr int BK = 64;      // k per LDS stage
  static constexpr int PITCH = 72;   // LDS row pitch (elements): 144 B keeps 16 B lane reads conflict-free
  static constexpr int MK = 16;      // k per MFMA
  static constexpr int DT = SF_DTYPE_BF16;
};

template <>
struct Tr<float> {
  static constexpr int VEC = 4;
  static constexpr int BK = 32;
  static constexpr int PITCH = 33;  // odd word pitch: 4-byte lane reads of 32 rows hit 32 banks
  static constexpr int MK = 2;
  static constexpr int DT = SF_DTYPE_F32;
};

// 16-byte vector as 4 dwords
struct V4 {
  uint32_t w[4];
};

__device__ __forceinline__ V4 ld16(const void* p) {
  uint4 v = *reinterpret_cast<const uint4*>(p);
  V4 r;
  r.w[0] = v.x; r.w[1] = v.y; r.w[2] = v.z; r.w[3] = v.w;
  return r;
}
__device__ __forceinline__ V4 zero16() {
  V4 r;
  r.w[0] = r.w[1] = r.w[2] = r.w[3] = 0u;
  return r;
}

// Apply mask (and scale) to a vector of B elements, with the reference's
// rounding: w = round(W * E) then round(w * s).
template <typename T>
__device__ __forceinline__ V4 apply_mask(V4 w, V4 e, bool has_scale, float s) {
  V4 o;
  if constexpr (sizeof(T) == 2) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float lo = bf16_to_f32(w.w[i] & 0xffffu) * bf16_to_f32(e.w[i] & 0xffffu);
      float hi = bf16_to_f32(w.w[i] >> 16) * bf16_to_f32(e.w[i] >> 16);
      if (has_scale) {
        lo = round_bf16(lo) * s;
        hi = round_bf16(hi) * s;
      }
      o.w[i] = static_cast<uint32_t>(f32_to_bf16(lo)) | (static_cast<uint32_t>(f32_to_bf16(hi)) << 16);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v = __uint_as_float(w.w[i]) * __uint_as_float(e.w[i]);
      if (has_scale) v = v * s;
      o.w[i] = __float_as_uint(v);
    }
  }
  return o;
}

// Transpose a VEC x VEC block held as VEC row vectors (row = k, lanes of the
// vector = m) into VEC vectors of k-values, one per m.
template <typename T>
__device__ __forceinline__ void transpose_block(V4 v[], V4 out[]) {
  if constexpr (sizeof(T) == 2) {
    // out[m].dword[j] = (in[2j][m], in[2j+1][m]) packed lo/hi
#pragma unroll
    for (int m = 0; m < 8; ++m) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t a = v[2 * j].w[m >> 1], b = v[2 * j + 1].w[m >> 1];
        // select the 16-bit half m & 1 of a (low result half) and of b (high result half)
        uint32_t sel = (m & 1) ? 0x07060302u : 0x05040100u;
        out[m].w[j] = __builtin_amdgcn_perm(b, a, sel);
      }
    }
  } else {
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int j = 0; j < 4; ++j) out[m].w[j] = v[j].w[m];
  }
}

// Per-thread staging of one operand tile (8 vectors of 16 bytes).
struct Stage {
  V4 v[8];
};

// Load the thread's share of a [256 rows x BK] tile of a K-contiguous operand.
// rows: the tile's first row; K limit k_end; mask optional.
template <typename T>
__device__ __forceinline__ void load_kc(Stage& st, const T* base, int64_t ld, int64_t row0, int64_t rows_total,
                                        int64_t k0, int64_t k_end, const T* mask, bool has_scale, float s) {
  constexpr int VEC = Tr<T>::VEC, BK = Tr<T>::BK, CPR = BK / VEC;  // chunks per row (8)
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int v = t + kThreads * i;
    const int r = v / CPR, c = v % CPR;
    const int64_t row = row0 + r, k = k0 + c * VEC;
    if (row < rows_total && k < k_end) {
      st.v[i] = ld16(base + row * ld + k);
      if (mask) st.v[i] = apply_mask<T>(st.v[i], ld16(mask + row * ld + k), has_scale, s);
    } else {
      st.v[i] = zero16();
    }
  }
}

template <typename T>
__device__ __forceinline__ void store_kc(const Stage& st, T* lds) {
  constexpr int VEC = Tr<T>::VEC, BK = Tr<T>::BK, CPR = BK / VEC, P = Tr<T>::PITCH;
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int v = t + kThreads * i;
    const int r = v / CPR, c = v % CPR;
    T* dst = lds + r * P + c * VEC;
    if constexpr (sizeof(T) == 2) {
      *reinterpret_cast<uint4*>(dst) = make_uint4(st.v[i].w[0], st.v[i].w[1], st.v[i].w[2], st.v[i].w[3]);
    } else {
      uint32_t* d = reinterpret_cast<uint32_t*>(dst);
      d[0] = st.v[i].w[0]; d[1] = st.v[i].w[1]; d[2] = st.v[i].w[2]; d[3] = st.v[i].w[3];
    }
  }
}

// Row-contiguous ("M/N-contiguous") operand: element (r, k) at base[k * ld + r].
// The tile is cut into VEC x VEC blocks; block b: kb = b % (BK/VEC), rb = b / (BK/VEC).
template <typename T>
__device__ __forceinline__ void load_rc(Stage& st, const T* base, int64_t ld, int64_t row0, int64_t rows_total,
                                        int64_t k0, int64_t k_end, const T* mask, bool has_scale, float s) {
  constexpr int VEC = Tr<T>::VEC, BK = Tr<T>::BK, KB = BK / VEC;
  constexpr int BLOCKS_PER_THREAD = 8 / VEC;  // 1 (bf16) or 2 (f32)
  const int t = threadIdx.x;
#pragma unroll
  for (int q = 0; q < BLOCKS_PER_THREAD; ++q) {
    const int b = t + kThreads * q;
    const int kb = b % KB, rb = b / KB;
    const int64_t r = row0 + rb * VEC;
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const int64_t k = k0 + kb * VEC + j;
      V4& dst = st.v[q * VEC + j];
      if (r < rows_total && k < k_end) {
        dst = ld16(base + k * ld + r);
        if (mask) dst = apply_mask<T>(dst, ld16(mask + k * ld + r), has_scale, s);
      } else {
        dst = zero16();
      }
    }
  }
}

template <typename T>
__device__ __forceinline__ void store_rc(const Stage& st, T* lds) {
  constexpr int VEC = Tr<T>::VEC, BK = Tr<T>::BK, KB = BK / VEC, P = Tr<T>::PITCH;
  constexpr int BLOCKS_PER_THREAD = 8 / VEC;
  const int t = threadIdx.x;
#pragma unroll
  for (int q = 0; q < BLOCKS_PER_THREAD; ++q) {
    const int b = t + kThreads * q;
    const int kb = b % KB, rb = b / KB;
    V4 in[VEC], out[VEC];
#pragma unroll
    for (int j = 0; j < VEC; ++j) in[j] = st.v[q * VEC + j];
    transpose_block<T>(in, out);
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      T* dst = lds + (rb * VEC + i) * P + kb * VEC;
      if constexpr (sizeof(T) == 2) {
        *reinterpret_cast<uint4*>(dst) = make_uint4(out[i].w[0], out[i].w[1], out[i].w[2], out[i].w[3]);
      } else {
        uint32_t* d = reinterpret_cast<uint32_t*>(dst);
        d[0] = out[i].w[0]; d[1] = out[i].w[1]; d[2] = out[i].w[2]; d[3] = out[i].w[3];
      }
    }
  }
}

__device__ __forceinline__ float load_elem(const void* p, int64_t i, int dtype) { return load_as_f32(p, i, dtype); }

template <typename T, int AL, int BL>
__global__ void __launch_bounds__(kThreads, 1) gemm_kernel(GemmArgs g) {
  constexpr int BK = Tr<T>::BK, P = Tr<T>::PITCH, MK = Tr<T>::MK;
  extern __shared__ __align__(16) unsigned char smem[];
  T* As = reinterpret_cast<T*>(smem);                   // [2][256][P]
  T* Bs = As + 2 * kTileM * P;                          // [2][256][P]

  // Tile order: consecutive workgroups walk N fastest within a band of rows so
  // that concurrently resident tiles share A rows and B columns in L2.
  const int64_t tile = blockIdx.x;
  const int64_t tm = tile / g.tiles_n, tn = tile % g.tiles_n;
  const int64_t m0 = tm * kTileM, n0 = tn * kTileN;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  const int64_t nk1 = ceil_div(g.K1, BK), nk2 = g.A2 ? ceil_div(g.K2, BK) : 0, nk = nk1 + nk2;

  f32x16_t acc[kFragM][kFragN];
#pragma unroll
  for (int i = 0; i < kFragM; ++i)
#pragma unroll
    for (int j = 0; j < kFragN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  Stage sa, sb;
  auto load_step = [&](int64_t s) {
    const bool seg2 = s >= nk1;
    const T* A = static_cast<const T*>(seg2 ? g.A2 : g.A1);
    const T* B = static_cast<const T*>(seg2 ? g.B2 : g.B1);
    const int64_t lda = seg2 ? g.lda2 : g.lda1, ldb = seg2 ? g.ldb2 : g.ldb1;
    const int64_t k0 = (seg2 ? s - nk1 : s) * BK, kend = seg2 ? g.K2 : g.K1;
    const T* msk = seg2 ? nullptr : static_cast<const T*>(g.bmask);
    const bool hs = !seg2 && g.has_scale;
    if (AL == 0)
      load_kc<T>(sa, A, lda, m0, g.M, k0, kend, nullptr, false, 1.0f);
    else
      load_rc<T>(sa, A, lda, m0, g.M, k0, kend, nullptr, false, 1.0f);
    if (BL == 0)
      load_kc<T>(sb, B, ldb, n0, g.N, k0, kend, msk, hs, g.bscale);
    else
      load_rc<T>(sb, B, ldb, n0, g.N, k0, kend, msk, hs, g.bscale);
  };
  auto store_step = [&](int buf) {
    T* a = As + buf * kTileM * P;
    T* b = Bs + buf * kTileN * P;
    if (AL == 0) store_kc<T>(sa, a); else store_rc<T>(sa, a);
    if (BL == 0) store_kc<T>(sb, b); else store_rc<T>(sb, b);
  };

  if (nk > 0) {
    load_step(0);
    store_step(0);
  }
  __syncthreads();

  for (int64_t s = 0; s < nk; ++s) {
    const int buf = static_cast<int>(s & 1);
    if (s + 1 < nk) load_step(s + 1);
    const T* a = As + buf * kTileM * P + (wm * kWaveM + (lane & 31)) * P;
    const T* b = Bs + buf * kTileN * P + (wn * kWaveN + (lane & 31)) * P;
#pragma unroll
    for (int kk = 0; kk < BK; kk += MK) {
      if constexpr (sizeof(T) == 2) {
        const int ko = kk + (lane >> 5) * 8;
        bf16x8_t fa[kFragM], fb[kFragN];
#pragma unroll
        for (int i = 0; i < kFragM; ++i) fa[i] = *reinterpret_cast<const bf16x8_t*>(a + i * 32 * P + ko);
#pragma unroll
        for (int j = 0; j < kFragN; ++j) fb[j] = *reinterpret_cast<const bf16x8_t*>(b + j * 32 * P + ko);
#pragma unroll
        for (int i = 0; i < kFragM; ++i)
#pragma unroll
          for (int j = 0; j < kFragN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
      } else {
        const int ko = kk + (lane >> 5);
        float fa[kFragM], fb[kFragN];
#pragma unroll
        for (int i = 0; i < kFragM; ++i) fa[i] = a[i * 32 * P + ko];
#pragma unroll
        for (int j = 0; j < kFragN; ++j) fb[j] = b[j * 32 * P + ko];
#pragma unroll
        for (int i = 0; i < kFragM; ++i)
#pragma unroll
          for (int j = 0; j < kFragN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i], fb[j], acc[i][j], 0, 0, 0);
      }
    }
    if (s + 1 < nk) store_step(buf ^ 1);
    __syncthreads();
  }

  // Epilogue.  32x32 accumulator layout: lane holds column (lane % 32) and
  // rows (e / 4) * 8 + (lane / 32) * 4 + e % 4, e = 0..15.
  const int cdt = g.c_dtype;
  const int edt = Tr<T>::DT;
#pragma unroll
  for (int i = 0; i < kFragM; ++i) {
#pragma unroll
    for (int j = 0; j < kFragN; ++j) {
      const int64_t col = n0 + wn * kWaveN + j * 32 + (lane & 31);
      if (col >= g.N) continue;
      const float bv = g.bias ? load_elem(g.bias, col, g.bias_dtype) : 0.0f;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int64_t row = m0 + wm * kWaveM + i * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
        if (row >= g.M) continue;
        const int64_t off = row * g.ldc + col;
        // result of the matmul in the output dtype, then the reference's follow-up ops
        float v = cdt == SF_DTYPE_BF16 ? round_bf16(acc[i][j][e]) : acc[i][j][e];
        if (g.bias) v = cdt == SF_DTYPE_BF16 ? round_bf16(v + bv) : v + bv;
        if (g.emask) {
          const float em = load_elem(g.emask, off, edt);
          if (g.dw) {
            if (em < 0.5f) {
              float d = g.decay * load_elem(g.dw, off, edt);
              if (cdt == SF_DTYPE_BF16) d = round_bf16(d);
              v = cdt == SF_DTYPE_BF16 ? round_bf16(v + d) : v + d;
            }
          } else {
            v = cdt == SF_DTYPE_BF16 ? round_bf16(v * em) : v * em;
          }
        }
        if (g.accumulate) {
          float o = load_elem(g.C, off, cdt);
          v = o + v;
        }
        store_from_f32(g.C, off, cdt, v);
      }
    }
  }
}

template <typename T>
constexpr size_t smem_bytes() {
  return sizeof(T) * 2ull * (kTileM + kTileN) * Tr<T>::PITCH;
}

template <typename T, int AL, int BL>
int launch_gemm(const GemmArgs& g, hipStream_t st) {
  static bool attr_set = false;  // per instantiation; host code runs the attribute call once
  auto kern = gemm_kernel<T, AL, BL>;
  const size_t smem = smem_bytes<T>();
  if (!attr_set) {
    SF_CHECK_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(smem)));
    attr_set = true;
  }
  const int64_t tiles = ceil_div(g.M, kTileM) * g.tiles_n;
  if (tiles == 0) return SF_OK;
  SF_CHECK_ARG(tiles < (1ll << 31), "GEMM grid too large");
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(tiles)), dim3(kThreads), smem, st, g);
  return launch_status("sf_gemm");
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace sf

using namespace sf;

extern "C" int sf_gemm(const sf_gemm_desc* d, void* stream) {
  SF_CHECK_ARG(d != nullptr, "null sf_gemm_desc");
  SF_CHECK_ARG(d->dtype == SF_DTYPE_BF16 || d->dtype == SF_DTYPE_F32, "bad element dtype %d", d->dtype);
  SF_CHECK_ARG(d->c_dtype == SF_DTYPE_BF16 || d->c_dtype == SF_DTYPE_F32, "bad output dtype %d", d->c_dtype);
  SF_CHECK_ARG(d->a_layout == SF_LAYOUT_K || d->a_layout == SF_LAYOUT_MN, "bad A layout");
  SF_CHECK_ARG(d->b_layout == SF_LAYOUT_K || d->b_layout == SF_LAYOUT_MN, "bad B layout");
  SF_CHECK_ARG(!(d->a_layout == SF_LAYOUT_MN && d->b_layout == SF_LAYOUT_K), "A M-contiguous with B K-contiguous is not built");
  SF_CHECK_ARG(d->M >= 0 && d->N >= 0 && d->K1 >= 0 && d->K2 >= 0, "negative GEMM size");
  if (d->M == 0 || d->N == 0) return SF_OK;
  SF_CHECK_ARG(d->C, "null C");
  SF_CHECK_ARG(d->K1 == 0 || (d->A1 && d->B1), "null A1/B1");
  SF_CHECK_ARG(d->K2 == 0 || (d->A2 && d->B2), "null A2/B2");
  const int vec = d->dtype == SF_DTYPE_BF16 ? 8 : 4;
  // every 16-byte vector must be aligned and lie inside its row: contiguous
  // extents and leading dimensions are multiples of the vector width.
  auto chk_operand = [&](const void* p, int64_t ld, int layout, int64_t rows, int64_t K) -> bool {
    if (!p || K == 0) return true;
    if (!al16(p) || ld % vec != 0) return false;
    if (layout == SF_LAYOUT_K) return K % vec == 0 && ld >= K;
    return rows % vec == 0 && ld >= rows;
  };
  SF_CHECK_ARG(chk_operand(d->A1, d->lda1, d->a_layout, d->M, d->K1) &&
                   chk_operand(d->A2, d->lda2, d->a_layout, d->M, d->K2) &&
                   chk_operand(d->B1, d->ldb1, d->b_layout, d->N, d->K1) &&
                   chk_operand(d->B2, d->ldb2, d->b_layout, d->N, d->K2) &&
                   chk_operand(d->bmask, d->ldb1, d->b_layout, d->N, d->K1),
               "GEMM operands must be 16-byte aligned with contiguous extents and leading dims that are multiples "
               "of %d elements (M=%lld N=%lld K1=%lld K2=%lld)",
               vec, (long long)d->M, (long long)d->N, (long long)d->K1, (long long)d->K2);
  SF_CHECK_ARG(d->ldc >= d->N, "ldc < N");
  SF_CHECK_ARG(!d->dw || d->emask, "the decay epilogue needs the effective mask");
  GemmArgs g;
  g.M = d->M; g.N = d->N; g.K1 = d->K1; g.K2 = d->K2;
  g.A1 = d->A1; g.lda1 = d->lda1; g.A2 = d->K2 ? d->A2 : nullptr; g.lda2 = d->lda2;
  g.B1 = d->B1; g.ldb1 = d->ldb1; g.B2 = d->B2; g.ldb2 = d->ldb2;
  g.bmask = d->bmask;
  g.bscale = d->bscale;
  g.has_scale = d->bscale != 1.0f;
  g.C = d->C; g.ldc = d->ldc; g.c_dtype = d->c_dtype;
  g.bias = d->bias; g.bias_dtype = d->bias_dtype;
  g.emask = d->emask; g.dw = d->dw; g.decay = d->decay;
  g.accumulate = d->accumulate;
  g.tiles_n = ceil_div(d->N, kTileN);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool bf = d->dtype == SF_DTYPE_BF16;
  if (d->a_layout == SF_LAYOUT_K && d->b_layout == SF_LAYOUT_K)
    return bf ? launch_gemm<uint16_t, 0, 0>(g, st) : launch_gemm<float, 0, 0>(g, st);
  if (d->a_layout == SF_LAYOUT_K)
    return bf ? launch_gemm<uint16_t, 0, 1>(g, st) : launch_gemm<float, 0, 1>(g, st);
  return bf ? launch_gemm<uint16_t, 1, 1>(g, st) : launch_gemm<float, 1, 1>(g, st);
}

// ---------------------------------------------------------------------------
// Column sums (bias gradient): a workgroup owns 64 columns; its 4 waves take
// interleaved rows and fold their partial sums in LDS in a fixed order.
// ---------------------------------------------------------------------------
namespace sf {
namespace {
__global__ void __launch_bounds__(256) column_sum_kernel(const void* __restrict__ A, int a_dtype, int64_t rows,
                                                         int64_t cols, void* __restrict__ out, int out_dtype) {
  __shared__ float part[4][64];
  const int c = threadIdx.x & 63, rg = threadIdx.x >> 6;
  const int64_t col = blockIdx.x * 64ll + c;
  float s = 0.0f;
  if (col < cols)
    for (int64_t r = rg; r < rows; r += 4) s += load_as_f32(A, r * cols + col, a_dtype);
  part[rg][c] = s;
  __syncthreads();
  if (rg == 0 && col < cols) store_from_f32(out, col, out_dtype, ((part[0][c] + part[1][c]) + part[2][c]) + part[3][c]);
}
}  // namespace
}  // namespace sf

extern "C" int sf_column_sum(const void* A, int a_dtype, int64_t rows, int64_t cols, void* out, int out_dtype,
                             void* stream) {
  SF_CHECK_ARG(rows >= 0 && cols >= 0, "negative shape");
  SF_CHECK_ARG((a_dtype == SF_DTYPE_F32 || a_dtype == SF_DTYPE_BF16) &&
                   (out_dtype == SF_DTYPE_F32 || out_dtype == SF_DTYPE_BF16),
               "bad dtype");
  if (cols == 0) return SF_OK;
  SF_CHECK_ARG(out && (rows == 0 || A), "null tensor");
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(column_sum_kernel, dim3(static_cast<unsigned>(ceil_div(cols, 64))), dim3(256), 0, st, A, a_dtype,
                     rows, cols, out, out_dtype);
  return launch_status("sf_column_sum");
}
