// Dense MFMA GEMM engine of the SparseLinear path (K1-K5) on gfx950.
//
//   C[M, N] = sum_k A(m, k) * B'(n, k)  (+ segment 2: sum_k A2(m, k) * B2(n, k))
//   B'(n, k) = B(n, k) * E(n, k) * s    (E: effective mask, optional)
//
// A is stored K-contiguous (A[m * lda + k]) or M-contiguous (A[k * lda + m]);
// B is stored K-contiguous (B[n * ldb + k]) or N-contiguous (B[k * ldb + n]).
// The three products of a masked linear map onto it as
//   forward    y  = x (W.E)^T : A K-contig (x [T, in]),   B K-contig (W [out, in])
//   input grad dx = dy (W.E)  : A K-contig (dy [T, out]), B N-contig (W [out, in])
//   weight grad dW = dy^T x   : A M-contig (dy [T, out]), B N-contig (x [T, in])
// The second K segment concatenates the SLoRB low-rank term into the same
// accumulators ([x | z] . [W.E | S]^T) instead of a separate GEMM + add.
//
// Tiling: 256 threads = 4 waves in a 2 x 2 grid; a workgroup owns a 256 x 256
// tile of C, each wave 128 x 128 as 4 x 4 blocks of v_mfma_f32_32x32x16_bf16
// (256 fp32 accumulators per lane, held in AGPRs).  One k-stage (64 k) of the
// A and B tiles is staged through double-buffered LDS laid out so that each
// MFMA fragment is one conflict-free 16-byte LDS read per lane.
//
// Two kernels share this tiling.  gemm_bf16_kernel (bf16 operands, the
// SparseLinear products) copies tiles global -> LDS with the buffer unit's
// direct-to-LDS loads (see its section below).  gemm_kernel (f32 operands, the
// block-sparse modes, masks whose rows are not 16-byte aligned) stages through
// registers: the global loads of stage s+2 are issued right after stage s+1 is
// written to LDS, and the mask multiply (B only) and, for M/N-contiguous
// operands, an 8 x 8 register transpose happen at the LDS write.  Neither
// writes a masked copy of W to memory.  Inside a stage the LDS reads of k-step
// kk+1 are issued before the MFMAs of kk.
//
// Tile order: dispatch ids are spread round-robin over the 8 XCDs; they are
// remapped so each XCD walks a contiguous range of tiles, ordered in bands of
// 8 M-tiles, which keeps the A and B k-slices of the concurrently resident
// tiles of one XCD in that XCD's L2.

#include <type_traits>

#include "sf_common.hpp"

namespace sf {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int kTileM = 256;
constexpr int kTileN = 256;
constexpr int kWaveM = 128;
constexpr int kWaveN = 128;
constexpr int kFragM = kWaveM / 32;  // 4
constexpr int kFragN = kWaveN / 32;  // 4
constexpr int kGroupM = 8;           // M-tiles per L2 band
constexpr int kXcds = 8;
constexpr int kEpiPitch = 132;     // f32 row pitch of the epilogue staging (64 rows x 128 cols per wave)

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
  int c_aligned;   // C is 16-byte aligned
  int64_t tiles_m, tiles_n;
  int splits;            // K splits (1: the kernel writes C itself)
  int64_t split_stages;  // segment-1 stages per split
  float* partial;        // splits > 1: [splits][M][N] f32 partial sums
  // block-sparse-16 B1 (B layouts 2 / 3): B1 is the blocks array, b_map its block map
  const int32_t* b_map;
  int64_t b_map_rows, b_map_cols;
  // block-sparse-16 C: the epilogue writes only the blocks c_map lists, into c_blocks
  void* c_blocks;
  const int32_t* c_map;
  int64_t c_map_rows, c_map_cols;
  int64_t ldbm;      // leading dimension of a K-major byte mask ([N][K1])
  int bmask_kmajor;  // bmask is K-major (input gradient: B = W^T, mask given transposed)
  int dma_mask_ok;   // the byte mask can be copied 16 bytes at a time (bf16 direct kernel)
};

// Element traits.  bf16 uses v_mfma_f32_32x32x16_bf16 (8 k-values per lane),
// f32 uses v_mfma_f32_32x32x2_f32 (1 k-value per lane).
template <typename T>
struct Tr;

template <>
struct Tr<uint16_t> {
  static constexpr int VEC = 8;     // elements per 16-byte vector
  static constexpr int BK = 64;     // k per LDS stage
  static constexpr int PITCH = 72;  // LDS row pitch (elements): 144 B keeps 16 B lane reads conflict-free
  static constexpr int MK = 16;     // k per MFMA
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
  r.w[0] = v.x;
  r.w[1] = v.y;
  r.w[2] = v.z;
  r.w[3] = v.w;
  return r;
}
__device__ __forceinline__ V4 zero16() {
  V4 r;
  r.w[0] = r.w[1] = r.w[2] = r.w[3] = 0u;
  return r;
}

// How B1 is masked while it is staged: not at all, by a multiplicative
// effective mask in the element dtype (rounded as the reference does), or by
// a byte and-mask (0x00 / 0xFF per element) for masks whose values are 0 or 1.
constexpr int kMaskNone = 0, kMaskMul = 1, kMaskByte = 2;

// Mask words that accompany one 16-byte operand vector.
template <typename T, int MK>
struct MaskWords {
  static constexpr int N = MK == kMaskMul ? 4 : (MK == kMaskByte ? (int)(16 / sizeof(T)) / 4 : 1);
};

// bf16 halves of a dword as f32, and the hardware round-to-nearest-even pack
// (v_cvt_pk_bf16_f32) back to two bf16.
__device__ __forceinline__ float lo_f(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_f(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  bf16x2_t v;
  v[0] = static_cast<__bf16>(lo);
  v[1] = static_cast<__bf16>(hi);
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ float hround(float x) { return static_cast<float>(static_cast<__bf16>(x)); }
__device__ __forceinline__ uint16_t hbits(float x) { return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x)); }

// Masked B vector.  Multiplicative mask, with the reference's rounding:
// w = round(W * E), then round(w * s) when a weight-scaling factor is set.
// Byte and-mask: each element is kept or zeroed (exactly W * E for E in {0, 1});
// v_perm widens mask bytes (b0, b1) to the dword (b0, b0, b1, b1).
template <typename T, int MK>
__device__ __forceinline__ V4 apply_mask(const V4& w, const uint32_t (&e)[MaskWords<T, MK>::N], bool has_scale,
                                         float s) {
  if constexpr (MK == kMaskNone) {
    return w;
  } else if constexpr (MK == kMaskByte) {
    V4 o;
    if constexpr (sizeof(T) == 2) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t m = e[i >> 1];
        o.w[i] = w.w[i] & __builtin_amdgcn_perm(m, m, (i & 1) ? 0x03030202u : 0x01010000u);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) o.w[i] = w.w[i] & __builtin_amdgcn_perm(e[0], e[0], 0x01010101u * i);
    }
    return o;
  } else {
    V4 o;
    if constexpr (sizeof(T) == 2) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float lo = lo_f(w.w[i]) * lo_f(e[i]);
        float hi = hi_f(w.w[i]) * hi_f(e[i]);
        if (has_scale) {
          lo = hround(lo) * s;
          hi = hround(hi) * s;
        }
        o.w[i] = pack2(lo, hi);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float v = __uint_as_float(w.w[i]) * __uint_as_float(e[i]);
        if (has_scale) v = v * s;
        o.w[i] = __float_as_uint(v);
      }
    }
    return o;
  }
}

// Transpose a VEC x VEC block held as VEC row vectors (row = k, lanes of the
// vector = m) into VEC vectors of k-values, one per m.
template <typename T>
__device__ __forceinline__ void transpose_block(const V4* v, V4* out) {
  if constexpr (sizeof(T) == 2) {
    // out[m].dword[j] = (in[2j][m], in[2j+1][m]) packed lo/hi
#pragma unroll
    for (int m = 0; m < 8; ++m) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t a = v[2 * j].w[m >> 1], b = v[2 * j + 1].w[m >> 1];
        const uint32_t sel = (m & 1) ? 0x07060302u : 0x05040100u;
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

// Per-thread share of one operand tile: 8 raw 16-byte vectors (+ their mask words).
template <typename T, int MK>
struct Stage {
  V4 v[8];
  uint32_t e[MK == kMaskNone ? 1 : 8][MaskWords<T, MK>::N];
};

// Raw buffer loads: an SGPR resource holds the tensor base and its byte
// extent; a lane offset at or past the extent reads zeros without touching
// memory, which is how rows past M/N and k past K are padded.
typedef __amdgpu_buffer_rsrc_t Rsrc;
constexpr uint32_t kOob = 0x80000000u;  // a lane offset past every operand's extent (extents are < 2^31 bytes)

__device__ __forceinline__ Rsrc make_rsrc(const void* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ V4 bload(Rsrc r, uint32_t voff, uint32_t soff) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0);
  V4 o;
  o.w[0] = x[0];
  o.w[1] = x[1];
  o.w[2] = x[2];
  o.w[3] = x[3];
  return o;
}

// Per-thread load state of one operand for one tile and one K segment.
//   K-contiguous (L == 0), element (r, k) at base[r * ld + k]: vector i of the
//   thread is row t / CPR + 32 i, k-chunk t % CPR; one lane offset per vector
//   (rows past the operand get an out-of-range offset), and the stage's k0 in
//   the scalar offset, which only ever moves in-range lanes to in-range bytes.
//   A wave reads 8 rows x 128 B per instruction.
//   Row-contiguous (L == 1), element (r, k) at base[k * ld + r]: the thread
//   owns VEC x VEC blocks (k-block t % KB, row-block t / KB [+ 32 for the second
//   f32 block]); one lane offset per loaded k-row, advanced by BK rows a stage.
template <typename T, int L>
struct Loader {
  static constexpr int VEC = Tr<T>::VEC, BK = Tr<T>::BK, CPR = BK / VEC;
  Rsrc rs, re;     // operand and (B1 only) its effective mask
  uint32_t off[8];  // lane byte offset of each of the thread's 8 vectors (kOob: padding)
  uint32_t k_step;  // row-contig: bytes one stage advances (BK rows)
  int kchunk;       // K-contig: first k of the thread's chunk within a stage
  int64_t k_end;

  // kstart: first k of the first stage this workgroup loads (row-contiguous
  // offsets advance from there; K-contiguous loads take k0 per call).
  __device__ __forceinline__ void init(const void* base, const void* emask, int64_t ld, int64_t row0,
                                       int64_t rows_total, int64_t kend, bool emask_bytes = false,
                                       int64_t kstart = 0) {
    const int t = threadIdx.x;
    k_end = kend;
    if constexpr (L == 0) {
      const int64_t bytes = rows_total * ld * (int64_t)sizeof(T);
      rs = make_rsrc(base, bytes);
      re = make_rsrc(emask ? emask : base, emask ? (emask_bytes ? bytes / (int64_t)sizeof(T) : bytes) : 0);
      kchunk = (t % CPR) * VEC;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int64_t row = row0 + t / CPR + 32 * i;
        off[i] = row < rows_total ? (uint32_t)((row * ld + kchunk) * (int64_t)sizeof(T)) : kOob;
      }
      k_step = 0;
    } else {
      const int64_t bytes = kend * ld * (int64_t)sizeof(T);
      rs = make_rsrc(base, bytes);
      re = make_rsrc(emask ? emask : base, emask ? (emask_bytes ? bytes / (int64_t)sizeof(T) : bytes) : 0);
      constexpr int KB = BK / VEC;
#pragma unroll
      for (int q = 0; q < 8 / VEC; ++q) {
        const int b = t + kThreads * q;
        const int kb = b % KB, rb = b / KB;
        const int64_t r = row0 + rb * VEC;
#pragma unroll
        for (int j = 0; j < VEC; ++j)
          off[q * VEC + j] =
              r < rows_total ? (uint32_t)(((kstart + kb * VEC + j) * ld + r) * (int64_t)sizeof(T)) : kOob;
      }
      k_step = (uint32_t)(BK * ld * (int64_t)sizeof(T));
      kchunk = 0;
    }
  }

  // Issue the loads of the stage starting at k0 (k0 advances by BK per call).
  // Mask words of the vector at operand byte offset o (scalar offset so):
  // the element-dtype mask shares the operand's offsets, the byte mask
  // takes them divided by the element size (kOob stays past its extent).
  template <int MK>
  __device__ __forceinline__ void load_mask(uint32_t (&e)[MaskWords<T, MK>::N], uint32_t o, uint32_t so) {
    if constexpr (MK == kMaskMul) {
      const V4 x = bload(re, o, so);
#pragma unroll
      for (int w = 0; w < 4; ++w) e[w] = x.w[w];
    } else if constexpr (MK == kMaskByte) {
      constexpr int sh = sizeof(T) == 2 ? 1 : 2;
      if constexpr (sizeof(T) == 2) {
        typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
        const u32x2 x = __builtin_amdgcn_raw_buffer_load_b64(re, (int)(o >> sh), (int)(so >> sh), 0);
        e[0] = x[0];
        e[1] = x[1];
      } else {
        e[0] = __builtin_amdgcn_raw_buffer_load_b32(re, (int)(o >> sh), (int)(so >> sh), 0);
      }
    }
  }

  template <int MK>
  __device__ __forceinline__ void load(Stage<T, MK>& st, int64_t k0) {
    if constexpr (L == 0) {
      const bool k_ok = k0 + kchunk < k_end;  // the k-tail chunk of the last stage reads zeros
      const uint32_t kb = (uint32_t)(k0 * (int64_t)sizeof(T));
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t o = k_ok ? off[i] : kOob;
        st.v[i] = bload(rs, o, kb);
        if constexpr (MK != kMaskNone) load_mask<MK>(st.e[i], o, kb);
      }
    } else {
      // k rows past K fall past the resource extent; lane offsets move by a stage afterwards
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        st.v[i] = bload(rs, off[i], 0);
        if constexpr (MK != kMaskNone) load_mask<MK>(st.e[i], off[i], 0);
        off[i] = off[i] >= kOob ? kOob : off[i] + k_step;
      }
    }
  }
  // Vector i of load(st, k0) alone (the same stage's vectors may be issued apart).
  template <int MK>
  __device__ __forceinline__ void load_one(Stage<T, MK>& st, int64_t k0, int i) {
    if constexpr (L == 0) {
      const bool k_ok = k0 + kchunk < k_end;
      const uint32_t kb = (uint32_t)(k0 * (int64_t)sizeof(T));
      const uint32_t o = k_ok ? off[i] : kOob;
      st.v[i] = bload(rs, o, kb);
      if constexpr (MK != kMaskNone) load_mask<MK>(st.e[i], o, kb);
    } else {
      st.v[i] = bload(rs, off[i], 0);
      if constexpr (MK != kMaskNone) load_mask<MK>(st.e[i], off[i], 0);
      off[i] = off[i] >= kOob ? kOob : off[i] + k_step;
    }
  }
};

// Vector i of store_kc (K-contiguous register path into a padded tile).
template <typename T, int MK>
__device__ __forceinline__ void store_kc_one(const Stage<T, MK>& st, T* lds, int i, bool has_scale, float s) {
  constexpr int VEC = Tr<T>::VEC, BK = Tr<T>::BK, CPR = BK / VEC, P = Tr<T>::PITCH;
  const int v = threadIdx.x + kThreads * i;
  V4 x = st.v[i];
  if constexpr (MK != kMaskNone) x = apply_mask<T, MK>(x, st.e[i], has_scale, s);
  T* dst = lds + (v / CPR) * P + (v % CPR) * VEC;
  *reinterpret_cast<uint4*>(dst) = make_uint4(x.w[0], x.w[1], x.w[2], x.w[3]);
}

template <typename T, int MK>
__device__ __forceinline__ void store_kc(const Stage<T, MK>& st, T* lds, bool has_scale, float s) {
  constexpr int VEC = Tr<T>::VEC, BK = Tr<T>::BK, CPR = BK / VEC, P = Tr<T>::PITCH;
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int v = t + kThreads * i;
    V4 x = st.v[i];
    if constexpr (MK != kMaskNone) x = apply_mask<T, MK>(x, st.e[i], has_scale, s);
    T* dst = lds + (v / CPR) * P + (v % CPR) * VEC;
    if constexpr (sizeof(T) == 2) {
      *reinterpret_cast<uint4*>(dst) = make_uint4(x.w[0], x.w[1], x.w[2], x.w[3]);
    } else {
      uint32_t* d = reinterpret_cast<uint32_t*>(dst);
      d[0] = x.w[0];
      d[1] = x.w[1];
      d[2] = x.w[2];
      d[3] = x.w[3];
    }
  }
}

template <typename T, int MK>
__device__ __forceinline__ void store_rc(const Stage<T, MK>& st, T* lds, bool has_scale, float s) {
  constexpr int VEC = Tr<T>::VEC, BK = Tr<T>::BK, KB = BK / VEC, P = Tr<T>::PITCH;
  constexpr int BLOCKS_PER_THREAD = 8 / VEC;
  const int t = threadIdx.x;
#pragma unroll
  for (int q = 0; q < BLOCKS_PER_THREAD; ++q) {
    const int b = t + kThreads * q;
    const int kb = b % KB, rb = b / KB;
    V4 in[VEC], out[VEC];
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      in[j] = st.v[q * VEC + j];
      if constexpr (MK != kMaskNone) in[j] = apply_mask<T, MK>(in[j], st.e[q * VEC + j], has_scale, s);
    }
    transpose_block<T>(in, out);
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      T* dst = lds + (rb * VEC + i) * P + kb * VEC;
      if constexpr (sizeof(T) == 2) {
        *reinterpret_cast<uint4*>(dst) = make_uint4(out[i].w[0], out[i].w[1], out[i].w[2], out[i].w[3]);
      } else {
        uint32_t* d = reinterpret_cast<uint32_t*>(dst);
        d[0] = out[i].w[0];
        d[1] = out[i].w[1];
        d[2] = out[i].w[2];
        d[3] = out[i].w[3];
      }
    }
  }
}

// Output vector m of transpose_block<uint16_t> alone (k-values of column m
// of the thread's 8 x 8 block), so the transpose can be spread over MFMAs.
__device__ __forceinline__ V4 transpose_one(const V4 (&v)[8], int m) {
  V4 o;
  const uint32_t sel = (m & 1) ? 0x07060302u : 0x05040100u;
#pragma unroll
  for (int j = 0; j < 4; ++j) o.w[j] = __builtin_amdgcn_perm(v[2 * j + 1].w[m >> 1], v[2 * j].w[m >> 1], sel);
  return o;
}
// LDS write of transposed vector m of the thread's block (the store_rc layout).
__device__ __forceinline__ void write_rc_one(const V4& x, uint16_t* lds, int m) {
  constexpr int VEC = 8, KB = 64 / VEC, P = Tr<uint16_t>::PITCH;
  const int b = threadIdx.x, kb = b % KB, rb = b / KB;
  uint16_t* dst = lds + (rb * VEC + m) * P + kb * VEC;
  *reinterpret_cast<uint4*>(dst) = make_uint4(x.w[0], x.w[1], x.w[2], x.w[3]);
}

// B operand gathered from a block-sparse-16 weight W: 16 x 16 blocks stored
// row-major in `blocks`, located through a block map [rows][cols] of block
// indices (-1: the block is pruned and reads as zeros).  TRANS = 0 (B layout
// 2): B(n, k) = W(n, k), the forward y = x W^T.  TRANS = 1 (B layout 3):
// B(n, k) = W(k, n), the input gradient dx = dy W.  Thread t owns 8
// consecutive 16-byte vectors of one block of the stage's tile (16 blocks
// along n x BK/16 along k), so a block's data is read as contiguous 128-byte
// runs; its map entry is fetched one stage ahead.
template <typename T, int TRANS>
struct BsrLoader {
  static constexpr int VEC = Tr<T>::VEC, BK = Tr<T>::BK, KBLK = BK / 16;
  static constexpr int VPB = 256 / VEC;     // vectors per block
  static constexpr int VPR = 16 / VEC;      // vectors per block row
  const T* blocks;
  const int32_t* map;
  int64_t nbr, nbc;  // block-map extent
  int64_t nb0;       // first block along n of the tile
  int bn, bk, w0;    // the thread's block (along n, along k within a stage) and first vector in it
  int32_t idx_next;  // map entry of the thread's block in the next stage to load

  __device__ __forceinline__ void init(const void* blk, const int32_t* m, int64_t rows, int64_t cols, int64_t n0,
                                       int64_t kstart) {
    blocks = static_cast<const T*>(blk);
    map = m;
    nbr = rows;
    nbc = cols;
    nb0 = n0 / 16;
    const int b = (threadIdx.x * 8) / VPB;
    bn = b / KBLK;
    bk = b % KBLK;
    w0 = (threadIdx.x * 8) % VPB;
    idx_next = lookup(kstart);
  }
  __device__ __forceinline__ int32_t lookup(int64_t k0) const {
    const int64_t kb = k0 / 16 + bk, n_b = nb0 + bn;
    const int64_t r = TRANS ? kb : n_b, c = TRANS ? n_b : kb;
    if (r >= nbr || c >= nbc) return -1;
    return map[r * nbc + c];
  }
  // Load the stage at k0 (its map entry was fetched by the previous call) and
  // prefetch the map entry of the stage after it.  Returns the block index.
  __device__ __forceinline__ int32_t load(Stage<T, kMaskNone>& st, int64_t k0) {
    const int32_t idx = idx_next;
    idx_next = lookup(k0 + BK);
    const T* src = blocks + (int64_t)(idx < 0 ? 0 : idx) * 256 + w0 * VEC;
#pragma unroll
    for (int i = 0; i < 8; ++i) st.v[i] = idx >= 0 ? ld16(src + i * VEC) : zero16();
    return idx;
  }
  // Write the staged vectors to the B tile of LDS ([n][k], pitch P), and the
  // block's presence flag (by the thread holding the block's first vectors).
  __device__ __forceinline__ void store(const Stage<T, kMaskNone>& st, int32_t idx, T* lds, uint8_t* pres) const {
    constexpr int P = Tr<T>::PITCH;
    if (w0 == 0) pres[bn * KBLK + bk] = idx >= 0 ? 1 : 0;
    if constexpr (TRANS == 0) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int w = w0 + i, row = w / VPR, ch = w % VPR;
        T* dst = lds + (bn * 16 + row) * P + bk * 16 + ch * VEC;
        if constexpr (sizeof(T) == 2) {
          *reinterpret_cast<uint4*>(dst) = make_uint4(st.v[i].w[0], st.v[i].w[1], st.v[i].w[2], st.v[i].w[3]);
        } else {
          uint32_t* d = reinterpret_cast<uint32_t*>(dst);
          d[0] = st.v[i].w[0];
          d[1] = st.v[i].w[1];
          d[2] = st.v[i].w[2];
          d[3] = st.v[i].w[3];
        }
      }
    } else {
      // the thread holds KR consecutive block rows (= k) x 16 columns (= n):
      // write, for each n, its KR k-values contiguously
      constexpr int KR = 8 / VPR;  // 4 (bf16) or 2 (f32)
      const int k_row0 = w0 / VPR;
#pragma unroll
      for (int n = 0; n < 16; ++n) {
        const int ch = n / VEC, e = n % VEC;
        T* dst = lds + (bn * 16 + n) * P + bk * 16 + k_row0;
        if constexpr (sizeof(T) == 2) {
          uint32_t h[KR];
#pragma unroll
          for (int r = 0; r < KR; ++r) {
            const uint32_t wd = st.v[r * VPR + ch].w[e >> 1];
            h[r] = (e & 1) ? (wd >> 16) : (wd & 0xffffu);
          }
          *reinterpret_cast<uint2*>(dst) = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
        } else {
          uint32_t* d = reinterpret_cast<uint32_t*>(dst);
#pragma unroll
          for (int r = 0; r < KR; ++r) d[r] = st.v[r * VPR + ch].w[e];
        }
      }
    }
  }
};

// Tile coordinates of workgroup `pid` (XCD-contiguous ranges, bands of kGroupM M-tiles).
__device__ __forceinline__ void tile_coords(int64_t pid, int64_t tiles_m, int64_t tiles_n, int64_t& tm, int64_t& tn) {
  const int64_t total = tiles_m * tiles_n;
  if (total % kXcds == 0) pid = (pid % kXcds) * (total / kXcds) + pid / kXcds;
  const int64_t band = kGroupM * tiles_n;
  const int64_t first_m = (pid / band) * kGroupM;
  const int64_t gm = tiles_m - first_m < kGroupM ? tiles_m - first_m : kGroupM;
  const int64_t r = pid % band;
  tm = first_m + r % gm;
  tn = r / gm;
}

__device__ __forceinline__ float load_elem(const void* p, int64_t i, int dtype) { return load_as_f32(p, i, dtype); }

// Epilogue shared by the GEMM kernels: the 4 x 4 accumulator blocks of each
// wave (its 128 x 128 share of the 256 x 256 tile) go to C, a split-K partial
// buffer or the kept blocks of a block-sparse C.
template <typename T>
__device__ __forceinline__ void gemm_epilogue(const GemmArgs& g, const f32x16_t (&acc)[kFragM * kFragN],
                                              unsigned char* smem, int64_t m0, int64_t n0, int64_t kz) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  // Epilogue.  32x32 accumulator layout: lane holds column (lane % 32) and
  // rows (e / 4) * 8 + (lane / 32) * 4 + e % 4, e = 0..15.  The accumulators
  // go through LDS in two halves of 64 rows per wave (the operand buffers are
  // free now); each lane then owns 8 consecutive columns of a row, so C is
  // read and written with 16-byte accesses and the optional epilogue operands
  // (bias, mask product, decay term, accumulation) are read coalesced.
  float* ep = reinterpret_cast<float*>(smem) + wave * (64 * kEpiPitch);
  const int64_t wrow0 = m0 + wm * kWaveM, wcol0 = n0 + wn * kWaveN;
  const bool cbf = g.c_dtype == SF_DTYPE_BF16;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    __syncthreads();
#pragma unroll
    for (int ii = 0; ii < 2; ++ii)
#pragma unroll
      for (int j = 0; j < kFragN; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int r = ii * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
          ep[r * kEpiPitch + j * 32 + (lane & 31)] = acc[(2 * h + ii) * kFragN + j][e];
        }
    __syncthreads();
    for (int it = 0; it < 16; ++it) {
      const int flat = it * 64 + lane;
      const int r = flat >> 4, c = (flat & 15) * 8;
      const int64_t row = wrow0 + h * 64 + r, col = wcol0 + c;
      if (row >= g.M || col >= g.N) continue;
      float v[8];
      const float4 p0 = *reinterpret_cast<const float4*>(ep + r * kEpiPitch + c);
      const float4 p1 = *reinterpret_cast<const float4*>(ep + r * kEpiPitch + c + 4);
      v[0] = p0.x; v[1] = p0.y; v[2] = p0.z; v[3] = p0.w;
      v[4] = p1.x; v[5] = p1.y; v[6] = p1.z; v[7] = p1.w;
      if (g.c_blocks) {
        // block-sparse C (the SDDMM weight gradient): only kept 16 x 16 blocks are written,
        // row (row % 16) of block c_map[row / 16][col / 16], 8 columns at a time
        const int64_t bi = (row / 16 < g.c_map_rows && col / 16 < g.c_map_cols)
                               ? g.c_map[(row / 16) * g.c_map_cols + col / 16] : -1;
        if (bi >= 0) {
          const int64_t o = bi * 256 + (row % 16) * 16 + (col % 16);
          if (g.c_dtype == SF_DTYPE_BF16) {
            *reinterpret_cast<uint4*>(static_cast<uint16_t*>(g.c_blocks) + o) =
                make_uint4(pack2(v[0], v[1]), pack2(v[2], v[3]), pack2(v[4], v[5]), pack2(v[6], v[7]));
          } else {
            float* cp = static_cast<float*>(g.c_blocks) + o;
            *reinterpret_cast<float4*>(cp) = make_float4(v[0], v[1], v[2], v[3]);
            *reinterpret_cast<float4*>(cp + 4) = make_float4(v[4], v[5], v[6], v[7]);
          }
        }
        continue;
      }
      if (g.splits > 1) {
        // split-K: raw f32 partial sums; sf_gemm's reduce kernel applies the epilogue
        float* pp = g.partial + (kz * g.M + row) * g.N + col;
        if (col + 8 <= g.N && (g.N & 3) == 0) {
          *reinterpret_cast<float4*>(pp) = make_float4(v[0], v[1], v[2], v[3]);
          *reinterpret_cast<float4*>(pp + 4) = make_float4(v[4], v[5], v[6], v[7]);
        } else {
          for (int q = 0; q < 8 && col + q < g.N; ++q) pp[q] = v[q];
        }
        continue;
      }
      const int64_t off = row * g.ldc + col;
      const bool vec = g.c_aligned && col + 8 <= g.N && (off & 7) == 0;
      if (!g.emask && vec) {
        // result of the matmul in the output dtype, then + bias (rounded again), then + C when
        // accumulating: the per-element sequence below, 8 outputs at a time
        if (g.bias) {
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            const float b = load_elem(g.bias, col + q, g.bias_dtype);
            v[q] = cbf ? hround(v[q]) + b : v[q] + b;
          }
        }
        if (g.accumulate) {
          float c[8];
          if (cbf) {
            const uint4 cw = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(g.C) + off);
            const uint32_t w4[4] = {cw.x, cw.y, cw.z, cw.w};
#pragma unroll
            for (int q = 0; q < 8; ++q) c[q] = bf16_to_f32(static_cast<uint16_t>(w4[q >> 1] >> (16 * (q & 1))));
          } else {
            const float4 c0 = *reinterpret_cast<const float4*>(static_cast<const float*>(g.C) + off);
            const float4 c1 = *reinterpret_cast<const float4*>(static_cast<const float*>(g.C) + off + 4);
            c[0] = c0.x; c[1] = c0.y; c[2] = c0.z; c[3] = c0.w;
            c[4] = c1.x; c[5] = c1.y; c[6] = c1.z; c[7] = c1.w;
          }
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            const float x = cbf ? hround(v[q]) : v[q];  // the product (+ bias) in the output dtype
            v[q] = c[q] + x;
          }
        }
        if (cbf) {
          *reinterpret_cast<uint4*>(static_cast<uint16_t*>(g.C) + off) =
              make_uint4(pack2(v[0], v[1]), pack2(v[2], v[3]), pack2(v[4], v[5]), pack2(v[6], v[7]));
        } else {
          float* cp = static_cast<float*>(g.C) + off;
          *reinterpret_cast<float4*>(cp) = make_float4(v[0], v[1], v[2], v[3]);
          *reinterpret_cast<float4*>(cp + 4) = make_float4(v[4], v[5], v[6], v[7]);
        }
        continue;
      }
      const int edt = Tr<T>::DT;
      for (int q = 0; q < 8; ++q) {
        if (col + q >= g.N) break;
        const int64_t o = off + q;
        float x = cbf ? hround(v[q]) : v[q];
        if (g.bias) {
          const float b = load_elem(g.bias, col + q, g.bias_dtype);
          x = cbf ? hround(x + b) : x + b;
        }
        if (g.emask) {
          const float em = load_elem(g.emask, o, edt);
          if (g.dw) {
            if (em < 0.5f) {
              float d = g.decay * load_elem(g.dw, o, edt);
              if (cbf) d = hround(d);
              x = cbf ? hround(x + d) : x + d;
            }
          } else {
            x = cbf ? hround(x * em) : x * em;
          }
        }
        if (g.accumulate) x = load_elem(g.C, o, g.c_dtype) + x;
        if (cbf)
          static_cast<uint16_t*>(g.C)[o] = hbits(x);
        else
          static_cast<float*>(g.C)[o] = x;
      }
    }
  }
}

template <typename T, int AL, int BL, int MASK>
__global__ void __launch_bounds__(kThreads, 1) gemm_kernel(GemmArgs g) {
  constexpr int BK = Tr<T>::BK, P = Tr<T>::PITCH, MK = Tr<T>::MK, KSTEPS = BK / MK;
  extern __shared__ __align__(16) unsigned char smem[];
  T* As = reinterpret_cast<T*>(smem);  // [2][256][P]
  T* Bs = As + 2 * kTileM * P;         // [2][256][P]

  // Split-K: workgroups [kz * tiles, (kz + 1) * tiles) take segment-1 stages
  // [kz * split_stages, (kz + 1) * split_stages); the last split also runs segment 2.
  const int64_t tiles = g.tiles_m * g.tiles_n;
  const int64_t kz = blockIdx.x / tiles;
  int64_t tm, tn;
  tile_coords(blockIdx.x - kz * tiles, g.tiles_m, g.tiles_n, tm, tn);
  const int64_t m0 = tm * kTileM, n0 = tn * kTileN;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  const int64_t nk1_all = ceil_div(g.K1, BK);
  const int64_t s_begin = kz * g.split_stages;
  const int64_t s_end = (s_begin + g.split_stages < nk1_all) ? s_begin + g.split_stages : nk1_all;
  const int64_t nk1 = s_end > s_begin ? s_end - s_begin : 0;  // segment-1 stages of this workgroup
  const int64_t nk2 = (g.A2 && kz == g.splits - 1) ? ceil_div(g.K2, BK) : 0;
  const int64_t kbase = s_begin * BK;
  const bool has_scale = g.has_scale != 0;
  const float bscale = g.bscale;

  f32x16_t acc[kFragM * kFragN];
#pragma unroll
  for (int i = 0; i < kFragM * kFragN; ++i) acc[i] = f32x16_t{};

  // Segment 1 (A1 . (B1.E.s)^T) runs through the pipelined loop below.
  constexpr bool kBsr = BL >= 2;  // B1 is a block-sparse-16 weight (layouts 2 / 3)
  constexpr int kBlkK = BK / 16;  // block columns of a stage along k
  uint8_t* pres = smem + 2 * (kTileM + kTileN) * P * sizeof(T);  // [2][16][kBlkK] presence of B blocks
  Loader<T, AL> la;
  Loader<T, (BL >= 2 ? 0 : BL)> lb;
  BsrLoader<T, (BL == 3 ? 1 : 0)> lbs;
  la.init(g.A1, nullptr, g.lda1, m0, g.M, g.K1, false, kbase);
  if constexpr (kBsr)
    lbs.init(g.B1, g.b_map, g.b_map_rows, g.b_map_cols, n0, kbase);
  else
    lb.init(g.B1, MASK != kMaskNone ? g.bmask : nullptr, g.ldb1, n0, g.N, g.K1, MASK == kMaskByte, kbase);
  Stage<T, kMaskNone> sa;
  Stage<T, MASK> sb;
  int32_t sb_idx = -1;  // block index of the staged B block (block-sparse B)
  auto load_b = [&](int64_t k0) {
    if constexpr (kBsr)
      sb_idx = lbs.load(sb, k0);
    else
      lb.load(sb, k0);
  };

  auto store_a = [&](const Stage<T, kMaskNone>& st, int buf) {
    T* a = As + buf * kTileM * P;
    if (AL == 0)
      store_kc<T, kMaskNone>(st, a, false, 1.0f);
    else
      store_rc<T, kMaskNone>(st, a, false, 1.0f);
  };
  auto store_b = [&](int buf) {
    T* b = Bs + buf * kTileN * P;
    if constexpr (kBsr)
      lbs.store(sb, sb_idx, b, pres + buf * 16 * kBlkK);
    else if (BL == 0)
      store_kc<T, MASK>(sb, b, has_scale, bscale);
    else
      store_rc<T, MASK>(sb, b, has_scale, bscale);
  };
  // block-sparse B: does N-fragment j of this wave meet a kept block at k-step kk?
  auto frag_live = [&](int buf, int j, int kk) -> bool {
    if constexpr (!kBsr) {
      return true;
    } else {
      const uint8_t* pr = pres + buf * 16 * kBlkK;
      const int nb = (wn * kWaveN + j * 32) / 16, kb = (kk * MK) / 16;
      return (pr[nb * kBlkK + kb] | pr[(nb + 1) * kBlkK + kb]) != 0;
    }
  };

  // MFMAs of one LDS stage; hook(kk) runs after the MFMAs of k-step kk are issued.
  auto mfma_stage = [&](int buf, auto&& hook) {
    const T* a = As + buf * kTileM * P + (wm * kWaveM + (lane & 31)) * P;
    const T* b = Bs + buf * kTileN * P + (wn * kWaveN + (lane & 31)) * P;
    if constexpr (sizeof(T) == 2) {
      bf16x8_t fa[2][kFragM], fb[2][kFragN];
      const int kl = (lane >> 5) * 8;
#pragma unroll
      for (int i = 0; i < kFragM; ++i) fa[0][i] = *reinterpret_cast<const bf16x8_t*>(a + i * 32 * P + kl);
#pragma unroll
      for (int j = 0; j < kFragN; ++j) fb[0][j] = *reinterpret_cast<const bf16x8_t*>(b + j * 32 * P + kl);
#pragma unroll
      for (int kk = 0; kk < KSTEPS; ++kk) {
        const int cur = kk & 1;
        if (kk + 1 < KSTEPS) {
          const int ko = (kk + 1) * MK + kl;
#pragma unroll
          for (int i = 0; i < kFragM; ++i) fa[cur ^ 1][i] = *reinterpret_cast<const bf16x8_t*>(a + i * 32 * P + ko);
#pragma unroll
          for (int j = 0; j < kFragN; ++j) fb[cur ^ 1][j] = *reinterpret_cast<const bf16x8_t*>(b + j * 32 * P + ko);
        }
#pragma unroll
        for (int j = 0; j < kFragN; ++j) {
          if (!frag_live(buf, j, kk)) continue;  // both 16-row blocks of the fragment pruned
#pragma unroll
          for (int i = 0; i < kFragM; ++i)
            acc[i * kFragN + j] =
                __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[cur][i], fb[cur][j], acc[i * kFragN + j], 0, 0, 0);
        }
        hook(kk * 4 / KSTEPS);
      }
    } else {
#pragma unroll
      for (int kk = 0; kk < KSTEPS; ++kk) {
        const int ko = kk * MK + (lane >> 5);
        float fa[kFragM], fb[kFragN];
#pragma unroll
        for (int i = 0; i < kFragM; ++i) fa[i] = a[i * 32 * P + ko];
#pragma unroll
        for (int j = 0; j < kFragN; ++j) fb[j] = b[j * 32 * P + ko];
#pragma unroll
        for (int j = 0; j < kFragN; ++j) {
          if (!frag_live(buf, j, kk)) continue;
#pragma unroll
          for (int i = 0; i < kFragM; ++i)
            acc[i * kFragN + j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i], fb[j], acc[i * kFragN + j], 0, 0, 0);
        }
        if (kk % (KSTEPS / 4) == 0) hook(kk * 4 / KSTEPS);
      }
    }
  };

  if (nk1 > 0) {
    la.load(sa, kbase);
    load_b(kbase);
    store_a(sa, 0);
    store_b(0);
  }
  if (nk1 > 1) {
    la.load(sa, kbase + BK);
    load_b(kbase + BK);
  }
  __syncthreads();

  // Stage s: MFMAs over LDS buffer s & 1.  Interleaved with them (one quarter
  // of the stage each): the raw registers of stage s+1 go to the other buffer
  // (A, then B, with the mask applied), and the loads of stage s+2 are issued
  // into the freed registers (A, then B).  The other buffer was last read in
  // stage s-1, which every wave finished at the barrier.
  for (int64_t s = 0; s < nk1; ++s) {
    const int buf = static_cast<int>(s & 1);
    const bool do_store = s + 1 < nk1, do_load = s + 2 < nk1;
    const int64_t k_next = kbase + (s + 2) * BK;
    mfma_stage(buf, [&](int q) {
      if (q == 0 && do_store) {
        store_a(sa, buf ^ 1);
        if (do_load) la.load(sa, k_next);
      }
      if (q == 1 && do_store) {
        store_b(buf ^ 1);
        if (do_load) load_b(k_next);
      }
    });
    __syncthreads();
  }

  // Segment 2 (the SLoRB term A2 . B2^T, a few stages, never masked): plain
  // load -> LDS -> MFMA steps through buffer 0.
  if (nk2 > 0) {
    Loader<T, AL> la2;
    Loader<T, (BL >= 2 ? 0 : BL)> lb2;
    la2.init(g.A2, nullptr, g.lda2, m0, g.M, g.K2);
    lb2.init(g.B2, nullptr, g.ldb2, n0, g.N, g.K2);
    for (int64_t s2 = 0; s2 < nk2; ++s2) {
      Stage<T, kMaskNone> ta, tb;
      la2.load(ta, s2 * BK);
      lb2.load(tb, s2 * BK);
      store_a(ta, 0);
      if (BL == 0)
        store_kc<T, kMaskNone>(tb, Bs, false, 1.0f);
      else
        store_rc<T, kMaskNone>(tb, Bs, false, 1.0f);
      __syncthreads();
      mfma_stage(0, [](int) {});
      __syncthreads();
    }
  }

  gemm_epilogue<T>(g, acc, smem, m0, n0, kz);
}

// ---------------------------------------------------------------------------
// bf16 kernel with direct-to-LDS staging (gfx950 `buffer_load_dwordx4 ... lds`).
//
// Operands are copied global -> LDS by the buffer unit without passing through
// registers; one wave instruction moves 64 x 16 B into 1 KiB of LDS.
//  * K-contiguous tiles (x, dy, W of the forward, the SLoRB operands): 256 rows
//    x 128 B, unpadded, chunks XOR-swizzled (slot s of row r holds chunk
//    s ^ f(r), f(r) = (r ^ r >> 3) & 7) so that the 16-byte fragment reads of 8
//    and of 16 consecutive rows fall in distinct banks.
//  * M/N-contiguous tiles (W of the input gradient, dy and x of the weight
//    gradient): 64 k-rows x 512 B with chunk c of row k at c ^ 4 (k & 3); the
//    MFMA fragments are read transposed with ds_read_b64_tr_b16.
//  * The hard 2:4 byte and-mask: K-major 256 rows x 64 B (the input-gradient
//    product reads its transposed copy, sf_transpose_u8), applied to the B
//    fragments with a byte permute + AND after they are read.
// Only a multiplicative (soft / mixed) mask keeps the register path for B:
// load, multiply, store into the padded 144-byte-pitch layout.
//
// Stage s (LDS buffer b = s & 1 holds it):
//   k-steps 0..2: MFMAs of k-step kk, fragment reads of k-step kk + 1
//   wait for this wave's copies into b ^ 1 and its fragment reads, barrier:
//     b ^ 1 (stage s + 1) is complete; b is no longer read by anyone
//   k-step 3: MFMAs interleaved with the fragment reads of k-step 0 of stage
//     s + 1 (from b ^ 1) and the copies of stage s + 2 into b
// LDS latency is covered by a k-step of MFMAs everywhere, and each copy has a
// whole stage to land.  A scheduling barrier after every MFMA keeps this
// interleave; the steady-state loop is unrolled twice so buffer offsets are
// immediates.
// ---------------------------------------------------------------------------
constexpr int kRowSw = 128;  // bytes per row of a swizzled (DMA) tile: 64 bf16
constexpr int kRowPad = 144; // bytes per row of a padded (register-path) tile

// One 16-byte-per-lane copy global -> LDS: lane l's 16 bytes land at lds + 16 l.
// Issued as inline assembly so the compiler does not track it: it would
// otherwise make every later LDS access that it cannot prove disjoint wait for
// all copies in flight.  The kernels wait for their copies themselves
// (s_waitcnt vmcnt(0) before the barrier that publishes a buffer).
__device__ __forceinline__ void dma16(Rsrc r, uint32_t lds, uint32_t voff, uint32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :: "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(voff), "s"(r), "s"(soff) : "memory", "m0");
}
// LDS byte address of a pointer into the kernel's dynamic LDS (`base` its start).
__device__ __forceinline__ uint32_t lds_addr(const unsigned char* base) {
  return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const unsigned char*)base;
}

// Direct copy of a K-contiguous bf16 operand tile (256 rows x 64 k) into a
// swizzled LDS tile.  Wave w copies rows [64 w, 64 w + 64) with 8 instructions;
// in instruction i lane l covers row 64 w + 8 i + l / 8, slot l % 8, i.e.
// chunk c = (l % 8) ^ f(row) = (l % 8) ^ (l / 8) ^ i.
struct DmaLoader {
  Rsrc rs;
  uint32_t off[8];  // lane byte offset (row, chunk) of instruction i; kOob for rows past the operand
  int64_t k_end;

  __device__ __forceinline__ void init(const void* base, int64_t ld, int64_t row0, int64_t rows_total,
                                       int64_t kend) {
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    rs = make_rsrc(base, rows_total * ld * 2);
    k_end = kend;
    const int c0 = (lane & 7) ^ (lane >> 3);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t row = row0 + w * 64 + i * 8 + (lane >> 3);
      off[i] = row < rows_total ? (uint32_t)((row * ld + (c0 ^ i) * 8) * 2) : kOob;
    }
  }
  // Instruction i of issue<false> alone.
  __device__ __forceinline__ void issue_one(uint32_t tile, int64_t k0, int i) const {
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    dma16(rs, tile + w * 64 * kRowSw + i * 8 * kRowSw, off[i], (uint32_t)(k0 * 2));
  }
  // Issue the copy of the stage at k0 into `tile` (256 rows x 128 B).  TAIL:
  // the stage may end past K (its chunks at or past K read zeros).
  template <bool TAIL>
  __device__ __forceinline__ void issue(uint32_t tile, int64_t k0) const {
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t dst = tile + w * 64 * kRowSw;
    const uint32_t soff = (uint32_t)(k0 * 2);
    if constexpr (!TAIL) {
#pragma unroll
      for (int i = 0; i < 8; ++i) dma16(rs, dst + i * 8 * kRowSw, off[i], soff);
    } else {
      const int64_t kv = k_end - k0;  // valid k of this stage
      const int c0 = (lane & 7) ^ (lane >> 3);
#pragma unroll
      for (int i = 0; i < 8; ++i) dma16(rs, dst + i * 8 * kRowSw, ((c0 ^ i) * 8 < kv) ? off[i] : kOob, soff);
    }
  }
};

// Direct copy of a byte and-mask tile (256 rows x 64 k, one byte per element)
// into LDS rows of 64 B.  Wave w copies rows [64 w, 64 w + 64) with 4
// instructions; in instruction i lane l covers row 64 w + 16 i + l / 4, slot
// l % 4, which holds 16-byte chunk (l % 4) ^ g(row), g(row) = (row >> 2) & 3
// = (l >> 4) & 3.
struct DmaMaskLoader {
  Rsrc rs;
  uint32_t off[4];
  int64_t k_end;

  __device__ __forceinline__ void init(const void* base, int64_t ld, int64_t row0, int64_t rows_total,
                                       int64_t kend) {
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    rs = make_rsrc(base, rows_total * ld);
    k_end = kend;
    const int c = (lane & 3) ^ ((lane >> 4) & 3);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t row = row0 + w * 64 + i * 16 + (lane >> 2);
      off[i] = row < rows_total ? (uint32_t)(row * ld + c * 16) : kOob;
    }
  }
  template <bool TAIL>
  __device__ __forceinline__ void issue(uint32_t tile, int64_t k0) const {
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t dst = tile + w * 64 * 64;
    const int64_t kv = k_end - k0;
    const int c = (lane & 3) ^ ((lane >> 4) & 3);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      dma16(rs, dst + i * 16 * 64, (!TAIL || c * 16 < kv) ? off[i] : kOob, (uint32_t)k0);
  }
  __device__ __forceinline__ void issue_one(uint32_t tile, int64_t k0, int i) const {
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    dma16(rs, tile + w * 64 * 64 + i * 16 * 64, off[i], (uint32_t)k0);
  }
};

// A bf16 fragment with its 8 mask bytes (0x00 / 0xFF) applied.
__device__ __forceinline__ bf16x8_t and_bytes(bf16x8_t x, uint2 m) {
  uint4 w = __builtin_bit_cast(uint4, x);
  w.x &= __builtin_amdgcn_perm(m.x, m.x, 0x01010000u);
  w.y &= __builtin_amdgcn_perm(m.x, m.x, 0x03030202u);
  w.z &= __builtin_amdgcn_perm(m.y, m.y, 0x01010000u);
  w.w &= __builtin_amdgcn_perm(m.y, m.y, 0x03030202u);
  return __builtin_bit_cast(bf16x8_t, w);
}

// Direct copy of an M/N-contiguous bf16 operand tile (64 k rows x 256 columns
// of a row-major [K, cols] matrix) into LDS rows of 512 B.  Wave w copies rows
// [16 w, 16 w + 16) with 8 instructions of 2 rows each; in instruction i lane l
// covers row 16 w + 2 i + l / 32, slot l % 32, which holds 16-byte column chunk
// (l % 32) ^ fmn(row), fmn(row) = 4 (row & 3).  Rows past K lie past the
// resource extent and read zeros; the offsets advance by a stage per copy.
struct DmaLoaderMN {
  Rsrc rs;
  uint32_t off[8];
  uint32_t k_step;

  __device__ __forceinline__ void init(const void* base, int64_t ld, int64_t col0, int64_t cols_total, int64_t kend,
                                       int64_t kstart) {
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    rs = make_rsrc(base, kend * ld * 2);
    k_step = (uint32_t)(64 * ld * 2);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = 16 * w + 2 * i + (lane >> 5);
      const int64_t col = col0 + 8 * ((lane & 31) ^ (4 * (row & 3)));
      off[i] = col < cols_total ? (uint32_t)(((kstart + row) * ld + col) * 2) : kOob;
    }
  }
  __device__ __forceinline__ void issue_one(uint32_t tile, int i) {
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    dma16(rs, tile + w * 16 * 512 + i * 1024, off[i], 0);
    off[i] = off[i] >= kOob ? kOob : off[i] + k_step;
  }
  __device__ __forceinline__ void issue(uint32_t tile) {
#pragma unroll
    for (int i = 0; i < 8; ++i) issue_one(tile, i);
  }
};

// Lane byte offset in an M/N-contiguous tile of the transposed reads of MFMA
// fragment rows [r0, r0 + 32) at k-step 0 (k-step kk adds kk * 8192, the
// second 4 k-values 2048).  ds_read_b64_tr_b16 hands lane 4q + c of each
// 16-lane group the c-th 16-bit value of the rows addressed by lanes
// q, q + 4, q + 8, q + 12; lane L therefore addresses row k = L / 4 (+ 8 for
// the second half-wave) at the 4 columns 4 (L % 4) of the group's 16.
__device__ __forceinline__ uint32_t mn_frag_base(int r0) {
  const int lane = threadIdx.x & 63, grp = lane >> 4, L = lane & 15, q = L >> 2;
  const int k = 8 * (grp >> 1) + q;
  const int col = r0 + 16 * (grp & 1) + 4 * (L & 3);
  return (uint32_t)(k * 512 + (((col >> 3) ^ (4 * q)) << 4) + (col & 7) * 2);
}
typedef short v4i16_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ bf16x8_t tr_frag(const unsigned char* p) {
  typedef __attribute__((address_space(3))) v4i16_t lds_v4;
  const v4i16_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4*)(p));
  const v4i16_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4*)(p + 2048));
  return __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

// Byte offset, within its tile, of the lane's fragment row `r` at k-step 0;
// k-step kk is at `base ^ (kk << 5)` (swizzled) or `base + kk * 32` (padded).
template <bool SW>
__device__ __forceinline__ uint32_t frag_base(int r) {
  const int h = (threadIdx.x & 63) >> 5;  // second 8-element half of the 16-k step
  if constexpr (SW) {
    const int g = ((r ^ (r >> 3)) & 7) ^ h;
    return (uint32_t)(r * kRowSw + (g << 4));
  } else {
    return (uint32_t)(r * kRowPad + h * 16);
  }
}
template <bool SW>
__device__ __forceinline__ uint32_t frag_at(uint32_t base, int kk) {
  if constexpr (SW)
    return base ^ (uint32_t)(kk << 5);
  else
    return base + (uint32_t)(kk * 32);
}

template <int AL, int BL, int MASK>
__global__ void __launch_bounds__(kThreads, 1) gemm_bf16_kernel(GemmArgs g) {
  using T = uint16_t;
  constexpr int BK = 64;
  constexpr bool DM = MASK == kMaskByte;  // byte mask: K-major tile in LDS, applied to the B fragments
  constexpr bool DB = MASK != kMaskMul;   // B copied by DMA (a multiplicative mask keeps the register path)
  constexpr uint32_t ABUF = 32768u, BBUF = DB ? 32768u : 256u * kRowPad, MBUF = 256u * 64;
  extern __shared__ __align__(16) unsigned char smem[];
  unsigned char* const As = smem;           // [2] A tiles (256 rows x 128 B swizzled, or 64 k x 512 B)
  unsigned char* const Bs = smem + 2 * ABUF;  // [2] B tiles (likewise, or padded for the register path)
  unsigned char* const Ms = Bs + 2 * BBUF;    // [2][256 rows][64 B] byte masks (DM)
  const uint32_t As_l = lds_addr(As), Bs_l = lds_addr(Bs), Ms_l = lds_addr(Ms);

  const int64_t tiles = g.tiles_m * g.tiles_n;
  const int64_t kz = blockIdx.x / tiles;
  int64_t tm, tn;
  tile_coords(blockIdx.x - kz * tiles, g.tiles_m, g.tiles_n, tm, tn);
  const int64_t m0 = tm * kTileM, n0 = tn * kTileN;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  const int64_t nk1_all = ceil_div(g.K1, BK);
  const int64_t s_begin = kz * g.split_stages;
  const int64_t s_end = (s_begin + g.split_stages < nk1_all) ? s_begin + g.split_stages : nk1_all;
  const int64_t nk = s_end > s_begin ? s_end - s_begin : 0;
  const int64_t nk2 = (g.A2 && kz == g.splits - 1) ? ceil_div(g.K2, BK) : 0;
  const int64_t kbase = s_begin * BK;
  const bool has_scale = g.has_scale != 0;
  const float bscale = g.bscale;

  f32x16_t acc[kFragM * kFragN];
#pragma unroll
  for (int i = 0; i < kFragM * kFragN; ++i) acc[i] = f32x16_t{};

  // Fragment offsets: K-contiguous tiles per (k-step, fragment); M/N-contiguous
  // tiles per fragment (k-steps are immediate offsets).
  uint32_t aoff[4][kFragM], boff[4][kFragN], moff[4][kFragN];
#pragma unroll
  for (int i = 0; i < kFragM; ++i) {
    const uint32_t base = AL == 0 ? frag_base<true>(wm * kWaveM + i * 32 + (lane & 31))
                                  : mn_frag_base(wm * kWaveM + i * 32);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) aoff[kk][i] = AL == 0 ? frag_at<true>(base, kk) : base + kk * 8192;
  }
#pragma unroll
  for (int j = 0; j < kFragN; ++j) {
    const int r = wn * kWaveN + j * 32 + (lane & 31);
    uint32_t base;
    if constexpr (!DB)
      base = frag_base<false>(r);
    else if constexpr (BL == 0)
      base = frag_base<true>(r);
    else
      base = mn_frag_base(wn * kWaveN + j * 32);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      if constexpr (!DB)
        boff[kk][j] = frag_at<false>(base, kk);
      else if constexpr (BL == 0)
        boff[kk][j] = frag_at<true>(base, kk);
      else
        boff[kk][j] = base + kk * 8192;
      moff[kk][j] = (uint32_t)(r * 64 + ((kk ^ ((r >> 2) & 3)) << 4) + (lane >> 5) * 8);
    }
  }

  bf16x8_t fa[2][kFragM], fb[2][kFragN];
  uint2 mk[2][kFragN];
  auto read_a = [&](int slot, int buf, int kk, int i) {
    const unsigned char* p = As + buf * ABUF + aoff[kk][i];
    if constexpr (AL == 0)
      fa[slot][i] = *reinterpret_cast<const bf16x8_t*>(p);
    else
      fa[slot][i] = tr_frag(p);
  };
  // MK: the B fragment's mask bytes too (segment 1 of a DM kernel; segment 2 is never masked)
  auto read_b = [&](auto mkc, int slot, int buf, int kk, int j) {
    const unsigned char* p = Bs + buf * BBUF + boff[kk][j];
    if constexpr (DB && BL == 1)
      fb[slot][j] = tr_frag(p);
    else
      fb[slot][j] = *reinterpret_cast<const bf16x8_t*>(p);
    if constexpr (decltype(mkc)::value) mk[slot][j] = *reinterpret_cast<const uint2*>(Ms + buf * MBUF + moff[kk][j]);
  };
  auto read_frags = [&](auto mkc, int slot, int buf, int kk) {
#pragma unroll
    for (int i = 0; i < kFragM; ++i) read_a(slot, buf, kk, i);
#pragma unroll
    for (int j = 0; j < kFragN; ++j) read_b(mkc, slot, buf, kk, j);
  };
  auto mfma1 = [&](int slot, int i, int j) {
    acc[i * kFragN + j] =
        __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[slot][i], fb[slot][j], acc[i * kFragN + j], 0, 0, 0);
  };
  auto apply_masks = [&](int slot) {
#pragma unroll
    for (int j = 0; j < kFragN; ++j) fb[slot][j] = and_bytes(fb[slot][j], mk[slot][j]);
  };
  auto mfmas = [&](int slot) {
#pragma unroll
    for (int j = 0; j < kFragN; ++j)
#pragma unroll
      for (int i = 0; i < kFragM; ++i) mfma1(slot, i, j);
  };
  using Masked = std::integral_constant<bool, DM>;
  using Plain = std::integral_constant<bool, false>;

  // Copy machinery of segment 1.
  DmaLoader dak, dbk;
  DmaLoaderMN dam, dbm;
  DmaMaskLoader dm;
  Loader<T, BL> lb;
  Stage<T, MASK> sb;
  if constexpr (AL == 0)
    dak.init(g.A1, g.lda1, m0, g.M, g.K1);
  else
    dam.init(g.A1, g.lda1, m0, g.M, g.K1, kbase);
  if constexpr (!DB)
    lb.init(g.B1, g.bmask, g.ldb1, n0, g.N, g.K1, false, kbase);
  else if constexpr (BL == 0)
    dbk.init(g.B1, g.ldb1, n0, g.N, g.K1);
  else
    dbm.init(g.B1, g.ldb1, n0, g.N, g.K1, kbase);
  if constexpr (DM) dm.init(g.bmask, g.ldbm, n0, g.N, g.K1);

  // A / B halves of copy piece p (the unmasked all-DMA case spreads them, below)
  auto dma_piece_a = [&](int buf, int64_t k0, int p) {
    if constexpr (AL == 0)
      dak.issue_one(As_l + buf * ABUF, k0, p);
    else
      dam.issue_one(As_l + buf * ABUF, p);
  };
  auto dma_piece_b = [&](int buf, int64_t k0, int p) {
    if constexpr (DB) {
      if constexpr (BL == 0)
        dbk.issue_one(Bs_l + buf * BBUF, k0, p);
      else
        dbm.issue_one(Bs_l + buf * BBUF, p);
    }
  };
  // piece p (0..7) of the DMA copy of the stage at k0 into buffer buf
  auto dma_piece = [&](int buf, int64_t k0, int p) {
    if constexpr (AL == 0)
      dak.issue_one(As_l + buf * ABUF, k0, p);
    else
      dam.issue_one(As_l + buf * ABUF, p);
    if constexpr (DB) {
      if constexpr (BL == 0)
        dbk.issue_one(Bs_l + buf * BBUF, k0, p);
      else
        dbm.issue_one(Bs_l + buf * BBUF, p);
    }
    if constexpr (DM) {
      if (p < 4) dm.issue_one(Ms_l + buf * MBUF, k0, p);
    }
  };
  // the whole copy; TAIL: the stage may end past K (K-contiguous chunks past K read zeros)
  auto dma_issue = [&](auto tail, int buf, int64_t k0) {
    constexpr bool TL = decltype(tail)::value;
    if constexpr (AL == 0)
      dak.template issue<TL>(As_l + buf * ABUF, k0);
    else
      dam.issue(As_l + buf * ABUF);
    if constexpr (DB) {
      if constexpr (BL == 0)
        dbk.template issue<TL>(Bs_l + buf * BBUF, k0);
      else
        dbm.issue(Bs_l + buf * BBUF);
    }
    if constexpr (DM) dm.template issue<TL>(Ms_l + buf * MBUF, k0);
  };
  auto reg_store = [&](int buf) {  // register path (multiplicative mask) into buffer `buf`
    if constexpr (!DB) {
      if constexpr (BL == 0)
        store_kc<T, MASK>(sb, reinterpret_cast<T*>(Bs + buf * BBUF), has_scale, bscale);
      else
        store_rc<T, MASK>(sb, reinterpret_cast<T*>(Bs + buf * BBUF), has_scale, bscale);
    }
  };
  auto reg_load = [&](int64_t k0) {
    if constexpr (!DB) lb.load(sb, k0);
  };
  using Tail = std::integral_constant<bool, true>;

  // Prologue: stages 0 and 1 into buffers 0 and 1, registers hold stage 2.
  if (nk > 0) {
    reg_load(kbase);
    dma_issue(Tail{}, 0, kbase);
    reg_store(0);
  }
  if (nk > 1) {
    reg_load(kbase + BK);
    dma_issue(Tail{}, 1, kbase + BK);
    reg_store(1);
  }
  if (nk > 2) reg_load(kbase + 2 * BK);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (nk > 0) {
    read_frags(Masked{}, 0, 0, 0);
    if constexpr (DM) apply_masks(0);
  }

  // Steady state: stages s (buffer 0) and s + 1 (buffer 1), each copying a
  // full stage s + 2 (and, on the register path, loading s + 3), with
  // compile-time LDS offsets and the instruction order fixed (a scheduling
  // barrier after every MFMA):
  //   k-steps 0..2: the next k-step's fragment reads after MFMAs 0..3
  //   k-step 3: the next stage's first fragment reads after MFMAs 0..3, then
  //   one eighth of the stage's copies after each of MFMAs 4..11
  //   (DM) after MFMAs 12..15 of every k-step the mask of the other slot's B
  //   fragments (read at its start), one fragment per MFMA.
  auto kstep = [&](int slot, auto&& after) {
#pragma unroll
    for (int idx = 0; idx < 16; ++idx) {
      mfma1(slot, idx & 3, idx >> 2);
      after(idx);
      if constexpr (DM) {
        if (idx >= 12) fb[slot ^ 1][idx - 12] = and_bytes(fb[slot ^ 1][idx - 12], mk[slot ^ 1][idx - 12]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  auto read_pair = [&](int slot, int buf, int kk, int idx) {  // fragments 2 idx, 2 idx + 1 (A 0..3, B 4..7)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int f = 2 * idx + h;
      if (f < kFragM)
        read_a(slot, buf, kk, f);
      else
        read_b(Masked{}, slot, buf, kk, f - kFragM);
    }
  };
  // SPREAD (A and B both copied by DMA, no byte mask): the 16 copy instructions of
  // a stage go one per MFMA slot, half in k-step 3 of stage s (pieces 0..3 of
  // stage s + 2) and half in k-step 0 of stage s + 1 (pieces 4..7), so the
  // buffer unit is never handed a whole stage's copies in one k-step.  They still
  // land before the barrier of stage s + 1 that publishes them.
  constexpr bool SPREAD = DB && !DM;
  auto spread_piece = [&](int buf, int64_t k0, int slot) {  // slot 0..7: A / B of pieces base + slot / 2
    if (slot & 1)
      dma_piece_b(buf, k0, slot >> 1);
    else
      dma_piece_a(buf, k0, slot >> 1);
  };
  auto steady = [&](auto bc, int64_t s) {
    constexpr int B = decltype(bc)::value;
    const bool pend = SPREAD && s > 0;  // pieces 4..7 of stage s + 1 (into B ^ 1) are still to be issued
    const int64_t k1 = kbase + (s + 1) * BK;
    kstep(0, [&](int idx) {
      if (idx < 4) read_pair(1, B, 1, idx);
      if constexpr (SPREAD) {
        if (pend && idx >= 4 && idx < 12) spread_piece(B ^ 1, k1, 8 + (idx - 4));
      }
    });
    kstep(1, [&](int idx) {
      if (idx < 4) read_pair(0, B, 2, idx);
    });
    kstep(0, [&](int idx) {
      if (idx < 4) read_pair(1, B, 3, idx);
    });
    // this wave's copies into B ^ 1 landed and its k-step 3 fragments are in registers
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    const int64_t k2 = kbase + (s + 2) * BK, k3 = kbase + (s + 3) * BK;
    kstep(1, [&](int idx) {
      if (idx < 4) read_pair(0, B ^ 1, 0, idx);  // the next stage's first fragments
      if constexpr (SPREAD) {
        if (idx >= 4 && idx < 12) spread_piece(B, k2, idx - 4);
      } else if (idx >= 4 && idx < 12) {
        const int p = idx - 4;
        if constexpr (!DB) {  // register path: one vector written, then its register reloaded
          if constexpr (BL == 0) {
            store_kc_one<T, MASK>(sb, reinterpret_cast<T*>(Bs + B * BBUF), p, has_scale, bscale);
            lb.load_one(sb, k3, p);
          }
        }
        dma_piece(B, k2, p);
      }
    });
    if constexpr (!DB && BL == 1) {  // N-contiguous multiplicative mask: block transpose, then reload
      store_rc<T, MASK>(sb, reinterpret_cast<T*>(Bs + B * BBUF), has_scale, bscale);
      lb.load(sb, k3);
    }
  };
  int64_t s = 0;
  for (; s + 5 <= nk; s += 2) {
    steady(std::integral_constant<int, 0>{}, s);
    steady(std::integral_constant<int, 1>{}, s + 1);
  }
  bool pend = SPREAD && s > 0;  // the last steady stage left pieces 4..7 of stage s + 1
  // The last (up to four) stages, with run-time buffer offsets.
  for (; s < nk; ++s) {
    const int b = static_cast<int>(s & 1);
    if constexpr (SPREAD) {
      if (pend) {
        for (int sl = 8; sl < 16; ++sl) spread_piece(b ^ 1, kbase + (s + 1) * BK, sl);
        pend = false;
      }
    }
    read_frags(Masked{}, 1, b, 1);
    mfmas(0);
    if constexpr (DM) apply_masks(1);
    read_frags(Masked{}, 0, b, 2);
    mfmas(1);
    if constexpr (DM) apply_masks(0);
    read_frags(Masked{}, 1, b, 3);
    mfmas(0);
    if constexpr (DM) apply_masks(1);
    if (s + 1 < nk) {
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      if (s + 2 < nk) {
        reg_store(b);
        if (s + 3 < nk) reg_load(kbase + (s + 3) * BK);
        dma_issue(Tail{}, b, kbase + (s + 2) * BK);
      }
      read_frags(Masked{}, 0, b ^ 1, 0);
    }
    mfmas(1);
    if constexpr (DM) apply_masks(0);
  }

  // Segment 2 (the SLoRB term A2 . B2^T, a few stages, never masked) through buffer 0.
  if (nk2 > 0) {
    DmaLoader da2k, db2k;
    DmaLoaderMN da2m, db2m;
    Loader<T, BL> lb2;
    if constexpr (AL == 0)
      da2k.init(g.A2, g.lda2, m0, g.M, g.K2);
    else
      da2m.init(g.A2, g.lda2, m0, g.M, g.K2, 0);
    if constexpr (!DB)
      lb2.init(g.B2, nullptr, g.ldb2, n0, g.N, g.K2);
    else if constexpr (BL == 0)
      db2k.init(g.B2, g.ldb2, n0, g.N, g.K2);
    else
      db2m.init(g.B2, g.ldb2, n0, g.N, g.K2, 0);
    for (int64_t s2 = 0; s2 < nk2; ++s2) {
      __syncthreads();  // every wave is done with buffer 0
      if constexpr (AL == 0)
        da2k.issue<true>(As_l, s2 * BK);
      else
        da2m.issue(As_l);
      if constexpr (!DB) {
        Stage<T, kMaskNone> tb;
        lb2.load(tb, s2 * BK);
        if constexpr (BL == 0)
          store_kc<T, kMaskNone>(tb, reinterpret_cast<T*>(Bs), false, 1.0f);
        else
          store_rc<T, kMaskNone>(tb, reinterpret_cast<T*>(Bs), false, 1.0f);
      } else if constexpr (BL == 0) {
        db2k.issue<true>(Bs_l, s2 * BK);
      } else {
        db2m.issue(Bs_l);
      }
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      read_frags(Plain{}, 0, 0, 0);
      read_frags(Plain{}, 1, 0, 1);
      mfmas(0);
      read_frags(Plain{}, 0, 0, 2);
      mfmas(1);
      read_frags(Plain{}, 1, 0, 3);
      mfmas(0);
      mfmas(1);
    }
  }

  gemm_epilogue<T>(g, acc, smem, m0, n0, kz);
}

// Split-K reduction: C = epilogue(sum over splits of the f32 partials), the
// splits summed in index order (deterministic), then the same output
// rounding, bias, mask product / decay term and accumulation as the GEMM
// epilogue.
__global__ void __launch_bounds__(256) splitk_reduce_kernel(GemmArgs g, int elem_dtype) {
  const int64_t total = g.M * g.N;
  const bool cbf = g.c_dtype == SF_DTYPE_BF16;
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = idx / g.N, col = idx - row * g.N;
    float x = 0.0f;
    for (int z = 0; z < g.splits; ++z) x += g.partial[z * total + idx];
    const int64_t o = row * g.ldc + col;
    if (cbf) x = hround(x);
    if (g.bias) {
      const float b = load_elem(g.bias, col, g.bias_dtype);
      x = cbf ? hround(x + b) : x + b;
    }
    if (g.emask) {
      const float em = load_elem(g.emask, o, elem_dtype);
      if (g.dw) {
        if (em < 0.5f) {
          float d = g.decay * load_elem(g.dw, o, elem_dtype);
          if (cbf) d = hround(d);
          x = cbf ? hround(x + d) : x + d;
        }
      } else {
        x = cbf ? hround(x * em) : x * em;
      }
    }
    if (g.accumulate) x = load_elem(g.C, o, g.c_dtype) + x;
    if (cbf)
      static_cast<uint16_t*>(g.C)[o] = hbits(x);
    else
      static_cast<float*>(g.C)[o] = x;
  }
}

// ---------------------------------------------------------------------------
// Block-sparse-16 products on bf16 operands (the BSR layout of
// convert_to_block_sparse plus its block map), DMA-staged like gemm_bf16_kernel.
//
// bsr_mm_kernel<DX>: C[T, n_out] = A[T, n_red] . B^T with B block-sparse.
//   forward (DX = 0):    A = x [T, in],  C = y [T, out];   B = W: block (o, r) of
//                        the tile is W block (row o, col r), read as stored.
//   input grad (DX = 1): A = dy [T, out], C = dx [T, in]; B = W^T: block (o, r)
//                        is W block (row r, col o), read transposed with
//                        ds_read_b64_tr_b16.
// A 256 x 256 tile (16 output blocks) over stages of 64 reduction values (4
// reduction blocks).  A is staged whole (the K-contiguous swizzled DMA tile of
// the dense kernel); of B only the present blocks are copied (an absent
// block's lanes read past the resource: zeros, no memory traffic) into 64
// slots of 512 B, slot o * 4 + r.  MFMAs are v_mfma_f32_32x32x16_bf16 with one
// reduction block per MFMA: the 32 output columns of a wave fragment are two
// adjacent output blocks, and the fragment's MFMAs run only when one of the two
// is present (a wave-uniform branch on a ballot of the block map); the other
// half then reads zeros.
// ---------------------------------------------------------------------------
template <int DX>
__global__ void __launch_bounds__(kThreads, 1) bsr_mm_kernel(GemmArgs g) {
  constexpr uint32_t ABUF = 32768u, BBUF = 32768u;
  extern __shared__ __align__(16) unsigned char smem[];
  unsigned char* const As = smem;
  unsigned char* const Bs = smem + 2 * ABUF;
  const uint32_t As_l = lds_addr(As), Bs_l = lds_addr(Bs);
  int64_t tm, tn;
  tile_coords(blockIdx.x, g.tiles_m, g.tiles_n, tm, tn);
  const int64_t m0 = tm * kTileM, n0 = tn * kTileN;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t ob0 = n0 / 16;                 // first output block of the tile
  const int64_t nk = ceil_div(g.K1, 64);       // reduction stages
  const int64_t out_blocks = DX ? g.b_map_cols : g.b_map_rows;
  const int64_t red_blocks = DX ? g.b_map_rows : g.b_map_cols;
  const int64_t nblocks = g.b_map_rows * g.b_map_cols;  // upper bound of block indices (extent of the blocks array)

  f32x16_t acc[kFragM * kFragN];
#pragma unroll
  for (int i = 0; i < kFragM * kFragN; ++i) acc[i] = f32x16_t{};

  // block index of tile slot (o, r) at stage s, or -1
  auto block_at = [&](int o, int r, int64_t s) -> int {
    const int64_t ob = ob0 + o, rb = s * 4 + r;
    if (ob >= out_blocks || rb >= red_blocks) return -1;
    return DX ? g.b_map[rb * g.b_map_cols + ob] : g.b_map[ob * g.b_map_cols + rb];
  };
  // DMA of B: wave w copies slots [16 w, 16 w + 16), two per instruction (lanes 0-31, 32-63).
  // The forward's blocks land with the 16-byte halves of rows 8..15 swapped, so that the
  // 16-byte fragment reads of rows 0..15 at one half fall in distinct banks.
  const int half = lane >> 5, part = lane & 31;
  const uint32_t chunk_off = DX ? (uint32_t)part * 16
                                : (uint32_t)((part >> 1) * 32 + (((part & 1) ^ ((part >> 4) & 1)) << 4));
  const Rsrc rsb = make_rsrc(g.B1, nblocks * 512);
  int nidx[8];
  auto load_idx = [&](int64_t s) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int slot = 16 * wave + 2 * i + half;
      nidx[i] = s < nk ? block_at(slot >> 2, slot & 3, s) : -1;
    }
  };
  auto issue_b = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t voff = nidx[i] >= 0 ? (uint32_t)nidx[i] * 512u + chunk_off : kOob;
      dma16(rsb, Bs_l + buf * BBUF + (uint32_t)(16 * wave + 2 * i) * 512u, voff, 0);
    }
  };
  // presence of this wave's output blocks 8 wn .. 8 wn + 7 at the 4 reduction blocks of a stage:
  // bit (o - 8 wn) * 4 + r of the ballot
  int pidx;
  auto load_pres = [&](int64_t s) { pidx = (s < nk && lane < 32) ? block_at(8 * wn + (lane >> 2), lane & 3, s) : -1; };

  DmaLoader dak;
  dak.init(g.A1, g.lda1, m0, g.M, g.K1);

  // fragment offsets: A as the dense kernel's K-contiguous tile; B per wave fragment j (output
  // blocks 8 wn + 2 j, + 1) at reduction block 0 (block r adds r * 512)
  uint32_t aoff[4][kFragM], boff[kFragN];
#pragma unroll
  for (int i = 0; i < kFragM; ++i) {
    const uint32_t base = frag_base<true>(wm * kWaveM + i * 32 + (lane & 31));
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) aoff[kk][i] = frag_at<true>(base, kk);
  }
#pragma unroll
  for (int j = 0; j < kFragN; ++j) {
    if constexpr (!DX) {
      const int o = 8 * wn + 2 * j + ((lane & 31) >> 4), row = lane & 15;
      boff[j] = (uint32_t)(o * 4 * 512 + row * 32 + ((half ^ (row >> 3)) << 4));
    } else {
      // ds_read_b64_tr_b16: lane 4q + c of a 16-lane group gets the c-th value of the 4-element rows
      // addressed by lanes q, q + 4, q + 8, q + 12.  Group G covers output columns 16 (G & 1) .. + 16
      // (block 8 wn + 2 j + (G & 1)) and reduction rows 8 (G >> 1) .. + 4 (the second read: + 4)
      const int G = lane >> 4, L = lane & 15;
      const int o = 8 * wn + 2 * j + (G & 1);
      boff[j] = (uint32_t)(o * 4 * 512 + (8 * (G >> 1) + (L >> 2)) * 32 + (L & 3) * 8);
    }
  }
  auto read_b = [&](int buf, int r, int j) -> bf16x8_t {
    const unsigned char* p = Bs + buf * BBUF + boff[j] + r * 512;
    if constexpr (!DX) {
      return *reinterpret_cast<const bf16x8_t*>(p);
    } else {
      typedef __attribute__((address_space(3))) v4i16_t lds_v4;
      const v4i16_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4*)(p));
      const v4i16_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4*)(p + 128));
      return __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    }
  };

  // Fragments are double-buffered over the 4 reduction blocks of a stage: the reads of block
  // r + 1 are issued before the MFMAs of block r, and the reads of the next stage's block 0 right
  // after the barrier that publishes it, before the MFMAs of block 3.  B fragments are read
  // whether or not their blocks are present (an absent block reads zeros); only the MFMAs branch.
  bf16x8_t fa[2][kFragM], fb[2][kFragN];
  auto load_frags = [&](int slot, int buf, int r) {
#pragma unroll
    for (int i = 0; i < kFragM; ++i) fa[slot][i] = *reinterpret_cast<const bf16x8_t*>(As + buf * ABUF + aoff[r][i]);
#pragma unroll
    for (int j = 0; j < kFragN; ++j) fb[slot][j] = read_b(buf, r, j);
  };
  auto mfmas = [&](int slot, int r, uint32_t pm) {
#pragma unroll
    for (int j = 0; j < kFragN; ++j) {
      if ((pm >> (8 * j + r)) & 0x11u) {
#pragma unroll
        for (int i = 0; i < kFragM; ++i)
          acc[i * kFragN + j] =
              __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[slot][i], fb[slot][j], acc[i * kFragN + j], 0, 0, 0);
      }
    }
  };

  // prologue: stage 0 into buffer 0; block indices of stage 1
  load_idx(0);
  load_pres(0);
  if (nk > 0) {
    dak.issue<true>(As_l, 0);
    issue_b(0);
  }
  int pres_cur = pidx;
  load_idx(1);
  load_pres(1);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (nk > 0) load_frags(0, 0, 0);
  for (int64_t s = 0; s < nk; ++s) {
    const int cur = static_cast<int>(s & 1);
    const uint32_t pmask = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)__ballot(pres_cur >= 0));
    const int pres_next = pidx;
    if (s + 1 < nk) {
      dak.issue<true>(As_l + (cur ^ 1) * ABUF, (s + 1) * 64);
      issue_b(cur ^ 1);
      load_idx(s + 2);
      load_pres(s + 2);
    }
    load_frags(1, cur, 1);
    mfmas(0, 0, pmask);
    load_frags(0, cur, 2);
    mfmas(1, 1, pmask);
    load_frags(1, cur, 3);
    mfmas(0, 2, pmask);
    // the next stage's copies (and index loads) landed; every wave's reads of this stage are in registers
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (s + 1 < nk) load_frags(0, cur ^ 1, 0);
    mfmas(1, 3, pmask);
    pres_cur = pres_next;
  }
  gemm_epilogue<uint16_t>(g, acc, smem, m0, n0, 0);
}

template <typename T>
constexpr size_t smem_bytes() {
  return sizeof(T) * 2ull * (kTileM + kTileN) * Tr<T>::PITCH + 2 * 16 * (Tr<T>::BK / 16);
}

// bf16 dense B: the direct-to-LDS kernel; its LDS also hosts the epilogue staging.
template <int AL, int BL, int MASK>
constexpr size_t smem_bytes_bf16() {
  constexpr size_t ops = 2ull * 32768 + 2ull * (MASK != kMaskMul ? 32768 : 256 * kRowPad) +
                         (MASK == kMaskByte ? 2ull * 256 * 64 : 0);
  constexpr size_t epi = 4ull * 64 * kEpiPitch * sizeof(float);
  return ops > epi ? ops : epi;
}

template <typename K>
int set_smem(K kern, size_t smem, bool& done) {
  if (!done) {
    SF_CHECK_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                     static_cast<int>(smem)));
    done = true;
  }
  return SF_OK;
}

template <typename T, int AL, int BL, int MASK>
int launch_gemm(const GemmArgs& g, hipStream_t st) {
  // bf16 dense B runs the direct-to-LDS kernel unless its byte mask cannot be copied as K-major rows
  constexpr bool kDirectT = sizeof(T) == 2 && BL < 2;
  const bool direct = kDirectT && (MASK != kMaskByte || g.dma_mask_ok);
  static bool attr_direct = false, attr_reg = false;  // per instantiation; host code sets the attribute once
  void (*kern)(GemmArgs);
  size_t smem;
  if constexpr (kDirectT) {
    if (direct) {
      kern = gemm_bf16_kernel<AL, (BL < 2 ? BL : 0), MASK>;
      smem = smem_bytes_bf16<AL, (BL < 2 ? BL : 0), MASK>();
      if (int rc = set_smem(kern, smem, attr_direct)) return rc;
    }
  }
  if (!direct) {
    kern = gemm_kernel<T, AL, BL, MASK>;
    smem = smem_bytes<T>();
    if (int rc = set_smem(kern, smem, attr_reg)) return rc;
  }
  const int64_t tiles = g.tiles_m * g.tiles_n;
  if (tiles == 0) return SF_OK;
  SF_CHECK_ARG(tiles * g.splits < (1ll << 31), "GEMM grid too large");
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(tiles * g.splits)), dim3(kThreads), smem, st, g);
  if (int rc = launch_status("sf_gemm")) return rc;
  if (g.splits > 1) {
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3(static_cast<unsigned>(elementwise_grid(g.M * g.N, 256))),
                       dim3(256), 0, st, g, Tr<T>::DT);
    return launch_status("sf_gemm (split-K reduce)");
  }
  return SF_OK;
}

// The bf16 block-sparse kernels (one 256 x 256 tile per workgroup, no split K).
constexpr size_t smem_bytes_bsr() {
  constexpr size_t ops = 4ull * 32768;
  constexpr size_t epi = 4ull * 64 * kEpiPitch * sizeof(float);
  return ops > epi ? ops : epi;
}
template <typename K>
int launch_bsr_kernel(K kern, bool& attr, const GemmArgs& g, hipStream_t st, const char* what) {
  const size_t smem = smem_bytes_bsr();
  if (int rc = set_smem(kern, smem, attr)) return rc;
  const int64_t tiles = g.tiles_m * g.tiles_n;
  if (tiles == 0) return SF_OK;
  SF_CHECK_ARG(tiles < (1ll << 31), "GEMM grid too large");
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(tiles)), dim3(kThreads), smem, st, g);
  return launch_status(what);
}

// ---------------------------------------------------------------------------
// Block-sparse-16 product with exact block skipping (bf16 operands and output):
//   C[T, R] = X[T, K] . S^T,   S [R, K] held as 16 x 16 blocks
// S's blocks come from `blocks` ([n][16][16], row-major) through `map`
// ([R / 16][K / 16]: block index, negative for an absent block).  The forward
// passes W (R = out, K = in) with the index convert_to_block_sparse builds;
// the input gradient passes the transposed matrix (sf_bsr_transpose: every
// block transposed, the map transposed), so one kernel serves both.
//
// v_mfma_f32_16x16x32_bf16 multiplies one block row (16 rows of S) by 16
// tokens over 32 k, i.e. two adjacent k-blocks; it is skipped when both are
// absent (a pair with one absent block multiplies zeros for that half).  Its
// S operand (lane l: row l % 16, k 8 (l / 16) .. + 8, so lanes 0-31 read the
// pair's first block and lanes 32-63 its second) is 16 contiguous bytes of a
// stored block row, loaded straight from the blocks array into registers:
// one instruction reads two whole 512-byte blocks, an absent block reads
// zeros through an out-of-range offset.  Only X goes through LDS: stages of
// 128 tokens x 64 k (4 k-blocks), double buffered, staged through registers
// (every load is a compiler-tracked one, so its waits are exact), shared by
// the 4 waves of the workgroup.  Wave w owns rows [128 w, 128 w + 128) of
// the workgroup's 512 (8 block rows) and all 128 tokens: 8 x 8 accumulator
// blocks of 16 x 16 (256 AGPRs).  The block map is read with scalar loads,
// one 16-byte row segment per block row and stage; the stage's S fragments
// are loaded one stage ahead.
// ---------------------------------------------------------------------------
constexpr int kBsWaveRows = 128;                   // rows of S per wave (8 block rows)
constexpr int kBsRows = 4 * kBsWaveRows;           // rows of S per workgroup
constexpr int kBsTok = 128;                        // tokens per workgroup (8 column blocks of 16)
constexpr int kBsStageK = 64;                      // k per stage: 4 k-blocks, 2 MFMA k-steps
constexpr uint32_t kBsXBuf = kBsTok * 128u;        // one X stage: 128 token rows x 128 B, chunk-swizzled
constexpr int kBsEpiPitch = kBsWaveRows * 2 + 16;  // bytes per token row of a wave's bf16 output staging

struct Bs16Args {
  const uint16_t* X;
  int64_t ldx, T, K;
  const uint16_t* blocks;
  const int32_t* map;
  int64_t nrb, nkb;
  uint16_t* C;
  int64_t ldc, R;
  int64_t tiles_t, tiles_r;
};

typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int bs_swz(int r) { return (r ^ (r >> 3)) & 7; }

__global__ void __launch_bounds__(kThreads, 1) bsr16_kernel(Bs16Args g) {
  extern __shared__ __align__(16) unsigned char smem[];
  int64_t tt, tr;
  tile_coords(blockIdx.x, g.tiles_t, g.tiles_r, tt, tr);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t t0 = tt * kBsTok;
  const int64_t rb0 = (tr * kBsRows + wave * kBsWaveRows) / 16;  // the wave's first block row
  const int64_t nk = g.K / kBsStageK;
  const Rsrc rx = make_rsrc(g.X, g.T * g.ldx * 2);
  const Rsrc rbk = make_rsrc(g.blocks, g.nrb * g.nkb * 512);

  // X copy: thread t moves 16-byte chunk t % 8 of token rows 32 i + t / 8, i = 0..3
  const int crow = threadIdx.x >> 3, cch = threadIdx.x & 7;
  uint32_t xoff[4], xlds[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 32 * i + crow;
    xoff[i] = t0 + row < g.T ? (uint32_t)(((t0 + row) * g.ldx + cch * 8) * 2) : kOob;
    xlds[i] = (uint32_t)(row * 128 + ((cch ^ bs_swz(row)) << 4));
  }
  // X fragment of k-step p, column block t: token row 16 t + lane % 16, chunk 4 p + lane / 16
  uint32_t boff[2][8];
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int row = 16 * t + (lane & 15);
      boff[p][t] = (uint32_t)(row * 128 + (((4 * p + (lane >> 4)) ^ bs_swz(row)) << 4));
    }
  // S fragment: row lane % 16 of the block, 16-byte half (lane / 16) % 2; lanes >= 32 take the second block
  const uint32_t aoff = (uint32_t)((lane & 15) * 32 + ((lane >> 4) & 1) * 16);
  const bool second = lane >= 32;

  f32x4_t acc[8][8];
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[j][t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  // Pipeline (every load compiler-tracked): at the start of stage s the X rows of stage s + 2, the
  // S fragments of stage s + 1 (from the block indices read a stage earlier) and the block indices
  // of stage s + 2 are loaded; the stage's MFMAs follow; at its end the X rows of stage s + 1
  // (loaded two stages earlier) are written to the other LDS buffer, and one barrier publishes them.
  // Lane l reads, per block row j and k-step p, the index of the block its half of the fragment
  // covers (block 2 p + (l >= 32) of the stage), so the skip test is a ballot.
  V4 xr[2][4];           // X rows of stage k in xr[k % 2]
  int32_t mv[2];         // block indices of stage k in mv[k % 2]: lane 4 j + kb holds block row j's
                         // entry kb of the stage (lanes 32-63 unused)
  bf16x8_t af[2][8][2];  // S fragments of stage k in af[k % 2]
  uint32_t live[2][8];   // per stage set and block row: bit p set when k-step p has a block
  const int mj = (lane >> 2) & 7, mk = lane & 3;
  auto load_map = [&](auto set_c, int64_t s) {
    constexpr int set = decltype(set_c)::value;
    const int64_t r = rb0 + mj;
    mv[set] = (lane < 32 && r < g.nrb) ? g.map[r * g.nkb + s * 4 + mk] : -1;
  };
  auto load_a = [&](auto set_c) {  // the fragments of the stage whose indices mv[set] holds
    constexpr int set = decltype(set_c)::value;
    const int32_t m = mv[set];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int e0 = __builtin_amdgcn_readlane(m, 4 * j), e1 = __builtin_amdgcn_readlane(m, 4 * j + 1);
      const int e2 = __builtin_amdgcn_readlane(m, 4 * j + 2), e3 = __builtin_amdgcn_readlane(m, 4 * j + 3);
      live[set][j] = ((e0 >= 0 || e1 >= 0) ? 1u : 0u) | ((e2 >= 0 || e3 >= 0) ? 2u : 0u);
      const int b0 = second ? e1 : e0, b1 = second ? e3 : e2;
      af[set][j][0] = __builtin_bit_cast(bf16x8_t, bload(rbk, b0 >= 0 ? (uint32_t)b0 * 512u + aoff : kOob, 0));
      af[set][j][1] = __builtin_bit_cast(bf16x8_t, bload(rbk, b1 >= 0 ? (uint32_t)b1 * 512u + aoff : kOob, 0));
    }
  };
  auto load_x = [&](auto set_c, int64_t s) {
    constexpr int set = decltype(set_c)::value;
#pragma unroll
    for (int i = 0; i < 4; ++i) xr[set][i] = bload(rx, xoff[i], (uint32_t)(s * kBsStageK * 2));
  };
  auto store_x = [&](auto set_c, int buf) {
    constexpr int set = decltype(set_c)::value;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint4 v;
      v.x = xr[set][i].w[0];
      v.y = xr[set][i].w[1];
      v.z = xr[set][i].w[2];
      v.w = xr[set][i].w[3];
      *reinterpret_cast<uint4*>(smem + buf * kBsXBuf + xlds[i]) = v;
    }
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  // stage s with set = s % 2 (compile time)
  auto stage = [&](auto set_c, int64_t s) {
    constexpr int set = decltype(set_c)::value;
    using Other = std::integral_constant<int, set ^ 1>;
    // Unconditional (past the last stage they re-read it): the compiler's wait counts then stay exact.
    // The fragments of stage s + 1 first (their indices, mv[(s + 1) % 2], were read two stages ago),
    // then X of stage s + 2, then the indices of stage s + 3 into the slot just consumed.
    const int64_t s2 = s + 2 < nk ? s + 2 : nk - 1, s3 = s + 3 < nk ? s + 3 : nk - 1;
    load_a(Other{});
    load_x(set_c, s2);
    load_map(Other{}, s3);
    const unsigned char* xb = smem + set * kBsXBuf;
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      bf16x8_t bf[8];
#pragma unroll
      for (int t = 0; t < 8; ++t) bf[t] = *reinterpret_cast<const bf16x8_t*>(xb + boff[p][t]);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (live[set][j] & (1u << p)) {
#pragma unroll
          for (int t = 0; t < 8; ++t)
            acc[j][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[set][j][p], bf[t], acc[j][t], 0, 0, 0);
        }
      }
    }
    store_x(Other{}, set ^ 1);  // X rows of stage s + 1, loaded at the start of stage s - 1 (past the end: unread)
    __syncthreads();
  };
  // prologue: stage 0's rows in LDS and fragments in registers, stage 1's rows and indices loading
  load_map(S0{}, 0);
  load_x(S0{}, 0);
  load_a(S0{});
  store_x(S0{}, 0);
  load_map(S1{}, nk > 1 ? 1 : 0);
  load_x(S1{}, nk > 1 ? 1 : 0);
  load_map(S0{}, nk > 2 ? 2 : nk - 1);
  __syncthreads();
  int64_t s = 0;
  for (; s + 1 < nk; s += 2) {
    stage(S0{}, s);
    stage(S1{}, s + 1);
  }
  if (s < nk) stage(S0{}, s);

  // Epilogue: lane l holds rows 16 j + 4 (l / 16) + e of token 16 t + l % 16.  Each wave stages its
  // 128 x 128 bf16 result token-major in LDS (the X buffers are free: the last stage ended in a
  // barrier), then writes 16 bytes (8 rows of one token) per lane.
  unsigned char* ep = smem + wave * (kBsTok * kBsEpiPitch);
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int tok = 16 * t + (lane & 15), row = 16 * j + 4 * (lane >> 4);
      uint2 v;
      v.x = pack2(acc[j][t][0], acc[j][t][1]);
      v.y = pack2(acc[j][t][2], acc[j][t][3]);
      *reinterpret_cast<uint2*>(ep + tok * kBsEpiPitch + row * 2) = v;
    }
  __syncthreads();
  const int64_t r0 = tr * kBsRows + wave * kBsWaveRows;
#pragma unroll 4
  for (int it = 0; it < kBsTok * 16 / 64; ++it) {
    const int id = it * 64 + lane, tok = id >> 4, cc = id & 15;
    const int64_t trow = t0 + tok, col = r0 + cc * 8;
    if (trow < g.T && col < g.R)
      *reinterpret_cast<uint4*>(g.C + trow * g.ldc + col) =
          *reinterpret_cast<const uint4*>(ep + tok * kBsEpiPitch + cc * 16);
  }
}

constexpr size_t smem_bytes_bs16() {
  constexpr size_t ops = 2ull * kBsXBuf, epi = 4ull * kBsTok * kBsEpiPitch;
  return ops > epi ? ops : epi;
}

// The block-sparse products bsr16_kernel takes: bf16 in and out, K a multiple of 64 (whole stages, the
// map's row segments 16-byte aligned), C 16-byte aligned rows, no epilogue operand.
bool bs16_ok(const GemmArgs& g) {
  return g.K1 % kBsStageK == 0 && g.c_dtype == SF_DTYPE_BF16 && !g.bias && !g.emask && !g.dw && !g.accumulate &&
         !g.c_blocks && g.c_aligned && g.ldc % 8 == 0 && g.N % 16 == 0 && g.b_map_rows * 16 == g.N &&
         g.b_map_cols * 16 == g.K1 && (reinterpret_cast<uintptr_t>(g.b_map) & 15u) == 0 && g.A2 == nullptr;
}

int launch_bs16(const GemmArgs& g, hipStream_t st) {
  static bool attr = false;
  const size_t smem = smem_bytes_bs16();
  if (int rc = set_smem(bsr16_kernel, smem, attr)) return rc;
  Bs16Args a;
  a.X = static_cast<const uint16_t*>(g.A1);
  a.ldx = g.lda1;
  a.T = g.M;
  a.K = g.K1;
  a.blocks = static_cast<const uint16_t*>(g.B1);
  a.map = g.b_map;
  a.nrb = g.b_map_rows;
  a.nkb = g.b_map_cols;
  a.C = static_cast<uint16_t*>(g.C);
  a.ldc = g.ldc;
  a.R = g.N;
  a.tiles_t = ceil_div(g.M, kBsTok);
  a.tiles_r = ceil_div(g.N, kBsRows);
  const int64_t tiles = a.tiles_t * a.tiles_r;
  if (tiles == 0) return SF_OK;
  SF_CHECK_ARG(tiles < (1ll << 31), "GEMM grid too large");
  hipLaunchKernelGGL(bsr16_kernel, dim3(static_cast<unsigned>(tiles)), dim3(kThreads), smem, st, a);
  return launch_status("sf_gemm (block-sparse, exact skip)");
}

// ---------------------------------------------------------------------------
// Skinny products: one side of C at most 64 wide (the SLoRB terms z = x P^T,
// dz = dy S, dP = dz^T x, dS = dy^T z at rank 64).  On the 256 x 256 tile
// three quarters of every MFMA would multiply padding, so these run on a
// 128 x 64 tile: C' [M', N' <= 64] = A' B'^T, 4 waves of 32 long-side rows by
// the 64 short-side columns (2 v_mfma_f32_32x32x16_bf16 per 16-k step), 64-k
// stages double-buffered in LDS through registers (the M/N-contiguous layouts
// are transposed while they are written to LDS), split-K over enough
// workgroups to fill the GPU, f32 partials reduced by splitk_reduce_kernel
// (which applies the output epilogue).  When C's short side is its rows
// (M <= 64) the roles swap (A' = B, B' = A) and so do the MFMA operands, so
// the accumulators come out in C's orientation and the partial stores stay
// coalesced.
// ---------------------------------------------------------------------------
constexpr int kSkM = 128, kSkN = 64, kSkK = 64, kSkPitch = kSkK + 8;  // LDS row: 64 bf16 + 16 B of padding

struct SkinnyArgs {
  const uint16_t* A;  // A' (long side M'): layout AL
  const uint16_t* B;  // B' (short side N' <= 64): layout BL
  int64_t lda, ldb;
  int64_t M, N, K;    // M' (long), N' (short), K
  int64_t split_stages;
  float* partial;     // [splits][C rows][C cols]
};

template <int AL, int BL, bool TOUT>
__global__ void __launch_bounds__(256) skinny_kernel(SkinnyArgs g) {
  __shared__ __align__(16) uint16_t As[2][kSkM][kSkPitch];  // [m][k]
  __shared__ __align__(16) uint16_t Bs[2][kSkN][kSkPitch];  // [n][k]
  const int64_t tiles = ceil_div(g.M, kSkM);
  const int64_t kz = blockIdx.x / tiles;
  const int64_t m0 = (blockIdx.x - kz * tiles) * kSkM;
  const int64_t nk = ceil_div(g.K, kSkK);
  const int64_t s0 = kz * g.split_stages;
  const int64_t s1 = s0 + g.split_stages < nk ? s0 + g.split_stages : nk;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  // Register stage of one K step.  K layout: 16-byte chunks of rows, stored as they are.
  // MN layout: A' as a 4 (k) x 8 (m) block per thread (k fastest over the threads), B' as
  // a 2 (k) x 8 (n) block; both are transposed in registers, so every LDS write is one
  // 8- or 4-byte word and both the writes and the MFMA operand reads are free of bank
  // conflicts at the 144-byte row pitch.
  struct Stage {
    uint4 a[4], b[2];
  };
  // Loads are unconditional, so the compiler's wait counts stay exact and two steps stay in
  // flight: a lane outside the split's K range or outside M' / N' reads the operand's first
  // chunk, and the store to LDS (where the data is first needed) replaces it with zeros.
  const int64_t kend = s1 * kSkK < g.K ? s1 * kSkK : g.K;
  auto a_ok = [&](int64_t k0, int i) {
    if constexpr (AL == 0) {
      const int c = t + 256 * i;
      return m0 + (c >> 3) < g.M && k0 + (c & 7) * 8 < kend;
    } else {
      return k0 + (t & 15) * 4 + i < kend && m0 + (t >> 4) * 8 < g.M;
    }
  };
  auto b_ok = [&](int64_t k0, int i) {
    if constexpr (BL == 0) {
      const int c = t + 256 * i;
      return (c >> 3) < g.N && k0 + (c & 7) * 8 < kend;
    } else {
      return k0 + (t & 31) * 2 + i < kend && (t >> 5) * 8 < g.N;
    }
  };
  auto gload = [&](Stage& r, int64_t k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {  // A' tile: 128 rows x 64 k
      int64_t off;
      if constexpr (AL == 0) {
        const int c = t + 256 * i;
        off = (m0 + (c >> 3)) * g.lda + k0 + (c & 7) * 8;
      } else {
        off = (k0 + (t & 15) * 4 + i) * g.lda + m0 + (t >> 4) * 8;
      }
      r.a[i] = *reinterpret_cast<const uint4*>(g.A + (a_ok(k0, i) ? off : 0));
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {  // B' tile: 64 rows x 64 k
      int64_t off;
      if constexpr (BL == 0) {
        const int c = t + 256 * i;
        off = (c >> 3) * g.ldb + k0 + (c & 7) * 8;
      } else {
        off = (k0 + (t & 31) * 2 + i) * g.ldb + (t >> 5) * 8;
      }
      r.b[i] = *reinterpret_cast<const uint4*>(g.B + (b_ok(k0, i) ? off : 0));
    }
  };
  auto zap = [](const uint4& v, bool ok) {
    return make_uint4(ok ? v.x : 0u, ok ? v.y : 0u, ok ? v.z : 0u, ok ? v.w : 0u);
  };
  // (lo16(x), lo16(y)) or (hi16(x), hi16(y)) packed into one word: element i of two rows.
  auto pair = [](uint32_t x, uint32_t y, int i) {
    return __builtin_amdgcn_perm(y, x, (i & 1) ? 0x07060302u : 0x05040100u);
  };
  auto word = [](const uint4& v, int i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; };
  auto sstore = [&](int buf, const Stage& raw, int64_t k0) {
    Stage r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r.a[i] = zap(raw.a[i], a_ok(k0, i));
#pragma unroll
    for (int i = 0; i < 2; ++i) r.b[i] = zap(raw.b[i], b_ok(k0, i));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (AL == 0) {
        const int c = t + 256 * i;
        *reinterpret_cast<uint4*>(&As[buf][c >> 3][(c & 7) * 8]) = r.a[i];
      }
    }
    if constexpr (AL != 0) {
      const int kq = (t & 15) * 4, mb = (t >> 4) * 8;
#pragma unroll
      for (int i = 0; i < 8; ++i) {  // row m = mb + i: k-values kq .. kq + 3
        const uint32_t lo = pair(word(r.a[0], i >> 1), word(r.a[1], i >> 1), i);
        const uint32_t hi = pair(word(r.a[2], i >> 1), word(r.a[3], i >> 1), i);
        *reinterpret_cast<uint2*>(&As[buf][mb + i][kq]) = make_uint2(lo, hi);
      }
    }
    if constexpr (BL == 0) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int c = t + 256 * i;
        *reinterpret_cast<uint4*>(&Bs[buf][c >> 3][(c & 7) * 8]) = r.b[i];
      }
    } else {
      const int kq = (t & 31) * 2, nb = (t >> 5) * 8;
#pragma unroll
      for (int i = 0; i < 8; ++i)  // row n = nb + i: k-values kq, kq + 1
        *reinterpret_cast<uint32_t*>(&Bs[buf][nb + i][kq]) = pair(word(r.b[0], i >> 1), word(r.b[1], i >> 1), i);
    }
  };
  f32x16_t acc[2] = {f32x16_t{}, f32x16_t{}};
  auto compute = [&](int buf) {
#pragma unroll
    for (int kk = 0; kk < kSkK / 16; ++kk) {
      const int kofs = kk * 16 + (lane >> 5) * 8;
      const bf16x8_t a = *reinterpret_cast<const bf16x8_t*>(&As[buf][wave * 32 + (lane & 31)][kofs]);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const bf16x8_t b = *reinterpret_cast<const bf16x8_t*>(&Bs[buf][j * 32 + (lane & 31)][kofs]);
        if constexpr (TOUT)
          acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b, a, acc[j], 0, 0, 0);  // rows n', columns m'
        else
          acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[j], 0, 0, 0);  // rows m', columns n'
      }
    }
  };
  // Two K steps of loads in flight: while step s is multiplied out of LDS buffer (s - s0) & 1,
  // step s + 1 waits in one register stage and step s + 2 is being fetched into the other.
  // The split runs an even number of steps; a step past kend loads zeros.
  Stage r0, r1;
  const int64_t se = s0 + ((s1 - s0 + 1) & ~int64_t(1));
  gload(r0, s0 * kSkK);
  gload(r1, (s0 + 1) * kSkK);
  sstore(0, r0, s0 * kSkK);
  __syncthreads();
  auto step = [&](int64_t s, Stage& next, Stage& ahead) {
    const int buf = static_cast<int>((s - s0) & 1);
    gload(ahead, (s + 2) * kSkK);
    compute(buf);
    sstore(buf ^ 1, next, (s + 1) * kSkK);
    __syncthreads();
  };
  for (int64_t s = s0; s < se; s += 2) {
    step(s, r1, r0);
    step(s + 1, r0, r1);
  }
  // 32x32 accumulator layout: lane holds column (lane % 32) and rows (e / 4) * 8 + (lane / 32) * 4 + e % 4
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int r = (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
      int64_t row, col, rows, cols;  // in C's coordinates
      if constexpr (TOUT) {
        row = j * 32 + r;
        col = m0 + wave * 32 + (lane & 31);
        rows = g.N;
        cols = g.M;
      } else {
        row = m0 + wave * 32 + r;
        col = j * 32 + (lane & 31);
        rows = g.M;
        cols = g.N;
      }
      if (row < rows && col < cols) g.partial[(kz * rows + row) * cols + col] = acc[j][e];
    }
}

// Splits of a skinny product.  A CU moves about the same bytes per unit time with one
// workgroup as with two, so the time of a split count is the number of workgroups on the
// busiest CU times the K steps each runs, plus about four steps of fixed cost (the first
// loads, the partial write); the count (1 .. 16) that minimises it wins.
int skinny_splits(int64_t long_side, int64_t K) {
  const int64_t tiles = ceil_div(long_side, kSkM), stages = ceil_div(K, kSkK);
  int64_t best = 1, best_cost = -1;
  for (int64_t sp = 1; sp <= 16 && sp <= stages; ++sp) {
    const int64_t cost = ceil_div(tiles * sp, 256) * (ceil_div(stages, sp) + 4);
    if (best_cost < 0 || cost < best_cost) {
      best = sp;
      best_cost = cost;
    }
  }
  return static_cast<int>(best);
}

// A product the skinny kernel takes: bf16, dense B, no effective mask, one K segment, dense C, a side of at most 64.
bool skinny_ok(const sf_gemm_desc* d) {
  return d->dtype == SF_DTYPE_BF16 && d->b_format == SF_BFMT_DENSE && !d->bmask && d->K2 == 0 && !d->c_blocks &&
         d->K1 > 0 && (d->N <= kSkN || d->M <= kSkN);
}

size_t skinny_workspace(const sf_gemm_desc* d) {
  const bool tout = d->N > kSkN;
  const int sp = skinny_splits(tout ? d->N : d->M, d->K1);
  return static_cast<size_t>(sp) * d->M * d->N * sizeof(float);
}

int launch_skinny(const sf_gemm_desc* d, GemmArgs g, hipStream_t st) {
  const bool tout = d->N > kSkN;  // C's short side is its rows: A' = B, B' = A
  SkinnyArgs a;
  a.A = static_cast<const uint16_t*>(tout ? d->B1 : d->A1);
  a.B = static_cast<const uint16_t*>(tout ? d->A1 : d->B1);
  a.lda = tout ? d->ldb1 : d->lda1;
  a.ldb = tout ? d->lda1 : d->ldb1;
  a.M = tout ? d->N : d->M;
  a.N = tout ? d->M : d->N;
  a.K = d->K1;
  const int al = tout ? d->b_layout : d->a_layout, bl = tout ? d->a_layout : d->b_layout;
  const int sp = skinny_splits(a.M, a.K);
  a.split_stages = ceil_div(ceil_div(a.K, kSkK), sp);
  a.partial = static_cast<float*>(d->workspace);
  const int64_t grid = ceil_div(a.M, kSkM) * sp;
  SF_CHECK_ARG(grid < (1ll << 31), "GEMM grid too large");
  const dim3 gd(static_cast<unsigned>(grid)), bd(256);
#define SF_SKINNY(AL_, BL_)                                                      \
  do {                                                                           \
    if (tout)                                                                    \
      hipLaunchKernelGGL((skinny_kernel<AL_, BL_, true>), gd, bd, 0, st, a);     \
    else                                                                         \
      hipLaunchKernelGGL((skinny_kernel<AL_, BL_, false>), gd, bd, 0, st, a);    \
  } while (0)
  if (al == SF_LAYOUT_K && bl == SF_LAYOUT_K)
    SF_SKINNY(0, 0);
  else if (al == SF_LAYOUT_K)
    SF_SKINNY(0, 1);
  else if (bl == SF_LAYOUT_K)
    SF_SKINNY(1, 0);
  else
    SF_SKINNY(1, 1);
#undef SF_SKINNY
  if (int rc = launch_status("sf_gemm (skinny)")) return rc;
  g.splits = sp;
  g.partial = a.partial;
  hipLaunchKernelGGL(splitk_reduce_kernel, dim3(static_cast<unsigned>(elementwise_grid(g.M * g.N, 256))), dim3(256), 0,
                     st, g, SF_DTYPE_BF16);
  return launch_status("sf_gemm (skinny reduce)");
}

template <typename T, int MASK>
int dispatch_layouts(const sf_gemm_desc* d, const GemmArgs& g, hipStream_t st) {
  if constexpr (MASK == kMaskNone) {
    if constexpr (sizeof(T) == 2) {
      if (d->b_format == SF_BFMT_BSR16 && g.splits == 1) {
        if (d->b_layout == SF_LAYOUT_K && bs16_ok(g)) return launch_bs16(g, st);
        static bool attr_f = false, attr_t = false;
        return d->b_layout == SF_LAYOUT_K
                   ? launch_bsr_kernel(bsr_mm_kernel<0>, attr_f, g, st, "sf_gemm (block-sparse)")
                   : launch_bsr_kernel(bsr_mm_kernel<1>, attr_t, g, st, "sf_gemm (block-sparse, transposed)");
      }
    }
    if (d->b_format == SF_BFMT_BSR16)
      return d->b_layout == SF_LAYOUT_K ? launch_gemm<T, 0, 2, MASK>(g, st) : launch_gemm<T, 0, 3, MASK>(g, st);
  }
  if (d->a_layout == SF_LAYOUT_K && d->b_layout == SF_LAYOUT_K) return launch_gemm<T, 0, 0, MASK>(g, st);
  if (d->a_layout == SF_LAYOUT_K) return launch_gemm<T, 0, 1, MASK>(g, st);
  return launch_gemm<T, 1, 1, MASK>(g, st);
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// K splits for a GEMM whose tile grid would leave most of the 256 CUs idle:
// enough splits to give about one workgroup per CU, each split keeping at
// least 8 stages of K, at most 16 splits.
int choose_splits(const sf_gemm_desc* d) {
  const int64_t tiles = ceil_div(d->M, kTileM) * ceil_div(d->N, kTileN);
  const int bk = d->dtype == SF_DTYPE_BF16 ? Tr<uint16_t>::BK : Tr<float>::BK;
  const int64_t stages = ceil_div(d->K1, bk);
  if (tiles >= 128 || stages < 16) return 1;
  int64_t sp = ceil_div(256, tiles);
  if (sp > stages / 8) sp = stages / 8;
  if (sp > 16) sp = 16;
  return sp < 2 ? 1 : static_cast<int>(sp);
}

}  // namespace
}  // namespace sf

using namespace sf;

extern "C" size_t sf_gemm_workspace_size(const sf_gemm_desc* d) {
  if (!d || d->M <= 0 || d->N <= 0 || d->K1 <= 0) return 0;
  if (d->dtype != SF_DTYPE_BF16 && d->dtype != SF_DTYPE_F32) return 0;
  if (skinny_ok(d)) return skinny_workspace(d);
  const int sp = choose_splits(d);
  return sp > 1 ? static_cast<size_t>(sp) * d->M * d->N * sizeof(float) : 0;
}

extern "C" int sf_gemm(const sf_gemm_desc* d, void* stream) {
  SF_CHECK_ARG(d != nullptr, "null sf_gemm_desc");
  SF_CHECK_ARG(d->dtype == SF_DTYPE_BF16 || d->dtype == SF_DTYPE_F32, "bad element dtype %d", d->dtype);
  SF_CHECK_ARG(d->c_dtype == SF_DTYPE_BF16 || d->c_dtype == SF_DTYPE_F32, "bad output dtype %d", d->c_dtype);
  SF_CHECK_ARG(d->a_layout == SF_LAYOUT_K || d->a_layout == SF_LAYOUT_MN, "bad A layout");
  SF_CHECK_ARG(d->b_layout == SF_LAYOUT_K || d->b_layout == SF_LAYOUT_MN, "bad B layout");
  SF_CHECK_ARG(!(d->a_layout == SF_LAYOUT_MN && d->b_layout == SF_LAYOUT_K),
               "A M-contiguous with B K-contiguous is not built");
  SF_CHECK_ARG(d->M >= 0 && d->N >= 0 && d->K1 >= 0 && d->K2 >= 0, "negative GEMM size");
  if (d->M == 0 || d->N == 0) return SF_OK;
  SF_CHECK_ARG(d->C || d->c_blocks, "null C");
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
  const bool bsr_b = d->b_format == SF_BFMT_BSR16;
  SF_CHECK_ARG(d->b_format == SF_BFMT_DENSE || bsr_b, "bad B format %d", d->b_format);
  if (bsr_b) {
    SF_CHECK_ARG(d->a_layout == SF_LAYOUT_K, "a block-sparse B needs a K-contiguous A");
    SF_CHECK_ARG(d->b_map && d->b_map_rows >= 0 && d->b_map_cols >= 0, "block-sparse B needs its block map");
    SF_CHECK_ARG(!d->bmask && d->K2 == 0, "block-sparse B takes no effective mask and no second K segment");
    SF_CHECK_ARG(d->K1 % 16 == 0, "block-sparse B: K (%lld) must be a multiple of 16", (long long)d->K1);
    SF_CHECK_ARG(d->K1 == 0 || (d->B1 && al16(d->B1)), "block-sparse B: blocks must be 16-byte aligned");
    SF_CHECK_ARG(d->b_map_rows * d->b_map_cols * 512 < (int64_t(1) << 31),
                 "block-sparse B: block arrays of 2 GiB or more are not supported");
  }
  if (d->bmask_kmajor) {
    SF_CHECK_ARG(d->bmask && d->bmask_bytes && d->b_layout == SF_LAYOUT_MN && d->dtype == SF_DTYPE_BF16,
                 "a K-major mask is a bf16 byte mask of an N-contiguous B");
    SF_CHECK_ARG(d->ldbm >= d->K1, "ldbm (%lld) < K1 (%lld)", (long long)d->ldbm, (long long)d->K1);
    SF_CHECK_ARG(al16(d->bmask) && d->ldbm % 16 == 0, "a K-major mask needs 16-byte aligned rows (ldbm %% 16 == 0)");
    SF_CHECK_ARG((int64_t)d->N * d->ldbm < (int64_t(1) << 31), "K-major mask of 2 GiB or more");
  }
  if (d->c_blocks) {
    SF_CHECK_ARG(d->c_map && d->M % 16 == 0 && d->N % 16 == 0 && al16(d->c_blocks),
                 "block-sparse C needs its block map, M and N multiples of 16 and 16-byte aligned blocks");
    SF_CHECK_ARG(!d->bias && !d->emask && !d->accumulate, "block-sparse C takes no bias, mask product or accumulation");
  }
  SF_CHECK_ARG(chk_operand(d->A1, d->lda1, d->a_layout, d->M, d->K1) &&
                   chk_operand(d->A2, d->lda2, d->a_layout, d->M, d->K2) &&
                   (bsr_b || chk_operand(d->B1, d->ldb1, d->b_layout, d->N, d->K1)) &&
                   chk_operand(d->B2, d->ldb2, d->b_layout, d->N, d->K2) &&
                   (d->bmask_bytes ? (!d->bmask || (reinterpret_cast<uintptr_t>(d->bmask) % vec == 0))
                               : chk_operand(d->bmask, d->ldb1, d->b_layout, d->N, d->K1)),
               "GEMM operands must be 16-byte aligned with contiguous extents and leading dims that are multiples "
               "of %d elements (M=%lld N=%lld K1=%lld K2=%lld)",
               vec, (long long)d->M, (long long)d->N, (long long)d->K1, (long long)d->K2);
  SF_CHECK_ARG(d->ldc >= d->N, "ldc < N");
  // operands are addressed with 32-bit buffer offsets; kOob must lie past every extent
  const int64_t es = d->dtype == SF_DTYPE_BF16 ? 2 : 4;
  auto extent = [&](const void* p, int64_t ld, int layout, int64_t rows, int64_t K) -> int64_t {
    if (!p || K == 0) return 0;
    return (layout == SF_LAYOUT_K ? rows : K) * ld * es;
  };
  const int64_t lim = int64_t(1) << 31;
  if (extent(d->A1, d->lda1, d->a_layout, d->M, d->K1) >= lim || extent(d->A2, d->lda2, d->a_layout, d->M, d->K2) >= lim ||
      (!bsr_b && extent(d->B1, d->ldb1, d->b_layout, d->N, d->K1) >= lim) ||
      extent(d->B2, d->ldb2, d->b_layout, d->N, d->K2) >= lim) {
    set_error("sf_gemm: operands of 2 GiB or more are not supported (M=%lld N=%lld K1=%lld)", (long long)d->M,
              (long long)d->N, (long long)d->K1);
    return SF_ERR_UNSUPPORTED;
  }
  SF_CHECK_ARG(!d->dw || d->emask, "the decay epilogue needs the effective mask");
  GemmArgs g;
  g.M = d->M;
  g.N = d->N;
  g.K1 = d->K1;
  g.K2 = d->K2;
  g.A1 = d->A1;
  g.lda1 = d->lda1;
  g.A2 = d->K2 ? d->A2 : nullptr;
  g.lda2 = d->lda2;
  g.B1 = d->B1;
  g.ldb1 = d->ldb1;
  g.B2 = d->B2;
  g.ldb2 = d->ldb2;
  g.bmask = d->K1 ? d->bmask : nullptr;
  g.bscale = d->bscale;
  g.has_scale = d->bscale != 1.0f;
  g.C = d->C;
  g.ldc = d->ldc;
  g.c_dtype = d->c_dtype;
  g.bias = d->bias;
  g.bias_dtype = d->bias_dtype;
  g.emask = d->emask;
  g.dw = d->dw;
  g.decay = d->decay;
  g.accumulate = d->accumulate;
  g.c_aligned = al16(d->C);
  g.b_map = bsr_b ? d->b_map : nullptr;
  g.b_map_rows = d->b_map_rows;
  g.b_map_cols = d->b_map_cols;
  g.c_blocks = d->c_blocks;
  g.c_map = d->c_map;
  g.c_map_rows = d->c_map_rows;
  g.c_map_cols = d->c_map_cols;
  g.bmask_kmajor = d->bmask_kmajor != 0;
  g.ldbm = d->b_layout == SF_LAYOUT_K ? d->ldb1 : (d->bmask_kmajor ? d->ldbm : d->ldb1);
  // the direct bf16 kernel copies a byte mask 16 bytes per lane from K-major rows
  g.dma_mask_ok = d->bmask && d->bmask_bytes && al16(d->bmask) && g.ldbm % 16 == 0 &&
                  (d->b_layout == SF_LAYOUT_K || g.bmask_kmajor);
  g.tiles_m = ceil_div(d->M, kTileM);
  g.tiles_n = ceil_div(d->N, kTileN);
  g.splits = 1;
  g.split_stages = ceil_div(d->K1, d->dtype == SF_DTYPE_BF16 ? Tr<uint16_t>::BK : Tr<float>::BK);
  g.partial = nullptr;
  {
    // as many of the chosen K splits as the workspace holds partials for (a caller running the product
    // beside another one can ask for fewer with a smaller workspace)
    int sp = choose_splits(d);
    const size_t per = static_cast<size_t>(d->M) * d->N * sizeof(float);
    if (d->workspace && sp > 1 && d->workspace_bytes < sp * per) sp = static_cast<int>(d->workspace_bytes / per);
    const size_t need = static_cast<size_t>(sp) * per;
    if (sp > 1 && !d->c_blocks && d->workspace && d->workspace_bytes >= need && al16(d->workspace)) {
      g.splits = sp;
      g.split_stages = ceil_div(g.split_stages, sp);
      g.partial = static_cast<float*>(d->workspace);
    }
  }
  // the weight-scaling factor is applied together with a multiplicative mask
  SF_CHECK_ARG(!g.has_scale || (g.bmask && !d->bmask_bytes), "bscale != 1 needs a multiplicative effective mask");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (skinny_ok(d) && d->workspace && d->workspace_bytes >= skinny_workspace(d) && al16(d->workspace))
    return launch_skinny(d, g, st);
  const bool bf = d->dtype == SF_DTYPE_BF16;
  if (g.bmask && d->bmask_bytes)
    return bf ? dispatch_layouts<uint16_t, kMaskByte>(d, g, st) : dispatch_layouts<float, kMaskByte>(d, g, st);
  if (g.bmask)
    return bf ? dispatch_layouts<uint16_t, kMaskMul>(d, g, st) : dispatch_layouts<float, kMaskMul>(d, g, st);
  return bf ? dispatch_layouts<uint16_t, kMaskNone>(d, g, st) : dispatch_layouts<float, kMaskNone>(d, g, st);
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
  if (rg == 0 && col < cols)
    store_from_f32(out, col, out_dtype, ((part[0][c] + part[1][c]) + part[2][c]) + part[3][c]);
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

// ---------------------------------------------------------------------------
// 2:4 packed weights and the sparse-MFMA forward (finalized / inference
// models: legacy/main_llama.py:2499-2568 hardens the masks and multiplies
// them into the weights; legacy/eval_wiki_ppl.py:548-651 then runs the plain
// forward).  A hardened 2:4 weight W [M = out, K = in] keeps two of every four
// consecutive k; it is stored as
//   vals bf16 (M * K / 2 values): the two kept values of each group in column
//        order, 8 per 16-column chunk; chunk 4 q + 2 kk + h of row
//        rb * 32 + r sits at [rb][q][kk][h * 32 + r][8] (vals_off);
//   idx  u32 [M / 32][K / 64][2][32]: for row block rb, 64-column chunk q, half
//        h and row rb * 32 + r, word (bits 2j + 1 : 2j = column in its group
//        of the j-th kept value, j = 0..7) for columns [q * 64 + 16 h, +16) in
//        the low 16 bits and [q * 64 + 32 + 16 h, +16) in the high 16 bits.
// Both are the operand layout of v_smfmac_f32_32x32x32_bf16 (A sparse, lane l:
// row l % 32, dense k [16 (l / 32), +16) as 8 values + 16 index bits, the
// index register's half picked by abid = the k-step), one 1 KiB (values) or
// 256-byte (indices) run per row block, stage and k-step, so the kernel loads
// its A fragments straight from memory into registers, fully coalesced.  The
// MFMA computes y^T tiles (out x tokens); the epilogue writes them transposed.
// ---------------------------------------------------------------------------
namespace sf {
namespace {

typedef __bf16 bf16x16_t __attribute__((ext_vector_type(16)));

struct Gemm24Args {
  const void* x;       // [N = tokens, K] bf16, row pitch ldx
  int64_t ldx;
  const void* vals;    // M * K / 2 bf16, fragment order (vals_off)
  const void* idx;     // u32 [M / 32][K / 64][2][32]
  int64_t M, N, K;
  const void* bias;    // [M] or null
  int bias_dtype;
  void* y;             // [N, M], row pitch ldy
  int y_dtype;
  int64_t ldy;
  int64_t tiles_m, tiles_n;
  int y_aligned;
  // optional dense second segment y^T += A2 . B2^T: A2 [M, K2] and B2 [N, K2] bf16, K-contiguous
  const void* A2;
  const void* B2;
  int64_t lda2, ldb2, K2;
};

constexpr int kEpi24Pitch = 68;  // f32 pitch of the transposed staging: 128 token rows x 64 out columns per wave
constexpr uint32_t k24XBuf = 256u * kRowSw;  // one x stage: 256 token rows x 128 B

__global__ void __launch_bounds__(kThreads, 1) gemm24_kernel(Gemm24Args g) {
  extern __shared__ __align__(16) unsigned char smem[];
  const uint32_t base_l = lds_addr(smem);
  int64_t tm, tn;
  tile_coords(blockIdx.x, g.tiles_m, g.tiles_n, tm, tn);
  const int64_t m0 = tm * kTileM, n0 = tn * kTileN;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t nk = g.K / 64;

  f32x16_t acc[kFragM * kFragN];
#pragma unroll
  for (int i = 0; i < kFragM * kFragN; ++i) acc[i] = f32x16_t{};

  // x stages (256 tokens x 64 k, swizzled rows of 128 B) double-buffered in LDS; the sparse A
  // operand (values + index words) loaded straight into registers.  Every load is compiler-tracked
  // and unconditional (past the last stage the clamped index re-reads it), so the compiler's wait
  // counts are exact: at the start of stage s the A fragments of stage s + 1 and the x rows of
  // stage s + 2 are issued; the x rows of stage s + 1 (loaded at the start of stage s - 1) are
  // written to the other buffer after the stage's MFMAs, and one barrier a stage publishes them.
  uint32_t boff[4][kFragN];
#pragma unroll
  for (int j = 0; j < kFragN; ++j) {
    const uint32_t b = frag_base<true>(wn * kWaveN + j * 32 + (lane & 31));
#pragma unroll
    for (int q = 0; q < 4; ++q) boff[q][j] = frag_at<true>(b, q);
  }
  // x copy: thread t moves 16-byte chunk t % 8 of token rows 32 i + t / 8, i = 0..7
  const Rsrc rx = make_rsrc(g.x, g.N * g.ldx * 2);
  const int crow = threadIdx.x >> 3, cch = threadIdx.x & 7;
  uint32_t xoff[8], xlds[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int row = 32 * i + crow;
    xoff[i] = n0 + row < g.N ? (uint32_t)(((n0 + row) * g.ldx + cch * 8) * 2) : kOob;
    xlds[i] = (uint32_t)(row * kRowSw + ((cch ^ ((row ^ (row >> 3)) & 7)) << 4));
  }
  // A fragments: row block rb = m0 / 32 + 4 wm + i, lane's 16 bytes of k-step kk at
  // vals + ((rb nk + s) 2 + kk) 1 KiB + 16 lane; its index word at idx + ((rb nk + s) 64 + lane) 4
  const Rsrc rv = make_rsrc(g.vals, g.M * g.K);
  const Rsrc ri = make_rsrc(g.idx, (g.M / 32) * nk * 256);
  uint32_t voff[kFragM], wioff[kFragM];
#pragma unroll
  for (int i = 0; i < kFragM; ++i) {
    const int64_t rb = m0 / 32 + wm * 4 + i;
    voff[i] = rb < g.M / 32 ? (uint32_t)((rb * nk * 2 * 64 + lane) * 16) : kOob;
    wioff[i] = rb < g.M / 32 ? (uint32_t)((rb * nk * 64 + lane) * 4) : kOob;
  }
  bf16x8_t fa[2][kFragM][2];  // [stage set][fragment][k-step]
  uint32_t fi[2][kFragM];
  V4 xr[2][8];
  auto load_a = [&](auto set_c, int64_t st) {
    constexpr int set = decltype(set_c)::value;
#pragma unroll
    for (int i = 0; i < kFragM; ++i) {
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
        fa[set][i][kk] = __builtin_bit_cast(bf16x8_t, bload(rv, voff[i], (uint32_t)((st * 2 + kk) * 1024)));
      fi[set][i] = __builtin_amdgcn_raw_buffer_load_b32(ri, (int)wioff[i], (int)(st * 256), 0);
    }
  };
  auto load_x = [&](auto set_c, int64_t st) {
    constexpr int set = decltype(set_c)::value;
#pragma unroll
    for (int i = 0; i < 8; ++i) xr[set][i] = bload(rx, xoff[i], (uint32_t)(st * 128));
  };
  auto store_x = [&](auto set_c, int buf) {
    constexpr int set = decltype(set_c)::value;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      uint4 v;
      v.x = xr[set][i].w[0];
      v.y = xr[set][i].w[1];
      v.z = xr[set][i].w[2];
      v.w = xr[set][i].w[3];
      *reinterpret_cast<uint4*>(smem + buf * k24XBuf + xlds[i]) = v;
    }
  };
  // B fragments: fb[kk] holds k-step kk of the current stage.  Stage s: fragments of k-step 1 read
  // during the k-step 0 MFMAs; x of stage s + 1 written to the other buffer; the barrier; the next
  // stage's k-step 0 fragments read during the k-step 1 MFMAs.
  bf16x16_t fb[2][kFragN];
  auto read_b = [&](int slot, int buf, int kk) {
    const unsigned char* xb = smem + buf * k24XBuf;
#pragma unroll
    for (int j = 0; j < kFragN; ++j) {
      const bf16x8_t lo = *reinterpret_cast<const bf16x8_t*>(xb + boff[2 * kk][j]);
      const bf16x8_t hi = *reinterpret_cast<const bf16x8_t*>(xb + boff[2 * kk + 1][j]);
      fb[slot][j] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15);
    }
  };
  auto mfmas = [&](auto set_c, auto kk_c) {
    constexpr int set = decltype(set_c)::value, kk = decltype(kk_c)::value;
#pragma unroll
    for (int j = 0; j < kFragN; ++j)
#pragma unroll
      for (int i = 0; i < kFragM; ++i)
        acc[i * kFragN + j] = __builtin_amdgcn_smfmac_f32_32x32x32_bf16(fa[set][i][kk], fb[kk][j], acc[i * kFragN + j],
                                                                       (int)fi[set][i], 0, kk);
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  auto stage = [&](auto set_c, int64_t st) {
    constexpr int set = decltype(set_c)::value;
    using Other = std::integral_constant<int, set ^ 1>;
    const int64_t s1 = st + 1 < nk ? st + 1 : nk - 1, s2 = st + 2 < nk ? st + 2 : nk - 1;
    load_a(Other{}, s1);
    load_x(set_c, s2);
    read_b(1, set, 1);
    store_x(Other{}, set ^ 1);  // x of stage s + 1 (past the end: written, never read)
    mfmas(set_c, S0{});
    // With one wave per SIMD nothing else feeds the MFMA pipe while a wave issues memory
    // instructions, so they go between the MFMAs (scheduling groups, in this order): k-step 0's 16
    // MFMAs each followed by one of 12 loads and by a fragment read (MFMAs 0-7) or a copy write
    // (8-15); after the barrier, k-step 1's MFMAs with the next stage's fragment reads (0-7) and
    // the remaining 8 loads (8-15).  Group sync ids 0 / 1 keep the two phases apart.
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      if (i < 12) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM read
      if (i < 8) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // DS read
      if (i >= 8) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // DS write
    }
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    read_b(0, set ^ 1, 0);      // the next stage's k-step 0 (past the end: unused)
    mfmas(set_c, S1{});
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
      if (i < 8) __builtin_amdgcn_sched_group_barrier(0x100, 1, 1);
      if (i >= 8) __builtin_amdgcn_sched_group_barrier(0x020, 1, 1);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  if (nk > 0) {
    load_a(S0{}, 0);
    load_x(S0{}, 0);
    store_x(S0{}, 0);
    load_x(S1{}, nk > 1 ? 1 : 0);
    __syncthreads();
    read_b(0, 0, 0);
    int64_t s = 0;
    for (; s + 1 < nk; s += 2) {
      stage(S0{}, s);
      stage(S1{}, s + 1);
    }
    if (s < nk) stage(S0{}, s);
  }

  // Segment 2 (dense, 64 k a stage through the first 64 KB of LDS): the low-rank term
  // A2 . B2^T accumulated into the same tile, operands in the swizzled K-contiguous layout of
  // the dense kernel.  It runs on the sparse instruction too (dense and sparse MFMAs on the
  // same accumulators do not fit the register file).  The 16 dense k of a k-step are the
  // kept values of 32 sparse k keeping columns 0 and 1 of every group of four: sparse k p
  // holds dense k 2 (p / 4) + p % 4.  The A fragment (lane half h: dense k [8 h, 8 h + 8),
  // sparse k [16 h, 16 h + 16)) is the dense one with index bits 0x4444; the B fragment
  // (lane half h: sparse k [8 h, 8 h + 8) and [16 + 8 h, 24 + 8 h)) takes dense k
  // [4 h, 4 h + 4) and [8 + 4 h, 12 + 4 h), each pair followed by two zeros.
  if (g.K2 > 0) {
    DmaLoader d2a, d2b;
    d2a.init(g.A2, g.lda2, m0, g.M, g.K2);
    d2b.init(g.B2, g.ldb2, n0, g.N, g.K2);
    const int64_t nk2 = ceil_div(g.K2, 64);
    const int hl = lane >> 5;
    for (int64_t s2 = 0; s2 < nk2; ++s2) {
      __syncthreads();  // every wave is done with the buffers
      d2a.issue<true>(base_l, s2 * 64);
      d2b.issue<true>(base_l + 32768u, s2 * 64);
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        bf16x8_t a[kFragM];
#pragma unroll
        for (int i = 0; i < kFragM; ++i)
          a[i] = *reinterpret_cast<const bf16x8_t*>(
              smem + frag_at<true>(frag_base<true>(wm * kWaveM + i * 32 + (lane & 31)), kk));
#pragma unroll
        for (int j = 0; j < kFragN; ++j) {
          const int r = wn * kWaveN + j * 32 + (lane & 31), sw = (r ^ (r >> 3)) & 7;
          const unsigned char* row = smem + 32768u + r * kRowSw + hl * 8;
          const uint2 p0 = *reinterpret_cast<const uint2*>(row + (((2 * kk) ^ sw) << 4));
          const uint2 p1 = *reinterpret_cast<const uint2*>(row + (((2 * kk + 1) ^ sw) << 4));
          const uint4 lo = make_uint4(p0.x, 0u, p0.y, 0u), hi = make_uint4(p1.x, 0u, p1.y, 0u);
          const bf16x16_t b = __builtin_shufflevector(__builtin_bit_cast(bf16x8_t, lo), __builtin_bit_cast(bf16x8_t, hi),
                                                      0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15);
#pragma unroll
          for (int i = 0; i < kFragM; ++i)
            acc[i * kFragN + j] =
                __builtin_amdgcn_smfmac_f32_32x32x32_bf16(a[i], b, acc[i * kFragN + j], 0x4444, 0, 0);
        }
      }
    }
  }

  // Epilogue: acc block (i, j) holds y^T rows (out) m = i * 32 + (e / 4) * 8 +
  // (lane / 32) * 4 + e % 4 and column (token) n = j * 32 + lane % 32.  Each
  // wave stages 64 out columns x its 128 tokens transposed, then every lane
  // writes 8 consecutive outputs of one token row.
  float* ep = reinterpret_cast<float*>(smem) + wave * (128 * kEpi24Pitch);
  const bool ybf = g.y_dtype == SF_DTYPE_BF16;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    __syncthreads();
#pragma unroll
    for (int ii = 0; ii < 2; ++ii)
#pragma unroll
      for (int j = 0; j < kFragN; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int o = ii * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
          ep[(j * 32 + (lane & 31)) * kEpi24Pitch + o] = acc[(2 * h + ii) * kFragN + j][e];
        }
    __syncthreads();
    for (int it = 0; it < 16; ++it) {
      const int flat = it * 64 + lane;
      const int t = flat >> 3, oc = (flat & 7) * 8;
      const int64_t row = n0 + wn * kWaveN + t, col = m0 + wm * kWaveM + h * 64 + oc;
      if (row >= g.N || col >= g.M) continue;
      float v[8];
      const float4 p0 = *reinterpret_cast<const float4*>(ep + t * kEpi24Pitch + oc);
      const float4 p1 = *reinterpret_cast<const float4*>(ep + t * kEpi24Pitch + oc + 4);
      v[0] = p0.x; v[1] = p0.y; v[2] = p0.z; v[3] = p0.w;
      v[4] = p1.x; v[5] = p1.y; v[6] = p1.z; v[7] = p1.w;
      const int64_t off = row * g.ldy + col;
      const int nv = col + 8 <= g.M ? 8 : static_cast<int>(g.M - col);
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        if (q < nv && g.bias) {
          const float bq = load_elem(g.bias, col + q, g.bias_dtype);
          v[q] = ybf ? hround(hround(v[q]) + bq) : v[q] + bq;
        }
      }
      if (nv == 8 && g.y_aligned && (off & 7) == 0) {
        if (ybf) {
          *reinterpret_cast<uint4*>(static_cast<uint16_t*>(g.y) + off) =
              make_uint4(pack2(v[0], v[1]), pack2(v[2], v[3]), pack2(v[4], v[5]), pack2(v[6], v[7]));
        } else {
          float* yp = static_cast<float*>(g.y) + off;
          *reinterpret_cast<float4*>(yp) = make_float4(v[0], v[1], v[2], v[3]);
          *reinterpret_cast<float4*>(yp + 4) = make_float4(v[4], v[5], v[6], v[7]);
        }
      } else {
        for (int q = 0; q < nv; ++q) {
          if (ybf)
            static_cast<uint16_t*>(g.y)[off + q] = hbits(v[q]);
          else
            static_cast<float*>(g.y)[off + q] = v[q];
        }
      }
    }
  }
}

constexpr size_t smem24_bytes() {
  constexpr size_t ops = 2ull * k24XBuf, epi = 4ull * 128 * kEpi24Pitch * sizeof(float);
  return ops > epi ? ops : epi;
}

// Element offset in `vals` of the 8 kept values of row `row`, 16-column chunk c16 (K / 64
// stages of 4 chunks): chunk c16 = 4 q + 2 kk + h of row block rb = row / 32 lands in the
// 2 KiB run (rb, q) at [kk][h * 32 + row % 32][8], the order of the sparse MFMA's A fragments.
__device__ __forceinline__ int64_t vals_off(int64_t row, int64_t c16, int64_t nk) {
  const int64_t q = c16 >> 2, sub = c16 & 3;
  return ((((row >> 5) * nk + q) * 2 + (sub >> 1)) * 64 + (sub & 1) * 32 + (row & 31)) * 8;
}

// Pack: one thread per (row, 16 columns): 4 groups -> 8 kept values (16 bytes)
// and a 16-bit index word.  A group keeping fewer than two columns is padded
// with zero values at its lowest unused columns; more than two is counted in
// `bad` (the caller treats a nonzero count as an error).
__global__ void __launch_bounds__(256) pack24_kernel(const void* __restrict__ W, int w_dtype, const void* __restrict__ mask,
                                                     int m_dtype, int64_t M, int64_t K, uint16_t* __restrict__ vals,
                                                     uint16_t* __restrict__ idx, unsigned long long* __restrict__ bad) {
  const int64_t per_row = K / 16, total = M * per_row, nk = K / 64;
  unsigned long long nbad = 0;
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = t / per_row, c16 = t - row * per_row;
    const int64_t e0 = row * K + c16 * 16;
    uint16_t out[8];
    uint32_t bits = 0;
#pragma unroll
    for (int grp = 0; grp < 4; ++grp) {
      int pos[2] = {-1, -1}, n = 0;
      float v[2] = {0.0f, 0.0f};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int64_t e = e0 + grp * 4 + c;
        const float m = load_as_f32(mask, e, m_dtype);
        if (m != 0.0f) {
          if (n < 2) {
            pos[n] = c;
            v[n] = load_as_f32(W, e, w_dtype) * m;
          }
          ++n;
        }
      }
      if (n > 2) ++nbad;
      // pad to two distinct columns with zero values
      for (int c = 0; c < 4 && (pos[0] < 0 || pos[1] < 0); ++c) {
        if (c == pos[0] || c == pos[1]) continue;
        if (pos[0] < 0) pos[0] = c;
        else pos[1] = c;
      }
      if (pos[1] < pos[0]) {  // column order
        const int tp = pos[0]; pos[0] = pos[1]; pos[1] = tp;
        const float tv = v[0]; v[0] = v[1]; v[1] = tv;
      }
      out[2 * grp] = f32_to_bf16(v[0]);
      out[2 * grp + 1] = f32_to_bf16(v[1]);
      bits |= (uint32_t)pos[0] << (4 * grp);
      bits |= (uint32_t)pos[1] << (4 * grp + 2);
    }
    uint16_t* vp = vals + vals_off(row, c16, nk);
#pragma unroll
    for (int q = 0; q < 8; ++q) vp[q] = out[q];
    const int64_t q64 = c16 >> 2, sub = c16 & 3;  // 16-column block inside its 64-column chunk
    const int64_t word = (((row >> 5) * nk + q64) * 2 + (sub & 1)) * 32 + (row & 31);
    idx[word * 2 + (sub >> 1)] = static_cast<uint16_t>(bits);
  }
  if (nbad) atomicAdd(bad, nbad);
}

// The hx = 0 training forward's weight pass: Wm = round(W * E) for a byte and-mask E (W
// bf16; the elementwise product of sf_apply_mask, kept for the input gradient) and, from
// the same loads, the packed 2:4 form of Wm (the kept bf16 values exactly, the index bits
// of pack24_kernel).  One thread per (row, 16 columns), 128 consecutive threads per (32-row block,
// 64 columns): thread w of the run takes row 32 rb + w % 32 and 16-column chunk 4 q + w / 32, so
// the run writes whole lines of every output (the 2 KiB value run and the index words of (rb, q),
// each row's 128 bytes of W . E) and reads whole 128-byte lines of W.
__global__ void __launch_bounds__(256) apply_pack24_kernel(const uint16_t* __restrict__ W, const uint8_t* __restrict__ E,
                                                           int64_t M, int64_t K, uint16_t* __restrict__ Wm,
                                                           uint16_t* __restrict__ vals, uint16_t* __restrict__ idx,
                                                           unsigned long long* __restrict__ bad) {
  const int64_t per_row = K / 16, total = M * per_row, nk = K / 64;
  unsigned long long nbad = 0;
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t run = t >> 7, rb = run / nk, q = run - rb * nk;
    const int w = static_cast<int>(t & 127);
    const int64_t row = rb * 32 + (w & 31), c16 = q * 4 + (w >> 5);
    const int64_t e0 = row * K + c16 * 16;
    const uint4 wa = *reinterpret_cast<const uint4*>(W + e0), wb = *reinterpret_cast<const uint4*>(W + e0 + 8);
    const uint4 mb = *reinterpret_cast<const uint4*>(E + e0);
    const uint32_t ww[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
    const uint32_t mw[4] = {mb.x, mb.y, mb.z, mb.w};
    uint32_t om[8], ov[4], bits = 0;
#pragma unroll
    for (int grp = 0; grp < 4; ++grp) {
      uint16_t kept[2] = {0, 0};
      int pos[2] = {-1, -1}, n = 0;
      uint16_t prod[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int e = grp * 4 + c;
        const uint16_t wbits = static_cast<uint16_t>(ww[e >> 1] >> (16 * (e & 1)));
        const bool keep = ((mw[grp] >> (8 * c)) & 0xffu) != 0;
        prod[c] = f32_to_bf16(bf16_to_f32(wbits) * (keep ? 1.0f : 0.0f));
        if (keep) {
          if (n < 2) {
            pos[n] = c;
            kept[n] = prod[c];
          }
          ++n;
        }
      }
      if (n > 2) ++nbad;
      for (int c = 0; c < 4 && (pos[0] < 0 || pos[1] < 0); ++c) {  // pad to two distinct columns, zero values
        if (c == pos[0] || c == pos[1]) continue;
        if (pos[0] < 0) pos[0] = c;
        else pos[1] = c;
      }
      if (pos[1] < pos[0]) {
        const int tp = pos[0]; pos[0] = pos[1]; pos[1] = tp;
        const uint16_t tv = kept[0]; kept[0] = kept[1]; kept[1] = tv;
      }
      om[2 * grp] = prod[0] | (static_cast<uint32_t>(prod[1]) << 16);
      om[2 * grp + 1] = prod[2] | (static_cast<uint32_t>(prod[3]) << 16);
      ov[grp] = kept[0] | (static_cast<uint32_t>(kept[1]) << 16);
      bits |= (uint32_t)pos[0] << (4 * grp);
      bits |= (uint32_t)pos[1] << (4 * grp + 2);
    }
    *reinterpret_cast<uint4*>(Wm + e0) = make_uint4(om[0], om[1], om[2], om[3]);
    *reinterpret_cast<uint4*>(Wm + e0 + 8) = make_uint4(om[4], om[5], om[6], om[7]);
    *reinterpret_cast<uint4*>(vals + vals_off(row, c16, nk)) = make_uint4(ov[0], ov[1], ov[2], ov[3]);
    const int64_t q64 = c16 >> 2, sub = c16 & 3;
    const int64_t word = (((row >> 5) * nk + q64) * 2 + (sub & 1)) * 32 + (row & 31);
    idx[word * 2 + (sub >> 1)] = static_cast<uint16_t>(bits);
  }
  if (nbad) atomicAdd(bad, nbad);
}

__global__ void __launch_bounds__(256) unpack24_kernel(const uint16_t* __restrict__ vals, const uint16_t* __restrict__ idx,
                                                       int64_t M, int64_t K, void* __restrict__ W, int w_dtype) {
  const int64_t per_row = K / 16, total = M * per_row, nk = K / 64;
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = t / per_row, c16 = t - row * per_row;
    const int64_t q64 = c16 >> 2, sub = c16 & 3;
    const int64_t word = (((row >> 5) * nk + q64) * 2 + (sub & 1)) * 32 + (row & 31);
    const uint32_t bits = idx[word * 2 + (sub >> 1)];
    float d[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) d[q] = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int p = (bits >> (2 * j)) & 3;
      d[(j >> 1) * 4 + p] += bf16_to_f32(vals[vals_off(row, c16, nk) + j]);
    }
#pragma unroll
    for (int q = 0; q < 16; ++q) store_from_f32(W, row * K + c16 * 16 + q, w_dtype, d[q]);
  }
}

}  // namespace
}  // namespace sf

extern "C" size_t sf_pack_2to4_sizes(int64_t out_features, int64_t in_features, size_t* idx_bytes) {
  if (idx_bytes) *idx_bytes = out_features > 0 && in_features > 0 ? (size_t)(out_features * in_features / 8) : 0;
  return out_features > 0 && in_features > 0 ? (size_t)(out_features * (in_features / 2) * 2) : 0;
}

extern "C" int sf_pack_2to4(const void* W, int w_dtype, const void* mask, int mask_dtype, int64_t out_features,
                            int64_t in_features, void* vals, void* idx, unsigned long long* bad_groups,
                            void* stream) {
  SF_CHECK_ARG((w_dtype == SF_DTYPE_F32 || w_dtype == SF_DTYPE_BF16) &&
                   (mask_dtype == SF_DTYPE_F32 || mask_dtype == SF_DTYPE_BF16),
               "bad dtype");
  SF_CHECK_ARG(out_features > 0 && in_features > 0, "empty weight");
  SF_CHECK_ARG(out_features % 32 == 0 && in_features % 64 == 0,
               "2:4 packing needs out %% 32 == 0 and in %% 64 == 0 (got %lld x %lld)", (long long)out_features,
               (long long)in_features);
  SF_CHECK_ARG(W && mask && vals && idx && bad_groups, "null tensor");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t work = out_features * (in_features / 16);
  pack24_kernel<<<elementwise_grid(work, 256), 256, 0, st>>>(W, w_dtype, mask, mask_dtype, out_features, in_features,
                                                            static_cast<uint16_t*>(vals), static_cast<uint16_t*>(idx),
                                                            bad_groups);
  return launch_status("sf_pack_2to4");
}

extern "C" int sf_unpack_2to4(const void* vals, const void* idx, int64_t out_features, int64_t in_features, void* W,
                              int w_dtype, void* stream) {
  SF_CHECK_ARG(w_dtype == SF_DTYPE_F32 || w_dtype == SF_DTYPE_BF16, "bad dtype");
  SF_CHECK_ARG(out_features > 0 && in_features > 0 && out_features % 32 == 0 && in_features % 64 == 0,
               "bad packed shape %lld x %lld", (long long)out_features, (long long)in_features);
  SF_CHECK_ARG(W && vals && idx, "null tensor");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t work = out_features * (in_features / 16);
  unpack24_kernel<<<elementwise_grid(work, 256), 256, 0, st>>>(static_cast<const uint16_t*>(vals),
                                                              static_cast<const uint16_t*>(idx), out_features,
                                                              in_features, W, w_dtype);
  return launch_status("sf_unpack_2to4");
}

namespace sf {
namespace {
int launch_gemm24(const void* x, int64_t ldx, int64_t tokens, const void* vals, const void* idx, int64_t out_features,
                  int64_t in_features, const void* z, int64_t ldz, const void* S, int64_t lds, int64_t rank,
                  const void* bias, int bias_dtype, void* y, int y_dtype, int64_t ldy, void* stream, const char* what) {
  SF_CHECK_ARG(y_dtype == SF_DTYPE_F32 || y_dtype == SF_DTYPE_BF16, "bad output dtype");
  SF_CHECK_ARG(!bias || bias_dtype == SF_DTYPE_F32 || bias_dtype == SF_DTYPE_BF16, "bad bias dtype");
  SF_CHECK_ARG(tokens >= 0 && out_features > 0 && in_features > 0 && rank >= 0, "bad shape");
  SF_CHECK_ARG(out_features % 32 == 0 && in_features % 64 == 0,
               "2:4 product needs out %% 32 == 0 and in %% 64 == 0 (got %lld x %lld)", (long long)out_features,
               (long long)in_features);
  if (tokens == 0) return SF_OK;
  SF_CHECK_ARG(x && vals && idx && y, "null tensor");
  SF_CHECK_ARG(ldx >= in_features && ldx % 8 == 0 && al16(x) && al16(vals) && al16(idx),
               "x rows, vals and idx must be 16-byte aligned (ldx %% 8 == 0)");
  SF_CHECK_ARG(ldy >= out_features, "ldy < out_features");
  SF_CHECK_ARG(tokens * ldx * 2 < (int64_t(1) << 31) && out_features * in_features < (int64_t(1) << 31),
               "2:4 product: operands of 2 GiB or more are not supported");
  if (rank > 0) {
    SF_CHECK_ARG(z && S, "null low-rank operand");
    SF_CHECK_ARG(rank % 8 == 0 && ldz >= rank && lds >= rank && ldz % 8 == 0 && lds % 8 == 0 && al16(z) && al16(S),
                 "low-rank operands: rank, ldz and lds must be multiples of 8 with 16-byte aligned rows");
    SF_CHECK_ARG(tokens * ldz * 2 < (int64_t(1) << 31) && out_features * lds * 2 < (int64_t(1) << 31),
                 "2:4 product: low-rank operands of 2 GiB or more are not supported");
  }
  Gemm24Args g;
  g.x = x;
  g.ldx = ldx;
  g.vals = vals;
  g.idx = idx;
  g.M = out_features;
  g.N = tokens;
  g.K = in_features;
  g.bias = bias;
  g.bias_dtype = bias_dtype;
  g.y = y;
  g.y_dtype = y_dtype;
  g.ldy = ldy;
  g.tiles_m = ceil_div(out_features, kTileM);
  g.tiles_n = ceil_div(tokens, kTileN);
  g.y_aligned = al16(y);
  g.A2 = S;
  g.B2 = z;
  g.lda2 = lds;
  g.ldb2 = ldz;
  g.K2 = rank > 0 ? rank : 0;
  static bool attr = false;
  if (int rc = set_smem(gemm24_kernel, smem24_bytes(), attr)) return rc;
  const int64_t tiles = g.tiles_m * g.tiles_n;
  SF_CHECK_ARG(tiles < (1ll << 31), "grid too large");
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(gemm24_kernel, dim3(static_cast<unsigned>(tiles)), dim3(kThreads), smem24_bytes(), st, g);
  return launch_status(what);
}
}  // namespace
}  // namespace sf

extern "C" int sf_gemm_2to4(const void* x, int64_t ldx, int64_t tokens, const void* vals, const void* idx,
                            int64_t out_features, int64_t in_features, const void* bias, int bias_dtype, void* y,
                            int y_dtype, int64_t ldy, void* stream) {
  return sf::launch_gemm24(x, ldx, tokens, vals, idx, out_features, in_features, nullptr, 0, nullptr, 0, 0, bias,
                           bias_dtype, y, y_dtype, ldy, stream, "sf_gemm_2to4");
}

extern "C" int sf_gemm_2to4_lowrank(const void* x, int64_t ldx, int64_t tokens, const void* vals, const void* idx,
                                    int64_t out_features, int64_t in_features, const void* z, int64_t ldz,
                                    const void* S, int64_t lds, int64_t rank, const void* bias, int bias_dtype,
                                    void* y, int y_dtype, int64_t ldy, void* stream) {
  return sf::launch_gemm24(x, ldx, tokens, vals, idx, out_features, in_features, z, ldz, S, lds, rank, bias,
                           bias_dtype, y, y_dtype, ldy, stream, "sf_gemm_2to4_lowrank");
}

extern "C" int sf_apply_mask_2to4(const void* W, const void* mask, int64_t out_features, int64_t in_features,
                                  void* Wm, void* vals, void* idx, unsigned long long* bad_groups, void* stream) {
  SF_CHECK_ARG(out_features > 0 && in_features > 0, "empty weight");
  SF_CHECK_ARG(out_features % 32 == 0 && in_features % 64 == 0,
               "2:4 packing needs out %% 32 == 0 and in %% 64 == 0 (got %lld x %lld)", (long long)out_features,
               (long long)in_features);
  SF_CHECK_ARG(W && mask && Wm && vals && idx && bad_groups, "null tensor");
  SF_CHECK_ARG(al16(W) && al16(mask) && al16(Wm) && al16(vals), "W, mask, Wm and vals must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t work = out_features * (in_features / 16);
  hipLaunchKernelGGL(apply_pack24_kernel, dim3(static_cast<unsigned>(elementwise_grid(work, 256))), dim3(256), 0, st,
                     static_cast<const uint16_t*>(W), static_cast<const uint8_t*>(mask), out_features, in_features,
                     static_cast<uint16_t*>(Wm), static_cast<uint16_t*>(vals), static_cast<uint16_t*>(idx),
                     bad_groups);
  return launch_status("sf_apply_mask_2to4");
}
