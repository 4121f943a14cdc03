// Block-sparse-16 format on gfx950 (K11): build the compressed block index of
// W * mask and its block map, replacing convert_to_block_sparse
// (legacy/triton_block_sparse.py:46-103), whose Python double loop issues one
// host sync per block.
//
// Format (same as the reference): blocks [nnz, bs, bs] (W * mask, row-major
// inside a block), row_ptr int32 [nbr + 1] (CSR over block rows), col_idx
// int32 [nnz] (ascending within a block row).  A block is kept iff
// sum(|W * mask|) over it is > 0 (:79-89): the product rounds in the weight
// dtype, and a block holding a NaN sums to NaN and is dropped, as there.
// block_map int32 [nbr, nbc] (the block's index in `blocks`, or -1) is the
// device-side lookup the block-sparse GEMMs use; it is derived from row_ptr /
// col_idx, so it exists for any CSR index, not only for ones built here.
//
//   sf_bsr_count   flags + per-block-row counts           (grid: block rows)
//   sf_bsr_scan    row_ptr = exclusive scan of the counts  (one workgroup)
//   sf_bsr_fill    col_idx, blocks, block_map              (grid: block rows)
//   sf_bsr_block_map  block_map from any row_ptr / col_idx
//   sf_bsr_transpose  the transposed matrix: every block transposed, map [nbc, nbr]

#include "sf_common.hpp"

namespace sf {
namespace {

constexpr int kBlock = 256;

__device__ __forceinline__ float rnd(float x, int dtype) { return dtype == SF_DTYPE_BF16 ? round_bf16(x) : x; }

// Flag of block (br, bc): any element of W * mask nonzero and none NaN.
__device__ __forceinline__ bool block_kept(const void* W, int w_dt, const void* M, int m_dt, int64_t cols, int64_t br,
                                           int64_t bc, int bs, int prod_dt) {
  bool any = false, nan = false;
  for (int i = 0; i < bs; ++i) {
    const int64_t base = (br * bs + i) * cols + bc * bs;
    for (int j = 0; j < bs; ++j) {
      const float p = rnd(load_as_f32(W, base + j, w_dt) * load_as_f32(M, base + j, m_dt), prod_dt);
      any |= p != 0.0f;
      nan |= p != p;
    }
  }
  return any && !nan;
}

__global__ void __launch_bounds__(kBlock) bsr_count_kernel(const void* W, int w_dt, const void* M, int m_dt,
                                                           int64_t cols, int64_t nbc, int bs, int prod_dt,
                                                           uint8_t* flags, int32_t* counts) {
  const int64_t br = blockIdx.x;
  int c = 0;
  for (int64_t bc = threadIdx.x; bc < nbc; bc += kBlock) {
    const bool k = block_kept(W, w_dt, M, m_dt, cols, br, bc, bs, prod_dt);
    flags[br * nbc + bc] = k ? 1 : 0;
    c += k ? 1 : 0;
  }
  __shared__ int red[kBlock];
  red[threadIdx.x] = c;
  __syncthreads();
  for (int off = kBlock / 2; off > 0; off >>= 1) {
    if (threadIdx.x < off) red[threadIdx.x] += red[threadIdx.x + off];
    __syncthreads();
  }
  if (threadIdx.x == 0) counts[br] = red[0];
}

// row_ptr[0] = 0, row_ptr[r + 1] = row_ptr[r] + counts[r]: chunked scan in one workgroup.
__global__ void __launch_bounds__(kBlock) bsr_scan_kernel(const int32_t* counts, int64_t nbr, int32_t* row_ptr) {
  __shared__ int32_t part[kBlock];
  __shared__ int32_t carry;
  if (threadIdx.x == 0) {
    carry = 0;
    row_ptr[0] = 0;
  }
  __syncthreads();
  for (int64_t base = 0; base < nbr; base += kBlock) {
    const int64_t i = base + threadIdx.x;
    int32_t v = i < nbr ? counts[i] : 0;
    part[threadIdx.x] = v;
    __syncthreads();
    for (int off = 1; off < kBlock; off <<= 1) {  // inclusive Hillis-Steele scan
      const int32_t add = threadIdx.x >= off ? part[threadIdx.x - off] : 0;
      __syncthreads();
      part[threadIdx.x] += add;
      __syncthreads();
    }
    if (i < nbr) row_ptr[i + 1] = carry + part[threadIdx.x];
    __syncthreads();
    if (threadIdx.x == 0) carry += part[kBlock - 1];
    __syncthreads();
  }
}

// One workgroup per block row: rank the kept blocks in column order (a scan of
// the flags, 256 columns at a time), write col_idx, the block data and the map.
__global__ void __launch_bounds__(kBlock) bsr_fill_kernel(const void* W, int w_dt, const void* M, int m_dt,
                                                          int64_t cols, int64_t nbc, int bs, int prod_dt,
                                                          const uint8_t* flags, const int32_t* row_ptr,
                                                          int32_t* col_idx, void* blocks, int b_dt,
                                                          int32_t* block_map) {
  const int64_t br = blockIdx.x;
  __shared__ int32_t part[kBlock];
  __shared__ int32_t carry;
  if (threadIdx.x == 0) carry = row_ptr[br];
  __syncthreads();
  for (int64_t base = 0; base < nbc; base += kBlock) {
    const int64_t bc = base + threadIdx.x;
    const int f = bc < nbc ? flags[br * nbc + bc] : 0;
    part[threadIdx.x] = f;
    __syncthreads();
    for (int off = 1; off < kBlock; off <<= 1) {
      const int32_t add = threadIdx.x >= off ? part[threadIdx.x - off] : 0;
      __syncthreads();
      part[threadIdx.x] += add;
      __syncthreads();
    }
    if (bc < nbc) {
      int32_t idx = -1;
      if (f) {
        idx = carry + part[threadIdx.x] - 1;
        col_idx[idx] = static_cast<int32_t>(bc);
        for (int i = 0; i < bs; ++i) {
          const int64_t src = (br * bs + i) * cols + bc * bs;
          const int64_t dst = (int64_t)idx * bs * bs + i * bs;
          for (int j = 0; j < bs; ++j)
            store_from_f32(blocks, dst + j, b_dt,
                           rnd(load_as_f32(W, src + j, w_dt) * load_as_f32(M, src + j, m_dt), prod_dt));
        }
      }
      if (block_map) block_map[br * nbc + bc] = idx;
    }
    __syncthreads();
    if (threadIdx.x == 0) carry += part[kBlock - 1];
    __syncthreads();
  }
}

__global__ void __launch_bounds__(kBlock) bsr_map_clear_kernel(int32_t* map, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    map[i] = -1;
}

__global__ void __launch_bounds__(kBlock) bsr_map_fill_kernel(const int32_t* row_ptr, const int32_t* col_idx,
                                                              int64_t nbr, int64_t nbc, int32_t* map) {
  const int64_t br = blockIdx.x;
  const int32_t b = row_ptr[br], e = row_ptr[br + 1];
  for (int32_t k = b + threadIdx.x; k < e; k += kBlock) {
    const int32_t c = col_idx[k];
    if (c >= 0 && c < nbc) map[br * nbc + c] = k;  // indices outside the block grid are ignored
  }
}

bool dt_ok(int d) { return d == SF_DTYPE_F32 || d == SF_DTYPE_BF16; }

// Every block transposed in place order: out[b][c][r] = in[b][r][c] (element size es bytes).
__global__ void __launch_bounds__(kBlock) bsr_transpose_blocks_kernel(const unsigned char* __restrict__ in,
                                                                      unsigned char* __restrict__ out, int64_t n,
                                                                      int es) {
  for (int64_t e = blockIdx.x * (int64_t)kBlock + threadIdx.x; e < n * 256; e += (int64_t)gridDim.x * kBlock) {
    const int64_t b = e >> 8;
    const int w = static_cast<int>(e & 255), r = w >> 4, c = w & 15;
    const unsigned char* src = in + (b * 256 + r * 16 + c) * es;
    unsigned char* dst = out + (b * 256 + c * 16 + r) * es;
    if (es == 2)
      *reinterpret_cast<uint16_t*>(dst) = *reinterpret_cast<const uint16_t*>(src);
    else
      *reinterpret_cast<uint32_t*>(dst) = *reinterpret_cast<const uint32_t*>(src);
  }
}

// map_t[c][r] = map[r][c].
__global__ void __launch_bounds__(kBlock) bsr_transpose_map_kernel(const int32_t* __restrict__ map, int64_t nbr,
                                                                   int64_t nbc, int32_t* __restrict__ map_t) {
  for (int64_t e = blockIdx.x * (int64_t)kBlock + threadIdx.x; e < nbr * nbc; e += (int64_t)gridDim.x * kBlock) {
    const int64_t r = e / nbc, c = e - r * nbc;
    map_t[c * nbr + r] = map[e];
  }
}

}  // namespace
}  // namespace sf

using namespace sf;

extern "C" int sf_bsr_count(const void* W, int w_dtype, const void* mask, int mask_dtype, int64_t rows, int64_t cols,
                            int block_size, uint8_t* flags, int32_t* counts, void* stream) {
  SF_CHECK_ARG(dt_ok(w_dtype) && dt_ok(mask_dtype), "bad dtype");
  SF_CHECK_ARG(block_size > 0 && rows >= 0 && cols >= 0, "bad shape");
  SF_CHECK_ARG(rows % block_size == 0 && cols % block_size == 0, "weight shape must be a multiple of the block size");
  const int64_t nbr = rows / block_size, nbc = cols / block_size;
  if (nbr == 0 || nbc == 0) return SF_OK;
  SF_CHECK_ARG(W && mask && flags && counts, "null tensor");
  const int prod_dt = (w_dtype == SF_DTYPE_F32 || mask_dtype == SF_DTYPE_F32) ? SF_DTYPE_F32 : SF_DTYPE_BF16;
  bsr_count_kernel<<<static_cast<unsigned>(nbr), kBlock, 0, static_cast<hipStream_t>(stream)>>>(
      W, w_dtype, mask, mask_dtype, cols, nbc, block_size, prod_dt, flags, counts);
  return launch_status("sf_bsr_count");
}

extern "C" int sf_bsr_scan(const int32_t* counts, int64_t nbr, int32_t* row_ptr, void* stream) {
  SF_CHECK_ARG(nbr >= 0 && row_ptr && (nbr == 0 || counts), "bad arguments");
  bsr_scan_kernel<<<1, kBlock, 0, static_cast<hipStream_t>(stream)>>>(counts, nbr, row_ptr);
  return launch_status("sf_bsr_scan");
}

extern "C" int sf_bsr_fill(const void* W, int w_dtype, const void* mask, int mask_dtype, int64_t rows, int64_t cols,
                           int block_size, const uint8_t* flags, const int32_t* row_ptr, int32_t* col_idx,
                           void* blocks, int blocks_dtype, int32_t* block_map, void* stream) {
  SF_CHECK_ARG(dt_ok(w_dtype) && dt_ok(mask_dtype) && dt_ok(blocks_dtype), "bad dtype");
  SF_CHECK_ARG(block_size > 0 && rows % block_size == 0 && cols % block_size == 0, "bad shape");
  const int64_t nbr = rows / block_size, nbc = cols / block_size;
  if (nbr == 0 || nbc == 0) return SF_OK;
  SF_CHECK_ARG(W && mask && flags && row_ptr && blocks, "null tensor");
  const int prod_dt = (w_dtype == SF_DTYPE_F32 || mask_dtype == SF_DTYPE_F32) ? SF_DTYPE_F32 : SF_DTYPE_BF16;
  bsr_fill_kernel<<<static_cast<unsigned>(nbr), kBlock, 0, static_cast<hipStream_t>(stream)>>>(
      W, w_dtype, mask, mask_dtype, cols, nbc, block_size, prod_dt, flags, row_ptr, col_idx, blocks, blocks_dtype,
      block_map);
  return launch_status("sf_bsr_fill");
}

extern "C" int sf_bsr_block_map(const int32_t* row_ptr, const int32_t* col_idx, int64_t nbr, int64_t nbc,
                                int32_t* block_map, void* stream) {
  SF_CHECK_ARG(nbr >= 0 && nbc >= 0, "bad shape");
  if (nbr == 0 || nbc == 0) return SF_OK;
  SF_CHECK_ARG(row_ptr && block_map, "null tensor");
  hipStream_t st = static_cast<hipStream_t>(stream);
  bsr_map_clear_kernel<<<elementwise_grid(nbr * nbc, kBlock), kBlock, 0, st>>>(block_map, nbr * nbc);
  bsr_map_fill_kernel<<<static_cast<unsigned>(nbr), kBlock, 0, st>>>(row_ptr, col_idx, nbr, nbc, block_map);
  return launch_status("sf_bsr_block_map");
}

extern "C" int sf_bsr_transpose(const void* blocks, int dtype, int64_t nblocks, const int32_t* block_map, int64_t nbr,
                                int64_t nbc, void* blocks_t, int32_t* block_map_t, void* stream) {
  SF_CHECK_ARG(nblocks >= 0 && nbr >= 0 && nbc >= 0, "bad shape");
  SF_CHECK_ARG(dtype == SF_DTYPE_F32 || dtype == SF_DTYPE_BF16, "bad dtype %d", dtype);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (nblocks > 0) {
    SF_CHECK_ARG(blocks && blocks_t, "null tensor");
    bsr_transpose_blocks_kernel<<<elementwise_grid(nblocks * 256, kBlock), kBlock, 0, st>>>(
        static_cast<const unsigned char*>(blocks), static_cast<unsigned char*>(blocks_t), nblocks,
        dtype == SF_DTYPE_F32 ? 4 : 2);
  }
  if (nbr > 0 && nbc > 0) {
    SF_CHECK_ARG(block_map && block_map_t, "null tensor");
    bsr_transpose_map_kernel<<<elementwise_grid(nbr * nbc, kBlock), kBlock, 0, st>>>(block_map, nbr, nbc, block_map_t);
  }
  return launch_status("sf_bsr_transpose");
}
