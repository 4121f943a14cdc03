// Fused mask-aware AdamW step (K10) on gfx950.
//
// One memory-bound pass per parameter tensor replaces the ~10 PyTorch ops
// per parameter of AdamW.step (legacy/adamw.py:79-174).  Per element, in the
// reference's op order and f32 arithmetic (each tensor op rounds to its
// result dtype; torch's add(alpha=) and addcmul are fused multiply-adds on
// the CPU, addcdiv is w + (value * y) / z with separate roundings):
//
//   p  <- p * (1 - lr wd)                                   (:85)
//   g  <- g + decay * (p * (1 - mask))        if mask       (:98-109)
//   m  <- m b1 + (1 - b1) g                                  (:151)
//   v  <- v b2 + ((1 - b2) g) g                              (:152)
//   vmax <- max(vmax, v)                      if amsgrad     (:153-155)
//   d  <- sqrt(v or vmax) / sqrt(bc2) + eps                  (:157-159)
//   p  <- p + (-lr / bc1) m / d                              (:161-163)
//   p  <- p - lr * (l1 sign(p) / d)           if l1 > 0, mask, 2-D (:171-174)
//
// Optionally the updated parameter is also written as a bf16 copy (an f32
// master parameter with the bf16 weight the GEMMs read).  Each thread owns
// 4 consecutive elements; 16-byte loads when every operand allows them.

#include "sf_common.hpp"

namespace sf {
namespace {

constexpr int kBlock = 256;

__device__ __forceinline__ float rnd(float x, int dtype) { return dtype == SF_DTYPE_BF16 ? round_bf16(x) : x; }

struct AdamArgs {
  void* p;
  const void* g;
  void* m;
  void* v;
  void* vmax;
  const void* mask;
  void* pcopy;
  int64_t n;
  int p_dt, g_dt, s_dt, m_dt;
  float c_wd;       // 1 - lr * wd
  float decay;      // SR-STE masked decay
  float b1, omb1;   // beta1, 1 - beta1
  float b2, omb2;   // beta2, 1 - beta2
  float sqrt_bc2;   // sqrt(1 - beta2^step)
  float eps;
  float neg_ss;     // -lr / (1 - beta1^step)
  float l1;         // adaptive L1 strength (0: off)
  float neg_lr;     // -lr
  int amsgrad;
};

__device__ __forceinline__ int promote(int a, int b) {
  return (a == SF_DTYPE_F32 || b == SF_DTYPE_F32) ? SF_DTYPE_F32 : SF_DTYPE_BF16;
}

template <int PD, int SD>
__device__ __forceinline__ void adam_element(const AdamArgs& a, float& p, float g, float& m, float& v, float& vmax,
                                             float mask, bool has_mask) {
  p = rnd(p * a.c_wd, PD);
  if (has_mask) {
    const int tdt = promote(PD, a.m_dt);  // dtype of p * (1 - mask)
    const float t = rnd(p * rnd(1.0f - mask, a.m_dt), tdt);
    g = rnd(fmaf(t, a.decay, g), promote(a.g_dt, tdt));
  }
  m = rnd(m * a.b1, SD);
  m = rnd(fmaf(g, a.omb1, m), SD);
  v = rnd(v * a.b2, SD);
  v = rnd(fmaf(a.omb2 * g, g, v), SD);
  float vv = v;
  if (a.amsgrad) {
    vmax = fmaxf(vmax, v);
    vv = vmax;
  }
  const float d = rnd(rnd(rnd(sqrtf(vv), SD) / a.sqrt_bc2, SD) + a.eps, SD);
  p = rnd(p + (a.neg_ss * m) / d, PD);
  if (a.l1 > 0.0f && has_mask) {
    const float sg = p > 0.0f ? 1.0f : (p < 0.0f ? -1.0f : p);  // torch.sign (NaN stays NaN)
    const float lt = rnd(rnd(a.l1 * sg, PD) / d, PD);
    p = rnd(fmaf(lt, a.neg_lr, p), PD);
  }
}

typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// 4 consecutive elements as f32: one 16-byte (f32) or 8-byte (bf16) access
// when `vec`, element by element (cnt of them) otherwise.  NT: non-temporal
// vector accesses (the multi-tensor step streams the whole optimizer arena once).
template <bool NT = false>
__device__ __forceinline__ void ld4(const void* b, int64_t i0, int dt, bool vec, int cnt, float o[4]) {
  if (vec) {
    if (dt == SF_DTYPE_F32) {
      const f32x4_t* q = reinterpret_cast<const f32x4_t*>(static_cast<const float*>(b) + i0);
      const f32x4_t x = NT ? __builtin_nontemporal_load(q) : *q;
      o[0] = x.x; o[1] = x.y; o[2] = x.z; o[3] = x.w;
    } else {
      const u32x2_t* q = reinterpret_cast<const u32x2_t*>(static_cast<const uint16_t*>(b) + i0);
      const u32x2_t x = NT ? __builtin_nontemporal_load(q) : *q;
      o[0] = bf16_to_f32(x.x & 0xffffu); o[1] = bf16_to_f32(x.x >> 16);
      o[2] = bf16_to_f32(x.y & 0xffffu); o[3] = bf16_to_f32(x.y >> 16);
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) o[j] = j < cnt ? load_as_f32(b, i0 + j, dt) : 0.0f;
}

template <bool NT = false>
__device__ __forceinline__ void st4(void* b, int64_t i0, int dt, bool vec, int cnt, const float v[4]) {
  if (vec) {
    if (dt == SF_DTYPE_F32) {
      f32x4_t* q = reinterpret_cast<f32x4_t*>(static_cast<float*>(b) + i0);
      const f32x4_t x{v[0], v[1], v[2], v[3]};
      if constexpr (NT)
        __builtin_nontemporal_store(x, q);
      else
        *q = x;
    } else {
      u32x2_t x;
      x.x = static_cast<uint32_t>(f32_to_bf16(v[0])) | (static_cast<uint32_t>(f32_to_bf16(v[1])) << 16);
      x.y = static_cast<uint32_t>(f32_to_bf16(v[2])) | (static_cast<uint32_t>(f32_to_bf16(v[3])) << 16);
      u32x2_t* q = reinterpret_cast<u32x2_t*>(static_cast<uint16_t*>(b) + i0);
      if constexpr (NT)
        __builtin_nontemporal_store(x, q);
      else
        *q = x;
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (j < cnt) store_from_f32(b, i0 + j, dt, v[j]);
}

template <int PD, int SD>
__global__ void __launch_bounds__(kBlock) adamw_kernel(AdamArgs a, bool aligned) {
  const int64_t nvec = (a.n + 3) / 4;
  const bool has_mask = a.mask != nullptr;
  for (int64_t iv = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; iv < nvec;
       iv += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i0 = iv * 4;
    const int cnt = a.n - i0 >= 4 ? 4 : static_cast<int>(a.n - i0);
    const bool vec = aligned && cnt == 4;
    float p[4], g[4], m[4], v[4], x[4] = {0, 0, 0, 0}, mk[4] = {0, 0, 0, 0};
    ld4(a.p, i0, PD, vec, cnt, p);
    ld4(a.g, i0, a.g_dt, vec, cnt, g);
    ld4(a.m, i0, SD, vec, cnt, m);
    ld4(a.v, i0, SD, vec, cnt, v);
    if (a.amsgrad) ld4(a.vmax, i0, SD, vec, cnt, x);
    if (has_mask) ld4(a.mask, i0, a.m_dt, vec, cnt, mk);
#pragma unroll
    for (int j = 0; j < 4; ++j) adam_element<PD, SD>(a, p[j], g[j], m[j], v[j], x[j], mk[j], has_mask);
    st4(a.p, i0, PD, vec, cnt, p);
    st4(a.m, i0, SD, vec, cnt, m);
    st4(a.v, i0, SD, vec, cnt, v);
    if (a.amsgrad) st4(a.vmax, i0, SD, vec, cnt, x);
    if (a.pcopy) st4(a.pcopy, i0, SF_DTYPE_BF16, vec, cnt, p);
  }
}

bool dt_ok(int d) { return d == SF_DTYPE_F32 || d == SF_DTYPE_BF16; }

// ---------------------------------------------------------------------------
// Multi-tensor step: one launch updates up to kMultiMax tensors.  The tensor
// table travels in the kernel arguments (no device table, nothing to copy or
// allocate); workgroup b belongs to the tensor i with first[i] <= b < first[i+1],
// found by a binary search over kernel-argument (scalar) loads, and updates
// that tensor's elements [(b - first[i]) * kMultiChunk, +kMultiChunk) with one
// 4-element vector per thread, as the single-tensor kernel does.
// ---------------------------------------------------------------------------
constexpr int kMultiMax = 40;               // tensors per launch (keeps the arguments under 4 KiB)
constexpr int kMultiChunk = 4 * kBlock;     // elements per workgroup

struct MultiTensor {
  void* p;
  const void* g;
  void* m;
  void* v;
  void* vmax;
  const void* mask;
  void* pcopy;
  int64_t n;
  int g_dt, m_dt;
  float l1;      // adaptive L1 strength of this tensor (0: off: no mask or < 2-D)
  int aligned;   // every operand allows the vector accesses
};

struct MultiArgs {
  AdamArgs a;                      // shared scalars (pointers and n unused)
  int count;
  int64_t first[kMultiMax + 1];    // first workgroup of each tensor; first[count] = grid
  MultiTensor t[kMultiMax];
};

template <int PD, int SD>
__global__ void __launch_bounds__(kBlock) adamw_multi_kernel(MultiArgs ma) {
  const int64_t b = blockIdx.x;
  int lo = 0, hi = ma.count - 1;  // last i with first[i] <= b (uniform across the workgroup)
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (ma.first[mid] <= b) lo = mid; else hi = mid - 1;
  }
  const MultiTensor& t = ma.t[lo];
  AdamArgs a = ma.a;
  a.g_dt = t.g_dt;
  a.m_dt = t.m_dt;
  a.l1 = t.l1;
  a.p = t.p;
  a.g = t.g;
  a.m = t.m;
  a.v = t.v;
  a.vmax = t.vmax;
  a.mask = t.mask;
  a.pcopy = t.pcopy;
  const bool has_mask = t.mask != nullptr;
  const int64_t i0 = (b - ma.first[lo]) * kMultiChunk + 4 * (int64_t)threadIdx.x;
  if (i0 >= t.n) return;
  const int cnt = t.n - i0 >= 4 ? 4 : static_cast<int>(t.n - i0);
  const bool vec = t.aligned && cnt == 4;
  float p[4], g[4], m[4], v[4], x[4] = {0, 0, 0, 0}, mk[4] = {0, 0, 0, 0};
  ld4<true>(t.p, i0, PD, vec, cnt, p);
  ld4<true>(t.g, i0, t.g_dt, vec, cnt, g);
  ld4<true>(t.m, i0, SD, vec, cnt, m);
  ld4<true>(t.v, i0, SD, vec, cnt, v);
  if (a.amsgrad) ld4<true>(t.vmax, i0, SD, vec, cnt, x);
  if (has_mask) ld4<true>(t.mask, i0, t.m_dt, vec, cnt, mk);
#pragma unroll
  for (int j = 0; j < 4; ++j) adam_element<PD, SD>(a, p[j], g[j], m[j], v[j], x[j], mk[j], has_mask);
  st4<true>(t.p, i0, PD, vec, cnt, p);
  st4<true>(t.m, i0, SD, vec, cnt, m);
  st4<true>(t.v, i0, SD, vec, cnt, v);
  if (a.amsgrad) st4<true>(t.vmax, i0, SD, vec, cnt, x);
  if (t.pcopy) st4<true>(t.pcopy, i0, SF_DTYPE_BF16, vec, cnt, p);
}

// Shared scalars of one step from the host hyper-parameters (the reference's Python doubles,
// then the f32 scalar operand of each tensor op).
void fill_scalars(const sf_adamw_params* hp, AdamArgs* a) {
  a->c_wd = static_cast<float>(1.0 - hp->lr * hp->weight_decay);
  a->decay = static_cast<float>(hp->decay);
  a->b1 = static_cast<float>(hp->beta1);
  a->omb1 = static_cast<float>(1.0 - hp->beta1);
  a->b2 = static_cast<float>(hp->beta2);
  a->omb2 = static_cast<float>(1.0 - hp->beta2);
  const double bc1 = 1.0 - pow(hp->beta1, static_cast<double>(hp->step));
  const double bc2 = 1.0 - pow(hp->beta2, static_cast<double>(hp->step));
  a->sqrt_bc2 = static_cast<float>(sqrt(bc2));
  a->eps = static_cast<float>(hp->eps);
  a->neg_ss = static_cast<float>(-(hp->lr / bc1));
  a->neg_lr = static_cast<float>(-hp->lr);
  a->amsgrad = hp->amsgrad;
}

int check_hp(const sf_adamw_params* hp) {
  SF_CHECK_ARG(hp != nullptr, "null sf_adamw_params");
  SF_CHECK_ARG(hp->step >= 1, "step must be >= 1 (the count after this step)");
  SF_CHECK_ARG(hp->lr >= 0.0 && hp->eps >= 0.0, "Invalid learning rate or epsilon value");
  SF_CHECK_ARG(hp->beta1 >= 0.0 && hp->beta1 < 1.0 && hp->beta2 >= 0.0 && hp->beta2 < 1.0,
               "Invalid beta parameter");
  return SF_OK;
}

bool al_ok(const void* q, int dt) {
  return !q || (reinterpret_cast<uintptr_t>(q) % (dt == SF_DTYPE_F32 ? 16 : 8)) == 0;
}

}  // namespace
}  // namespace sf

using namespace sf;

extern "C" int sf_adamw_step(void* param, int param_dtype, const void* grad, int grad_dtype, void* exp_avg,
                             void* exp_avg_sq, void* max_exp_avg_sq, int state_dtype, const void* mask, int mask_dtype,
                             void* param_bf16_copy, int64_t n, const sf_adamw_params* hp, void* stream) {
  if (int rc = check_hp(hp)) return rc;
  SF_CHECK_ARG(n >= 0, "negative element count");
  SF_CHECK_ARG(dt_ok(param_dtype) && dt_ok(grad_dtype) && dt_ok(state_dtype) && (!mask || dt_ok(mask_dtype)),
               "bad dtype");
  if (n == 0) return SF_OK;
  SF_CHECK_ARG(param && grad && exp_avg && exp_avg_sq, "null tensor");
  SF_CHECK_ARG(!hp->amsgrad || max_exp_avg_sq, "amsgrad needs max_exp_avg_sq");
  AdamArgs a;
  a.p = param;
  a.g = grad;
  a.m = exp_avg;
  a.v = exp_avg_sq;
  a.vmax = hp->amsgrad ? max_exp_avg_sq : nullptr;
  a.mask = mask;
  a.pcopy = param_bf16_copy;
  a.n = n;
  a.p_dt = param_dtype;
  a.g_dt = grad_dtype;
  a.s_dt = state_dtype;
  a.m_dt = mask ? mask_dtype : SF_DTYPE_F32;
  fill_scalars(hp, &a);
  a.l1 = mask && hp->apply_l1 ? static_cast<float>(hp->l1) : 0.0f;
  hipStream_t st = static_cast<hipStream_t>(stream);
  // one 4-element vector per thread (no grid-stride reuse of a thread): measured faster than a
  // capped grid for this 10-stream read / write mix
  const int64_t blocks = ceil_div((n + 3) / 4, kBlock);
  const int grid = static_cast<int>(blocks < (1ll << 30) ? blocks : (1ll << 30));
  const bool aligned = al_ok(param, param_dtype) && al_ok(grad, grad_dtype) && al_ok(exp_avg, state_dtype) &&
                       al_ok(exp_avg_sq, state_dtype) && al_ok(a.vmax, state_dtype) && al_ok(mask, a.m_dt) &&
                       al_ok(param_bf16_copy, SF_DTYPE_BF16);
  if (param_dtype == SF_DTYPE_F32 && state_dtype == SF_DTYPE_F32)
    adamw_kernel<SF_DTYPE_F32, SF_DTYPE_F32><<<grid, kBlock, 0, st>>>(a, aligned);
  else if (param_dtype == SF_DTYPE_F32)
    adamw_kernel<SF_DTYPE_F32, SF_DTYPE_BF16><<<grid, kBlock, 0, st>>>(a, aligned);
  else if (state_dtype == SF_DTYPE_F32)
    adamw_kernel<SF_DTYPE_BF16, SF_DTYPE_F32><<<grid, kBlock, 0, st>>>(a, aligned);
  else
    adamw_kernel<SF_DTYPE_BF16, SF_DTYPE_BF16><<<grid, kBlock, 0, st>>>(a, aligned);
  return launch_status("sf_adamw_step");
}

extern "C" int sf_adamw_step_multi(const sf_adamw_tensor* tensors, int count, int param_dtype, int state_dtype,
                                   const sf_adamw_params* hp, void* stream) {
  if (int rc = check_hp(hp)) return rc;
  SF_CHECK_ARG(count >= 0 && (count == 0 || tensors), "bad tensor list");
  SF_CHECK_ARG(dt_ok(param_dtype) && dt_ok(state_dtype), "bad dtype");
  for (int i = 0; i < count; ++i) {
    const sf_adamw_tensor& t = tensors[i];
    SF_CHECK_ARG(t.n >= 0, "tensor %d: negative element count", i);
    SF_CHECK_ARG(dt_ok(t.grad_dtype) && (!t.mask || dt_ok(t.mask_dtype)), "tensor %d: bad dtype", i);
    if (t.n == 0) continue;
    SF_CHECK_ARG(t.param && t.grad && t.exp_avg && t.exp_avg_sq, "tensor %d: null tensor", i);
    SF_CHECK_ARG(!hp->amsgrad || t.max_exp_avg_sq, "tensor %d: amsgrad needs max_exp_avg_sq", i);
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  MultiArgs ma;
  memset(&ma, 0, sizeof(ma));
  fill_scalars(hp, &ma.a);
  auto flush = [&]() -> int {
    if (ma.count == 0) return SF_OK;
    const int64_t grid = ma.first[ma.count];
    SF_CHECK_ARG(grid < (1ll << 31), "launch of %lld workgroups exceeds the grid limit", (long long)grid);
    if (param_dtype == SF_DTYPE_F32 && state_dtype == SF_DTYPE_F32)
      adamw_multi_kernel<SF_DTYPE_F32, SF_DTYPE_F32><<<static_cast<unsigned>(grid), kBlock, 0, st>>>(ma);
    else if (param_dtype == SF_DTYPE_F32)
      adamw_multi_kernel<SF_DTYPE_F32, SF_DTYPE_BF16><<<static_cast<unsigned>(grid), kBlock, 0, st>>>(ma);
    else if (state_dtype == SF_DTYPE_F32)
      adamw_multi_kernel<SF_DTYPE_BF16, SF_DTYPE_F32><<<static_cast<unsigned>(grid), kBlock, 0, st>>>(ma);
    else
      adamw_multi_kernel<SF_DTYPE_BF16, SF_DTYPE_BF16><<<static_cast<unsigned>(grid), kBlock, 0, st>>>(ma);
    ma.count = 0;
    ma.first[0] = 0;
    return launch_status("sf_adamw_step_multi");
  };
  constexpr int64_t kGridCap = (1ll << 31) - kMultiChunk;  // a launch stays under the grid limit
  for (int i = 0; i < count; ++i) {
    const sf_adamw_tensor& src = tensors[i];
    if (src.n == 0) continue;
    const int64_t blocks = ceil_div(src.n, static_cast<int64_t>(kMultiChunk));
    if (ma.count == kMultiMax || ma.first[ma.count] + blocks > kGridCap)
      if (int rc = flush()) return rc;
    SF_CHECK_ARG(blocks <= kGridCap, "tensor %d of %lld elements exceeds the grid limit", i, (long long)src.n);
    MultiTensor& t = ma.t[ma.count];
    t.p = src.param;
    t.g = src.grad;
    t.m = src.exp_avg;
    t.v = src.exp_avg_sq;
    t.vmax = hp->amsgrad ? src.max_exp_avg_sq : nullptr;
    t.mask = src.mask;
    t.pcopy = src.param_bf16_copy;
    t.n = src.n;
    t.g_dt = src.grad_dtype;
    t.m_dt = src.mask ? src.mask_dtype : SF_DTYPE_F32;
    t.l1 = src.mask && src.apply_l1 ? static_cast<float>(hp->l1) : 0.0f;
    t.aligned = al_ok(src.param, param_dtype) && al_ok(src.grad, src.grad_dtype) && al_ok(src.exp_avg, state_dtype) &&
                al_ok(src.exp_avg_sq, state_dtype) && al_ok(t.vmax, state_dtype) && al_ok(src.mask, t.m_dt) &&
                al_ok(src.param_bf16_copy, SF_DTYPE_BF16);
    ma.first[ma.count + 1] = ma.first[ma.count] + blocks;
    ++ma.count;
  }
  return flush();
}
