/*
 * sparseforge_amd — C ABI of the MI355X (gfx950) sparse-training hot path.
 *
 * Every entry point takes plain device pointers, element counts and a
 * hipStream_t passed as `void*` (NULL = the legacy default stream), enqueues
 * its kernels on that stream and returns without synchronising.  Tensors are
 * dense and row-major ([rows, cols] with row stride == cols) unless stated.
 * Nothing here allocates device memory: entry points that need scratch
 * take a `workspace` pointer whose minimum size the matching *_workspace_size
 * function reports.  Return value: SF_OK or a negative SF_ERR_* code; the
 * message of the most recent failure on the calling thread is returned by
 * sf_last_error().
 *
 * The reference implementation is Python (liuhanzuo/SparseForge,
 * legacy/sparse_modeling.py, legacy/utils.py, legacy/adamw.py,
 * legacy/triton_block_sparse.py); each declaration names the reference lines
 * whose behaviour it reproduces.  A ctypes binding of this header is
 * sparseforge_amd/_lib.py.
 */
#ifndef SPARSEFORGE_AMD_H
#define SPARSEFORGE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
#define SF_OK 0
#define SF_ERR_INVALID (-1)     /* bad argument (shape, dtype, null pointer) */
#define SF_ERR_UNSUPPORTED (-2) /* valid in the reference, not built on device */
#define SF_ERR_HIP (-3)         /* HIP runtime / launch failure */

/* ---- element types ----------------------------------------------------- */
#define SF_DTYPE_F32 0
#define SF_DTYPE_BF16 1
#define SF_DTYPE_U8 2 /* byte and-mask (0x00 / 0xFF per element); sf_effective_mask output only */

/* ---- hard-mask projections (SparseLinear._hard_mask_from_soft) --------- */
#define SF_HARD_NONE 0         /* all ones                       (:523-524)  */
#define SF_HARD_THRESHOLD 1    /* soft > 0.5                     (:526-531)  */
#define SF_HARD_NM_TAIL_KEEP 2 /* top-N of each M-group, tail columns = 1 (nm_2_4, :578-603) */
#define SF_HARD_NM_STRICT 3    /* top-N of each M-group, cols % M == 0 required (structured, :720-735) */

/* ---- importance metrics (compute_gate_target scores, :1041-1079) ------- */
#define SF_METRIC_MAGNITUDE 0
#define SF_METRIC_HESSIAN_OBD 1
#define SF_METRIC_HESSIAN_RATIO 2
#define SF_METRIC_HESSIAN 3
#define SF_METRIC_WANDA 4
#define SF_METRIC_MOVEMENT 5
#define SF_METRIC_WEIGHT_SQUARED 6 /* W * W in W's dtype: hessian_obd when hessian_diag is a placeholder
                                      (:1049-1055; legacy/utils.py:506-511) */

/* ---- gate-target forms ------------------------------------------------- */
#define SF_GATE_UNSTRUCTURED 0 /* sigmoid((z - tau) / (T + 1e-8)), global tau  (:1097-1162) */
#define SF_GATE_STRUCTURED 1   /* sigmoid((z - tau_g) / (T + 1e-8)), tau_g = N-th largest of group (:1164-1185) */
#define SF_GATE_STRUCTURED_EXACT 2 /* top-N scatter of ones (:1176-1182) */
#define SF_GATE_ZSCORE 3 /* z = ((s - mu) / sigma) in the score dtype: the input the block_sparse gate
                            pools per block (:1083-1088, :1122-1131); sf_gate_target only */

/* ---- penalty pull applied to G inside update_mask (:1291-1573) ---------- */
#define SF_PENALTY_NONE 0
#define SF_PENALTY_MID 1            /* G -= c * (1 - 2 m)                 (:1567-1570) */
#define SF_PENALTY_NM_2_4 2         /* G -= c * (m - top2(G)), tail target 1 (:1350-1393) */
#define SF_PENALTY_STRUCTURED_TOPN 3 /* G -= c * (m - topN(G)), cols % M == 0 (:1531-1565) */
#define SF_PENALTY_TARGET 4 /* G -= c * (m - target), target given: the block16 / block_sparse16 /
                               block_sparse32 modes (:1298-1347, :1395-1529); sf_apply_gate only */

/* ---- per-block statistics (bs x bs tiles of the fully covered core) ---- */
#define SF_BLOCK_MEAN 0 /* mean(x)            (_blockify_tensor :495-497; block penalty :1436-1438) */
#define SF_BLOCK_RMS 1  /* sqrt(mean(x * x))  (block_sparse hard mask :632-633; block gate :1131)   */

const char* sf_last_error(void);
int sf_version(void);

/*
 * Hard projection of a soft mask.  Replaces SparseLinear._hard_mask_from_soft
 * (legacy/sparse_modeling.py:510-735) for hard types none / unstructured /
 * nm_2_4 / structured.  Ties inside a group resolve exactly as torch.topk on
 * the CPU does.  Device support: m_group == 4, 1 <= n_keep <= 3.
 * soft: [rows, cols] (soft_dtype); hard: [rows, cols] (hard_dtype), values {0, 1}.
 */
int sf_hard_mask(const void* soft, int soft_dtype, void* hard, int hard_dtype, int64_t rows,
                 int64_t cols, int kind, int n_keep, int m_group, void* stream);

/*
 * Parameters of one gate-target / mask-update call.  Host scalars are the
 * values SparseLinear computes from its config and the step
 * (legacy/sparse_modeling.py:932-985, :1242-1666).
 */
typedef struct sf_mask_params {
  int64_t rows, cols;
  int metric;          /* SF_METRIC_* */
  int gate;            /* SF_GATE_* */
  int n_keep, m_group; /* N, M of the structured gate and of topN penalties */
  int hard_kind;       /* SF_HARD_* used for the flip count */
  int hard_n, hard_m;  /* N, M of that hard projection */
  int penalty;         /* SF_PENALTY_* (only when penalty_coef != 0) */
  int has_frozen;      /* frozen_mask_flags is a full [rows, cols] tensor */
  int snap_high;       /* step >= 2000: freeze_high snaps to 1 (:1632-1636) */
  int score_dtype;     /* dtype the reference holds scores in (promotion of W, H) */
  float temperature;   /* _temperature(step) */
  float eps_metric;    /* 1e-8 */
  float movement_temp; /* cfg.temperature (movement metric) */
  float beta_struct;   /* _beta_structural(step) */
  float mask_lr;       /* a of the EMA */
  float penalty_coef;  /* mask_penalty_lr * lambda_mid */
  float binarize;      /* mask_binarize_decay */
  float freeze_low, freeze_high;
  int apply_freeze;    /* freeze_low > 0 or freeze_high < 1 */
} sf_mask_params;

/*
 * Workspace bytes needed by sf_score_stats / sf_gate_target / sf_update_mask
 * for a [rows, cols] layer and a tau sample of `sample_size` elements.
 */
size_t sf_mask_workspace_size(int64_t rows, int64_t cols, int64_t sample_size);

/*
 * Global mean and population std (+1e-6) of the layer's scores
 * (legacy/sparse_modeling.py:1083-1088).  stats_out: device float[2] = {mu, sigma}.
 * W: weight, H: hessian_diag (or NULL), aux: scaler_row [cols] for wanda or
 * grad_ema [rows, cols] for movement (or NULL).
 */
int sf_score_stats(const sf_mask_params* p, const void* W, int w_dtype, const void* H, int h_dtype,
                   const void* aux, int aux_dtype, float* stats_out, void* workspace,
                   size_t workspace_bytes, void* stream);

/*
 * Unstructured threshold tau = torch.quantile(z[sample_idx], q) with linear
 * interpolation (legacy/sparse_modeling.py:987-1015).  sample_idx: device
 * int64[sample_size] (NULL: use every element, sample_size must equal
 * rows*cols).  stats: device {mu, sigma} from sf_score_stats.  tau_out: device float[1].
 */
int sf_tau_quantile(const sf_mask_params* p, const void* W, int w_dtype, const void* H, int h_dtype,
                    const void* aux, int aux_dtype, const float* stats, const int64_t* sample_idx,
                    int64_t sample_size, float q, float* tau_out, void* workspace,
                    size_t workspace_bytes, void* stream);

/*
 * sf_tau_quantile without a workspace argument: allocates nothing (no
 * hipMalloc, no allocating library call), for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid allocation).  No counterpart in the reference.  The scratch
 * lives in a static device array of the library (about 4.2 MiB per GPU, held
 * until the process ends), one copy per GPU; the device is the stream's
 * (NULL stream: the current device).  Samples above SF_TAU_NOALLOC_MAX_SAMPLE
 * elements are rejected with SF_ERR_INVALID.  Every call on one GPU shares
 * that scratch: calls that overlap on one GPU (different streams without
 * ordering between them) race and must not be issued.  Results equal
 * sf_tau_quantile's for the same inputs.
 */
#define SF_TAU_NOALLOC_MAX_SAMPLE (1 << 20)
int sf_tau_quantile_noalloc(const sf_mask_params* p, const void* W, int w_dtype, const void* H, int h_dtype,
                            const void* aux, int aux_dtype, const float* stats, const int64_t* sample_idx,
                            int64_t sample_size, float q, float* tau_out, void* stream);

/*
 * Sample indices for the tau quantile: idx[i] uniform in [0, n) from the
 * counter-based generator (seed, i).  Replaces torch.randint at :993.
 */
int sf_sample_indices(int64_t* idx, int64_t sample_size, int64_t n, uint64_t seed, void* stream);

/*
 * Sorted sample indices for the tau quantile: `count` independent lists of
 * sample_size indices, list c (at idx + c * sample_size) distributed as
 * sample_size independent uniform draws from [0, n[c]) -- torch.randint's
 * law at :993 -- and delivered in non-decreasing order (the quantile of a
 * sample does not depend on its order).  seeds[c] seeds list c's counter
 * generator; n and seeds are host arrays.  sf_update_mask_multi reads a
 * sorted sample's keys from its statistics pass instead of gathering them.
 * workspace: sf_sample_indices_sorted_workspace_size(sample_size, count)
 * bytes.  sample_size < 2^28.
 */
size_t sf_sample_indices_sorted_workspace_size(int64_t sample_size, int count);
int sf_sample_indices_sorted(int64_t* idx, int64_t sample_size, const int64_t* n, const uint64_t* seeds,
                             int count, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Gate target G (compute_gate_target, legacy/sparse_modeling.py:1018-1239):
 * scores -> z-norm -> gate form -> beta structural mix -> frozen override.
 * G: [rows, cols] in g_dtype.  stats / tau: device scalars from the calls above
 * (tau unused for structured gates).  mask and frozen are read only for the
 * frozen override.
 */
int sf_gate_target(const sf_mask_params* p, const void* W, int w_dtype, const void* H, int h_dtype,
                   const void* aux, int aux_dtype, const void* mask, int mask_dtype,
                   const void* frozen, int frozen_dtype, const float* stats, const float* tau, void* G,
                   int g_dtype, void* stream);

/*
 * Fused periodic mask update (SparseLinear.update_mask body after the
 * step gating, legacy/sparse_modeling.py:1288-1661): gate target, penalty
 * pull + clamp, binarisation push, EMA mask <- clamp((1-a) m + a G), freeze
 * snaps and flags, and the hard-mask flip count.  One read of W/H/mask, one
 * write of mask.  flips: device int64[1], incremented (caller zeroes it).
 */
int sf_update_mask(const sf_mask_params* p, const void* W, int w_dtype, const void* H, int h_dtype,
                   const void* aux, int aux_dtype, void* mask, int mask_dtype, void* frozen,
                   int frozen_dtype, const float* stats, const float* tau, int64_t* flips,
                   void* stream);

/*
 * One layer of sf_update_mask_multi: its operands (as sf_update_mask takes
 * them) and its outputs.
 */
typedef struct sf_mask_layer {
  int64_t rows, cols;
  const void* W;
  const void* H;              /* hessian_diag, or NULL */
  const void* aux;            /* scaler_row / grad_ema, or NULL */
  void* mask;
  void* frozen;               /* frozen flags (when p->has_frozen), or NULL */
  const int64_t* sample_idx;  /* tau sample indices, or NULL for every element */
  int64_t sample_size;        /* tau sample size (rows * cols when sample_idx is NULL) */
  float* stats;               /* out: device float[2] {mu, sigma} */
  float* tau;                 /* out: device float[1] (unstructured gate), else may be NULL */
  int64_t* flips;             /* device int64[1], incremented, or NULL */
} sf_mask_layer;

/*
 * Workspace bytes of sf_update_mask_multi over these layers.
 */
size_t sf_update_mask_multi_workspace_size(const sf_mask_layer* layers, int count);

/*
 * The mask update of every SparseLinear of a model in a handful of launches:
 * calculate_model_mask (legacy/utils.py:184-310) calls update_mask
 * (legacy/sparse_modeling.py:1242-1666) layer after layer, and each call here
 * would be sf_score_stats + sf_tau_quantile(q) (unstructured gate) +
 * sf_update_mask.  For layers whose parameters are equal but for their shape
 * (p->rows / p->cols are ignored: each layer brings its own), this runs all
 * three stages of up to 28 layers per launch, and every output (stats, tau,
 * mask, frozen flags, flip counts) equals that of the three single-layer
 * calls bit for bit.  Empty layers are skipped.  `stages` (SF_MULTI_*) picks
 * the stages to run: a stage run alone reads what earlier calls wrote to the
 * layers' stats / tau.
 */
#define SF_MULTI_STATS 1  /* sf_score_stats: layers' stats */
#define SF_MULTI_TAU 2    /* sf_tau_quantile (unstructured gate only): layers' tau */
#define SF_MULTI_UPDATE 4 /* sf_update_mask: masks, frozen flags, flips */
#define SF_MULTI_ALL 7
int sf_update_mask_multi(const sf_mask_params* p, float q, const sf_mask_layer* layers, int count,
                         int stages, int w_dtype, int h_dtype, int aux_dtype, int mask_dtype,
                         int frozen_dtype, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Count of positions whose hard projection differs between two soft masks
 * (legacy/sparse_modeling.py:1659-1661).  flips: device int64[1], incremented.
 */
int sf_hard_flip_count(const void* prev, const void* now, int dtype, int64_t rows, int64_t cols,
                       int kind, int n_keep, int m_group, int64_t* flips, void* stream);

/*
 * Importance scores of one layer (_compute_importance_scores,
 * legacy/utils.py:482-533; the score half of compute_gate_target,
 * legacy/sparse_modeling.py:1041-1079): magnitude |W|, hessian_obd
 * (H + eps) W^2, hessian_ratio |W| / sqrt(H + eps), hessian H, wanda
 * |W| sqrt(scaler + eps), movement |W g| / max(temperature, eps), each
 * reference op rounded to its result dtype, the result rounded to s_dtype.
 * S: [rows, cols].
 */
int sf_importance_scores(const sf_mask_params* p, const void* W, int w_dtype, const void* H, int h_dtype,
                         const void* aux, int aux_dtype, void* S, int s_dtype, void* stream);

/*
 * Joint importance score of a GLU gate/up pair: S = score(gate) + score(up),
 * each from its own layer's metric, eps and operands
 * (_compute_importance_scores, legacy/utils.py:480-533, summed at :415-420),
 * the sum rounded in s_dtype (the promotion of the two score dtypes).  Both
 * layers share the operand dtypes.  S: [rows, cols], written.
 */
int sf_joint_scores(const sf_mask_params* gate_p, const void* gate_W, const void* gate_H,
                    const void* gate_aux, const sf_mask_params* up_p, const void* up_W, const void* up_H,
                    const void* up_aux, int w_dtype, int h_dtype, int aux_dtype, void* S, int s_dtype,
                    void* stream);

/*
 * Joint mask update of a GLU gate/up pair (legacy/utils.py:422-479 with
 * _compute_joint_gate_target :536-613 and _apply_mid_penalty_to_gate
 * :615-643): one pass computes G from the joint score S (z-scored with
 * `stats` of S and rounded in the mask dtype, so p->score_dtype must equal
 * mask_dtype), the gate layer's frozen flags and mask, the penalty against
 * the gate mask (SF_PENALTY_MID or SF_PENALTY_STRUCTURED_TOPN), the
 * binarisation push, then the EMA of BOTH masks with that G.  No freeze step
 * (the reference's joint path has none).  Flip counts use p->hard_kind /
 * hard_n for the gate and up_hard_kind / up_hard_n for the up layer; each
 * counter is device int64[1], incremented (NULL skips it).
 */
int sf_glu_update_masks(const sf_mask_params* p, const void* S, int s_dtype, void* gate_mask,
                        void* up_mask, int mask_dtype, const void* gate_frozen, int frozen_dtype,
                        const float* stats, const float* tau, int up_hard_kind, int up_hard_n,
                        int64_t* gate_flips, int64_t* up_flips, void* stream);

/*
 * dst[c][r] = src[r][c] for a byte mask (src [rows, cols], dst [cols, rows]):
 * the K-major form of the effective byte mask that the input-gradient GEMM
 * reads beside the transposed weight tile (sf_gemm_desc.bmask_kmajor).  No
 * counterpart of its own in the reference; part of the mask application of
 * FusedMaskedLinearSTE.backward (legacy/sparse_modeling.py:113-115).
 */
int sf_transpose_u8(const uint8_t* src, int64_t rows, int64_t cols, uint8_t* dst, void* stream);

/*
 * Block statistic of each bs x bs block (bs = 16 or 32) of the fully covered
 * core [:rows/bs*bs, :cols/bs*bs] of x [rows, cols]: out[br * (cols/bs) + bc]
 * (device float[(rows/bs) * (cols/bs)]), SF_BLOCK_MEAN or SF_BLOCK_RMS.  The
 * sum runs in f64 and is rounded to f32 once (torch sums in f32, so results
 * agree to a few ulp and exactly for blocks of equal elements).  Replaces the
 * tile means of _blockify_tensor (legacy/sparse_modeling.py:488-497), of the
 * block_sparse penalty (:1431-1438) and the block RMS of the block_sparse hard
 * mask (:624-633) and gate (:1126-1131).
 */
int sf_block_stat(const void* x, int x_dtype, int64_t rows, int64_t cols, int bs, int stat, float* out,
                  void* stream);

/*
 * keep[i] = 1.0f for the k largest entries of v[n] (device floats), else 0.0f:
 * the torch.topk(flat, k) + scatter of the block_sparse hard mask
 * (legacy/sparse_modeling.py:641-655, :699-713) and penalty target
 * (:1441-1451).  NaN ranks largest, -0 == +0.  Equal values are kept exactly
 * as torch.topk's CPU kernel keeps them: its selection (std::nth_element, or
 * std::partial_sort when k * 64 <= n, over (value, index) pairs compared by
 * value; GCC libstdc++'s introselect / heap select) is reproduced step for
 * step.  k <= 0: all 0; k >= n: all 1.  workspace: device memory of
 * sf_topk_keep_workspace_size(n) bytes, 16-byte aligned (contents undefined
 * on entry and exit).
 */
size_t sf_topk_keep_workspace_size(int64_t n);
int sf_topk_keep(const float* v, int64_t n, int64_t k, float* keep, void* workspace, size_t workspace_bytes,
                 void* stream);

/*
 * block16 projection: in each 16 x 16 tile of the core of x [rows, cols] the k
 * largest elements become 1 and the rest 0; elements outside the core become
 * 1 (legacy/sparse_modeling.py:537-575 for the hard mask, :1318-1341 for the
 * block16 penalty target).  Ties as sf_topk_keep over the tile's 256 entries
 * in row-major order (torch.topk along the flattened tile).  bs must be 16.  out: [rows, cols] in out_dtype.
 */
int sf_tile_topk(const void* x, int x_dtype, int64_t rows, int64_t cols, int bs, int64_t k, void* out,
                 int out_dtype, void* stream);

/*
 * Expand per-block values over the core of out [rows, cols]:
 *   out = (bvals[block]).to(out dtype), or with tau (device float[1])
 *   out = sigmoid((bvals[block] - *tau) / (temperature + 1e-8)) in f32, then cast
 *   (the block_sparse gate, legacy/sparse_modeling.py:1144-1154).
 * Outside the core: unchanged (edge_write = 0, as _blockify_tensor :505-507)
 * or edge_val (hard masks, targets and G keep 1 there).  Where ov_flags != 0
 * the element takes ov_src instead, cast to the out dtype (the frozen override
 * G[frozen] = mask[frozen], :1227-1229).  Used for blockify (bvals = block
 * means, edge_write 0), block hard masks / targets (bvals = sf_topk_keep
 * flags, edge_val 1) and the block gate.
 */
int sf_block_fill(const float* bvals, int64_t rows, int64_t cols, int bs, const float* tau, float temperature,
                  void* out, int out_dtype, int edge_write, float edge_val, const void* ov_src, int ov_src_dtype,
                  const void* ov_flags, int ov_flags_dtype, void* stream);

/*
 * The update half of update_mask for a gate target G already in memory
 * (p->score_dtype): penalty pull (p->penalty, with SF_PENALTY_TARGET reading
 * `target`), clamp, binarisation push, EMA of `mask` and, with do_freeze, the
 * freeze snaps and flags (legacy/sparse_modeling.py:1291-1642 without the
 * flip count).  The staged path of the block hard types and block penalty
 * modes uses it; blockify and sf_freeze_mask follow when the hard type is
 * block_sparse16/32.
 */
int sf_apply_gate(const sf_mask_params* p, const void* G, const void* target, int target_dtype, void* mask,
                  int mask_dtype, void* frozen, int frozen_dtype, int do_freeze, void* stream);

/*
 * Freeze snaps and flags of update_mask (legacy/sparse_modeling.py:1621-1642)
 * as a pass of its own: after the mask blockify of the block_sparse types.
 */
int sf_freeze_mask(const sf_mask_params* p, void* mask, int mask_dtype, void* frozen, int frozen_dtype,
                   void* stream);

/* ---- effective mask for the masked GEMMs (SparseLinear.forward, :759-771) */
#define SF_EFF_SOFT 0 /* E = mask.to(weight dtype)                                  */
#define SF_EFF_MIX 1  /* E = (hx * mask + (1 - hx) * hard(mask)).to(weight dtype)     */
#define SF_EFF_HARD 2 /* E = hard(mask) (the hx = 0 case of MIX), any eff dtype; with
                         eff_dtype SF_DTYPE_U8 it is written as a byte and-mask        */

/*
 * Effective mask E of a forward call, written in the weight dtype (the
 * reference's `mask_cast`, legacy/sparse_modeling.py:72-73 and :759-771).
 * mode SF_EFF_MIX uses the hard projection `hard_kind` (SF_HARD_*) with N:M =
 * hard_n:hard_m; the arithmetic rounds in the mask dtype as the reference does.
 */
int sf_effective_mask(const void* mask, int mask_dtype, void* eff, int eff_dtype, int64_t rows, int64_t cols,
                      int mode, float hx, int hard_kind, int hard_n, int hard_m, void* stream);

/*
 * sf_effective_mask with the hard projection given as a tensor (`hard`,
 * [rows, cols], values {0, 1}) instead of computed per group: the block hard
 * types, whose projection is not group-local (legacy/sparse_modeling.py:770).
 */
int sf_effective_mask_given(const void* mask, int mask_dtype, const void* hard, int hard_dtype, void* eff,
                            int eff_dtype, int64_t rows, int64_t cols, int mode, float hx, void* stream);

/* ---- distillation KL (Distill_Model.kl_loss, legacy/sparse_modeling.py:1749-1828) ---- */

/* Token rows per chunk of the reference's loop for a vocabulary size: 128 above
 * 100000, 512 above 50000, else 2048 (:1772-1777). */
int64_t sf_kl_chunk_rows(int64_t vocab);

/* Workspace bytes of sf_kl_forward for `rows` token rows. */
size_t sf_kl_workspace_size(int64_t rows);

/*
 * KL(P_teacher || Q_student) of Distill_Model.kl_loss: logits [rows, vocab]
 * (dtype), clamped to +-100 and divided by `temperature`, log-softmax per row;
 * per chunk of `chunk_rows` rows the sum of p (log p - log q) is added unless a
 * log-probability of the chunk is NaN or the sum is not finite; the loss
 * (total * T^2 / rows in f32) is written to out[0] in out_dtype, or 0 if not
 * finite.  row_lse: device double[rows][2] = log-sum-exp of student and teacher
 * rows; row_scale: device float[rows] = T / rows for rows of kept chunks, else
 * 0; both are inputs of sf_kl_backward.  Sums run in f64; the reference sums
 * in f32, so losses agree to about 1e-6 relative.
 */
int sf_kl_forward(const void* student, const void* teacher, int dtype, int64_t rows, int64_t vocab,
                  float temperature, int64_t chunk_rows, void* out, int out_dtype, double* row_lse,
                  float* row_scale, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Gradient of that loss with respect to the student logits (the autograd of
 * the reference's chunk loop): grad_student = g * row_scale[r] * (q - p) where
 * -100 <= s <= 100, else 0 (clamp's gradient), in the logits dtype.
 * grad_out: the loss gradient g (device scalar, grad_out_dtype).
 */
int sf_kl_backward(const void* student, const void* teacher, int dtype, int64_t rows, int64_t vocab,
                   float temperature, const double* row_lse, const float* row_scale, const void* grad_out,
                   int grad_out_dtype, void* grad_student, void* stream);

/*
 * Masked weight W_eff = (W * E).to(W dtype), then (W_eff * scale).to(W dtype)
 * when scale != 1: the `w = weight * mask_cast` (and `* scale_factor`) of
 * FusedMaskedLinearSTE.forward (legacy/sparse_modeling.py:72-81); with scale 1
 * the `weight * mask_cast` of its backward (:113-115).  E: an SF_DTYPE_U8 byte
 * and-mask (0x00 / 0xFF, from sf_effective_mask) or an effective mask in the
 * weight dtype.  W, E, out: [rows, cols].  The GEMMs then run unmasked.
 */
int sf_apply_mask(const void* W, int w_dtype, const void* E, int e_dtype, float scale, void* out, int64_t rows,
                  int64_t cols, void* stream);

/* ---- attention softmax of the retraining model (cfg5; legacy/model_llama.py:39-55 eager attention,
 *      legacy/main_llama.py:194 autocast; differentiated twice by the Hutchinson HVP, legacy/utils.py:714-869) */

/*
 * p = softmax(x, dim=-1, dtype=float32).to(x dtype) over rows of `cols`
 * columns (x, p: [rows, cols], dtype f32 or bf16).  causal: row r keeps columns
 * 0 .. r % cols (the rows of [batches, S, S] attention scores whose masked
 * entries are -inf), the rest of the row gets probability 0 and is not read.
 * y is computed in f32 and rounded to nearest even.  cols <= 4096.
 */
int sf_softmax_rows(const void* x, int dtype, int64_t rows, int64_t cols, int causal, void* p, void* stream);

/*
 * The backward of that softmax and cast from the scores x (y recomputed, bit
 * for bit the forward's): grad_x = (y (g - sum(g y))).to(x dtype), g =
 * grad_p in f32 (torch's _softmax_backward_data after ToCopyBackward).
 */
int sf_softmax_rows_backward(const void* x, const void* grad_p, int dtype, int64_t rows, int64_t cols, int causal,
                             void* grad_x, void* stream);

/*
 * The backward of sf_softmax_rows_backward with respect to grad_p and x, given
 * the gradient grad_grad_x of its output: with y, g as above, h = grad_grad_x
 * in f32, c = sum g y, d = sum h y, u = g h - c h - d g, e = sum u y:
 *   grad_grad_p = (y (h - d)).to(dtype), grad2_x = (y (u - e)).to(dtype)
 * (torch's SoftmaxBackwardDataBackward0 with its softmax_double_backward, and
 * the softmax backward that carries u to the scores).
 */
int sf_softmax_rows_double_backward(const void* x, const void* grad_p, const void* grad_grad_x, int dtype,
                                    int64_t rows, int64_t cols, int causal, void* grad_grad_p, void* grad2_x,
                                    void* stream);

/* ---- RMSNorm of the retraining model (cfg5; HuggingFace LlamaRMSNorm of the LlamaForCausalLM the reference
 *      retrains, legacy/model_llama.py:18-57; differentiated twice by the Hutchinson HVP, legacy/utils.py:714-869) */

/*
 * y = weight * (x32 * rsqrt(mean(x32^2, -1) + eps)).to(dtype), x32 = x in f32,
 * over rows of `cols` columns (x, y: [rows, cols]; weight: [cols]; one dtype,
 * f32 or bf16).  rstd: f32[rows] receives 1 / sqrt(mean + eps), which the two
 * backward passes take.  cols: a multiple of 8, at most 4096; every pointer
 * 16-byte aligned.  The row sums run in another order than torch's.
 */
int sf_rmsnorm_forward(const void* x, const void* weight, int dtype, int64_t rows, int64_t cols, float eps, void* y,
                       float* rstd, void* stream);

/* f32 scratch of the weight-gradient column sums of the two calls below. */
size_t sf_rmsnorm_workspace_size(int64_t rows, int64_t cols);

/*
 * The backward of sf_rmsnorm_forward (torch's op sequence: the DT-rounded
 * grad_y * weight, the rsqrt / mean / pow chain in f32, the cast back):
 * grad_x [rows, cols] and grad_weight [cols] (the column sums of the rounded
 * grad_y * n, added in f32 in a fixed order).
 */
int sf_rmsnorm_backward(const void* x, const void* weight, const void* grad_y, const float* rstd, int dtype,
                        int64_t rows, int64_t cols, void* grad_x, void* grad_weight, void* workspace,
                        size_t workspace_bytes, void* stream);

/*
 * The backward of sf_rmsnorm_backward with respect to grad_y, x and weight,
 * given the gradients grad_grad_x / grad_grad_weight (null: zero) of its
 * outputs: the closed-form derivatives evaluated in f32, cast to the dtype.
 */
int sf_rmsnorm_double_backward(const void* x, const void* weight, const void* grad_y, const float* rstd,
                               const void* grad_grad_x, const void* grad_grad_weight, int dtype, int64_t rows,
                               int64_t cols, void* grad_grad_y, void* grad2_x, void* grad2_weight, void* workspace,
                               size_t workspace_bytes, void* stream);

/* ---- gated MLP product of the retraining model (cfg5; HuggingFace LlamaMLP's silu(gate) * up, the
 *      LlamaForCausalLM of legacy/model_llama.py:18-57; differentiated twice by the Hutchinson HVP) */

/*
 * y = silu(g).to(dtype) * u over n elements (g, u, y: one dtype, f32 or bf16;
 * n a multiple of 8; 16-byte aligned), torch's silu and mul in f32 with the
 * cast to the dtype after each.
 */
int sf_swiglu_forward(const void* g, const void* u, int dtype, int64_t n, void* y, void* stream);

/*
 * Its backward: grad_g = silu_backward((grad_y * u).to(dtype), g), grad_u =
 * grad_y * silu(g).to(dtype), each cast to the dtype.
 */
int sf_swiglu_backward(const void* g, const void* u, const void* grad_y, int dtype, int64_t n, void* grad_g,
                       void* grad_u, void* stream);

/*
 * The backward of sf_swiglu_backward with respect to grad_y, g and u, given
 * the gradients grad_grad_g / grad_grad_u (null: zero) of its outputs: the
 * closed-form derivatives (silu's first and second) in f32, cast to the dtype.
 */
int sf_swiglu_double_backward(const void* g, const void* u, const void* grad_y, const void* grad_grad_g,
                              const void* grad_grad_u, int dtype, int64_t n, void* grad_grad_y, void* grad2_g,
                              void* grad2_u, void* stream);

/*
 * Per-head operands of the retraining model's attention (HuggingFace eager
 * LlamaAttention, legacy/model_llama.py:39-55: q/k/v views [B, S, H, D]
 * transposed to [B, H, S, D], apply_rotary_pos_emb on q and k).  x is
 * [B, S, H * D] (the projections' rows); y is [B * H, S, D], or [B * H, D, S]
 * when `transposed` (the key operand of q k^T).
 *   sf_to_heads:   y = scale * rot(x), or scale * x without `rotate`
 *   sf_from_heads: its adjoint, x_grad [B, S, H * D] = rot^T(scale * g)
 * rot(x)[d] = x[d] c[d] + x[(d + D/2) % D] ss[d] with c = cos, ss = -sin on
 * the first half and sin on the second (cos, sin: f32 tables [S, D], rounded
 * to the dtype), each product rounded to the dtype, then their sum; the
 * adjoint rounds the same way, so the pair equals torch's ops and their
 * derivatives bit for bit.  dtype f32 or bf16, D a multiple of 16 up to 128,
 * 16-byte aligned tensors, scale 1 or a power of two.
 */
int sf_to_heads(const void* x, int dtype, int64_t B, int64_t S, int64_t H, int64_t D, const float* cos,
                const float* sin, int rotate, int transposed, float scale, void* y, void* stream);
int sf_from_heads(const void* g, int dtype, int64_t B, int64_t S, int64_t H, int64_t D, const float* cos,
                  const float* sin, int rotate, int transposed, float scale, void* x_grad, void* stream);

/*
 * dst[b] = src[b]^T for `batch` row-major [rows, cols] matrices of 2- or
 * 4-byte elements (dst: [batch, cols, rows]): the contiguous transposed
 * operands of the attention products' derivatives (torch.bmm gets contiguous
 * operands only).  16-byte aligned, not aliased.
 */
int sf_transpose_batched(const void* src, int elem_bytes, int64_t batch, int64_t rows, int64_t cols, void* dst,
                         void* stream);

/* ---- GEMM engine (FusedMaskedLinearSTE, :56-132, and the SLoRB F.linear pair, :790-794) */
#define SF_LAYOUT_K 0  /* operand stored K-contiguous: X[row * ld + k]                        */
#define SF_LAYOUT_MN 1 /* operand stored M/N-contiguous: X[k * ld + row] (a transposed view)  */

typedef struct sf_gemm_desc {
  int dtype;              /* element dtype of A1, A2, B1, B2, bmask, emask, dw            */
  int a_layout, b_layout; /* SF_LAYOUT_*; (MN, K) is not built                            */
  int64_t M, N, K1, K2;   /* K2 = 0: no second segment                                    */
  const void* A1;
  int64_t lda1;
  const void* B1;
  int64_t ldb1;
  const void* A2;
  int64_t lda2;
  const void* B2;
  int64_t ldb2;
  const void* bmask; /* effective mask E applied to B1 (B1's layout and ld), or NULL  */
  float bscale;      /* weight-scaling factor applied after E (1 = none)              */
  void* C;           /* [M, N] row-major                                              */
  int64_t ldc;
  int c_dtype;
  const void* bias; /* [N] added after rounding to c_dtype, or NULL                    */
  int bias_dtype;
  const void* emask; /* [M, N] (ld = ldc): C *= emask, or the test of the decay term   */
  const void* dw;    /* [M, N] (ld = ldc): C += decay * dw * (emask < 0.5), or NULL   */
  float decay;
  int accumulate; /* C += result                                                        */
  int bmask_bytes; /* bmask is a byte and-mask (SF_EFF_HARD with SF_DTYPE_U8): B1 elements
                      are kept or zeroed; requires bscale == 1                          */
  void* workspace; /* optional scratch of sf_gemm_workspace_size(desc) bytes, 16-byte
                      aligned: lets a GEMM with few output tiles split K (f32 partial
                      sums reduced in a fixed order); NULL runs it unsplit; a smaller
                      workspace limits the splits to the M x N f32 partials it holds  */
  size_t workspace_bytes;
  /* Block-sparse-16 operands (the compressed layout of convert_to_block_sparse,
     legacy/triton_block_sparse.py:46-103, plus its block map from sf_bsr_*): */
  int b_format;           /* SF_BFMT_*.  BSR16: B1 is the blocks array [nnz][16][16] of a
                             weight W; b_layout SF_LAYOUT_K gives B = W (forward, W is
                             [N, K1]), SF_LAYOUT_MN gives B = W^T (input gradient, W is
                             [K1, N]); pruned blocks are skipped, no bmask / K2     */
  const int32_t* b_map;   /* [b_map_rows][b_map_cols] block indices of W, -1 = pruned   */
  int64_t b_map_rows, b_map_cols;
  void* c_blocks;         /* non-NULL: C is written only at the blocks c_map lists, into
                             c_blocks [nnz][16][16] (the SDDMM weight gradient)        */
  const int32_t* c_map;   /* [M/16][N/16] block indices of C, -1 = not stored            */
  int64_t c_map_rows, c_map_cols;
  int bmask_kmajor;       /* with b_layout SF_LAYOUT_MN and a byte bmask: 1 = bmask is given
                             K-major, [N][K1] with leading dimension ldbm (the transpose
                             of B1's layout), so the input-gradient GEMM reads it beside
                             the transposed weight tile; 0 = bmask has B1's layout      */
  int64_t ldbm;
} sf_gemm_desc;

#define SF_BFMT_DENSE 0
#define SF_BFMT_BSR16 1

/*
 * C = A1 . (B1 * E * s)^T + A2 . B2^T (+ bias), bf16 or f32 MFMA on gfx950.
 * Replaces the cuBLAS matmuls of FusedMaskedLinearSTE.forward/backward
 * (legacy/sparse_modeling.py:79-87, :113-125) with the mask applied inside
 * the kernel, and folds the SLoRB term (:790-794) into the same accumulators.
 */
int sf_gemm(const sf_gemm_desc* d, void* stream);

/*
 * Scratch bytes sf_gemm would use for this descriptor's split-K (0: no split).
 * Depends only on dtype, M, N and K1.
 */
size_t sf_gemm_workspace_size(const sf_gemm_desc* d);

/*
 * out[c] = sum_r A[r, c] for a row-major [rows, cols] matrix (bias gradient,
 * legacy/sparse_modeling.py:127-129).  f32 accumulation, result in out_dtype.
 */
int sf_column_sum(const void* A, int a_dtype, int64_t rows, int64_t cols, void* out, int out_dtype, void* stream);

/* ---- block-sparse-16 index (convert_to_block_sparse, legacy/triton_block_sparse.py:46-103) ----
 * A block is kept iff sum(|W * mask|) over it is > 0 (a block holding a NaN is
 * dropped, as the reference's sum > 0 test does).  Building a layout:
 * sf_bsr_count -> sf_bsr_scan -> (read row_ptr[nbr] = nnz, allocate) -> sf_bsr_fill. */

/* flags [nbr * nbc] (1 = kept) and counts [nbr] of kept blocks per block row. */
int sf_bsr_count(const void* W, int w_dtype, const void* mask, int mask_dtype, int64_t rows, int64_t cols,
                 int block_size, uint8_t* flags, int32_t* counts, void* stream);

/* row_ptr [nbr + 1] = exclusive scan of counts (row_ptr[0] = 0). */
int sf_bsr_scan(const int32_t* counts, int64_t nbr, int32_t* row_ptr, void* stream);

/* col_idx [nnz] (ascending per block row), blocks [nnz][bs][bs] = W * mask in
 * blocks_dtype, and optionally block_map [nbr][nbc] (index or -1). */
int sf_bsr_fill(const void* W, int w_dtype, const void* mask, int mask_dtype, int64_t rows, int64_t cols,
                int block_size, const uint8_t* flags, const int32_t* row_ptr, int32_t* col_idx, void* blocks,
                int blocks_dtype, int32_t* block_map, void* stream);

/* block_map [nbr][nbc] from any CSR block index (row_ptr must be a valid scan
 * over col_idx; out-of-range columns are ignored). */
int sf_bsr_block_map(const int32_t* row_ptr, const int32_t* col_idx, int64_t nbr, int64_t nbc, int32_t* block_map,
                     void* stream);

/* The transposed block-sparse matrix, for the input gradient x_grad = dy . (W . M)
 * (the reference's BlockSparseLinear is forward-only, legacy/triton_block_sparse.py:290-470;
 * its CSR layout is :86-101): blocks_t[b] = blocks[b]^T for b < nblocks (same order,
 * so the indices stay valid) and block_map_t [nbc][nbr] = block_map^T.  The
 * block-sparse GEMM then multiplies by W^T with the forward's kernel. */
int sf_bsr_transpose(const void* blocks, int dtype, int64_t nblocks, const int32_t* block_map, int64_t nbr,
                     int64_t nbc, void* blocks_t, int32_t* block_map_t, void* stream);

/* ---- mask-aware AdamW (AdamW.step, legacy/adamw.py:65-176) ------------- */
typedef struct sf_adamw_params {
  double lr, weight_decay, beta1, beta2, eps;
  double decay; /* SR-STE masked-decay strength: the optimizer's `decay` (:51, :76-77, :101) */
  double l1;    /* adaptive_l1_decay (:56)                                                   */
  int amsgrad;
  int apply_l1; /* the parameter is >= 2-D (the l1 term also needs a mask, :171-172)        */
  int64_t step; /* state['step'] after this step's increment (:146)                         */
} sf_adamw_params;

/*
 * One AdamW step of one parameter tensor of n elements, in place: param,
 * exp_avg, exp_avg_sq (and max_exp_avg_sq when amsgrad), replacing the
 * per-parameter body of AdamW.step (legacy/adamw.py:84-174) with one fused
 * pass.  mask (the parameter's `mask` attribute, :99) may be NULL: no
 * masked decay and no L1 term.  param_bf16_copy (may be NULL) receives the
 * updated parameter rounded to bf16 (an f32 master parameter with its bf16
 * working copy).  Scalars follow the reference's Python doubles.
 */
int sf_adamw_step(void* param, int param_dtype, const void* grad, int grad_dtype, void* exp_avg, void* exp_avg_sq,
                  void* max_exp_avg_sq, int state_dtype, const void* mask, int mask_dtype, void* param_bf16_copy,
                  int64_t n, const sf_adamw_params* hp, void* stream);

/*
 * One tensor of a multi-tensor AdamW step (the per-parameter operands of
 * sf_adamw_step).  apply_l1: the parameter is >= 2-D (the L1 term also needs
 * a mask).  Tensors with n == 0 are skipped.
 */
typedef struct sf_adamw_tensor {
  void* param;             /* [n] param_dtype, updated in place           */
  const void* grad;        /* [n] grad_dtype                               */
  void* exp_avg;           /* [n] state_dtype                              */
  void* exp_avg_sq;        /* [n] state_dtype                              */
  void* max_exp_avg_sq;    /* [n] state_dtype when amsgrad, else NULL      */
  const void* mask;        /* [n] mask_dtype (the parameter's `mask`) or NULL */
  void* param_bf16_copy;   /* [n] bf16 copy of the updated parameter or NULL */
  int64_t n;
  int grad_dtype, mask_dtype;
  int apply_l1;
  int reserved;
} sf_adamw_tensor;

/*
 * The AdamW step of a whole parameter list in one pass over HBM
 * (AdamW.step's loop over parameters, legacy/adamw.py:79-174, fused): the
 * per-element arithmetic of sf_adamw_step for every tensor of `tensors` (a
 * HOST array of `count` entries that share param_dtype, state_dtype and the
 * hyper-parameters, including step).  The list travels in the kernel
 * arguments: one launch per 40 tensors, nothing allocated or copied.
 */
int sf_adamw_step_multi(const sf_adamw_tensor* tensors, int count, int param_dtype, int state_dtype,
                        const sf_adamw_params* hp, void* stream);

/* ---- Hutchinson Hessian diagonal (update_hessian_hutchinson, legacy/utils.py:710-869) ----
 * Probe v(seed, i) = +-1 from bit i % 64 of output i / 64 of the SplitMix64
 * stream seeded with `seed`: a pure function, regenerated wherever needed.  It
 * replaces the torch.randint draw of _rademacher_like (:710-711). */

/* v[0..n) = v(seed, i) in dtype (the tensor the backward of the probe dot needs). */
int sf_rademacher(void* v, int dtype, int64_t n, uint64_t seed, void* stream);

/* Scratch bytes of sf_rademacher_dot. */
size_t sf_rademacher_dot_workspace_size(void);

/*
 * out (device float[1]) = sum_i g[i] * v_i, the per-weight term of the probe
 * dot (legacy/utils.py:781-788); v from (seed, i), or from `v` when not NULL.
 * f64 partial sums in a fixed order (deterministic).
 */
int sf_rademacher_dot(const void* g, int g_dtype, const void* v, int v_dtype, int64_t n, uint64_t seed, float* out,
                      void* workspace, size_t workspace_bytes, void* stream);

/*
 * H <- beta * H + (1 - beta) * clamp(hvp * v, min=0), in place, one pass
 * (legacy/utils.py:806-868 single-GPU branch).  v from (seed, i), or from `v`
 * when not NULL (the reference's own probes in parity tests).
 */
int sf_hutchinson_update(void* H, int h_dtype, const void* hvp, int hvp_dtype, const void* v, int v_dtype, int64_t n,
                         uint64_t seed, double beta, void* stream);

/* One tensor of sf_hutchinson_update_multi (probe regenerated from its seed). */
typedef struct sf_hutch_tensor {
  void* H;          /* hessian_diag, updated in place */
  const void* hvp;  /* the Hessian-vector product */
  int64_t n;        /* elements, a multiple of 4; H and hvp 4-element aligned */
  uint64_t seed;
  double beta;
} sf_hutch_tensor;

/*
 * sf_hutchinson_update over many tensors (the per-weight loop of
 * update_hessian_hutchinson, legacy/utils.py:806-868), 48 tensors per
 * launch; every element gets the value sf_hutchinson_update gives it.
 */
int sf_hutchinson_update_multi(const sf_hutch_tensor* tensors, int count, int h_dtype, int hvp_dtype,
                               void* stream);

/* ---------------------------------------------------------------------------
 * Mask statistics and penalties: one fused pass per mask tensor
 * (legacy/utils.py mid_penalty :876-938, sparsity_penalty :942-1025,
 * nm_2_4_tile_stats :1029-1234, mask_stats :2069-2280).  Each call writes the
 * SF_MSTAT_COUNT sums of one tensor (device doubles, in a fixed order, so the
 * result is deterministic); the host composes the reference's scalars from
 * the rows of all layers after a single copy.
 * ------------------------------------------------------------------------- */
#define SF_MSTAT_SUM 0        /* sum m                                                        */
#define SF_MSTAT_SUM2 1       /* sum m * m                                                    */
#define SF_MSTAT_ENTROPY 2    /* sum -(c log c) - ((1 - c) log(1 - c)), c = clamp(m, eps, 1 - eps)
                                 in the mask dtype; terms in f32, summed in f64 (the reference
                                 takes f64 logs: a few f32 ulp per term); NaN once some c == 1 */
#define SF_MSTAT_LT05 3       /* count m < 0.5   (each threshold rounded to the mask dtype)   */
#define SF_MSTAT_LT01 4       /* count m < 0.1                                                */
#define SF_MSTAT_LT001 5      /* count m < 0.01                                               */
#define SF_MSTAT_GT90 6       /* count m > 0.9                                                */
#define SF_MSTAT_GT99 7       /* count m > 0.99                                               */
#define SF_MSTAT_GT05 8       /* count m > 0.5                                                */
#define SF_MSTAT_SUM_LT05 9   /* sum of m over m < 0.5                                        */
#define SF_MSTAT_SUM_GT05 10  /* sum of m over m > 0.5                                        */
#define SF_MSTAT_MID 11       /* sum m * (1 - m), 1 - m and the product rounded to the mask dtype */
#define SF_MSTAT_NONFINITE 12 /* count of NaN and +-inf                                       */
#define SF_MSTAT_TOP2 13      /* over every full group of 4 along a row: sum of its 2 largest
                                 (descending sort order, NaN largest)                         */
#define SF_MSTAT_BOT2 14      /* ... sum of its 2 smallest                                    */
#define SF_MSTAT_TAIL_LT05 15 /* count m < 0.5 in columns >= tail_col                         */
#define SF_MSTAT_COUNT 16

/* Scratch bytes of sf_mask_stats (per-workgroup partial sums). */
size_t sf_mask_stats_workspace_size(void);

/*
 * out[0..SF_MSTAT_COUNT) (device doubles) = the sums above over mask [rows, cols]
 * (row-major, dtype SF_DTYPE_F32 or SF_DTYPE_BF16).  eps: the entropy clamp of
 * mask_stats (:2131-2132).  tail_col: first column of the sparsity_penalty
 * threshold tail, (cols / M) * M (:983-993).  Groups of 4 for TOP2 / BOT2 start
 * at column 0 of every row; the partial last group of a row is left out, as
 * nm_2_4_tile_stats does (:1099-1104).
 */
int sf_mask_stats(const void* mask, int dtype, int64_t rows, int64_t cols, int64_t tail_col, float eps, double* out,
                  void* workspace, size_t workspace_bytes, void* stream);

/*
 * hist[b] += number of idx[i] (i < take) with lo <= x <= hi and
 * b = (int)((x - lo) * bins / (hi - lo)) (clamped to bins - 1), x = mask[idx[i]]
 * as f32: the torch.histc of the sampled mask values in mask_stats
 * (:2147-2152) with its device binning formula; NaN and values outside
 * [lo, hi] are not counted.  hist: device uint64[bins], accumulated.
 */
int sf_mask_hist(const void* mask, int dtype, int64_t n, const int64_t* idx, int64_t take, int bins, float lo,
                 float hi, unsigned long long* hist, void* stream);

/*
 * out[0] = sum of v[i] with keep[i] != 0, out[1] = sum of the others (device
 * doubles, fixed order): the upper- and lower-half sums of the sorted block
 * means in mask_stats (:2158-2181), with keep = sf_topk_keep(v, n - n / 2).
 */
int sf_keep_split_sum(const float* v, const float* keep, int64_t n, double* out, void* stream);

/* ---------------------------------------------------------------------------
 * 2:4 packed weights and the sparse-MFMA forward of finalized models.  The
 * reference hardens every mask and multiplies it into its weight at the end
 * of training (legacy/main_llama.py:2499-2568) and then runs the plain
 * forward F.linear(x, W_hard) (legacy/eval_wiki_ppl.py:548-651); for a 2:4
 * hard mask the build stores W_hard as
 *   vals [out, in / 2] bf16: the two kept values of every group of 4, in
 *        column order;
 *   idx  u32 [out / 32][in / 64][2][32] (out * in / 8 bytes): for row block
 *        rb, 64-column chunk q, half h, row rb * 32 + r: bits 2j + 1 : 2j give
 *        the column inside its group of the j-th kept value (j = 0..7) of
 *        columns [64 q + 16 h, +16) in the low 16 bits and of
 *        [64 q + 32 + 16 h, +16) in the high 16 bits,
 * the operand layout of gfx950's v_smfmac_f32_32x32x32_bf16.  Needs
 * out % 32 == 0 and in % 64 == 0.
 * ------------------------------------------------------------------------- */

/* Bytes of vals (returned) and of idx (*idx_bytes) for an out x in weight. */
size_t sf_pack_2to4_sizes(int64_t out_features, int64_t in_features, size_t* idx_bytes);

/*
 * Pack W * mask (columns with mask != 0 kept; W, mask [out, in], f32 or bf16)
 * into vals / idx.  A group with fewer than two kept columns is padded with
 * zeros; groups with more than two are added to *bad_groups (device uint64,
 * accumulated): the caller rejects the packing when it is nonzero.
 */
int sf_pack_2to4(const void* W, int w_dtype, const void* mask, int mask_dtype, int64_t out_features,
                 int64_t in_features, void* vals, void* idx, unsigned long long* bad_groups, void* stream);

/* Dense W [out, in] (f32 or bf16) from vals / idx: the inverse of sf_pack_2to4. */
int sf_unpack_2to4(const void* vals, const void* idx, int64_t out_features, int64_t in_features, void* W, int w_dtype,
                   void* stream);

/*
 * y [tokens, out] (row pitch ldy, f32 or bf16) = x [tokens, in] (bf16, row
 * pitch ldx) . W_hard^T (+ bias [out]) with W_hard given packed: the forward
 * F.linear(x, W * M_hard, b) of a finalized SparseLinear
 * (legacy/sparse_modeling.py:737-739 dense_forward after
 * legacy/eval_wiki_ppl.py:548-651).  f32 accumulation; a bf16 y is the
 * rounded product plus the bias, rounded again.
 */
int sf_gemm_2to4(const void* x, int64_t ldx, int64_t tokens, const void* vals, const void* idx, int64_t out_features,
                 int64_t in_features, const void* bias, int bias_dtype, void* y, int y_dtype, int64_t ldy,
                 void* stream);

/*
 * The training forward of a SparseLinear whose effective mask is a 2:4 hard
 * mask (hardening_x = 0 in legacy/sparse_modeling.py:56-81
 * FusedMaskedLinearSTE.forward, with E from _hard_mask_from_soft :578-603 /
 * :720-735 and the SLoRB pair of :790-794), on the sparse MFMA.
 *
 * sf_apply_mask_2to4: Wm = W * mask (W bf16 [out, in], mask a byte and-mask,
 * 0 = pruned; the elementwise product sf_apply_mask writes, which the input
 * gradient reuses) and the packed vals / idx of Wm in one pass.  Groups with
 * more than two kept columns are added to *bad_groups (device uint64,
 * accumulated); a mask from the N:M hard projection with N = 2, M = 4 has none.
 * Pruned columns do not enter the packed product, so a non-finite weight there
 * does not reach y (the dense product of Wm would carry its NaN).
 *
 * sf_gemm_2to4_lowrank: sf_gemm_2to4 plus the low-rank term z S^T
 * (z [tokens, rank] row pitch ldz, S [out, rank] row pitch lds, bf16,
 * rank % 8 == 0; rank 0: none) accumulated in f32 before the output rounding,
 * i.e. y = x Wm^T + z S^T (+ bias) as the dense forward computes it.
 */
int sf_apply_mask_2to4(const void* W, const void* mask, int64_t out_features, int64_t in_features, void* Wm,
                       void* vals, void* idx, unsigned long long* bad_groups, void* stream);
int sf_gemm_2to4_lowrank(const void* x, int64_t ldx, int64_t tokens, const void* vals, const void* idx,
                         int64_t out_features, int64_t in_features, const void* z, int64_t ldz, const void* S,
                         int64_t lds, int64_t rank, const void* bias, int bias_dtype, void* y, int y_dtype,
                         int64_t ldy, void* stream);

/*
 * Sustained MFMA rate probe, a measurement aid with no counterpart in the
 * reference (bench.py reports the rate beside the published dense peak):
 * `blocks` workgroups of 4 waves, each wave iters x 16
 * v_mfma_f32_32x32x16_bf16 on register operands distributed like a GEMM's
 * (about N(0, 1) and N(0, 0.02)), no memory traffic in the loop; FLOPs = blocks * 4 * iters * 16 * 32768.  out: device
 * float[blocks * 256] checksums.
 */
int sf_mfma_probe(int iters, int blocks, float* out, void* stream);

/*
 * Sustained HBM rate probe, a measurement aid with no counterpart in the
 * reference (bench.py reports the rates beside the mask kernels' GB/s): a
 * grid-stride stream over n elements (n % 4 == 0, 16-byte aligned operands)
 * with a token FMA per element.  pattern 0: the fused mask update's traffic
 * (read W bf16, H f32, M f32; write M f32: 14 B / element); 1: the score
 * statistics' (read W, H: 6 B / element; M receives blocks * 256 floats);
 * 2: a copy (read H, write M: 8 B / element).
 */
int sf_hbm_probe(int pattern, const void* W, const void* H, void* M, int64_t n, int blocks, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SPARSEFORGE_AMD_H */
