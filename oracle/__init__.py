"""CPU oracle of the SparseForge sparse-training hot path — TEST INFRASTRUCTURE ONLY.

A plain numpy restatement of the reference functions (liuhanzuo/SparseForge,
legacy/*.py), each citing the reference lines it follows.  It is the checker
the GPU parity tests compare the HIP library against, and the "port" CPU
baseline that bench.py times.  Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg may import it; the product package
(sparseforge_amd) never does.

How each module is pinned (checks that would fail on a dropped term, a wrong
sign or index, or a transposed operand):

  masks.py      top-N selection: against torch.topk itself over every weak
                ordering of 4 values and over random tie-heavy tensors
                (tests/test_oracle_masks.py); gate target / update_mask:
                against golden vectors written by the reference code
                (tests/golden/make_reference_golden.py) and against closed-form
                invariants (2nd-largest of a group gets G = 0.5 exactly,
                G in (0, 1), exactly N ones per full group).
  select.py     torch.topk's CPU selection (libstdc++ introselect / heap
                select): against torch.topk itself on tie-heavy inputs with NaN
                and -0 through both branches (tests/test_oracle_select.py).
  quantile      against torch.quantile (linear interpolation).
  adamw.py      against torch.optim.AdamW(foreach=False) for decay = 0 and
                l1 = 0, and against reference golden vectors for decay != 0,
                l1 > 0.
  hutchinson.py clamp/EMA closed form; SplitMix64 against its published
                first outputs for seed 1234567.
  linear.py     masked linear fwd/bwd against torch.matmul closed forms and
                torch.autograd on the dense equivalent.
  bsr.py        CSR build against the reference's own output
                (tests/golden/ref_bsr_basic_f32.npz) and a brute-force dense
                scan; BSR products against the dense masked product.
  masks.glu_joint_update  against the reference's own output for three
                consecutive steps (tests/golden/ref_glu_joint_f32.npz) and
                the shared-target invariants.
  stats.py      mid_penalty / sparsity_penalty / nm_2_4_tile_stats /
                mask_stats against the reference's own outputs on small models
                (tests/golden/ref_stats_*.npz: f32 and bf16 masks, threshold
                neighbours, ragged rows, NaN and exact-1 entries), the group
                sort against sorted(), the histogram binning against
                torch.histc, and constant-mask closed forms.
"""
