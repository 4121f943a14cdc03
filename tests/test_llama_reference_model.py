"""The cfg5 model against the model the reference retrains: transformers' LlamaForCausalLM (CPU).

The reference wraps HuggingFace's LlamaForCausalLM (legacy/model_llama.py:39-55), loads it in bf16
(:120), runs it under torch.amp.autocast(bf16) (legacy/main_llama.py:194) with eager attention
(:383-388).  One tiny LlamaConfig (2 layers, 4 heads of 16, non-unit RMSNorm weights, 24 positions)
and one set of random weights go into all three models:

* float64: transformers' forward equals the oracle's dense forward (oracle/retrain.forward, the
  float64 restatement the end-to-end GPU test is checked against) within 1e-12 of the logits' scale,
  which pins the rotary convention and tables, the RMSNorm placement, the attention scale and mask,
  SwiGLU and the residual order, and the three places where that model computes in float32 whatever
  its dtype (rotary tables, RMSNorm's normalisation, the softmax);
* float32: sparseforge_amd.llama.LlamaDecoder (the dense teacher; the student's masked linears are
  the teacher's at unit masks on the GPU) within 1e-5 of transformers' float64 logits;
* bf16 weights under CPU autocast: LlamaDecoder against transformers' eager attention under the same
  autocast, which pins the bf16 operation sequence (rotation in bf16, bf16 products, the float32
  softmax cast back): within half a bf16 ulp of the logits' scale (the same CPU kernels give the
  same bits), while running the attention in float32 on the same bf16 activations lands more than
  twice that away.  The parameters are converted to bf16 and the rotary buffer is left in full
  precision, as from_pretrained(torch_dtype=bf16) (legacy/model_llama.py:120) leaves it.
"""
import numpy as np
import pytest
import torch

transformers = pytest.importorskip("transformers")

V, HID, FFN, LAYERS, HEADS, SEQ = 97, 64, 96, 2, 4, 24


def _models(seed=0):
    from transformers import LlamaConfig, LlamaForCausalLM

    from sparseforge_amd.llama import LlamaShape

    cfg = LlamaConfig(vocab_size=V, hidden_size=HID, intermediate_size=FFN, num_hidden_layers=LAYERS,
                      num_attention_heads=HEADS, num_key_value_heads=HEADS, rms_norm_eps=1e-5, rope_theta=10000.0,
                      max_position_embeddings=64, tie_word_embeddings=False, attn_implementation="eager")
    torch.manual_seed(seed)
    hf = LlamaForCausalLM(cfg).double().eval()
    g = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        for name, p in hf.named_parameters():
            if name.endswith("norm.weight"):
                p.copy_(1.0 + 0.1 * torch.randn(p.shape, generator=g, dtype=torch.float64))
            else:
                p.copy_(0.05 * torch.randn(p.shape, generator=g, dtype=torch.float64))
    shape = LlamaShape(vocab_size=V, hidden_size=HID, intermediate_size=FFN, num_hidden_layers=LAYERS,
                       num_attention_heads=HEADS, rms_norm_eps=1e-5, rope_theta=10000.0)
    # transformers' names are ours under "model." (lm_head aside)
    params = {(k[len("model."):] if k.startswith("model.") else k): v.detach() for k, v in hf.named_parameters()}
    return hf, shape, params


def _ours(shape, params, dtype):
    from sparseforge_amd.llama import LlamaDecoder

    m = LlamaDecoder(shape, None, device="cpu", dtype=dtype)
    sd = m.state_dict()
    assert set(sd) == set(params), sorted(set(sd) ^ set(params))
    m.load_state_dict({k: v.to(dtype) for k, v in params.items()})
    return m.eval()


def _idx():
    return torch.randint(0, V, (2, SEQ), generator=torch.Generator().manual_seed(7))


def test_float64_oracle_forward_equals_transformers():
    from oracle import retrain as orc

    hf, shape, params = _models()
    idx = _idx()
    with torch.no_grad():
        ref = hf(input_ids=idx).logits
        got = orc.forward(params, None, shape, idx, False, False)
    err = float((got - ref).abs().max() / ref.abs().max())
    assert err < 1e-12, err


def test_oracle_pin_detects_convention_changes():
    """The float64 comparison separates plausible mistakes: rotary tables in float64 instead of float32,
    an interleaved (GPT-J) rotation instead of the half split, and RMSNorm's weight inside the
    normalised quantity all move the logits by far more than the bar."""
    from oracle import retrain as orc

    hf, shape, params = _models()
    idx = _idx()
    with torch.no_grad():
        ref = hf(input_ids=idx).logits

    def err_with(patch, fn):
        orig = getattr(orc, patch)
        setattr(orc, patch, fn)
        try:
            with torch.no_grad():
                got = orc.forward(params, None, shape, idx, False, False)
        finally:
            setattr(orc, patch, orig)
        return float((got - ref).abs().max() / ref.abs().max())

    def rope64(seq, d, theta):
        inv = 1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.float64) / d))
        ang = torch.arange(seq, dtype=torch.float64)[:, None] * inv[None, :]
        ang = torch.cat([ang, ang], dim=-1)
        return ang.cos(), ang.sin()

    def rot_interleaved(x, cos, sin):
        x2 = torch.stack([-x[..., 1::2], x[..., 0::2]], dim=-1).flatten(-2)
        c = cos[..., : cos.shape[-1] // 2].repeat_interleave(2, -1)
        s = sin[..., : sin.shape[-1] // 2].repeat_interleave(2, -1)
        return x * c + x2 * s

    def rms_weight_first(x, w, eps):
        y = x * w
        return y * torch.rsqrt(y.pow(2).mean(-1, keepdim=True) + eps)

    assert err_with("rope", rope64) > 1e-9
    assert err_with("_rot", rot_interleaved) > 1e-3
    assert err_with("rmsnorm", rms_weight_first) > 1e-3


def test_float32_decoder_matches_transformers():
    hf, shape, params = _models()
    idx = _idx()
    ours = _ours(shape, params, torch.float32)
    with torch.no_grad():
        ref = hf(input_ids=idx).logits
        got, _loss, _ = ours(idx)
    err = float((got.double() - ref).abs().max() / ref.abs().max())
    assert err < 1e-5, err


def test_bf16_decoder_follows_transformers_eager_sequence():
    from sparseforge_amd import llama

    hf, shape, params = _models()
    idx = _idx()
    for p in hf.parameters():
        p.data = p.data.to(torch.bfloat16)
    ours = _ours(shape, params, torch.bfloat16)
    with torch.no_grad(), torch.autocast("cpu", dtype=torch.bfloat16):
        ref = hf(input_ids=idx).logits.double()
        got = ours(idx)[0].double()
        orig = llama.causal_attention

        def f32_attention(q, k, v, cos, sin):  # the float32 sequence on the same bf16 activations
            return orig(q.float(), k.float(), v.float(), cos, sin).to(q.dtype)

        llama.causal_attention = f32_attention
        try:
            alt = ours(idx)[0].double()
        finally:
            llama.causal_attention = orig
    scale = float(ref.abs().max())
    err = float((got - ref).abs().max()) / scale
    err_f32 = float((alt - ref).abs().max()) / scale
    print(f"bf16 sequence: {err:.3e} of scale; float32 attention: {err_f32:.3e}")
    assert err <= 2.0 ** -9, err
    assert err_f32 > 2 * 2.0 ** -9, (err, err_f32)
