"""HF ``Qwen2ForCausalLM`` eager run over the oracle's weights.

Oracle (test infrastructure only).  This is the reference's own acceptance
oracle for the decoder step: history/attempts/g4c-attempt69b-b4-eager/
batched_decoder_step.py:477-518 runs ``AutoModelForCausalLM`` eager with a
DynamicCache one token at a time and compares logits and written K/V at
rtol=atol=5e-3 (DEC:34-35).  Here the model is built from a local
``Qwen2Config`` (never a downloaded checkpoint) and loaded with the same
seeded weights as the oracle, so a mistake in the restatement (a dropped
term, a wrong sign in ``rotate_half``, a transposed operand, a wrong GQA
head mapping) shows as a logits or K/V mismatch.
"""
from __future__ import annotations

import torch

from .decoder import ModelDims


def build_hf_model(dims: ModelDims, weights: dict[str, torch.Tensor], max_positions: int = 4096):
    from transformers import Qwen2Config, Qwen2ForCausalLM

    config = Qwen2Config(
        vocab_size=dims.vocab,
        hidden_size=dims.hidden,
        intermediate_size=dims.intermediate,
        num_hidden_layers=dims.num_layers,
        num_attention_heads=dims.num_heads,
        num_key_value_heads=dims.num_kv_heads,
        max_position_embeddings=max_positions,
        rms_norm_eps=dims.rms_eps,
        rope_theta=dims.rope_theta,
        tie_word_embeddings=False,
        use_sliding_window=False,
        attn_implementation="eager",
    )
    config.rope_parameters = {"rope_type": "default", "rope_theta": dims.rope_theta}
    model = Qwen2ForCausalLM(config).to(dims.torch_dtype).eval()
    # ``.to(dtype)`` also casts the rotary ``inv_freq`` buffer; a checkpoint
    # loaded with ``torch_dtype`` (the reference's gate, DEC:485-491) keeps
    # it in fp32, as DEC:213-217 computes it.  Restore the fp32 values.
    rotary = model.model.rotary_emb
    fp32_inv_freq, _ = rotary.compute_default_rope_parameters(config)
    rotary.register_buffer("inv_freq", fp32_inv_freq, persistent=False)
    state = {"model.embed_tokens.weight": weights["embedding"], "model.norm.weight": weights["final_norm"], "lm_head.weight": weights["lm_head"]}
    local = {
        "input_norm": "input_layernorm.weight",
        "post_norm": "post_attention_layernorm.weight",
        "q_weight": "self_attn.q_proj.weight",
        "q_bias": "self_attn.q_proj.bias",
        "k_weight": "self_attn.k_proj.weight",
        "k_bias": "self_attn.k_proj.bias",
        "v_weight": "self_attn.v_proj.weight",
        "v_bias": "self_attn.v_proj.bias",
        "o_weight": "self_attn.o_proj.weight",
        "gate_weight": "mlp.gate_proj.weight",
        "up_weight": "mlp.up_proj.weight",
        "down_weight": "mlp.down_proj.weight",
    }
    for layer in range(dims.num_layers):
        for ours, theirs in local.items():
            state[f"model.layers.{layer}.{theirs}"] = weights[f"layers_{layer}_{ours}"]
    missing, unexpected = model.load_state_dict(state, strict=False)
    missing = [m for m in missing if "rotary" not in m]
    if missing or unexpected:
        raise RuntimeError(f"HF state mismatch: missing={missing} unexpected={unexpected}")
    return model


def cache_layer(cache, index: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Keys and values [B, KVH, S, d] of one layer of a DynamicCache (the
    keys are cached after RoPE)."""
    layer = cache.layers[index]
    return layer.keys, layer.values


@torch.no_grad()
def hf_incremental(model, token_ids: list[int]) -> tuple[list[torch.Tensor], list[torch.Tensor], list[torch.Tensor]]:
    """One token per call with a growing cache, as DEC:488-518.

    Returns per step the last logits (fp32 [V]) and, as the reference's gate
    records them (DEC:506-511), the key and value each layer wrote at that
    step: [layers, KVH, d] in the model dtype.
    """
    from transformers import DynamicCache

    cache = DynamicCache()
    logits, keys, values = [], [], []
    layers = model.config.num_hidden_layers
    for step, token in enumerate(token_ids):
        outputs = model(
            input_ids=torch.tensor([[token]], dtype=torch.int64),
            position_ids=torch.tensor([[step]], dtype=torch.int64),
            past_key_values=cache,
            use_cache=True,
        )
        cache = outputs.past_key_values
        logits.append(outputs.logits[0, -1].float().clone())
        ks, vs = zip(*(cache_layer(cache, i) for i in range(layers)))
        keys.append(torch.stack([k[0, :, step] for k in ks]).clone())
        values.append(torch.stack([v[0, :, step] for v in vs]).clone())
    return logits, keys, values
