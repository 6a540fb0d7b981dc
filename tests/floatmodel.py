"""A small random Qwen3 float model (transformers, built offline) for the
quantiser tests."""

import torch


def small_float_model(seed=0, outliers=False):
    """A 2-layer Qwen3 (hidden 256, 4/2 heads, vocab 1000) with random weights
    and non-trivial norm gains and per-channel activation scales. outliers:
    a few channels scaled up by orders of magnitude at every smoothing site
    (the RMSNorm inputs, K after its norm, the inputs of o and down), so the
    smoothing factors reach their clamp."""
    from transformers import Qwen3Config, Qwen3ForCausalLM
    torch.manual_seed(seed)
    cfg = Qwen3Config(vocab_size=1000, hidden_size=256, intermediate_size=512,
                      num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
                      head_dim=128, max_position_embeddings=1024, tie_word_embeddings=True,
                      rope_theta=1e6, eos_token_id=999)
    cfg._attn_implementation = "eager"
    m = Qwen3ForCausalLM(cfg).float().eval()
    with torch.no_grad():
        for layer in m.model.layers:
            for norm in (layer.input_layernorm, layer.post_attention_layernorm,
                         layer.self_attn.q_norm, layer.self_attn.k_norm):
                norm.weight.mul_(1 + 0.3 * torch.randn_like(norm.weight))
            for lin in (layer.self_attn.q_proj, layer.self_attn.k_proj, layer.self_attn.v_proj,
                        layer.self_attn.o_proj, layer.mlp.gate_proj, layer.mlp.up_proj,
                        layer.mlp.down_proj):
                lin.weight.mul_(3.0)
        m.model.norm.weight.mul_(1 + 0.3 * torch.randn_like(m.model.norm.weight))
        m.model.embed_tokens.weight.mul_(torch.exp(torch.randn(1, 256)))
        if outliers:
            m.model.embed_tokens.weight[:, :3].mul_(1e6)
            for layer in m.model.layers:
                layer.self_attn.k_norm.weight[:4].mul_(3e3)
                layer.self_attn.q_norm.weight[4:6].mul_(3e3)
                layer.self_attn.v_proj.weight[:2].mul_(1e4)
                layer.mlp.up_proj.weight[:2].mul_(1e4)
                layer.mlp.gate_proj.weight[:, 5:8].mul_(1e-4)
                layer.mlp.up_proj.weight[:, 5:8].mul_(1e-4)
    return m
