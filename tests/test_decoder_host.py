"""Host-side checks of the decode harness: the SmolLM2-135M geometry and the
weight names an in-code Hugging Face Llama expects (no GPU needed)."""
import torch

from voom_amd.decoder import DecoderConfig, random_weights


def test_default_config_is_smollm2_135m():
    cfg = DecoderConfig()
    # 134,515,008 parameters with tied embeddings
    assert cfg.param_count == 134_515_008
    assert cfg.num_attention_heads * cfg.head_dim == cfg.hidden_size


def test_weights_use_hf_llama_names_and_shapes():
    from transformers import LlamaConfig, LlamaForCausalLM

    cfg = DecoderConfig(num_hidden_layers=2, vocab_size=512)
    w = random_weights(cfg, seed=0)
    hcfg = LlamaConfig(vocab_size=512, hidden_size=cfg.hidden_size,
                       intermediate_size=cfg.intermediate_size, num_hidden_layers=2,
                       num_attention_heads=cfg.num_attention_heads,
                       num_key_value_heads=cfg.num_key_value_heads, head_dim=cfg.head_dim,
                       tie_word_embeddings=True)
    ref = LlamaForCausalLM(hcfg).state_dict()
    assert set(w) == set(ref) - {"lm_head.weight"}
    for k, v in w.items():
        assert tuple(v.shape) == tuple(ref[k].shape), k
    assert sum(v.numel() for v in w.values()) == cfg.param_count
    # seeded: the same values on every call
    assert torch.equal(random_weights(cfg, seed=0)["model.layers.1.mlp.up_proj.weight"],
                       w["model.layers.1.mlp.up_proj.weight"])
    std = w["model.layers.0.mlp.gate_proj.weight"].float().std().item()
    assert abs(std - 0.02) < 1e-3
