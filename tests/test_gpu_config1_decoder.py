"""Config 1 at its stated size: the SmolLM2-135M-shaped decoder (30 layers,
hidden 576, 9 q / 3 kv heads, head_dim 64, SwiGLU 1536, vocab 49152, random
N(0, 0.02) bf16 weights, seed 0) over a 512-token prompt (seed 1) through
PagedKVCache with 64-token pages, against an in-code Hugging Face
LlamaForCausalLM in fp32 on the same weights.

Teacher forcing: the logits at every one of the 512 prompt positions (the
causal prefill through the paged kernel) and at the first 16 decode
positions, each decode step replayed from the captured HIP graph that the
bench times, with the HF model's own next input fed in.  The bar is the one
tests/test_gpu_decoder.py states: per position relative L2 <= 3e-2 and max abs
<= 8e-2 (about twice what bf16 arithmetic alone costs the HF model at 30
layers).  The reference's loop is runtime/engine.py:8459-8503 over
runtime/layer_runner.py:48-182.
"""
import numpy as np
import pytest
import torch

from voom_amd.decoder import DecoderConfig, PagedDecoder, random_weights

pytestmark = pytest.mark.gpu

PROMPT, DECODE = 512, 16


def hf_logits(cfg, weights, ids):
    from transformers import LlamaConfig, LlamaForCausalLM

    hcfg = LlamaConfig(vocab_size=cfg.vocab_size, hidden_size=cfg.hidden_size,
                       intermediate_size=cfg.intermediate_size,
                       num_hidden_layers=cfg.num_hidden_layers,
                       num_attention_heads=cfg.num_attention_heads,
                       num_key_value_heads=cfg.num_key_value_heads, head_dim=cfg.head_dim,
                       rms_norm_eps=cfg.rms_norm_eps, rope_theta=cfg.rope_theta,
                       tie_word_embeddings=True, max_position_embeddings=4096)
    m = LlamaForCausalLM(hcfg).eval()
    missing, unexpected = m.load_state_dict({k: v.float() for k, v in weights.items()},
                                            strict=False)
    assert not unexpected and set(missing) <= {"lm_head.weight"}
    with torch.no_grad():
        return m(ids).logits[0].numpy()


def check(got, ref, where):
    rel = np.linalg.norm(got - ref, axis=-1) / np.linalg.norm(ref, axis=-1)
    err = np.abs(got - ref).max()
    agree = float((got.argmax(-1) == ref.argmax(-1)).mean())
    print(f"[config1] {where}: rel L2 max {rel.max():.4f}, abs max {err:.4f}, "
          f"argmax agreement {agree:.3f}", flush=True)
    assert rel.max() <= 3e-2, (where, int(rel.argmax()), float(rel.max()))
    assert err <= 8e-2, (where, float(err))


def test_config1_full_size_teacher_forced_prefill_and_graph_decode():
    cfg = DecoderConfig()
    assert cfg.num_hidden_layers == 30 and cfg.vocab_size == 49152
    weights = random_weights(cfg, seed=0)
    ids = torch.randint(0, cfg.vocab_size, (1, PROMPT + DECODE),
                        generator=torch.Generator().manual_seed(1))
    print("[config1] HF fp32 reference over 528 positions (CPU)", flush=True)
    ref = hf_logits(cfg, weights, ids)
    dec = PagedDecoder(cfg, weights)
    kv = dec.new_cache(page_positions=64)
    print("[config1] prefill of 512 tokens through the paged kernel", flush=True)
    got = dec.forward(ids[:, :PROMPT].cuda(), kv)[0].cpu().numpy()
    check(got, ref[:PROMPT], "prefill")
    logits = torch.empty((1, cfg.vocab_size), dtype=torch.float32, device="cuda")
    graph, tok, _ = dec.capture_decode(kv, PROMPT + DECODE, logits=logits)
    rows = []
    for t in range(PROMPT, PROMPT + DECODE):
        tok.fill_(int(ids[0, t]))
        graph.replay()
        kv.advance(1)
        rows.append(logits[0].cpu().numpy().copy())
    assert kv.offset == PROMPT + DECODE
    check(np.stack(rows), ref[PROMPT:], "graph decode")
    assert sum(len(p) for p in kv._pages) == cfg.num_hidden_layers * ((PROMPT + DECODE) // 64)
    assert all(p.resident for pages in kv._pages for p in pages)
