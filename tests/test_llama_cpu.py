"""CPU checks of the Llama harness model (no GPU, no HIP library): the layer
math against Hugging Face's LlamaForCausalLM on the same weights, and the
static-cache decode step against the prefill logits."""
import pytest
import torch

from int4_hip.llama import LlamaConfig, LlamaForCausalLM

TINY = LlamaConfig(vocab_size=97, hidden_size=64, intermediate_size=160, num_hidden_layers=2,
                   num_attention_heads=8, num_key_value_heads=2, head_dim=8, rope_theta=500000.0,
                   rope_scaling=(32.0, 1.0, 4.0, 64))


def _model(seed=0):
    m = LlamaForCausalLM(TINY)
    m.init_weights(seed)
    g = torch.Generator().manual_seed(seed + 100)
    with torch.no_grad():  # non-trivial norm weights
        for layer in m.model.layers:
            layer.input_layernorm.weight.uniform_(0.5, 1.5, generator=g)
            layer.post_attention_layernorm.weight.uniform_(0.5, 1.5, generator=g)
        m.model.norm.weight.uniform_(0.5, 1.5, generator=g)
    m.allocate_cache(40, torch.float32, "cpu")
    return m.eval()


def test_matches_hf_llama():
    transformers = pytest.importorskip("transformers")
    m = _model()
    hc = transformers.LlamaConfig(
        vocab_size=TINY.vocab_size, hidden_size=TINY.hidden_size, intermediate_size=TINY.intermediate_size,
        num_hidden_layers=TINY.num_hidden_layers, num_attention_heads=TINY.num_attention_heads,
        num_key_value_heads=TINY.num_key_value_heads, head_dim=TINY.head_dim, rms_norm_eps=TINY.rms_norm_eps,
        rope_theta=TINY.rope_theta, max_position_embeddings=128, tie_word_embeddings=True,
        rope_scaling={"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
                      "original_max_position_embeddings": 64},
        attn_implementation="eager")
    hf = transformers.LlamaForCausalLM(hc).eval()
    missing, unexpected = hf.load_state_dict(
        {k: v for k, v in m.state_dict().items() if not k.startswith(("kc", "vc"))}, strict=False)
    assert not unexpected and all("rotary" in k for k in missing), (missing, unexpected)
    ids = torch.randint(0, TINY.vocab_size, (1, 33), generator=torch.Generator().manual_seed(3))
    with torch.no_grad():
        ref = hf(ids).logits[0]
        got = m.prefill(ids[0])
    torch.testing.assert_close(got, ref, rtol=1e-4, atol=1e-4)


def test_decode_steps_match_prefill():
    m = _model(1)
    ids = torch.randint(0, TINY.vocab_size, (30,), generator=torch.Generator().manual_seed(4))
    full = m.prefill(ids)
    m2 = _model(1)
    m2.prefill(ids[:10])
    for t in range(10, 30):
        step = m2.decode_step(ids[t:t + 1], torch.tensor([t]))
        torch.testing.assert_close(step[0], full[t], rtol=1e-4, atol=1e-4)
