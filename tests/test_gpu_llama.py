"""GPU end-to-end: the Llama harness with every decoder linear converted by
quantize_model_linears (HIP W4A16 kernels) against the same model in the
reference's fake mode (dequantized weights in nn.Linear, torch matmul), and
graph-replayed decoding against eager decoding."""
import pytest
import torch

import int4_hip
from int4_hip.llama import GraphDecoder, LlamaConfig, LlamaForCausalLM, argmax_last, run_eval

pytestmark = pytest.mark.gpu
DEV = "cuda"
SMALL = LlamaConfig(vocab_size=1024, hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                    num_attention_heads=8, num_key_value_heads=2, head_dim=64)


def _model(quant: str, seed: int = 0):
    with torch.device(DEV):
        m = LlamaForCausalLM(SMALL)
    m.init_weights(seed)
    m = m.to(torch.bfloat16).eval()
    if quant == "w4":
        int4_hip.quantize_model_linears(m, 128)
    elif quant == "fake":
        int4_hip.quantize_model_linears(m, 128, fake=True)
    m.allocate_cache(96, torch.bfloat16, DEV)
    return m


def test_w4_matches_fake_quant_logits():
    print("[llama] w4 vs fake prefill logits", flush=True)
    ids = torch.randint(0, SMALL.vocab_size, (80,), device=DEV, generator=torch.Generator(DEV).manual_seed(5))
    w4, fake = _model("w4"), _model("fake")
    assert isinstance(w4.model.layers[0].self_attn.q_proj, int4_hip.Int4Linear)
    assert not isinstance(w4.lm_head, int4_hip.Int4Linear)  # skip=("lm_head",)
    a, b = w4.prefill(ids).float(), fake.prefill(ids).float()
    torch.cuda.synchronize()
    # bf16 activations through 2 layers: compare against the logit scale
    err = (a - b).abs().max().item() / b.abs().max().item()
    assert err < 3e-2, err
    assert (a.argmax(-1) == b.argmax(-1)).float().mean().item() > 0.9


def test_graph_decode_matches_eager():
    print("[llama] graph vs eager decode", flush=True)
    ids = torch.randint(0, SMALL.vocab_size, (40,), device=DEV, generator=torch.Generator(DEV).manual_seed(6))
    m = _model("w4", seed=1)
    first = m.prefill(ids)[-1:].argmax(-1)
    eager = GraphDecoder(m, DEV)
    eager.start(first, 40)
    want = [eager.step().clone() for _ in range(24)]
    g = GraphDecoder(m, DEV)
    g.start(first, 40)
    g.capture()
    m.prefill(ids)  # the capture's warm-up steps advanced the cache
    g.start(first, 40)
    got = [g.step().clone() for _ in range(24)]
    torch.cuda.synchronize()
    assert torch.equal(torch.cat(got), torch.cat(want))


@pytest.mark.parametrize("lm_head", [False, True])
def test_run_eval_small(lm_head):
    print(f"[llama] run_eval small lm_head={lm_head}", flush=True)
    r = run_eval(prompt_len=48, new_tokens=8, cfg=SMALL, reps=1, quantize_lm_head=lm_head)
    assert r["linear_weight_bytes"] < r["linear_weight_bytes_before"] / 3
    for k in ("bf16_prefill_tokens_per_s", "w4_prefill_tokens_per_s", "bf16_decode_tokens_per_s",
              "w4_decode_tokens_per_s", "prefill_top1_agreement", "prefill_kl_mean"):
        assert r[k] == r[k] and r[k] >= 0, (k, r[k])
    assert r["vs_fake_prefill_top1_agreement"] > 0.9 and r["vs_fake_prefill_kl_mean"] < 1e-2, r


def test_argmax_last_first_index():
    for seed in range(8):
        g = torch.Generator(DEV).manual_seed(seed)
        x = torch.randint(0, 5, (1, 128256), device=DEV, generator=g).to(torch.bfloat16)
        assert argmax_last(x).item() == x.argmax(-1).item() == (x[0] == x.max()).nonzero()[0].item()
