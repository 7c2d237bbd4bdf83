"""GPU end-to-end: the Llama harness with every decoder linear converted by
quantize_model_linears (HIP W4A16 kernels) against the same model in the
reference's fake mode (dequantized weights in nn.Linear, torch matmul), and
graph-replayed decoding against eager decoding -- on a small model and on the
full Llama-3.2-1B architecture; and the on-disk format
of Int4Linear (state_dict save -> weights-only load -> same output bits)."""
import copy
import io
from pathlib import Path

import numpy as np
import pytest
import torch

import int4_hip
from _checks import _check, _decode
from _synth import randn
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


# ----------------------------------------------------------------- on-disk format
# int4_triton/qlinear.py:18-21 registers qweight/scales/zeros/bias as buffers in
# the GPTQ-style layout of int4_triton/quantize.py:8-12, so a state dict carries
# a quantized layer
@pytest.mark.parametrize("bias", [False, True])
def test_int4linear_state_dict_round_trip(bias):
    print(f"[state dict] bias={bias}", flush=True)
    lin = torch.nn.Linear(2048, 512, bias=bias, dtype=torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(randn((512, 2048), seed=31, sigma=0.02))
        if bias:
            lin.bias.copy_(randn((512,), seed=32, sigma=0.1))
    q = int4_hip.Int4Linear.from_linear(lin.to(DEV), 128)
    x = randn((3, 7, 2048), seed=33).to(DEV)
    want = q(x)
    blob = io.BytesIO()
    torch.save(q.state_dict(), blob)
    for where in (DEV, "cpu"):  # loaded onto the GPU directly, or onto the CPU and moved
        blob.seek(0)
        sd = torch.load(blob, map_location=where, weights_only=True)
        assert list(sd) == (["qweight", "scales", "zeros"] + (["bias"] if bias else []))
        fresh = int4_hip.Int4Linear(2048, 512, group_size=128, bias=bias, device=where)
        fresh.load_state_dict(sd)
        if where == "cpu":  # dequantize works on the CPU copy, bit-identical to the GPU kernel
            assert torch.equal(fresh.dequantize().view(torch.int16).to(DEV),
                               q.dequantize().view(torch.int16))
            fresh = fresh.to(DEV)
        got = fresh(x)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), where


def test_int4linear_from_reference_written_buffers():
    """Buffers the reference's own quantize_int4_ref wrote (tests/golden) load
    into an Int4Linear; its forward matches the CPU oracle on them."""
    g = np.load(Path(__file__).resolve().parent / "golden" / "quantize_golden.npz")
    name = "normal_bf16_g128"
    qw = torch.from_numpy(g[name + "__qweight"])
    s = torch.from_numpy(g[name + "__scales"].astype(np.int16)).view(torch.float16)
    z = torch.from_numpy(g[name + "__zeros"].astype(np.int16)).view(torch.float16)
    K, N = qw.shape[0] * 8, qw.shape[1]
    layer = int4_hip.Int4Linear(K, N, group_size=K // s.shape[0], device=DEV)
    layer.load_state_dict({"qweight": qw, "scales": s, "zeros": z})
    for M in (1, 5, 40, 130):
        print(f"[golden buffers] M={M}", flush=True)
        x = randn((M, K), seed=40 + M).to(DEV)
        _check(layer(x), x, layer.qweight, layer.scales, layer.zeros, ref_unrounded=False,
               exact_w=_decode(M, K // s.shape[0], N, K))


# ------------------------------------------------- full-size Llama-3.2-1B
def test_llama_1b_full_size_w4_vs_fake_and_graph_decode():
    """LlamaConfig() defaults: 16 layers, hidden 2048, 32/8 heads of 64, SwiGLU
    8192, vocab 128256, tied embedding, RMSNorm 1e-5, RoPE theta 500000; every
    decoder linear an Int4Linear (G=128).  A 512-token prefill against the same
    model in fake mode (same int4 weights dequantized into nn.Linear, torch
    bf16 matmul), then graph-replayed greedy decoding against eager decoding
    (eval_llama.py:120-183)."""
    cfg = LlamaConfig()
    assert (cfg.num_hidden_layers, cfg.hidden_size, cfg.vocab_size) == (16, 2048, 128256)
    print("[llama-1b] building", flush=True)
    with torch.device(DEV):
        base = LlamaForCausalLM(cfg)
    base.init_weights(0)
    base = base.to(torch.bfloat16).eval()
    fake = copy.deepcopy(base)
    w4 = int4_hip.quantize_model_linears(base, 128)
    int4_hip.quantize_model_linears(fake, 128, fake=True)
    assert sum(isinstance(m, int4_hip.Int4Linear) for m in w4.modules()) == 7 * 16
    prompt_len, steps = 512, 16
    for m in (w4, fake):
        m.allocate_cache(prompt_len + 2 * steps + 8, torch.bfloat16, DEV)
    ids = torch.randint(0, cfg.vocab_size, (prompt_len,), device=DEV, generator=torch.Generator(DEV).manual_seed(3))
    print("[llama-1b] prefill w4 vs fake", flush=True)
    a = w4.prefill(ids).float()
    b = fake.prefill(ids).float()
    del fake
    rel = ((a - b).abs().max() / b.abs().max()).item()
    la, lb = torch.log_softmax(a, -1), torch.log_softmax(b, -1)
    kl = (lb.exp() * (lb - la)).sum(-1).mean().item()
    top1 = (a.argmax(-1) == b.argmax(-1)).float().mean().item()
    print(f"[llama-1b] max rel logit err {rel:.3e}, KL {kl:.3e}, top-1 {top1:.4f}", flush=True)
    assert rel < 5e-2 and kl < 1e-3 and top1 > 0.9, (rel, kl, top1)
    del la, lb, b
    print("[llama-1b] eager vs graph decode", flush=True)
    first = a[-1:].argmax(-1)
    eager = GraphDecoder(w4, DEV)
    eager.start(first, prompt_len)
    want = [eager.step().clone() for _ in range(steps)]
    w4.prefill(ids)
    g = GraphDecoder(w4, DEV)
    g.start(first, prompt_len)
    g.capture()
    w4.prefill(ids)  # the capture's warm-up steps advanced the cache
    g.start(first, prompt_len)
    got = [g.step().clone() for _ in range(steps)]
    torch.cuda.synchronize()
    assert torch.equal(torch.cat(got), torch.cat(want))
