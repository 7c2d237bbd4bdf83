"""A Llama-3.2-1B-architecture decoder, random-initialised from a seed, for the
end-to-end W4A16 check of ``Int4Linear`` / ``quantize_model_linears``.

It stands in for the Hugging Face model that the reference's evaluation script
downloads (benchmarks/eval_llama.py:206-211; no network here): same module
names (``model.layers.{i}.self_attn.q_proj`` ... ``lm_head``), so the
reference's conversion call and its ``skip=("lm_head",)`` rule apply
unchanged, and the same measurements (eval_llama.py:112-183):

  * prefill: one forward over the prompt, writing the static KV cache;
  * decode: greedy single-token steps captured once in a HIP graph, with the
    next-token copy and the position increment inside the graph
    (eval_llama.py:132-143, 162-167);
  * weight bytes of the decoder linears before and after conversion
    (eval_llama.py:52-62).

Layer math follows the Llama architecture: RMSNorm (fp32 statistics), rotary
embeddings with the Llama-3 frequency scaling, grouped-query attention
(32 query / 8 key-value heads of 64), SwiGLU MLP, tied embedding / lm_head.
Attention is computed in fp32 from contiguous operands: the KV cache is fp32
and keeps K transposed ([kv_heads, head_dim, positions]), so no bf16 batched
product with a transposed operand is issued.

With Int4Linear projections, q/k/v (into one buffer when decoding) and
gate/up each go through one grouped W4A16 call (``w4a16_matmul_grouped``), so
a layer makes 4 W4A16 launches instead of 7.
"""
from __future__ import annotations

import math
import time
from dataclasses import dataclass, asdict

import torch
import torch.nn as nn
import torch.nn.functional as F


@dataclass
class LlamaConfig:
    vocab_size: int = 128256
    hidden_size: int = 2048
    intermediate_size: int = 8192
    num_hidden_layers: int = 16
    num_attention_heads: int = 32
    num_key_value_heads: int = 8
    head_dim: int = 64
    rms_norm_eps: float = 1e-5
    rope_theta: float = 500000.0
    # Llama-3 rotary scaling (factor, low/high frequency factors, original context)
    rope_scaling: tuple | None = (32.0, 1.0, 4.0, 8192)
    initializer_range: float = 0.02
    tie_word_embeddings: bool = True


class RMSNorm(nn.Module):
    def __init__(self, n: int, eps: float):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(n))
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        # one fused kernel; fp32 statistics (the weight is applied before the
        # final rounding, where the Hugging Face layer rounds first)
        return F.rms_norm(x, (x.shape[-1],), self.weight, self.eps)


def rope_inv_freq(cfg: LlamaConfig) -> torch.Tensor:
    inv = 1.0 / (cfg.rope_theta ** (torch.arange(0, cfg.head_dim, 2, dtype=torch.float64) / cfg.head_dim))
    if cfg.rope_scaling is not None:
        factor, low, high, orig = cfg.rope_scaling
        wavelen = 2 * math.pi / inv
        low_wl, high_wl = orig / low, orig / high
        smooth = (orig / wavelen - low) / (high - low)
        scaled = torch.where(wavelen > low_wl, inv / factor, inv)
        mid = (wavelen <= low_wl) & (wavelen >= high_wl)
        inv = torch.where(mid, (1 - smooth) * inv / factor + smooth * inv, scaled)
    return inv.float()


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x [T, heads, D]; cos/sin [T, D/2] (fp32).  Rotates the two halves of D; fp32 result."""
    d2 = x.shape[-1] // 2
    xf = x.float()
    x1, x2 = xf[..., :d2], xf[..., d2:]
    c, s = cos[:, None, :], sin[:, None, :]
    return torch.cat((x1 * c - x2 * s, x2 * c + x1 * s), dim=-1)


def _all_int4(mods) -> bool:
    from .qlinear import Int4Linear
    return all(isinstance(m, Int4Linear) for m in mods) and len({m.group_size for m in mods}) == 1


def _grouped(x: torch.Tensor, mods, buf: torch.Tensor | None = None) -> list:
    """Outputs of several Int4Linear (no bias) on one input from one grouped W4A16
    call; with ``buf`` (a single row, [1, sum N]) they are slices of it."""
    from .gemm import w4a16_matmul_grouped
    outs = None
    if buf is not None:
        outs, o = [], 0
        for m in mods:
            outs.append(buf[:, o:o + m.out_features])
            o += m.out_features
    return w4a16_matmul_grouped([x] * len(mods), [(m.qweight, m.scales, m.zeros) for m in mods], out=outs)


class Attention(nn.Module):
    def __init__(self, cfg: LlamaConfig):
        super().__init__()
        h, d = cfg.hidden_size, cfg.head_dim
        self.nh, self.nkv, self.d = cfg.num_attention_heads, cfg.num_key_value_heads, d
        self.q_proj = nn.Linear(h, self.nh * d, bias=False)
        self.k_proj = nn.Linear(h, self.nkv * d, bias=False)
        self.v_proj = nn.Linear(h, self.nkv * d, bias=False)
        self.o_proj = nn.Linear(self.nh * d, h, bias=False)

    def forward(self, x, cos, sin, kc, vc, pos0: int | None, pos_t: torch.Tensor | None, mask_bias):
        """Prefill (pos0 = 0, T tokens) or one decode token (pos_t = device position,
        mask_bias [positions] = 0 up to pos_t, -inf past it)."""
        T = x.shape[0]
        nq, nk = self.nh * self.d, self.nkv * self.d
        g = self.nh // self.nkv
        scale = 1.0 / math.sqrt(self.d)
        mods = (self.q_proj, self.k_proj, self.v_proj)
        if pos_t is None:
            qo, ko, vo = _grouped(x, mods) if _all_int4(mods) else [m(x) for m in mods]
            q = apply_rope(qo.view(T, self.nh, self.d), cos, sin)
            k = apply_rope(ko.view(T, self.nkv, self.d), cos, sin)
            v = vo.view(T, self.nkv, self.d)
            kc[:, :, pos0:pos0 + T] = k.permute(1, 2, 0)
            vc[:, pos0:pos0 + T] = v.transpose(0, 1)
            L = pos0 + T
            kt = kc[:, :, :L].contiguous()                                # [kv, D, L]
            vv = vc[:, :L].contiguous()                                   # [kv, L, D]
            qg = q.view(T, self.nkv, g, self.d).permute(1, 2, 0, 3).reshape(self.nkv, g * T, self.d)
            s = torch.bmm(qg.contiguous(), kt) * scale                    # [kv, g*T, L]
            qpos = torch.arange(T, device=x.device).repeat(g) + pos0
            causal = torch.arange(L, device=x.device)[None, :] > qpos[:, None]
            s = s.masked_fill(causal[None], float("-inf"))
            o = torch.bmm(torch.softmax(s, dim=-1), vv)                   # [kv, g*T, D]
            o = o.view(self.nkv, g, T, self.d).permute(2, 0, 1, 3).reshape(T, nq)
        else:
            if _all_int4(mods):
                qkv = torch.empty((1, nq + 2 * nk), dtype=x.dtype, device=x.device)
                _grouped(x, mods, qkv)
            else:
                qkv = torch.cat([m(x) for m in mods], dim=-1)
            qk = apply_rope(qkv[:, :nq + nk].view(1, self.nh + self.nkv, self.d), cos, sin)[0]
            kc.index_copy_(2, pos_t, qk[self.nh:, :, None])
            vc.index_copy_(1, pos_t, qkv[:, nq + nk:].view(self.nkv, 1, self.d).float())
            s = torch.baddbmm(mask_bias, qk[:self.nh].view(self.nkv, g, self.d), kc, alpha=scale)  # [kv, g, Lmax]
            o = torch.bmm(torch.softmax(s, dim=-1), vc).reshape(1, nq)
        return self.o_proj(o.to(x.dtype))


class MLP(nn.Module):
    def __init__(self, cfg: LlamaConfig):
        super().__init__()
        h, i = cfg.hidden_size, cfg.intermediate_size
        self.gate_proj = nn.Linear(h, i, bias=False)
        self.up_proj = nn.Linear(h, i, bias=False)
        self.down_proj = nn.Linear(i, h, bias=False)

    def forward(self, x):
        if _all_int4((self.gate_proj, self.up_proj)):
            g, u = _grouped(x, (self.gate_proj, self.up_proj))
            return self.down_proj(F.silu(g) * u)
        return self.down_proj(F.silu(self.gate_proj(x)) * self.up_proj(x))


class DecoderLayer(nn.Module):
    def __init__(self, cfg: LlamaConfig):
        super().__init__()
        self.input_layernorm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)
        self.self_attn = Attention(cfg)
        self.post_attention_layernorm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)
        self.mlp = MLP(cfg)


class LlamaBody(nn.Module):
    def __init__(self, cfg: LlamaConfig):
        super().__init__()
        self.embed_tokens = nn.Embedding(cfg.vocab_size, cfg.hidden_size)
        self.layers = nn.ModuleList(DecoderLayer(cfg) for _ in range(cfg.num_hidden_layers))
        self.norm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)


class LlamaForCausalLM(nn.Module):
    """Batch-1 causal LM with a static KV cache of ``max_len`` positions."""

    def __init__(self, cfg: LlamaConfig):
        super().__init__()
        self.config = cfg
        self.model = LlamaBody(cfg)
        self.lm_head = nn.Linear(cfg.hidden_size, cfg.vocab_size, bias=False)
        if cfg.tie_word_embeddings:
            self.lm_head.weight = self.model.embed_tokens.weight
        self.kc = self.vc = None

    @torch.no_grad()
    def init_weights(self, seed: int):
        """N(0, initializer_range) for every linear and the embedding, ones for the norms."""
        g = torch.Generator(device=self.lm_head.weight.device).manual_seed(seed)
        std = self.config.initializer_range
        for m in self.modules():
            if isinstance(m, (nn.Linear, nn.Embedding)):
                m.weight.normal_(0.0, std, generator=g)
            elif isinstance(m, RMSNorm):
                m.weight.fill_(1.0)

    def allocate_cache(self, max_len: int, dtype: torch.dtype, device):
        """Static fp32 KV cache of max_len positions (dtype: the activation dtype)."""
        c = self.config
        nl = c.num_hidden_layers
        self.max_len = max_len
        self.kc = torch.zeros((nl, c.num_key_value_heads, c.head_dim, max_len), dtype=torch.float32, device=device)
        self.vc = torch.zeros((nl, c.num_key_value_heads, max_len, c.head_dim), dtype=torch.float32, device=device)
        inv = rope_inv_freq(c).to(device)
        ang = torch.arange(max_len, device=device, dtype=torch.float32)[:, None] * inv[None, :]
        self.cos, self.sin = ang.cos(), ang.sin()
        self.key_pos = torch.arange(max_len, device=device)

    def _layers(self, x, cos, sin, pos0, pos_t):
        mask_bias = None
        if pos_t is not None:
            mask_bias = torch.zeros(self.max_len, device=x.device).masked_fill_(self.key_pos > pos_t, float("-inf"))
        for i, layer in enumerate(self.model.layers):
            x = x + layer.self_attn(layer.input_layernorm(x), cos, sin, self.kc[i], self.vc[i], pos0, pos_t,
                                    mask_bias)
            x = x + layer.mlp(layer.post_attention_layernorm(x))
        return self.lm_head(self.model.norm(x))

    @torch.no_grad()
    def prefill(self, ids: torch.Tensor) -> torch.Tensor:
        """Logits [T, vocab] of a 1-D prompt; fills cache positions 0..T-1."""
        T = ids.shape[0]
        assert T <= self.max_len
        x = self.model.embed_tokens(ids)
        return self._layers(x, self.cos[:T], self.sin[:T], 0, None)

    @torch.no_grad()
    def decode_step(self, ids: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
        """Logits [1, vocab] of token ids[0] at device position pos[0] (cache updated in place)."""
        x = self.model.embed_tokens(ids)
        cos, sin = self.cos.index_select(0, pos), self.sin.index_select(0, pos)
        return self._layers(x, cos, sin, None, pos)


def linear_weight_bytes(model: nn.Module, include_lm_head: bool = False) -> int:
    """Bytes of the decoder linears' weights (eval_llama.py:52-62)."""
    from .qlinear import Int4Linear
    total = 0
    for name, m in model.named_modules():
        if "lm_head" in name and not include_lm_head:
            continue
        if isinstance(m, Int4Linear):
            total += sum(b.numel() * b.element_size() for b in (m.qweight, m.scales, m.zeros))
        elif isinstance(m, nn.Linear):
            total += m.weight.numel() * m.weight.element_size()
    return total


def model_bytes(model: nn.Module) -> int:
    seen, total = set(), 0
    for t in list(model.parameters()) + list(model.buffers()):
        if t.data_ptr() in seen:  # tied embedding / lm_head
            continue
        seen.add(t.data_ptr())
        total += t.numel() * t.element_size()
    return total


def argmax_last(logits: torch.Tensor) -> torch.Tensor:
    """argmax over the last dim of [1, V] logits (first index of the maximum), as
    two reductions over [V/256, 256] when V allows: one [1, 128256] argmax is a
    single long reduction (tens of microseconds)."""
    V = logits.shape[-1]
    if logits.shape[0] != 1 or V % 256:
        return logits.argmax(-1)
    vals, idx = logits.view(V // 256, 256).max(-1)
    row = vals.argmax(-1, keepdim=True)
    return (row * 256 + idx.gather(0, row)).view(1)


class GraphDecoder:
    """Greedy decoding with one captured step: ids <- argmax(logits), pos += 1
    inside the graph (eval_llama.py:132-143, 162-167)."""

    def __init__(self, model: LlamaForCausalLM, device):
        self.model = model
        self.ids = torch.zeros(1, dtype=torch.long, device=device)
        self.pos = torch.zeros(1, dtype=torch.long, device=device)
        self.graph = None

    def _step(self):
        logits = self.model.decode_step(self.ids, self.pos)
        nxt = argmax_last(logits)
        self.ids.copy_(nxt)
        self.pos.add_(1)
        return nxt

    def start(self, first_token: torch.Tensor, pos: int):
        self.ids.copy_(first_token.reshape(1))
        self.pos.fill_(pos)

    def capture(self):
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):  # warm-up: workspaces and library handles
            for _ in range(2):
                self._step()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        # captured on the warm-up stream: the library's split-K workspace is
        # kept per stream, and the warm-up allocated it for this one
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=side):
            self.out = self._step()

    def step(self) -> torch.Tensor:
        if self.graph is None:
            return self._step()
        self.graph.replay()
        return self.out


@torch.no_grad()
def run_eval(prompt_len: int = 512, new_tokens: int = 128, group_size: int = 128, seed: int = 0,
             cfg: LlamaConfig | None = None, quantize_lm_head: bool = False, reps: int = 3) -> dict:
    """configs[4]-style end-to-end run: bf16 model, then the same weights converted
    with ``quantize_model_linears``; prefill and graph decode timings for both,
    and top-1 / KL agreement of the W4 logits with the bf16 ones."""
    from .qlinear import quantize_model_linears
    dev = torch.device("cuda")
    cfg = cfg or LlamaConfig()
    dtype = torch.bfloat16
    with torch.device(dev):
        model = LlamaForCausalLM(cfg)
    model.init_weights(seed)
    model = model.to(dtype).eval()
    if quantize_lm_head:  # untie: the embedding stays full precision (eval_llama.py:209-211)
        model.lm_head.weight = nn.Parameter(model.lm_head.weight.detach().clone())
    model.allocate_cache(prompt_len + new_tokens + 8, dtype, dev)
    g = torch.Generator(device=dev).manual_seed(seed + 1)
    prompt = torch.randint(0, cfg.vocab_size, (prompt_len,), device=dev, generator=g)

    def measure(tag):
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        model.prefill(prompt)  # warm-up (workspaces, library handles)
        torch.cuda.synchronize()
        best = float("inf")
        for _ in range(reps):
            ev[0].record()
            logits = model.prefill(prompt)
            ev[1].record()
            torch.cuda.synchronize()
            best = min(best, ev[0].elapsed_time(ev[1]))
        dec = GraphDecoder(model, dev)
        dec.start(logits[-1:].argmax(-1), prompt_len)
        dec.capture()
        # re-run the prompt so that the timed decode starts from a clean cache
        logits = model.prefill(prompt)
        dec.start(logits[-1:].argmax(-1), prompt_len)
        toks = []
        torch.cuda.synchronize()
        ev[0].record()
        for _ in range(new_tokens):
            toks.append(dec.step().clone())
        ev[1].record()
        torch.cuda.synchronize()
        dms = ev[0].elapsed_time(ev[1])
        tokens = torch.cat(toks).tolist()
        return logits.float(), tokens, {
            f"{tag}_prefill_ms": best, f"{tag}_prefill_tokens_per_s": prompt_len / best * 1e3,
            f"{tag}_decode_ms_per_token": dms / new_tokens, f"{tag}_decode_tokens_per_s": new_tokens / dms * 1e3,
        }

    res = {"config": asdict(cfg), "prompt_len": prompt_len, "new_tokens": new_tokens, "group_size": group_size,
           "quantize_lm_head": quantize_lm_head, "seed": seed, "data": "synthetic (seeded random weights and prompt)"}
    res["linear_weight_bytes_before"] = linear_weight_bytes(model, quantize_lm_head)
    ref_logits, ref_tokens, r = measure("bf16")
    res.update(r)
    skip = () if quantize_lm_head else ("lm_head",)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    quantize_model_linears(model, group_size, skip=skip)
    torch.cuda.synchronize()
    res["quantize_time_s"] = time.perf_counter() - t0
    res["linear_weight_bytes"] = linear_weight_bytes(model, quantize_lm_head)
    res["model_bytes"] = model_bytes(model)
    w4_logits, w4_tokens, r = measure("w4")
    res.update(r)

    def agree(a, b):
        la, lb = torch.log_softmax(a, -1), torch.log_softmax(b, -1)
        return float((a.argmax(-1) == b.argmax(-1)).float().mean()), float((la.exp() * (la - lb)).sum(-1).mean())

    # quantization error: W4 kernels vs the unquantized bf16 model
    res["prefill_top1_agreement"], res["prefill_kl_mean"] = agree(ref_logits, w4_logits)
    same = [a == b for a, b in zip(ref_tokens, w4_tokens)]
    res["decode_token_agreement"] = sum(same) / len(same)
    res["decode_first_divergence"] = same.index(False) if False in same else len(same)
    # kernel error alone: W4 kernels vs the reference's fake mode (the same int4
    # weights dequantized into nn.Linear, torch matmul)
    dequantize_model_linears(model)
    fake_logits = model.prefill(prompt).float()
    res["vs_fake_prefill_top1_agreement"], res["vs_fake_prefill_kl_mean"] = agree(fake_logits, w4_logits)
    return res


@torch.no_grad()
def dequantize_model_linears(model: nn.Module) -> nn.Module:
    """Replace every Int4Linear by an nn.Linear holding its dequantized weight
    (the state quantize_model_linears(..., fake=True) produces)."""
    from .qlinear import Int4Linear
    for prefix, parent in list(model.named_modules()):
        for name, child in list(parent.named_children()):
            if isinstance(child, Int4Linear):
                w = child.dequantize(torch.bfloat16)
                lin = nn.Linear(child.in_features, child.out_features, bias=child.bias is not None,
                                device=w.device, dtype=w.dtype)
                lin.weight.copy_(w)
                if child.bias is not None:
                    lin.bias.copy_(child.bias)
                setattr(parent, name, lin)
    return model


if __name__ == "__main__":
    import argparse
    import json
    ap = argparse.ArgumentParser(description="random-init Llama-3.2-1B W4A16 end-to-end run")
    ap.add_argument("--prompt-len", type=int, default=512)
    ap.add_argument("--new-tokens", type=int, default=128)
    ap.add_argument("--group-size", type=int, default=128)
    ap.add_argument("--quantize-lm-head", action="store_true")
    a = ap.parse_args()
    print(json.dumps(run_eval(a.prompt_len, a.new_tokens, a.group_size, quantize_lm_head=a.quantize_lm_head)))
