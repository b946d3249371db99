"""Oracle for the decoder forward and greedy generation (TEST INFRASTRUCTURE ONLY).

A CPU restatement of the reference ``EdgeRagDecoder`` (``edgerag/core/model.py:72-152``) and its
blocks (``edgerag/core/layers.py:27-374``) for one request, with a plain concatenating KV cache:

* :func:`rms_norm` -- ``layers.py:40-47`` (fp32 variance, cast before the weight multiply);
* :func:`rope_cos_sin` -- ``layers.py:64-90`` (``inv_freq @ positions`` in fp32, ``cat(f, f)``);
* :func:`apply_rope` -- ``layers.py:93-114`` (halves convention, ``[-x2, x1]``);
* :class:`OracleDecoder.forward` -- ``model.py:105-152`` with ``Attention.forward``
  (``layers.py:285-322``: projections, RoPE before the cache write, ``sdpa_attention`` with
  ``build_causal_mask(S, past)``), ``SwiGLUMLP`` (``:341``) and ``DecoderLayer`` (``:360-374``);
  quant projections are ``dequantize -> F.linear`` (``linear.py:186-196``).

Weights are taken from a built ``edgerag_amd`` decoder (the packed codes and fp16 scales it
quantised, its fp16 embeddings, norms and lm_head), so both sides run the same numbers; the oracle
evaluates in float32 (or float64) on the CPU.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F

from oracle import attention as oa
from oracle import quant as oq


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    input_dtype = x.dtype
    xf = x.to(torch.float32)
    variance = xf.pow(2).mean(-1, keepdim=True)
    xf = xf * torch.rsqrt(variance + eps)
    return weight * xf.to(input_dtype)


def rope_cos_sin(positions: torch.Tensor, head_dim: int, theta: float,
                 dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor]:
    """``(S, d)`` cos/sin for logical ``positions (S,)``."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim))
    freqs = (inv_freq[:, None] @ positions[None, :].float()).T
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """``x (1, H, S, d)``, ``cos``/``sin`` ``(S, d)``."""
    return x * cos[None, None] + rotate_half(x) * sin[None, None]


@dataclass
class LayerWeights:
    wq: torch.Tensor
    wk: torch.Tensor
    wv: torch.Tensor
    wo: torch.Tensor
    wgate: torch.Tensor
    wup: torch.Tensor
    wdown: torch.Tensor
    norm1: torch.Tensor
    norm2: torch.Tensor


class OracleDecoder:
    """Reference-semantics decoder for one request at a time, on the CPU."""

    def __init__(self, model, dtype: torch.dtype = torch.float32) -> None:
        spec = model.spec
        self.spec = spec
        self.dtype = dtype
        d = spec.head_dim
        q_out, kv_out = spec.n_q_heads * d, spec.n_kv_heads * d
        inter = spec.intermediate_size

        def deq(lin):
            w = oq.dequantized(lin.packed.detach().cpu(), lin.scales.detach().cpu(),
                               lin.in_features,
                               oq.QuantConfig(lin.config.group_size, lin.config.bits))
            return w.to(dtype)

        self.layers = []
        for layer in model.layers:
            wqkv, wgu = deq(layer.qkv), deq(layer.gate_up)
            self.layers.append(LayerWeights(
                wq=wqkv[:q_out], wk=wqkv[q_out : q_out + kv_out], wv=wqkv[q_out + kv_out :],
                wo=deq(layer.o_proj), wgate=wgu[:inter], wup=wgu[inter:],
                wdown=deq(layer.down_proj),
                norm1=layer.input_layernorm.weight.detach().cpu().to(dtype),
                norm2=layer.post_attention_layernorm.weight.detach().cpu().to(dtype)))
        self.embed = model.embed_tokens.detach().cpu().to(dtype)  # model or random_weights()
        self.norm = model.norm.weight.detach().cpu().to(dtype)
        self.lm_head = model.lm_head.detach().cpu().to(dtype)
        self.reset()

    def reset(self) -> None:
        self.k_cache: list[torch.Tensor | None] = [None] * len(self.layers)
        self.v_cache: list[torch.Tensor | None] = [None] * len(self.layers)
        self.seq_len = 0

    @torch.no_grad()
    def forward(self, token_ids: list[int]) -> torch.Tensor:
        """Append ``token_ids`` to the cache; return their logits ``(S, vocab)``."""
        spec = self.spec
        S, d = len(token_ids), spec.head_dim
        past = self.seq_len
        hidden = self.embed[torch.tensor(token_ids)][None]  # (1, S, h)
        cos, sin = rope_cos_sin(torch.arange(past, past + S), d, spec.rope_theta, self.dtype)
        mask = oa.build_causal_mask(S, past, self.dtype)
        for i, w in enumerate(self.layers):
            x = rms_norm(hidden, w.norm1, spec.rms_norm_eps)
            q = F.linear(x, w.wq).view(1, S, spec.n_q_heads, d).transpose(1, 2)
            k = F.linear(x, w.wk).view(1, S, spec.n_kv_heads, d).transpose(1, 2)
            v = F.linear(x, w.wv).view(1, S, spec.n_kv_heads, d).transpose(1, 2)
            q, k = apply_rope(q, cos, sin), apply_rope(k, cos, sin)
            self.k_cache[i] = k if self.k_cache[i] is None else torch.cat([self.k_cache[i], k], 2)
            self.v_cache[i] = v if self.v_cache[i] is None else torch.cat([self.v_cache[i], v], 2)
            attn = oa.sdpa_attention(q, self.k_cache[i], self.v_cache[i], mask, d**-0.5,
                                     spec.n_rep)
            hidden = hidden + F.linear(attn.reshape(1, S, -1), w.wo)
            x = rms_norm(hidden, w.norm2, spec.rms_norm_eps)
            hidden = hidden + F.linear(F.silu(F.linear(x, w.wgate)) * F.linear(x, w.wup), w.wdown)
        self.seq_len += S
        return F.linear(rms_norm(hidden, self.norm, spec.rms_norm_eps), self.lm_head)[0]

    def generate(self, prompt: list[int], max_new_tokens: int,
                 chunk_size: int | None = None) -> list[int]:
        """Greedy generation the reference executor performs: (chunked) prefill, the first token
        from the last prompt position, then one token per step."""
        self.reset()
        chunk = chunk_size or len(prompt)
        logits = None
        for start in range(0, len(prompt), chunk):
            logits = self.forward(prompt[start : start + chunk])
        out = [int(logits[-1].argmax())]
        while len(out) < max_new_tokens:
            out.append(int(self.forward([out[-1]])[-1].argmax()))
        return out


def random_weights(spec, seed: int, bits: int = 8, group_size: int | None = None,
                   std: float = 0.02, dtype: torch.dtype = torch.float16):
    """Seeded CPU weights in the layout an ``edgerag_amd`` decoder holds (fused q/k/v and
    gate/up rows, quantised with the reference rule), as plain namespaces. Norm weights are
    ``1 + 0.1 N(0,1)`` so a norm applied in the wrong place changes the answer."""
    from types import SimpleNamespace

    g = torch.Generator().manual_seed(seed)
    h, d, inter = spec.hidden_size, spec.head_dim, spec.intermediate_size
    q_out, kv_out = spec.n_q_heads * d, spec.n_kv_heads * d

    def lin(n, k):
        cfg = oq.QuantConfig(k if group_size is None else group_size, bits)
        packed, scales = oq.quantize_for_layer(torch.randn(n, k, generator=g) * std, cfg)
        return SimpleNamespace(packed=packed, scales=scales, in_features=k,
                               config=SimpleNamespace(group_size=cfg.group_size, bits=bits))

    def norm():
        return SimpleNamespace(weight=(1 + 0.1 * torch.randn(h, generator=g)).to(dtype))

    layers = [SimpleNamespace(qkv=lin(q_out + 2 * kv_out, h), o_proj=lin(h, q_out),
                              gate_up=lin(2 * inter, h), down_proj=lin(h, inter),
                              input_layernorm=norm(), post_attention_layernorm=norm())
              for _ in range(spec.n_layers)]
    return SimpleNamespace(
        spec=spec, layers=layers, norm=norm(),
        embed_tokens=(torch.randn(spec.vocab_size, h, generator=g) * std).to(dtype),
        lm_head=(torch.randn(spec.vocab_size, h, generator=g) * std).to(dtype),
    )
