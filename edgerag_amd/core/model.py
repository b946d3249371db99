"""The language decoder over a packed ragged batch: embeddings -> N blocks -> norm -> lm_head.

Same architecture and arithmetic as the reference ``EdgeRagDecoder`` (``edgerag/core/model.py:
31-152``, blocks from ``edgerag/core/layers.py:257-374``): pre-norm blocks, grouped-query attention
with RoPE applied before the cache write (keys are cached post-RoPE, ``layers.py:301-306``),
SwiGLU MLP, fp16 embeddings / norms / lm_head (the quantisation skip list, ``linear.py:229-241``)
and weight-only INT8 or INT4 projections.

What changes is the execution shape. The reference runs one request per forward and one forward
per request per iteration (``serve/executor.py:116-154``). Here every request of an iteration --
chunked-prefill slices and single-token decodes alike -- is packed token-major into one forward:

* q/k/v are one fused quant linear (their rows stacked: exact, each row keeps its codes and scale),
  gate/up another, so a layer runs four weight-streaming launches whatever the batch holds;
* K/V of every new token are scattered into the shared paged pool by slot (``kv_append``);
* attention is one ragged launch over all requests (``paged_attention`` with the step's plan):
  causal inside each chunk, full over the cached prefix, per request -- exactly the per-request
  ``build_causal_mask`` + SDPA of the reference;
* only the rows whose logits are read (each request's last token) go through the final norm and
  the lm_head (the reference's ``last_token_only``, ``model.py:150-152``).
"""

from __future__ import annotations

from dataclasses import dataclass
from functools import partial

import torch
from torch import nn

from edgerag_amd import kernels
from edgerag_amd.core.layers import RMSNorm, RotaryTable
from edgerag_amd.core.linear import LinearBase, QuantLinear
from edgerag_amd.core.quant import QuantConfig
from edgerag_amd.core.spec import ModelSpec


@dataclass
class StepInputs:
    """Device-side inputs of one packed forward (built and uploaded once per step)."""

    token_ids: torch.Tensor  # (T,) int32
    positions: torch.Tensor  # (T,) int32 logical positions
    slots: torch.Tensor  # (T,) int32 pool slot of every new token
    logit_rows: torch.Tensor  # (R',) int32 rows of the packed batch whose logits are needed
    plan: kernels.AttentionPlan | kernels.FixedAttention  # eager plan, or graph-stable staging
    #: (T, hidden) input rows replacing the embedding lookup (prompt embeddings), or None.
    hidden: torch.Tensor | None = None
    #: Every row of the batch emits, in order (``logit_rows`` is then 0..T-1): no row gather.
    all_rows: bool = False


def _config(bits: int, group_size: int | None, in_features: int) -> QuantConfig:
    """``group_size=None`` is per-output-channel quantisation: one group spanning the input."""
    return QuantConfig(group_size=in_features if group_size is None else group_size, bits=bits)


class DecoderLayer(nn.Module):
    def __init__(self, spec: ModelSpec, bits: int, group_size: int | None, device, dtype) -> None:
        super().__init__()
        h, d = spec.hidden_size, spec.head_dim
        self.q_out, self.kv_out = spec.n_q_heads * d, spec.n_kv_heads * d
        self.intermediate = inter = spec.intermediate_size
        self.qkv = QuantLinear(h, self.q_out + 2 * self.kv_out, config=_config(bits, group_size, h),
                               device=device)
        self.o_proj = QuantLinear(self.q_out, h, config=_config(bits, group_size, self.q_out),
                                  device=device)
        self.gate_up = QuantLinear(h, 2 * inter, config=_config(bits, group_size, h), device=device)
        self.down_proj = QuantLinear(inter, h, config=_config(bits, group_size, inter),
                                     device=device)
        self.input_layernorm = RMSNorm(h, spec.rms_norm_eps, device, dtype)
        self.post_attention_layernorm = RMSNorm(h, spec.rms_norm_eps, device, dtype)

    def load(self, q, k, v, o, gate, up, down) -> None:
        """Quantise the reference's seven projection weights (``(out, in)`` each) into the fused
        layout: rows of q/k/v stacked, rows of gate/up stacked."""
        self.qkv.load_weight(torch.cat([q, k, v], dim=0))
        self.o_proj.load_weight(o)
        self.gate_up.load_weight(torch.cat([gate, up], dim=0))
        self.down_proj.load_weight(down)


class EdgeRagDecoder(nn.Module):
    # Largest batch whose q/k/v and gate/up projections use the fused streaming epilogues.
    STREAM_EPILOGUE_MAX_TOKENS = 32
    # Smallest batch whose q/k/v and gate/up projections use the tiled GEMM's fused epilogues.
    TILED_EPILOGUE_MIN_TOKENS = 65

    def __init__(
        self,
        spec: ModelSpec,
        bits: int = 8,
        group_size: int | None = None,
        device: torch.device | str = "cuda",
        dtype: torch.dtype = torch.float16,
    ) -> None:
        """``bits`` 8 or 4; ``group_size=None`` quantises per output channel (
        INT8 per-channel), an integer gives group-wise scales along K."""
        super().__init__()
        self.spec = spec
        self.device = torch.device(device)
        self.dtype = dtype
        self.bits, self.group_size = bits, group_size
        h = spec.hidden_size
        self.embed_tokens = nn.Parameter(
            torch.zeros(spec.vocab_size, h, device=self.device, dtype=dtype), requires_grad=False
        )
        self.layers = nn.ModuleList(
            [DecoderLayer(spec, bits, group_size, self.device, dtype) for _ in range(spec.n_layers)]
        )
        self.norm = RMSNorm(h, spec.rms_norm_eps, self.device, dtype)
        self.lm_head = nn.Parameter(
            torch.zeros(spec.vocab_size, h, device=self.device, dtype=dtype), requires_grad=False
        )
        self.rotary = RotaryTable(spec.head_dim, spec.rope_theta, spec.max_position_embeddings,
                                  self.device, dtype)
        self.scaling = spec.head_dim**-0.5

    # --- weights ----------------------------------------------------------------------------------

    @torch.no_grad()
    def init_random(self, seed: int = 0, std: float = 0.02) -> None:
        """Seeded random weights (no checkpoint is available offline): N(0, std) projections,
        embeddings and lm_head, quantised on the device with the reference's rule; unit norms."""
        g = torch.Generator(device=self.device).manual_seed(seed)
        spec = self.spec
        h, inter = spec.hidden_size, spec.intermediate_size
        q_out, kv_out = spec.n_q_heads * spec.head_dim, spec.n_kv_heads * spec.head_dim

        def w(n, k):
            return torch.randn(n, k, generator=g, device=self.device) * std

        self.embed_tokens.copy_(w(spec.vocab_size, h).to(self.dtype))
        for layer in self.layers:
            layer.load(w(q_out, h), w(kv_out, h), w(kv_out, h), w(h, q_out), w(inter, h),
                       w(inter, h), w(h, inter))
            layer.input_layernorm.weight.fill_(1.0)
            layer.post_attention_layernorm.weight.fill_(1.0)
        self.norm.weight.fill_(1.0)
        self.lm_head.copy_(w(spec.vocab_size, h).to(self.dtype))

    @torch.no_grad()
    def load_quantized(self, weights) -> None:
        """Take already-quantised weights laid out like this decoder (per layer ``qkv``,
        ``o_proj``, ``gate_up``, ``down_proj`` with ``packed``/``scales``, norm weights, fp16
        ``embed_tokens`` and ``lm_head``) without re-quantising."""
        for layer, src in zip(self.layers, weights.layers):
            for name in ("qkv", "o_proj", "gate_up", "down_proj"):
                lin = getattr(src, name)
                getattr(layer, name).load_quantized(lin.packed.to(self.device),
                                                    lin.scales.to(self.device))
            layer.input_layernorm.weight.copy_(src.input_layernorm.weight)
            layer.post_attention_layernorm.weight.copy_(src.post_attention_layernorm.weight)
        self.norm.weight.copy_(weights.norm.weight)
        self.embed_tokens.copy_(weights.embed_tokens)
        self.lm_head.copy_(weights.lm_head)

    def weight_bytes(self) -> int:
        total = 0
        for layer in self.layers:
            for lin in (layer.qkv, layer.o_proj, layer.gate_up, layer.down_proj):
                total += lin.weight_bytes()
        total += 2 * self.embed_tokens.numel() * self.embed_tokens.element_size()
        return total

    # --- forward --------------------------------------------------------------------------------

    def _norm_fused(self, T: int) -> bool:
        """Whether a batch of T tokens runs residual add + RMSNorm inside the projections (decode
        batches: producers ``quant_linear_residual``, consumers with a normed input)."""
        spec, layer = self.spec, self.layers[0]
        h, cfg = spec.hidden_size, layer.o_proj.config
        if self.dtype != torch.float16 or cfg.bits != 8 or T > 16:
            return False
        parts = [kernels.quant_residual_parts(T, lin.in_features, h, 8, lin.config.group_size)
                 for lin in (layer.o_proj, layer.down_proj)]
        gu = layer.gate_up
        return (
            all(0 < p <= 256 for p in parts)
            and kernels.quant_swiglu_fused(T, gu.in_features, gu.out_features, gu.config.bits,
                                           gu.config.group_size, normed=True)
            and kernels.quant_rope_fused(T, layer.qkv.in_features, layer.qkv.config.bits,
                                         layer.qkv.config.group_size, spec.n_q_heads,
                                         spec.n_kv_heads, spec.head_dim, normed=True)
        )

    @torch.inference_mode()
    def forward_hidden(self, step: StepInputs, key_pool: list[torch.Tensor],
                       value_pool: list[torch.Tensor]) -> torch.Tensor:
        """Run every layer over the packed batch; return the final-norm hidden of ``logit_rows``.

        Per layer: fused q/k/v linear with RoPE + KV append (one launch for decode batches, two
        otherwise) -> ragged attention -> o_proj -> residual add + RMSNorm -> fused gate/up linear
        with SiLU * up (one launch for decode batches) -> down_proj -> residual add + the next
        RMSNorm. Decode batches of up to 16 tokens fold each residual add into o_proj / down_proj
        (which update the residual stream in place and leave per-workgroup sums of squares) and
        each RMSNorm into the next projection; otherwise the residual add + RMSNorm is one launch."""
        spec = self.spec
        T = step.token_ids.shape[0]
        d, eps = spec.head_dim, spec.rms_norm_eps
        n_layers = len(self.layers)
        qkv0 = self.layers[0].qkv
        # The fused streaming epilogues (q/k/v + RoPE + append, gate/up + SiLU * up) serve batches
        # of up to 32 tokens; larger batches run the tiled GEMM and the elementwise launch apart,
        # which is faster there.
        # Batches past 64 tokens run the tiled GEMM, whose epilogues take RoPE + append and
        # SiLU * up where the library covers the shape (the same bits as the elementwise launches
        # apart); batches of 33-64 tokens run the projection and the elementwise launch apart.
        stream_epi = T <= self.STREAM_EPILOGUE_MAX_TOKENS
        tiled_epi = T >= self.TILED_EPILOGUE_MIN_TOKENS
        want_rows = ((stream_epi or tiled_epi) and isinstance(qkv0, QuantLinear)
                     and kernels.quant_rope_fused(T, qkv0.in_features, qkv0.config.bits,
                                                  qkv0.config.group_size, spec.n_q_heads,
                                                  spec.n_kv_heads, d, self.dtype))
        rows = None
        w0 = self.layers[0].input_layernorm.weight
        # The residual stream is updated in place, so it is always a fresh tensor of this step.
        if step.hidden is None and kernels.embed_rmsnorm_fits(self.embed_tokens):
            # Token ids: the embedding rows, the first RMSNorm and the step's rotary rows in one
            # launch (the same bits as index_select, rmsnorm and rope_rows).
            hidden, x, rows = kernels.embed_rmsnorm(
                step.token_ids, self.embed_tokens, w0, eps,
                rope=(step.positions, self.rotary.cos, self.rotary.sin) if want_rows else None)
        else:
            hidden = (self.embed_tokens.index_select(0, step.token_ids) if step.hidden is None
                      else step.hidden)
            x = kernels.rmsnorm(hidden, w0, eps)
            if want_rows:
                rows = kernels.rope_rows(step.positions, self.rotary.cos, self.rotary.sin)
        q = torch.empty((T, spec.n_q_heads, d), device=self.device, dtype=self.dtype)
        attn_out = torch.empty_like(q)
        fused = rows is not None and self._norm_fused(T)
        partials = (torch.empty(T * 256, dtype=torch.float32, device=self.device) if fused
                    else None)
        xw = torch.empty_like(hidden) if fused else None  # fp16(norm weight * hidden)
        gu0 = self.layers[0].gate_up
        gemm_swiglu = (tiled_epi and isinstance(gu0, QuantLinear)
                       and self.dtype == torch.float16
                       and kernels.quant_swiglu_fused(T, gu0.in_features, gu0.out_features,
                                                      gu0.config.bits, gu0.config.group_size))
        gemm_rope = tiled_epi and rows is not None
        norm = None  # the normed input of the next q/k/v projection (None: x is normalised)
        for idx, layer in enumerate(self.layers):
            rope_append = layer.qkv.rope_append if stream_epi or gemm_rope else partial(
                LinearBase.rope_append, layer.qkv)
            rope_append(xw if norm is not None else x, step.positions, self.rotary.cos,
                        self.rotary.sin, spec.n_q_heads, spec.n_kv_heads, d, step.slots,
                        key_pool[idx], value_pool[idx], q_out=q, rows=rows, norm=norm)
            if isinstance(step.plan, kernels.FixedAttention):
                step.plan.launch(q, key_pool[idx], value_pool[idx], self.scaling, attn_out)
            else:
                kernels.paged_attention(q, key_pool[idx], value_pool[idx], step.plan,
                                        self.scaling, out=attn_out)
            next_norm = (self.layers[idx + 1].input_layernorm.weight if idx + 1 < n_layers
                         else self.norm.weight)
            if fused:
                parts = layer.o_proj.residual(attn_out.view(T, layer.q_out), hidden, partials,
                                              layer.post_attention_layernorm.weight, xw)
                act = layer.gate_up.swiglu(xw, norm=kernels.NormedInput(partials, parts, eps))
                last = idx + 1 == n_layers
                parts = layer.down_proj.residual(act, hidden, partials,
                                                 None if last else next_norm, None if last else xw)
                if last:
                    x = kernels.rmsnorm(hidden, next_norm, eps)
                else:
                    norm = kernels.NormedInput(partials, parts, eps)
                continue
            o = layer.o_proj(attn_out.view(T, layer.q_out))
            x = kernels.rmsnorm(hidden, layer.post_attention_layernorm.weight, eps, delta=o,
                                h_out=hidden)
            act = (layer.gate_up.swiglu(x) if stream_epi or gemm_swiglu
                   else LinearBase.swiglu(layer.gate_up, x))
            down = layer.down_proj(act)
            x = kernels.rmsnorm(hidden, next_norm, eps, delta=down, h_out=hidden)
        return x if step.all_rows else x.index_select(0, step.logit_rows)

    @torch.inference_mode()
    def logits(self, step: StepInputs, key_pool, value_pool) -> torch.Tensor:
        """``(R', vocab)`` logits of the rows in ``step.logit_rows``."""
        return self.greedy(step, key_pool, value_pool)[0]

    @torch.inference_mode()
    def greedy(self, step: StepInputs, key_pool, value_pool) -> tuple[torch.Tensor, torch.Tensor]:
        """Logits ``(R', vocab)`` of the rows in ``step.logit_rows`` and their greedy tokens
        (int32 ``(R',)``). fp16 batches of up to 16 rows run the fused lm_head GEMV + argmax
        (the 201 MB weight streamed once, no separate argmax pass) where the kernel takes the
        width; others the vendor GEMM and ``edgerag_argmax_rows``."""
        h = self.forward_hidden(step, key_pool, value_pool)
        rows = h.shape[0]
        if self.dtype == torch.float16 and rows >= 1 and kernels.lm_head_fused(h):
            logits = torch.empty((rows, self.spec.vocab_size), dtype=self.dtype,
                                 device=self.device)
            return kernels.lm_head_argmax(h, self.lm_head, logits)
        logits = nn.functional.linear(h, self.lm_head)
        return logits, kernels.argmax_rows(logits)
