"""Oracle for decode / chunked-prefill attention over the paged pool (test infrastructure only).

Restates, in torch CPU:

* ``repeat_kv`` -- ``edgerag/core/layers.py:117-134`` (consecutive, repeat_interleave order);
* ``build_causal_mask`` -- ``edgerag/core/layers.py:227-254`` (additive, ``finfo.min``);
* ``sdpa_attention`` -- ``edgerag/core/layers.py:137-167``;
* ``eager_attention`` -- ``edgerag/core/layers.py:192-224`` (fp32 softmax, cast back);
* ``paged_attention_reference`` -- ``edgerag/cache/fused.py:89-167`` (blockwise online softmax);
* ``sdpa_over_gather`` -- ``tests/test_fused_attention.py:44-65``;
* ``ragged_reference`` -- the per-request loop of ``ModelExecutor.execute``
  (``edgerag/serve/executor.py:116-154``): each request's queries attend its gathered history
  through ``build_causal_mask(c, L - c)``.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from oracle.paged import gather_pool


def repeat_kv(x: torch.Tensor, n_rep: int) -> torch.Tensor:
    """``(B, H_kv, S, d) -> (B, H_kv * n_rep, S, d)``, each kv head repeated consecutively."""
    if n_rep == 1:
        return x
    b, h, s, d = x.shape
    return x[:, :, None].expand(b, h, n_rep, s, d).reshape(b, h * n_rep, s, d)


def build_causal_mask(seq_len: int, past_len: int, dtype: torch.dtype) -> torch.Tensor:
    """``(1, 1, S, past+S)``: 0 where ``k <= past + i``, ``finfo(dtype).min`` elsewhere."""
    total = past_len + seq_len
    q_pos = torch.arange(past_len, total).unsqueeze(1)
    k_pos = torch.arange(total).unsqueeze(0)
    mask = torch.zeros((seq_len, total), dtype=dtype).masked_fill_(k_pos > q_pos,
                                                                   torch.finfo(dtype).min)
    return mask[None, None]


def sdpa_attention(q, k, v, attn_mask, scaling: float, n_rep: int) -> torch.Tensor:
    """layers.py:137-167 -> ``(B, S, H_q, d)``."""
    k = repeat_kv(k, n_rep)
    v = repeat_kv(v, n_rep)
    if attn_mask is not None:
        attn_mask = attn_mask[..., : k.shape[-2]]
    out = F.scaled_dot_product_attention(q, k, v, attn_mask=attn_mask, scale=scaling)
    return out.transpose(1, 2).contiguous()


def eager_attention(q, k, v, attn_mask, scaling: float, n_rep: int) -> torch.Tensor:
    """layers.py:192-224: explicit scores, fp32 softmax, cast to the query dtype."""
    k = repeat_kv(k, n_rep)
    v = repeat_kv(v, n_rep)
    w = torch.matmul(q, k.transpose(2, 3)) * scaling
    if attn_mask is not None:
        w = w + attn_mask[..., : k.shape[-2]]
    w = F.softmax(w, dim=-1, dtype=torch.float32).to(q.dtype)
    return torch.matmul(w, v).transpose(1, 2).contiguous()


def paged_attention_reference(
    query: torch.Tensor,
    key_pool: torch.Tensor,
    value_pool: torch.Tensor,
    block_ids: torch.Tensor,
    seq_len: int,
    scaling: float,
    n_rep: int = 1,
) -> torch.Tensor:
    """fused.py:89-167: walk the blocks, carry (max, denom, acc) in fp32, divide at the end."""
    if query.shape[2] != 1:
        raise ValueError(
            f"fused paged attention is the decode path: expected 1 query position, got "
            f"{query.shape[2]}"
        )
    n_kv_heads, _, block_size, head_dim = key_pool.shape
    n_q_heads = query.shape[1]
    if n_q_heads != n_kv_heads * n_rep:
        raise ValueError(f"{n_q_heads} query heads against {n_kv_heads} kv heads at n_rep={n_rep}")
    if seq_len <= 0:
        return torch.zeros((1, 1, n_q_heads, head_dim), dtype=query.dtype)

    q = query[0, :, 0, :].float()
    m = torch.full((n_q_heads,), -math.inf)
    denom = torch.zeros(n_q_heads)
    acc = torch.zeros(n_q_heads, head_dim)
    for logical, block in enumerate(block_ids.tolist()):
        start = logical * block_size
        valid = min(block_size, seq_len - start)
        if valid <= 0:
            break
        keys = key_pool[:, block, :valid].float()
        values = value_pool[:, block, :valid].float()
        if n_rep > 1:
            keys = keys.repeat_interleave(n_rep, dim=0)
            values = values.repeat_interleave(n_rep, dim=0)
        scores = torch.einsum("hd,hkd->hk", q, keys) * scaling
        new_m = torch.maximum(m, scores.max(dim=-1).values)
        alpha = torch.nan_to_num(torch.exp(m - new_m), nan=0.0)
        probs = torch.exp(scores - new_m.unsqueeze(-1))
        denom = denom * alpha + probs.sum(dim=-1)
        acc = acc * alpha.unsqueeze(-1) + torch.einsum("hk,hkd->hd", probs, values)
        m = new_m
    out = acc / denom.clamp_min(torch.finfo(torch.float32).tiny).unsqueeze(-1)
    return out.to(query.dtype).reshape(1, 1, n_q_heads, head_dim)


def sdpa_over_gather(query, key_pool, value_pool, block_ids, seq_len, scaling, n_rep):
    """test_fused_attention.py:44-65: gather, slice, repeat_interleave, SDPA."""
    n_kv_heads, _, _, head_dim = key_pool.shape
    keys = key_pool[:, block_ids].reshape(n_kv_heads, -1, head_dim)[:, :seq_len].unsqueeze(0)
    values = value_pool[:, block_ids].reshape(n_kv_heads, -1, head_dim)[:, :seq_len].unsqueeze(0)
    if n_rep > 1:
        keys = keys.repeat_interleave(n_rep, dim=1)
        values = values.repeat_interleave(n_rep, dim=1)
    out = F.scaled_dot_product_attention(query, keys, values, scale=scaling)
    return out.transpose(1, 2).contiguous()


def ragged_reference(
    query: torch.Tensor,
    key_pool: torch.Tensor,
    value_pool: torch.Tensor,
    query_start_loc: list[int],
    context_lens: list[int],
    block_tables: list[list[int]],
    scaling: float,
) -> torch.Tensor:
    """Per request: gather (paged.py:229-238), causal mask (layers.py:227-254), SDPA in fp32.

    ``query`` is packed ``(T, H_q, d)``; returns fp32 ``(T, H_q, d)``. Inputs are upcast to fp32
    first, so an fp16 pool is compared against exact fp32 arithmetic on the same fp16 values.
    """
    n_kv_heads = key_pool.shape[0]
    n_q_heads, head_dim = query.shape[1], query.shape[2]
    n_rep = n_q_heads // n_kv_heads
    out = torch.zeros(query.shape, dtype=torch.float32)
    for r, table in enumerate(block_tables):
        q0, q1 = query_start_loc[r], query_start_loc[r + 1]
        c, L = q1 - q0, context_lens[r]
        if c == 0:
            continue
        k = gather_pool(key_pool, table, L).float().unsqueeze(0)
        v = gather_pool(value_pool, table, L).float().unsqueeze(0)
        q = query[q0:q1].float().transpose(0, 1).unsqueeze(0)  # (1, H_q, c, d)
        mask = build_causal_mask(c, L - c, torch.float32)
        out[q0:q1] = sdpa_attention(q, k, v, mask, scaling, n_rep)[0]
    return out


def attention_f64(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, past_len: int,
                  scaling: float) -> torch.Tensor:
    """Textbook float64 softmax attention for one head: the closed form that pins the rest.

    ``q (c, d)``, ``k/v (L, d)``; query ``i`` sees keys ``[0, past_len + i]``.
    """
    q, k, v = q.double(), k.double(), v.double()
    s = (q @ k.T) * scaling
    c, L = s.shape
    visible = torch.arange(L)[None, :] <= (past_len + torch.arange(c))[:, None]
    s = torch.where(visible, s, torch.tensor(-math.inf, dtype=torch.float64))
    p = torch.exp(s - s.max(dim=-1, keepdim=True).values)
    p = torch.where(visible, p, torch.zeros((), dtype=torch.float64))
    return (p @ v) / p.sum(dim=-1, keepdim=True)
