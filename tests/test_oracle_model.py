"""Pins for the decoder oracle (CPU): RMSNorm and RoPE closed forms with planted mistakes caught,
incremental (cached) decoding equal to full recompute, chunked prefill equal to single-shot
(``tests/test_executor.py:114-130`` and ``tests/test_batched.py:80-119`` in the reference)."""

from __future__ import annotations

import math

import torch

from edgerag_amd.core.spec import ModelSpec
from oracle import model as om

TOY = ModelSpec("toy", "llama", 2, 128, 4, 2, 32, 256, 512, 10000.0, pad_token_id=0,
                intermediate_size=256)


def test_rms_norm_closed_form_and_cast_order() -> None:
    x = torch.full((3, 64), 2.0)
    w = torch.linspace(0.5, 1.5, 64)
    eps = 1e-5
    expected = w * (2.0 / math.sqrt(4.0 + eps))
    torch.testing.assert_close(om.rms_norm(x, w, eps), expected.expand(3, 64))
    # fp16: the weight multiplies the already-cast normalised value (layers.py:46-47)
    xh = torch.randn(4, 2048, generator=torch.Generator().manual_seed(0)).half()
    wh = (1 + 0.1 * torch.randn(2048, generator=torch.Generator().manual_seed(1))).half()
    got = om.rms_norm(xh, wh, eps)
    xf = xh.float()
    planted = (wh.float() * (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps))).half()
    assert got.dtype == torch.float16 and not torch.equal(got, planted)


def test_rope_rotates_pairs_and_depends_only_on_relative_position() -> None:
    d, theta = 64, 130000.0
    g = torch.Generator().manual_seed(0)
    q = torch.randn(1, 1, 1, d, generator=g, dtype=torch.float64)
    k = torch.randn(1, 1, 1, d, generator=g, dtype=torch.float64)

    def rot(x, p):
        c, s = om.rope_cos_sin(torch.tensor([p]), d, theta, torch.float64)
        return om.apply_rope(x, c, s)

    half = d // 2
    r = rot(q, 17)
    pair_norm = lambda x: x[..., :half] ** 2 + x[..., half:] ** 2  # noqa: E731
    torch.testing.assert_close(pair_norm(r), pair_norm(q))
    dots = [float((rot(q, m) * rot(k, m - 5)).sum()) for m in (5, 40, 300)]
    assert max(dots) - min(dots) < 1e-4  # fp32 inv_freq, as the reference computes it
    # planted: the interleaved-pairs convention is a different rotation
    c, s = om.rope_cos_sin(torch.tensor([17]), d, theta, torch.float64)
    inter = torch.stack((-q[..., 1::2], q[..., 0::2]), dim=-1).flatten(-2)
    assert not torch.allclose(q * c + inter * s, r)


def test_incremental_decode_equals_full_recompute() -> None:
    o = om.OracleDecoder(om.random_weights(TOY, 3), torch.float64)
    ids = list(range(3, 40))
    full = o.forward(ids)
    o.reset()
    o.forward(ids[:30])
    step = [o.forward([t])[-1] for t in ids[30:]]
    torch.testing.assert_close(torch.stack(step), full[30:], rtol=1e-9, atol=1e-9)


def test_chunked_prefill_equals_single_shot_generation() -> None:
    o = om.OracleDecoder(om.random_weights(TOY, 4), torch.float32)
    prompt = list(range(7, 47))
    ref = o.generate(prompt, 6)
    for chunk in (1, 4, 16):
        assert o.generate(prompt, 6, chunk_size=chunk) == ref
