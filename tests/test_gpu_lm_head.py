"""edgerag_lm_head_argmax: the fp16 output head of a decode step with the greedy choice fused in
(edgerag/core/model.py:150-152 + the executor's argmax, edgerag/serve/executor.py:136, :154).

Logits are checked against a float64 product at the linear tolerance (rtol 1e-2 / atol 2e-3,
north_star); tokens exactly against torch.argmax over the written fp16 logits (first index of the
maximum, a NaN counting as the maximum), and against the float64 reference's argmax wherever its
top two are not a near tie.
"""

from __future__ import annotations

import pytest
import torch

from edgerag_amd import _lib, kernels

pytestmark = pytest.mark.gpu

TOL = dict(rtol=1e-2, atol=2e-3)


def _weight(vocab, k, seed, device):
    g = torch.Generator(device=device).manual_seed(seed)
    return (torch.randn(vocab, k, generator=g, device=device) * 0.02).half()


@pytest.mark.parametrize("m", [1, 3, 8, 16])
def test_smollm2_head_logits_and_tokens(device, m) -> None:
    w = _weight(49152, 2048, 1, device)
    g = torch.Generator(device=device).manual_seed(100 + m)
    x = torch.randn(m, 2048, generator=g, device=device).half()
    logits = torch.empty(m, 49152, dtype=torch.float16, device=device)
    _, tokens = kernels.lm_head_argmax(x, w, logits)
    ref = x.double() @ w.double().T
    torch.testing.assert_close(logits.double(), ref, **TOL)
    assert torch.equal(tokens.long(), logits.float().argmax(dim=-1))
    top2 = torch.topk(ref, 2, dim=-1).values
    clear = (top2[:, 0] - top2[:, 1]) > 4e-3
    assert torch.equal(tokens.long()[clear], ref.argmax(dim=-1)[clear])


def test_ties_take_the_first_index_and_nan_wins(device) -> None:
    """Rows 100 and 5000 of the weight are equal and dominant: the tie goes to 100. A NaN row
    (row 777, and a later one) beats everything for the rows where it appears."""
    w = _weight(8192, 256, 2, device)
    w[100] = 0.5
    w[5000] = 0.5
    x = torch.full((4, 256), 0.01, device=device, dtype=torch.float16)
    logits = torch.empty(4, 8192, dtype=torch.float16, device=device)
    _, tokens = kernels.lm_head_argmax(x, w, logits)
    assert tokens.tolist() == [100] * 4
    w[777] = float("nan")
    w[3000] = float("nan")
    _, tokens = kernels.lm_head_argmax(x, w, logits)
    assert tokens.tolist() == [777] * 4
    assert torch.equal(tokens.long(), logits.float().argmax(dim=-1))


@pytest.mark.parametrize("vocab,k,m", [(1000, 64, 5), (64, 32, 16), (49, 96, 2)])
def test_edge_shapes_and_no_logits(device, vocab, k, m) -> None:
    """A vocabulary that is no multiple of the 64-row slices, the smallest k, and the launch
    without logits (tokens only)."""
    w = _weight(vocab, k, 3, device)
    g = torch.Generator(device=device).manual_seed(vocab)
    x = torch.randn(m, k, generator=g, device=device).half()
    logits = torch.empty(m, vocab, dtype=torch.float16, device=device)
    _, t1 = kernels.lm_head_argmax(x, w, logits)
    _, t2 = kernels.lm_head_argmax(x, w)
    assert torch.equal(t1, t2)
    torch.testing.assert_close(logits.double(), x.double() @ w.double().T, **TOL)
    assert torch.equal(t1.long(), logits.float().argmax(dim=-1))


def test_row_limit_and_graph_replay(device) -> None:
    """More than 16 rows is refused; a captured call replays to the eager result."""
    w = _weight(4096, 512, 4, device)
    x = torch.randn(17, 512, device=device).half()
    with pytest.raises(ValueError):
        kernels.lm_head_argmax(x, w)
    lib = _lib.load()
    assert lib.edgerag_lm_head_workspace_bytes(17, 4096) == 0
    x = x[:8].contiguous()
    logits = torch.empty(8, 4096, dtype=torch.float16, device=device)
    tokens = torch.empty(8, dtype=torch.int32, device=device)
    kernels.lm_head_argmax(x, w, logits, tokens)
    eager_l, eager_t = logits.clone(), tokens.clone()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        kernels.lm_head_argmax(x, w, logits, tokens)
    for _ in range(3):
        logits.zero_()
        tokens.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(logits, eager_l) and torch.equal(tokens, eager_t)
