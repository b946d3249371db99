"""Committed golden fixtures (tests/golden/): config 1 decode step and small INT8/INT4 quant cases.

CPU tests: the oracle still reproduces the fixtures (a change in the oracle, or in torch's
arithmetic, shows up here). GPU tests: the HIP kernels, called through the C ABI, reproduce them --
slot writes and quantisation bit for bit, fp32 attention within 1e-5, the linear within the
north_star rtol 1e-2 (fp16) and 1e-5 (fp32 activations).
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import paged as op
from oracle import quant as oq
from tests.golden.make_golden import CFG1, cfg1_inputs, quant_inputs

GOLDEN = Path(__file__).resolve().parent / "golden"


def _cfg1():
    return dict(np.load(GOLDEN / "cfg1_decode.npz"))


def _quant():
    return dict(np.load(GOLDEN / "quant_small.npz"))


def _tables(bt: np.ndarray) -> list[list[int]]:
    return [[int(b) for b in row if b >= 0] for row in bt]


def test_cfg1_inputs_are_the_frozen_ones() -> None:
    fx = _cfg1()
    kp, vp, tables, new_k, new_v, q, slots = cfg1_inputs()
    assert tables == _tables(fx["block_tables"])
    assert np.array_equal(slots, fx["slots"])
    assert np.array_equal(new_k, fx["new_k"]) and np.array_equal(q, fx["q"])
    assert abs(float(kp.std()) - 1.0) < 0.02 and abs(float(kp.mean())) < 0.02  # N(0, 1)


def test_oracle_reproduces_cfg1_fixture() -> None:
    fx = _cfg1()
    kp, vp, tables, new_k, new_v, q, slots = cfg1_inputs()
    kpt, vpt = torch.from_numpy(kp), torch.from_numpy(vp)
    lens = fx["lens"].tolist()
    for r, L in enumerate(lens):
        op.write_slots(kpt, torch.from_numpy(new_k[r : r + 1]).transpose(0, 1)[None], tables[r], L - 1)
        op.write_slots(vpt, torch.from_numpy(new_v[r : r + 1]).transpose(0, 1)[None], tables[r], L - 1)
    bs = CFG1["bs"]
    assert np.array_equal(kpt.numpy()[:, slots // bs, slots % bs], fx["k_rows"])
    assert np.array_equal(vpt.numpy()[:, slots // bs, slots % bs], fx["v_rows"])
    out = oa.ragged_reference(torch.from_numpy(q), kpt, vpt, list(range(len(lens) + 1)), lens,
                              tables, CFG1["scale"])
    torch.testing.assert_close(out, torch.from_numpy(fx["out"]), rtol=0, atol=1e-6)


@pytest.mark.parametrize("bits,g", [(8, 256), (4, 128)])
def test_oracle_reproduces_quant_fixture(bits, g) -> None:
    fx = _quant()
    w, x = quant_inputs()
    cfg = oq.QuantConfig(group_size=g, bits=bits)
    codes, scales = oq.quantize_groupwise(torch.from_numpy(w), cfg)
    packed, _ = oq.quantize_for_layer(torch.from_numpy(w), cfg)
    tag = f"int{bits}"
    assert np.array_equal(codes.numpy(), fx[f"{tag}_codes"])
    assert np.array_equal(packed.numpy(), fx[f"{tag}_packed"])
    assert np.array_equal(scales.numpy().view(np.int16), fx[f"{tag}_scales"].view(np.int16))
    deq = oq.dequantize_groupwise(codes, scales, cfg)
    assert np.array_equal(deq.numpy().view(np.int16), fx[f"{tag}_deq"].view(np.int16))


@pytest.mark.gpu
def test_kernels_reproduce_cfg1_fixture(device) -> None:
    from edgerag_amd import kernels
    from edgerag_amd.cache.fused import ragged_paged_attention

    fx = _cfg1()
    kp, vp, tables, new_k, new_v, q, slots = cfg1_inputs()
    dk, dv = torch.from_numpy(kp).to(device), torch.from_numpy(vp).to(device)
    kernels.kv_append(torch.from_numpy(new_k).to(device), torch.from_numpy(new_v).to(device),
                      torch.from_numpy(slots).to(device), dk, dv)
    bs = CFG1["bs"]
    assert np.array_equal(dk.cpu().numpy()[:, slots // bs, slots % bs], fx["k_rows"])
    assert np.array_equal(dv.cpu().numpy()[:, slots // bs, slots % bs], fx["v_rows"])
    # every other slot of the pool is untouched
    mask = np.ones((CFG1["nb"], bs), bool)
    mask[slots // bs, slots % bs] = False
    assert np.array_equal(dk.cpu().numpy()[:, mask], kp[:, mask])
    lens = fx["lens"]
    out = ragged_paged_attention(torch.from_numpy(q).to(device), dk, dv,
                                 np.arange(len(lens) + 1, dtype=np.int32), lens,
                                 fx["block_tables"], CFG1["scale"])
    torch.testing.assert_close(out.cpu(), torch.from_numpy(fx["out"]), rtol=0, atol=1e-5)


@pytest.mark.gpu
@pytest.mark.parametrize("bits,g", [(8, 256), (4, 128)])
def test_kernels_reproduce_quant_fixture(device, bits, g) -> None:
    from edgerag_amd import kernels

    fx = _quant()
    w, x = quant_inputs()
    tag = f"int{bits}"
    packed, scales = kernels.quantize(torch.from_numpy(w).to(device), bits, g)
    assert np.array_equal(packed.cpu().numpy(), fx[f"{tag}_packed"])
    assert np.array_equal(scales.cpu().numpy().view(np.int16), fx[f"{tag}_scales"].view(np.int16))
    deq = kernels.dequantize(packed, scales, 256, bits, g)
    assert np.array_equal(deq.cpu().numpy().view(np.int16), fx[f"{tag}_deq"].view(np.int16))
    y = kernels.quant_linear(torch.from_numpy(x).to(device), packed, scales, None, 256, 64, bits, g)
    torch.testing.assert_close(y.float().cpu(), torch.from_numpy(fx[f"{tag}_y"]), rtol=1e-2,
                               atol=2e-3)
    y32 = kernels.quant_linear(torch.from_numpy(x).float().to(device), packed, scales, None, 256,
                               64, bits, g)
    torch.testing.assert_close(y32.cpu(), torch.from_numpy(fx[f"{tag}_y"]), rtol=1e-5, atol=1e-5)
