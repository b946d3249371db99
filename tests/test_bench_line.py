"""The full bench record fits the last 2,000 characters of the run's output (the part of the
output a round-end record keeps), with every contract field and every secondary table."""

from __future__ import annotations

import json

import bench


def _verbose_record() -> dict:
    rows4 = []
    for k, n, bits in ((2048, 2048, 8), (2048, 8192, 8), (8192, 2048, 8), (1152, 1152, 4),
                       (1152, 4608, 4)):
        for m in (1, 8, 32, 64, 512, 544):
            rows4.append([k, n, bits, m, 41.05, 0.1234, 52.31, 24645.4])
    single = [[L, 12.34, 3456.7, 0.4321, 512, 1] for L in bench.SINGLE_SEQ_LENS]
    summ = {"output_tok_per_s": 2384.47, "iterations": 1516, "iteration_ms_p50": 2.024,
            "iteration_ms_p99": 6.221, "ttft_s_p50": 1.979, "ttft_s_p99": 4.0,
            "gpu_busy_s": 4.395}
    return {
        "metric": "paged-attn step KV GB/s (% HBM peak); quant GEMV GB/s; decoder output tok/s",
        "value": 6391.8, "unit": "GB/s", "n_gpus": 1, "steps": 50, "warmup": 10,
        "ms_per_step": 0.1688, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16", "data": "synthetic",
        "config": {"workload": "cfg2", "context_tokens": 131644, "step_bytes": 1078984900,
                   "hbm_frac": 0.799, "plan_us": 32.3, "planner_us": 11.0, "attn_items": 4640,
                   "copy_gbs_1gib": 5112.2},
        "roofline": {"bound": "hbm", "kernel": "attn_decode_kernel", "achieved": 6121.1,
                     "peak": 8000.0, "unit": "GB/s", "frac": 0.7651, "traffic": 1082419000,
                     "algorithmic_bytes": 1078984900, "launch_us": 176.27,
                     "frac_of_gather_ceiling": 0.9842},
        "ceilings": {"stream_read_1GiB_gbs": 5978.0},
        "cpu_baseline": {"value": 10.265, "unit": "GB/s", "cores": 16, "kind": "port",
                         "ms_per_step": 105.11, "sample": "the full cfg2 step ..."},
        "cfg3": {"ms_per_step": 0.2043, "step_bytes": 828473316, "gbs": 4055.8,
                 "hbm_frac": 0.507, "attn_us": 218.4, "items": 1280,
                 "cpu_baseline": {"value": 7.796, "unit": "GB/s", "cores": 16, "kind": "port",
                                  "runs": 28}},
        "single_seq": {"cols": bench.SINGLE_SEQ_COLS, "b1": single, "b2": single},
        "cfg4": {"cols": ["k", "n", "bits", "m", "us", "frac", "ref_us", "cpu_us"],
                 "rows": rows4},
        "lm_head": {"cols": ["m", "us", "vendor_us", "read_us", "frac"],
                    "rows": [[m, 43.65, 58.3, 35.48, 0.5768] for m in (1, 8, 16)]},
        "cfg5": {"requests": 64, "offered_load": dict(summ), "saturated": dict(summ),
                 "weight_bytes": 2014543872,
                 "cpu_baseline": {"value": 3.271, "unit": "output tok/s"}},
    }


def test_full_record_fits_the_output_tail() -> None:
    out = bench.compact_line(_verbose_record())
    text = json.dumps(out, separators=(",", ":"))
    # Numbers here are wider than real ones; the stderr of a run adds ~100 characters.
    assert len(text) <= 1900, len(text)
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
                "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config",
                "roofline", "cpu_baseline"):
        assert key in out, key
    assert {"bound", "achieved", "peak", "unit", "frac", "traffic"} <= set(out["roofline"])
    assert {"value", "unit", "cores", "kind", "sample"} <= set(out["cpu_baseline"])
    assert out["cfg3"]["ms_per_step"] == 0.2043 and out["cfg3"]["hbm_frac"] == 0.507
    assert out["cfg4"]["m"] == [1, 8, 32, 64, 512, 544]
    assert len(out["cfg4"]["us"]) == 5 and all(len(v) == 6 for v in out["cfg4"]["us"].values())
    # One read-probe time per shape, then hipBLASLt at M = 512 and 544.
    assert all(len(v) == 3 for v in out["cfg4"]["ref"].values())
    assert out["single_seq"]["L"] == list(bench.SINGLE_SEQ_LENS)
    assert set(out["cfg5"]) == {"offered", "saturated", "cpu_tok_s"}
