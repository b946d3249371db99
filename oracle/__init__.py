"""CPU oracle -- TEST INFRASTRUCTURE ONLY.

A restatement, in PyTorch-CPU (and a small C file for the byte/integer parts), of the reference
EdgeRAG algorithms on the decoder-step path. Every function cites the reference file:line it
follows (paths relative to the reference checkout, Tejas544/edgerag).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
this package, and only as the checker or the timed CPU baseline -- never as the thing measured
on the GPU or shipped. The product package ``edgerag_amd`` never imports it.

How each function is pinned (beyond "it reads like the reference"):

* ``paged.write_slots`` / ``paged.gather_pool``: closed-form slot arithmetic and a per-token
  brute-force loop (tests/test_oracle_paged.py), plus the C restatement in ``oracle/c``.
* ``attention.paged_attention_reference``: float64 textbook softmax and
  ``F.scaled_dot_product_attention`` over the gathered history, the reference's own boundary
  sweep / poison / GQA / scattered-table / overflow / empty cases (tests/test_oracle_attention.py).
* ``attention.ragged_reference``: the single-chunk, past=0 case equals SDPA ``is_causal=True``;
  float64 brute force of ``k <= past + i``; chunked == unchunked.
* ``quant.*``: the reference test suite's known-answer vectors and error bands, the C
  restatement, and closed forms (tests/test_oracle_quant.py).
* ``model.*``: RMSNorm / RoPE closed forms and small-case float64 comparisons
  (tests/test_oracle_model.py).
"""
