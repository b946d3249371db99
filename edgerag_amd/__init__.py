"""edgerag_amd: MI355X-native ragged decoder step for EdgeRAG.

Slot-mapped KV append, fused paged attention over mixed decode / chunked-prefill batches, and
weight-only INT8 / INT4 linears, as hand-written gfx950 HIP kernels behind a C ABI
(``include/edgerag_amd.h``), with a Python host layer that mirrors the reference's seams
(``PagedKVCache``, ``fused_paged_attention``, ``QuantLinear``, ``ModelExecutor``).
"""

__version__ = "0.1.0"
