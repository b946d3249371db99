"""Model shape: the integers the KV pool, the attention kernels and the linears are sized by.

Field names and the ``n_rep`` / ``kv_bytes_per_token`` arithmetic follow the reference
``ModelSpec`` (``edgerag/core/spec.py:67-140``), so a spec built for the reference constructs
unchanged. The vision-tower fields are accepted (with defaults) but unused: the vision tower is
outside the decoder step.
"""

from __future__ import annotations

from dataclasses import dataclass

DTYPE_BYTES: dict[str, int] = {"float32": 4, "float16": 2, "bfloat16": 2, "int8": 1, "int4": 1}


@dataclass(frozen=True)
class ModelSpec:
    model_id: str
    model_type: str
    n_layers: int
    hidden_size: int
    n_q_heads: int
    n_kv_heads: int
    head_dim: int
    vocab_size: int
    max_position_embeddings: int
    rope_theta: float
    vision_layers: int = 0
    vision_hidden: int = 0
    vision_image_size: int = 0
    vision_patch_size: int = 1
    scale_factor: int = 1
    image_token_id: int = 0
    pad_token_id: int = 2
    rms_norm_eps: float = 1e-5
    intermediate_size: int = 0
    hidden_act: str = "silu"

    def __post_init__(self) -> None:
        if not 0 <= self.pad_token_id < self.vocab_size:
            raise ValueError(
                f"{self.model_id}: pad_token_id={self.pad_token_id} is outside "
                f"vocab_size={self.vocab_size}"
            )

    @property
    def uses_gqa(self) -> bool:
        return self.n_kv_heads < self.n_q_heads

    @property
    def n_rep(self) -> int:
        """Query heads per kv head (1 = MHA)."""
        if self.n_q_heads % self.n_kv_heads:
            raise ValueError(
                f"{self.model_id}: {self.n_q_heads} query heads is not divisible by "
                f"{self.n_kv_heads} kv heads"
            )
        return self.n_q_heads // self.n_kv_heads

    def kv_bytes_per_token(self, dtype: str = "float16") -> int:
        """K and V bytes one token occupies across every layer."""
        return 2 * self.n_layers * self.n_kv_heads * self.head_dim * DTYPE_BYTES[dtype]

    def kv_bytes(self, seq_len: int, batch: int = 1, dtype: str = "float16") -> int:
        return self.kv_bytes_per_token(dtype) * seq_len * batch


#: The SmolLM2-1.7B-shaped text decoder the serving benchmark runs (24 layers, hidden 2048,
#: 32/32 heads of 64, SwiGLU 8192, RoPE theta 130000, vocab 49152).
SMOLLM2_1_7B = ModelSpec(
    model_id="smollm2-1.7b-shaped",
    model_type="llama",
    n_layers=24,
    hidden_size=2048,
    n_q_heads=32,
    n_kv_heads=32,
    head_dim=64,
    vocab_size=49152,
    max_position_embeddings=8192,
    rope_theta=130000.0,
    pad_token_id=2,
    rms_norm_eps=1e-5,
    intermediate_size=8192,
)
