"""`DeBERTaV2Configuration` (Configuration.swift:3-48)."""

from __future__ import annotations

from dataclasses import dataclass

from . import _native as N


@dataclass(frozen=True)
class DeBERTaV2Configuration:
    hidden_size: int = 1024
    intermediate_size: int = 4096
    num_hidden_layers: int = 24
    num_attention_heads: int = 16
    layer_norm_eps: float = 1e-7
    position_buckets: int = 256
    max_relative_positions: int = -1
    hidden_act: str = "gelu"
    pad_token_id: int = 0
    # Not in the Swift struct: fixed there by the checkpoint shapes
    # (word embeddings [128011, C], DeBERTa.swift:199-202; classifier.0 C -> 2048).
    vocab_size: int = 128011
    classifier_hidden: int = 2048

    @property
    def head_size(self) -> int:  # Configuration.swift:36
        return self.hidden_size // self.num_attention_heads

    @classmethod
    def default(cls) -> "DeBERTaV2Configuration":  # Configuration.swift:38-48
        return cls()

    def to_native(self) -> N.GdConfig:
        if self.hidden_act != "gelu":
            raise N.GlinerDecideError(N.GD_ERR_UNSUPPORTED, f"hidden_act {self.hidden_act!r} (only exact gelu)")
        return N.GdConfig(self.hidden_size, self.intermediate_size, self.num_hidden_layers, self.num_attention_heads,
                          self.layer_norm_eps, self.position_buckets, self.max_relative_positions, self.pad_token_id,
                          self.vocab_size, self.classifier_hidden)
