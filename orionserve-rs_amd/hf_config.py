"""Hugging Face ``config.json`` parsing, restated from the reference's
crates/orion-models/src/config.rs: the same accepted field names and aliases,
defaults, architecture detection and consistency checks, normalised into the
metadata the HIP model is created from.  Host-side only (no device code).
"""
from __future__ import annotations

import json
import os
from dataclasses import dataclass, field
from typing import Any, Dict, List, Optional


class ModelError(Exception):
    """orion_core::ModelError (crates/orion-core/src/error.rs): the variant is
    the subclass, its message names what was wrong."""


class PathNotFound(ModelError):
    pass


class MissingFile(ModelError):
    pass


class Malformed(ModelError):
    pass


class UnsupportedArchitecture(ModelError):
    pass


class UnsupportedDtype(ModelError):
    pass


class TensorNotFound(ModelError):
    pass


class ShapeMismatch(ModelError):
    pass


# serde field aliases of HfConfig (config.rs:20-80)
_ALIASES = {
    "num_hidden_layers": ("num_hidden_layers", "n_layer", "num_layers"),
    "num_attention_heads": ("num_attention_heads", "n_head"),
    "max_position_embeddings": ("max_position_embeddings", "n_positions", "max_sequence_length"),
    "rms_norm_eps": ("rms_norm_eps", "layer_norm_eps", "rms_norm_epsilon"),
}


def _field(raw: Dict[str, Any], name: str, required: bool = False):
    for key in _ALIASES.get(name, (name,)):
        if key in raw:
            return raw[key]
    if required:
        raise Malformed(f"config.json: missing field `{name}`")
    return None


ARCH_LLAMA, ARCH_QWEN2 = "llama", "qwen2"


@dataclass
class HfConfig:
    """The subset of config.json the engine understands (config.rs:20-80);
    unknown fields are ignored."""

    hidden_size: int
    num_hidden_layers: int
    num_attention_heads: int
    vocab_size: int
    architectures: List[str] = field(default_factory=list)
    model_type: Optional[str] = None
    num_key_value_heads: Optional[int] = None
    head_dim: Optional[int] = None
    intermediate_size: Optional[int] = None
    max_position_embeddings: Optional[int] = None
    rope_theta: Optional[float] = None
    rms_norm_eps: Optional[float] = None
    torch_dtype: Optional[str] = None
    eos_token_id: Any = None
    bos_token_id: Optional[int] = None
    tie_word_embeddings: Optional[bool] = None

    @classmethod
    def from_json(cls, text: str) -> "HfConfig":
        try:
            raw = json.loads(text)
        except json.JSONDecodeError as e:
            raise Malformed(f"config.json: {e}") from None
        if not isinstance(raw, dict):
            raise Malformed("config.json: not an object")

        def opt_int(name):
            v = _field(raw, name)
            if v is not None and (not isinstance(v, int) or isinstance(v, bool) or v < 0):
                raise Malformed(f"config.json: `{name}` must be a non-negative integer")
            return v

        def req_int(name):
            v = _field(raw, name, required=True)
            if not isinstance(v, int) or isinstance(v, bool) or v < 0:
                raise Malformed(f"config.json: `{name}` must be a non-negative integer")
            return v

        def opt_float(name):
            v = _field(raw, name)
            if v is not None and (isinstance(v, bool) or not isinstance(v, (int, float))):
                raise Malformed(f"config.json: `{name}` must be a number")
            return None if v is None else float(v)

        eos = raw.get("eos_token_id")
        if eos is not None and not (isinstance(eos, int) or
                                    (isinstance(eos, list) and all(isinstance(t, int) for t in eos))):
            raise Malformed("config.json: `eos_token_id` must be an id or a list of ids")
        return cls(
            hidden_size=req_int("hidden_size"),
            num_hidden_layers=req_int("num_hidden_layers"),
            num_attention_heads=req_int("num_attention_heads"),
            vocab_size=req_int("vocab_size"),
            architectures=list(raw.get("architectures") or []),
            model_type=raw.get("model_type"),
            num_key_value_heads=opt_int("num_key_value_heads"),
            head_dim=opt_int("head_dim"),
            intermediate_size=opt_int("intermediate_size"),
            max_position_embeddings=opt_int("max_position_embeddings"),
            rope_theta=opt_float("rope_theta"),
            rms_norm_eps=opt_float("rms_norm_eps"),
            torch_dtype=raw.get("torch_dtype"),
            eos_token_id=eos,
            bos_token_id=raw.get("bos_token_id"),
            tie_word_embeddings=raw.get("tie_word_embeddings"),
        )

    @classmethod
    def load(cls, directory: str) -> "HfConfig":
        """HfConfig::load (config.rs:158-172)."""
        path = os.path.join(directory, "config.json")
        if not os.path.exists(path):
            raise MissingFile(f"missing file: {path}")
        with open(path, "r", encoding="utf-8") as f:
            return cls.from_json(f.read())

    def architecture(self) -> str:
        """Architecture::detect (config.rs:110-131): the architectures list
        first, then model_type; anything else is refused."""
        for a in self.architectures:
            if a in ("LlamaForCausalLM", "MistralForCausalLM"):
                return ARCH_LLAMA
            if a == "Qwen2ForCausalLM":
                return ARCH_QWEN2
        if self.model_type in ("llama", "mistral"):
            return ARCH_LLAMA
        if self.model_type == "qwen2":
            return ARCH_QWEN2
        name = (self.architectures[0] if self.architectures else self.model_type) or "<unspecified>"
        raise UnsupportedArchitecture(name)

    def ffn_dim(self) -> int:  # config.rs:234-238
        return self.intermediate_size if self.intermediate_size is not None else 4 * self.hidden_size

    def ties_embeddings(self) -> bool:  # config.rs:240-243
        return bool(self.tie_word_embeddings) if self.tie_word_embeddings is not None else False

    def eos_token_ids(self) -> List[int]:
        if self.eos_token_id is None:
            return []
        return [self.eos_token_id] if isinstance(self.eos_token_id, int) else list(self.eos_token_id)

    def dtype(self) -> str:
        """parse_dtype (config.rs:148-156)."""
        s = self.torch_dtype
        if s is None or s in ("float32", "float"):
            return "f32"
        if s in ("float16", "half"):
            return "f16"
        if s == "bfloat16":
            return "bf16"
        raise UnsupportedDtype(f"unsupported dtype: {s}")

    def to_metadata(self, name: str = "model"):
        """HfConfig::to_metadata (config.rs:176-231): defaults and checks."""
        from orion_hip import ModelMetadata  # the binding's metadata type

        arch = self.architecture()
        kv = self.num_key_value_heads if self.num_key_value_heads is not None else self.num_attention_heads
        head_dim = (self.head_dim if self.head_dim is not None
                    else self.hidden_size // max(self.num_attention_heads, 1))
        if self.num_attention_heads == 0 or self.num_hidden_layers == 0:
            raise Malformed("config.json: num_attention_heads and num_hidden_layers must be non-zero")
        if kv == 0:
            raise Malformed("config.json: num_key_value_heads must be non-zero")
        if self.num_attention_heads % kv:
            raise Malformed(f"config.json: num_attention_heads ({self.num_attention_heads}) must "
                            f"be a multiple of num_key_value_heads ({kv})")
        if head_dim == 0:
            raise Malformed("config.json: head_dim resolved to zero")
        if self.vocab_size == 0:
            raise Malformed("config.json: vocab_size must be non-zero")
        self.dtype()  # validates torch_dtype
        return ModelMetadata(
            hidden_size=self.hidden_size, num_layers=self.num_hidden_layers,
            num_attention_heads=self.num_attention_heads, num_kv_heads=kv, head_dim=head_dim,
            vocab_size=self.vocab_size, intermediate_size=self.ffn_dim(),
            max_position_embeddings=(self.max_position_embeddings
                                     if self.max_position_embeddings is not None else 2048),
            rope_theta=self.rope_theta if self.rope_theta is not None else 10000.0,
            rms_norm_eps=self.rms_norm_eps if self.rms_norm_eps is not None else 1e-5,
            architecture=arch, name=name, tied_lm_head=self.ties_embeddings())
