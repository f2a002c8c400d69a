"""Qwen3_5Config -- same fields, defaults and derived dims as the reference family config.

Reference: src/qwen3_5/config.py:15-109 (field list :16-40, derived dims :42-68,
`from_hf` parsing of `text_config` / `rope_parameters` :70-101, GGUF hard-fail
:104-109).  Kept field-for-field so a reference config dict parses identically.
"""

from __future__ import annotations

from dataclasses import dataclass, field


@dataclass
class Qwen3_5Config:
    vocab_size: int
    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    rms_norm_eps: float
    rope_theta: float
    partial_rotary_factor: float
    tie_word_embeddings: bool
    hidden_act: str
    layer_types: list = field(default_factory=list)
    full_attention_interval: int = 4
    attn_output_gate: bool = True
    output_gate_type: str = "sigmoid"
    linear_num_key_heads: int = 16
    linear_num_value_heads: int = 32
    linear_key_head_dim: int = 128
    linear_value_head_dim: int = 128
    linear_conv_kernel_dim: int = 4

    # -- derived (config.py:42-65) --
    @property
    def n_rep(self) -> int:
        return self.num_attention_heads // self.num_key_value_heads

    @property
    def rotary_dim(self) -> int:
        return int(self.head_dim * self.partial_rotary_factor)

    @property
    def key_dim(self) -> int:
        return self.linear_key_head_dim * self.linear_num_key_heads

    @property
    def value_dim(self) -> int:
        return self.linear_value_head_dim * self.linear_num_value_heads

    @property
    def conv_dim(self) -> int:
        return 2 * self.key_dim + self.value_dim

    @property
    def v_per_k(self) -> int:
        return self.linear_num_value_heads // self.linear_num_key_heads

    def layer_type(self, i: int) -> str:
        return self.layer_types[i]

    @classmethod
    def from_hf(cls, raw: dict) -> "Qwen3_5Config":
        t = raw.get("text_config", raw)
        hidden = t["hidden_size"]
        n_head = t["num_attention_heads"]
        rp = t.get("rope_parameters", {})
        return cls(
            vocab_size=t["vocab_size"],
            hidden_size=hidden,
            intermediate_size=t["intermediate_size"],
            num_hidden_layers=t["num_hidden_layers"],
            num_attention_heads=n_head,
            num_key_value_heads=t.get("num_key_value_heads", n_head),
            head_dim=t.get("head_dim", hidden // n_head),
            rms_norm_eps=t.get("rms_norm_eps", 1e-6),
            rope_theta=rp.get("rope_theta", t.get("rope_theta", 1e7)),
            partial_rotary_factor=rp.get("partial_rotary_factor",
                                         t.get("partial_rotary_factor", 1.0)),
            tie_word_embeddings=t.get("tie_word_embeddings",
                                      raw.get("tie_word_embeddings", False)),
            hidden_act=t.get("hidden_act", "silu"),
            layer_types=list(t["layer_types"]),
            full_attention_interval=t.get("full_attention_interval", 4),
            attn_output_gate=t.get("attn_output_gate", True),
            output_gate_type=t.get("output_gate_type", "sigmoid"),
            linear_num_key_heads=t["linear_num_key_heads"],
            linear_num_value_heads=t["linear_num_value_heads"],
            linear_key_head_dim=t["linear_key_head_dim"],
            linear_value_head_dim=t["linear_value_head_dim"],
            linear_conv_kernel_dim=t["linear_conv_kernel_dim"],
        )


def build_config(raw: dict, fmt: str) -> Qwen3_5Config:
    if fmt != "hf":
        raise NotImplementedError(
            f"qwen3_5 loads checkpoints in the hf (safetensors) format only, not {fmt!r}: "
            "there is no agreed GGUF tensor layout for the Gated DeltaNet layers")
    return Qwen3_5Config.from_hf(raw)


def _schedule(n_layers: int, interval: int = 4) -> list:
    return ["full_attention" if i % interval == interval - 1 else "linear_attention"
            for i in range(n_layers)]


def tiny_config_dict() -> dict:
    """The tiny CPU-runnable hybrid decoder: hidden 1024, 8 layers [GDN x3, attn] x2,
    GDN 8 qk / 16 v heads of dim 128 (conv 4), attention 8 q / 2 kv heads of dim 256
    with a sigmoid output gate, SwiGLU 3072, vocab 32768, one MTP layer."""
    return {
        "model_type": "qwen3_5", "vocab_size": 32768, "hidden_size": 1024,
        "intermediate_size": 3072, "num_hidden_layers": 8, "num_attention_heads": 8,
        "num_key_value_heads": 2, "head_dim": 256, "rms_norm_eps": 1e-6,
        "rope_parameters": {"rope_theta": 1e7, "partial_rotary_factor": 0.25},
        "tie_word_embeddings": True, "hidden_act": "silu", "layer_types": _schedule(8),
        "full_attention_interval": 4, "linear_num_key_heads": 8,
        "linear_num_value_heads": 16, "linear_key_head_dim": 128,
        "linear_value_head_dim": 128, "linear_conv_kernel_dim": 4,
        "mtp_num_hidden_layers": 1,
    }


def dense_8b_config_dict() -> dict:
    """The 8B-class dense hybrid decoder of the end-to-end speculative workload:
    hidden 4096, 32 layers (3:1 GDN:attention), GDN 16 qk / 32 v heads of dim 128,
    attention 32 q / 4 kv heads of dim 256 (gated), SwiGLU 12288, vocab 151936,
    one MTP layer."""
    return {
        "model_type": "qwen3_5", "vocab_size": 151936, "hidden_size": 4096,
        "intermediate_size": 12288, "num_hidden_layers": 32, "num_attention_heads": 32,
        "num_key_value_heads": 4, "head_dim": 256, "rms_norm_eps": 1e-6,
        "rope_parameters": {"rope_theta": 1e7, "partial_rotary_factor": 0.25},
        "tie_word_embeddings": True, "hidden_act": "silu", "layer_types": _schedule(32),
        "full_attention_interval": 4, "linear_num_key_heads": 16,
        "linear_num_value_heads": 32, "linear_key_head_dim": 128,
        "linear_value_head_dim": 128, "linear_conv_kernel_dim": 4,
        "mtp_num_hidden_layers": 1,
    }


def micro_config_dict() -> dict:
    """A very small hybrid decoder for fast parity tests (same structure as the tiny
    one: [GDN x3, attn] x1, GDN 2 qk / 4 v heads of dim 128, attention 4 q / 2 kv
    heads of dim 256, hidden 256, vocab 512)."""
    return {
        "model_type": "qwen3_5", "vocab_size": 512, "hidden_size": 256,
        "intermediate_size": 512, "num_hidden_layers": 4, "num_attention_heads": 4,
        "num_key_value_heads": 2, "head_dim": 256, "rms_norm_eps": 1e-6,
        "rope_parameters": {"rope_theta": 1e7, "partial_rotary_factor": 0.25},
        "tie_word_embeddings": True, "hidden_act": "silu", "layer_types": _schedule(4),
        "full_attention_interval": 4, "linear_num_key_heads": 2,
        "linear_num_value_heads": 4, "linear_key_head_dim": 128,
        "linear_value_head_dim": 128, "linear_conv_kernel_dim": 4,
        "mtp_num_hidden_layers": 1,
    }
