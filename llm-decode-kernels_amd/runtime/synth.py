"""Synthetic Llama-architecture weights (random init; there is no network for checkpoints).

``SyntheticLlama(shape, seed, device)`` is a read-only mapping with the Hugging Face Llama state-dict keys that the
decode runtime consumes (runtime/model.py:93-110 of the reference): embed_tokens, per-layer q/k/v/o and
gate/up/down projections, the two RMSNorm weights per layer, the final norm and lm_head. Each tensor is generated
on access from its own seed (base seed + CRC32 of the key) with torch's generator on ``device``, so it is
deterministic per key and independent of access order, and a large model never has to sit in memory as fp16 all at
once. Linear weights ~ N(0, std^2) (std 0.02, the HF initializer range); RMSNorm weights are 1 + norm_std * N(0, 1)
(norm_std 0 gives HF's all-ones init).
"""
import zlib
from collections.abc import Mapping
from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class LlamaShape:
    """The attributes of a Hugging Face LlamaConfig that the runtime reads."""
    hidden_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    intermediate_size: int
    vocab_size: int
    rms_norm_eps: float = 1e-5
    rope_theta: float = 10000.0

    @property
    def head_dim(self):
        return self.hidden_size // self.num_attention_heads


# BASELINE configs 4 and 5
TINYLLAMA = LlamaShape(2048, 22, 32, 4, 5632, 32000, 1e-5, 10000.0)
LLAMA3_8B = LlamaShape(4096, 32, 32, 8, 14336, 128256, 1e-5, 500000.0)


class SyntheticLlama(Mapping):
    def __init__(self, shape: LlamaShape, seed: int = 0, device="cuda", std: float = 0.02, norm_std: float = 0.0,
                 dtype=torch.float16):
        self.shape, self.seed, self.device, self.std, self.norm_std, self.dtype = \
            shape, seed, torch.device(device), std, norm_std, dtype
        s = shape
        D = s.head_dim
        self._shapes = {"model.embed_tokens.weight": (s.vocab_size, s.hidden_size),
                        "model.norm.weight": (s.hidden_size,),
                        "lm_head.weight": (s.vocab_size, s.hidden_size)}
        for i in range(s.num_hidden_layers):
            p = f"model.layers.{i}."
            self._shapes.update({
                p + "input_layernorm.weight": (s.hidden_size,),
                p + "post_attention_layernorm.weight": (s.hidden_size,),
                p + "self_attn.q_proj.weight": (s.num_attention_heads * D, s.hidden_size),
                p + "self_attn.k_proj.weight": (s.num_key_value_heads * D, s.hidden_size),
                p + "self_attn.v_proj.weight": (s.num_key_value_heads * D, s.hidden_size),
                p + "self_attn.o_proj.weight": (s.hidden_size, s.num_attention_heads * D),
                p + "mlp.gate_proj.weight": (s.intermediate_size, s.hidden_size),
                p + "mlp.up_proj.weight": (s.intermediate_size, s.hidden_size),
                p + "mlp.down_proj.weight": (s.hidden_size, s.intermediate_size)})

    def __getitem__(self, key):
        shp = self._shapes[key]
        g = torch.Generator(device=self.device).manual_seed(self.seed * 1_000_003 + zlib.crc32(key.encode()))
        if key.endswith("norm.weight"):
            t = torch.randn(shp, generator=g, device=self.device, dtype=torch.float32) * self.norm_std + 1.0
        else:
            t = torch.randn(shp, generator=g, device=self.device, dtype=torch.float32) * self.std
        return t.to(self.dtype)

    def __iter__(self):
        return iter(self._shapes)

    def __len__(self):
        return len(self._shapes)
