"""Shapes of the Qwen3.5 hybrid models this build runs, and seeded synthetic Q4K weights.

QWEN35_08B is the 0.8B shape (engine/FORMAT.md:14-33): 24 layers, every fourth one gated full
attention (layers 3, 7, ..., 23), the others Gated DeltaNet; hidden 1024, FFN 3584, vocab
248320, 8 query / 2 KV heads of 256, Gated DeltaNet 16 heads of 128, conv kernel 4.
"""
from __future__ import annotations

from dataclasses import dataclass


@dataclass(frozen=True)
class Shape:
    hidden: int = 1024
    layers: int = 24
    ffn: int = 3584
    vocab: int = 248320
    n_heads: int = 8
    n_kv: int = 2
    head_dim: int = 256
    rot: int = 64
    lin_k_heads: int = 16
    lin_v_heads: int = 16
    lin_k_dim: int = 128
    lin_v_dim: int = 128
    conv_k: int = 4
    full_every: int = 4          # layer i is full attention when i % full_every == full_every - 1
    eos_id: int = 248044
    rms_eps: float = 1e-6
    rope_theta: float = 1e7

    def is_full(self, layer: int) -> bool:
        return layer % self.full_every == self.full_every - 1

    @property
    def conv_dim(self) -> int:
        return 2 * self.lin_k_heads * self.lin_k_dim + self.lin_v_heads * self.lin_v_dim

    @property
    def vd(self) -> int:
        return self.lin_v_heads * self.lin_v_dim

    def layer_mats(self, layer: int) -> list[tuple[str, int, int]]:
        """(name, rows, cols) of every Q4K matrix of a layer, in launch order."""
        H, F = self.hidden, self.ffn
        if self.is_full(layer):
            hd = self.head_dim
            mix = [("self_attn.q_proj", self.n_heads * hd * 2, H),
                   ("self_attn.k_proj", self.n_kv * hd, H),
                   ("self_attn.v_proj", self.n_kv * hd, H),
                   ("self_attn.o_proj", H, self.n_heads * hd)]
        else:
            mix = [("linear_attn.in_proj_qkv", self.conv_dim, H),
                   ("linear_attn.in_proj_z", self.vd, H),
                   ("linear_attn.in_proj_b", self.lin_v_heads, H),
                   ("linear_attn.in_proj_a", self.lin_v_heads, H),
                   ("linear_attn.out_proj", H, self.vd)]
        return mix + [("mlp.gate_proj", F, H), ("mlp.up_proj", F, H), ("mlp.down_proj", H, F)]

    def q4k_bytes(self) -> int:
        """Q4K bytes of all layers plus the (tied) head."""
        b = sum(r // 4 * (c // 256) * 576 for l in range(self.layers) for _, r, c in self.layer_mats(l))
        return b + self.vocab // 4 * (self.hidden // 256) * 576


QWEN35_08B = Shape()
