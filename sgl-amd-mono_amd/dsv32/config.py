"""Geometry of one GPU's TP=4 share of a DeepSeek-V3.2 DSA decoder layer.

The reference's layer kernel is parameterised by ``LayerConfig``
(``sgl_amd_mono/glm53/gfx950/config.py:144-197``) at GLM-5.3 sizes; the same structure
at DeepSeek-V3.2 sizes (hidden 7168, q_lora 1536, 128 heads of 128 + 64, kv 512 + 64,
256 experts top-8, expert intermediate 2048, 61 layers; V4-Pro shares hidden, q_lora
and depth: ``deepseek_v4/gfx950/config.py:10-25``) is what the kernels here carry.
"""

from __future__ import annotations

from dataclasses import dataclass

TP = 4


@dataclass(frozen=True)
class LayerConfig:
    hidden: int = 7168
    q_lora: int = 1536
    kv_lora: int = 512
    rope_dim: int = 64
    nope_dim: int = 128
    v_dim: int = 128
    heads: int = 128 // TP  # local attention heads
    index_heads: int = 64  # replicated on every rank
    index_dim: int = 128
    index_topk: int = 2048
    page: int = 64
    experts: int = 256
    top_k: int = 8
    inter: int = 2048 // TP  # local expert intermediate (FP8)
    route_scale: float = 2.5
    # group-limited routing (DeepSeek-V3's n_group / topk_group); 1, 1: plain top-8, the
    # benchmark configs' router; the DeepSeek-V3.2 checkpoint routes with 8, 4
    n_group: int = 1
    topk_group: int = 1
    rms_eps: float = 1e-6
    layers: int = 61

    @property
    def qk_dim(self) -> int:
        return self.nope_dim + self.rope_dim

    @property
    def kv_row(self) -> int:
        """Values of a KV cache row: the latent plus the rotary key."""
        return self.kv_lora + self.rope_dim

    @property
    def softmax_scale(self) -> float:
        return self.qk_dim ** -0.5


DSV32 = LayerConfig()


@dataclass(frozen=True)
class Mxfp4MoeConfig:
    """Config 4: the MXFP4 expert block at one GPU's TP=4 share."""

    hidden: int = 3072
    experts: int = 256
    top_k: int = 8
    inter: int = 1536 // TP
    route_scale: float = 2.5
    n_group: int = 1
    topk_group: int = 1


MXFP4_MOE = Mxfp4MoeConfig()

# rows a MoE launch takes (the north star's decode widths are 1..16)
MAX_ROWS = 16
