"""Model geometry (the fields of the reference's ModelConfig, model/configs.py:14-72) and the
synthetic configurations the GPU path is measured on.

Every synthetic configuration uses plain RoPE (yarn_factor 1): the float reference the GPU path
is checked against (model/fastref.py:64-65) has no YaRN correction.
"""

import dataclasses
from dataclasses import dataclass


@dataclass
class ModelConfig:
    name: str
    n_layer: int
    n_embd: int
    n_head: int
    n_kv_head: int
    head_dim: int
    ffn_dim: int
    vocab: int
    rope_theta: float = 1000000.0
    rms_eps: float = 1e-6
    max_ctx: int = 2048
    tie_embeddings: bool = False
    yarn_factor: float = 1.0
    yarn_orig_ctx: int = 0
    layer_types: tuple = ()
    dn_num_v_heads: int = 0
    dn_num_k_heads: int = 0
    dn_k_head_dim: int = 0
    dn_v_head_dim: int = 0
    dn_conv_kernel: int = 0
    rope_dims: int = 0
    attn_gated: bool = False
    hadamard_block: int = 0
    hadamard_signs: dict = None

    def vocab_padded(self, n_channels):
        """The vocabulary rounded up to a multiple of the channel count: row-sharded embedding and
        LM head tensors get zero rows there (model/configs.py:69-72)."""
        return -(-self.vocab // n_channels) * n_channels

    def layer_type(self, l):
        return self.layer_types[l] if self.layer_types else "attn"

    @property
    def n_dn_layers(self):
        return sum(1 for t in self.layer_types if t == "deltanet")

    @property
    def q_dim(self):
        return self.n_head * self.head_dim

    @property
    def kv_dim(self):
        return self.n_kv_head * self.head_dim

    def replace(self, **kw):
        return dataclasses.replace(self, **kw)


# The tiny random Qwen3 model the token loop is checked on: hidden 256, 4 layers, 4 q / 2 kv heads
# of 64, SwiGLU 768, vocab 2048, tied fp16 embedding. max_ctx covers the 16-token prompt plus 64
# generated tokens.
TINY = ModelConfig(name="tiny-qwen3", n_layer=4, n_embd=256, n_head=4, n_kv_head=2, head_dim=64,
                   ffn_dim=768, vocab=2048, max_ctx=128, tie_embeddings=True)

# Qwen3-1.7B shape (ternary tied embedding/LM head: 0.38 GB of weights per token with trit5).
QWEN3_1P7B = ModelConfig(name="qwen3-1.7b-shape", n_layer=28, n_embd=2048, n_head=16,
                         n_kv_head=8, head_dim=128, ffn_dim=6144, vocab=151936, max_ctx=1024,
                         tie_embeddings=True)

# Qwen3-8B shape (separate ternary LM head), fp16 KV cache to context 4096.
QWEN3_8B = ModelConfig(name="qwen3-8b-shape", n_layer=36, n_embd=4096, n_head=32, n_kv_head=8,
                       head_dim=128, ffn_dim=12288, vocab=151936, max_ctx=4096)

# Qwen3.5-27B hybrid shape: three Gated DeltaNet layers then one gated full-attention layer.
QWEN35_27B = ModelConfig(name="qwen3.5-27b-shape", n_layer=64, n_embd=5120, n_head=24,
                         n_kv_head=4, head_dim=256, ffn_dim=17408, vocab=248320, max_ctx=2048,
                         rope_theta=10000000.0,
                         layer_types=tuple(("deltanet", "deltanet", "deltanet", "attn") * 16),
                         dn_num_v_heads=48, dn_num_k_heads=16, dn_k_head_dim=128,
                         dn_v_head_dim=128, dn_conv_kernel=4, rope_dims=64, attn_gated=True)

# A tiny hybrid with the 27B's traits (DeltaNet + gated attention with partial RoPE), for
# correctness of the hybrid path.
TINY_HYBRID = ModelConfig(name="tiny-hybrid", n_layer=4, n_embd=256, n_head=4, n_kv_head=2,
                          head_dim=64, ffn_dim=512, vocab=1024, max_ctx=128, rope_theta=10000000.0,
                          layer_types=("deltanet", "deltanet", "deltanet", "attn"),
                          dn_num_v_heads=8, dn_num_k_heads=2, dn_k_head_dim=64, dn_v_head_dim=64,
                          dn_conv_kernel=4, rope_dims=16, attn_gated=True, tie_embeddings=True)

CONFIGS = {c.name: c for c in (TINY, QWEN3_1P7B, QWEN3_8B, QWEN35_27B, TINY_HYBRID)}

# Isolated GEMV shapes (rows, cols) of the Qwen3-1.7B layers.
MICROBENCH_SHAPES = ((2048, 2048), (1024, 2048), (6144, 2048), (2048, 6144))
