"""Block configuration and the attention dispatcher.

``ModelConfig`` carries the fields of the reference dataclass that shape the
attention block (reference models.py:21-37); ``build_attention`` is the
counterpart of the reference ``_build_attention`` (reference models.py:465-488)
but forwards every block field, including ``local_block_size`` and
``latent_query_block_size`` that the reference dispatcher drops.
"""
from __future__ import annotations

from dataclasses import dataclass


@dataclass
class ModelConfig:
    vocab_size: int = 128
    max_seq_len: int = 1024
    d_model: int = 128
    n_heads: int = 4
    n_layers: int = 4
    d_ff: int = 256
    dropout: float = 0.0
    local_window: int = 64
    local_block_size: int = 256
    latent_tokens: int = 16
    latent_d_model: int = 64
    latent_heads: int = 2
    latent_query_block_size: int = 0
    checkpoint_blocks: bool = False
    use_triton_kernel: bool = True


# architecture presets of the reference trainer (reference train.py:71-93); the
# window / block / latent-count knobs keep their CLI defaults (reference train.py:130-135)
MODEL_PRESETS = {
    "0.55b": dict(d_model=1408, n_heads=16, n_layers=22, d_ff=4096, latent_d_model=512, latent_heads=8),
    "0.60b": dict(d_model=1536, n_heads=16, n_layers=22, d_ff=4096, latent_d_model=384, latent_heads=8),
}


def build_attention(config: ModelConfig):
    """Return the HIP attention block for ``config``.

    Raises ``RuntimeError`` when ``use_triton_kernel`` is False: the PyTorch
    reference path is not part of this package, and ``dropout`` must be 0
    (the reference never sets it, reference models.py:29).
    """
    if not config.use_triton_kernel:
        raise RuntimeError("build_attention builds the fused HIP block only (use_triton_kernel=True)")
    if config.dropout != 0.0:
        raise ValueError("the fused block implements dropout = 0 only")
    from .module import LocalLatentAttentionTriton
    return LocalLatentAttentionTriton(
        d_model=config.d_model, n_heads=config.n_heads, latent_heads=config.latent_heads,
        latent_dim=config.latent_d_model, n_latents=config.latent_tokens, window=config.local_window,
        local_block_size=config.local_block_size, latent_query_block_size=config.latent_query_block_size)
