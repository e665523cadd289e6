"""CPU restatement of the MiniCPM4.1 decoder pieces around the LeanSelect layer (oracle).

Test infrastructure only: ``tests/`` and ``bench.py``'s CPU-baseline leg may use
it.  Each function restates the reference's torch expression with the same
rounding points (every torch op that returns a 16-bit tensor rounds once, RNE);
float32 intermediates are kept in float32 exactly where the reference keeps
them.  Paths are relative to the LeanSelect repository root.
"""
from __future__ import annotations

import math

import torch

__all__ = [
    "rotary_tables",
    "longrope_scale",
    "rms_layernorm",
    "apply_rotary_pos_emb",
    "silu_mul",
    "scaled_residual",
    "embed_scale",
]


def rotary_tables(head_dim: int, max_pos: int, base: float = 10000.0, ext_factors=None,
                  scale: float = 1.0):
    """``(cos, sin)`` float32 ``[max_pos, head_dim]``.

    ``MiniCPMRotaryEmbedding._set_cos_sin_cache`` (minicpm.py:804-838):
    ``inv_freq = 1 / base ** (arange(0, dim, 2) / dim)``, ``freqs = outer(t,
    inv_freq)``, ``emb = cat(freqs, freqs)``, then ``cos``/``sin`` in float32.
    With ``ext_factors``, ``MiniCPMLongRoPE._set_cos_sin_cache`` (minicpm.py:917-939):
    ``freqs = outer(t, 1 / ext_factors) * inv_freq`` and ``cos``/``sin`` times ``scale``
    (``longrope_scale``).
    """
    inv_freq = 1.0 / base ** (torch.arange(0, head_dim, 2).float() / head_dim)
    t = torch.arange(max_pos, dtype=inv_freq.dtype)
    if ext_factors is None:
        freqs = torch.outer(t, inv_freq)
        emb = torch.cat((freqs, freqs), dim=-1)
        return emb.cos().to(torch.float32), emb.sin().to(torch.float32)
    ext = torch.tensor(ext_factors, dtype=torch.float32)
    freqs = torch.mul(torch.outer(t, 1.0 / ext), inv_freq.to(torch.float32))
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(torch.float32) * scale, emb.sin().to(torch.float32) * scale


def longrope_scale(max_position_embeddings: int, original_max_position_embeddings: int) -> float:
    """``MiniCPMLongRoPE.__init__``'s ``scaling_factor`` (minicpm.py:908-914)."""
    s = max_position_embeddings / original_max_position_embeddings
    return math.sqrt(1 + math.log(s) / math.log(original_max_position_embeddings))


def rms_layernorm(hidden: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """``rms_layernorm`` (minicpm.py:772-788), un-chunked branch."""
    old_dtype = hidden.dtype
    variance = hidden.to(torch.float32).pow(2).mean(dim=-1, keepdim=True)
    hidden = (hidden * torch.rsqrt(variance + eps)).to(old_dtype)
    return hidden * weight


def _rotate_half(x: torch.Tensor) -> torch.Tensor:
    """``rotate_half`` (minicpm.py:1027-1031)."""
    x1 = x[..., : x.shape[-1] // 2]
    x2 = x[..., x.shape[-1] // 2:]
    return torch.cat((-x2, x1), dim=-1)


def apply_rotary_pos_emb(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                         positions: torch.Tensor) -> torch.Tensor:
    """``apply_rotary_pos_emb`` on one of q/k (minicpm.py:1034-1070), un-chunked branch.

    ``x [n, heads, D]``; ``positions [n]``.  The product and the sum are each
    float32 operations, then one rounding to ``x.dtype``.
    """
    c = cos[positions].unsqueeze(1)
    s = sin[positions].unsqueeze(1)
    xf = x.to(torch.float32)
    return (xf * c + _rotate_half(xf) * s).to(x.dtype)


def silu_mul(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """``act_fn(gate_proj(x)) * up_proj(x)`` (minicpm.py:1098-1135, ``hidden_act="silu"``)."""
    return torch.nn.functional.silu(gate) * up


def scaled_residual(residual: torch.Tensor, h: torch.Tensor, scale_depth: float,
                    num_layers: int) -> torch.Tensor:
    """``residual + hidden_states * (scale_depth / sqrt(num_layers))`` (minicpm.py:3616-3625)."""
    return residual + h * (scale_depth / math.sqrt(num_layers))


def embed_scale(ids: torch.Tensor, table: torch.Tensor, scale: float) -> torch.Tensor:
    """``embed_tokens(input_ids) * scale_emb`` (minicpm.py:3773-3774)."""
    return torch.nn.functional.embedding(ids.long(), table) * scale
