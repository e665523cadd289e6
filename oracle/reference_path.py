"""The reference's own torch formulation of the LeanSelect prefill path, on the
CPU in the activation dtype (test infrastructure: the CPU baseline that
``bench.py`` times beside the GPU, and a cross-check of the float64 oracle).

Where ``leanselect_oracle`` accumulates every contraction in float64 and rounds
once, this module runs the same steps with the reference's torch operations
and dtypes, as ``_lightweight_compressed_attention`` does on its device:

* ``fused_weights`` (``leanselect/selector.py:144-158``): the einsum of the
  float32 masters, cast to the activation dtype;
* ``project_queries`` / ``project_atom_keys`` / ``score_pages``
  (``selector.py:160-214``): einsums in the activation dtype;
* ``pool_atoms_to_pages(reduce="max")`` (``leanselect/pages.py:146-187``):
  ``-inf`` padding and ``max_pool1d`` (kernel 5, stride 4);
* visibility, forcing and ``torch.topk(sorted=False)``
  (``leanselect/models/minicpm.py:3094-3141``);
* ``CompressK.forward`` (``minicpm.py:1158-1185``): the mean of each window in
  the key dtype.

Sequences are processed one at a time as in the reference; the query rows of a
long sequence are cut into chunks so the atom-score matrix of one chunk, not of
the whole sequence, is held at once (the values are the same).

Only ``tests/`` and ``bench.py``'s CPU-baseline leg use this module.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

__all__ = ["reference_compress_k", "reference_select_prefill", "reference_sparse_attention_rows"]


def _fused(head_mix, kv_head_mix, q_proj, k_proj, dtype):
    H, G, D = head_mix.shape[0], kv_head_mix.shape[0], q_proj.shape[1]
    qf = torch.einsum("hr,rdj->hdrj", head_mix, q_proj).reshape(H, D, -1).to(dtype)
    kf = torch.einsum("hr,rdj->hdrj", kv_head_mix, k_proj).reshape(G, D, -1).to(dtype)
    return qf.contiguous(), kf.contiguous()


def reference_compress_k(k: torch.Tensor, cu_seqlens: list[int], kernel_size: int = 32,
                         kernel_stride: int = 16):
    """``([sum A, G, D], cu_seqlens_compressed)``: window means in ``k.dtype``."""
    out, cu_c = [], [0]
    for b in range(len(cu_seqlens) - 1):
        s, e = cu_seqlens[b], cu_seqlens[b + 1]
        n = (e - s - kernel_size) // kernel_stride + 1 if e - s >= kernel_size else 0
        if n > 0:
            win = k[s:e].unfold(0, kernel_size, kernel_stride)[:n]  # [n, G, D, kernel]
            out.append(win.mean(dim=-1))
        cu_c.append(cu_c[-1] + n)
    kc = torch.cat(out, 0) if out else k.new_empty((0,) + tuple(k.shape[1:]))
    return kc, cu_c


def reference_select_prefill(q: torch.Tensor, kc: torch.Tensor, cu_q: list[int],
                             cu_k: list[int], masters, *, topk: int, block_size: int = 64,
                             kernel_stride: int = 16, init_blocks: int = 1,
                             local_blocks: int = 4, chunk_rows: int = 16384) -> torch.Tensor:
    """``topk_idx [G, total_q, take]`` int32 as the reference computes it (ids of a
    row in ``torch.topk(sorted=False)`` order, ``-1`` for invalid slots)."""
    head_mix, kv_head_mix, q_proj, k_proj = masters
    dt = q.dtype
    qf, kf = _fused(head_mix, kv_head_mix, q_proj, k_proj, dt)
    total_q, H, D = q.shape
    G = kf.shape[0]
    gs = H // G
    max_pages = max(((cu_q[b + 1] - cu_q[b] + block_size - 1) // block_size
                     for b in range(len(cu_q) - 1)), default=0)
    take = min(int(topk), max_pages)
    out = torch.full((G, total_q, take), -1, dtype=torch.int32)
    s_pool = block_size // kernel_stride
    for b in range(len(cu_q) - 1):
        q0, q1, k0, k1 = cu_q[b], cu_q[b + 1], cu_k[b], cu_k[b + 1]
        n = q1 - q0
        if n <= 0 or k1 <= k0:
            continue
        kt = torch.einsum("agd,gdf->gaf", kc[k0:k1], kf)  # project_atom_keys
        n_atoms = kt.shape[1]
        n_pages = (n + block_size - 1) // block_size
        padded = (n_pages - 1) * s_pool + s_pool + 1
        right = max(padded - (n_atoms + 1), 0)
        page_ids = torch.arange(n_pages)
        bt = min(take, n_pages)
        for c0 in range(0, n, chunk_rows):
            c1 = min(n, c0 + chunk_rows)
            qg = q[q0 + c0 : q0 + c1].reshape(c1 - c0, G, gs, D)
            qt = torch.einsum("ngsd,gsdf->gnf", qg, qf.reshape(G, gs, D, -1))  # project_queries
            atom = torch.einsum("gnf,gaf->gna", qt, kt)
            flat = F.pad(atom.reshape(-1, 1, n_atoms), (1, right), value=float("-inf"))
            pages = F.max_pool1d(flat, kernel_size=s_pool + 1, stride=s_pool)[..., :n_pages]
            pages = pages.reshape(G, c1 - c0, n_pages)
            qp = torch.arange(c0, c1) // block_size
            visible = page_ids[None] <= qp[:, None]
            local = visible & (page_ids[None] + local_blocks >= qp[:, None])
            forced = (page_ids < init_blocks)[None] | local
            pages = pages.masked_fill(~visible, float("-inf"))
            pages = pages.masked_fill(forced & visible, float("inf"))
            vals, idx = torch.topk(pages, bt, dim=-1, largest=True, sorted=False)
            invalid = torch.isnan(vals) | torch.isneginf(vals)
            out[:, q0 + c0 : q0 + c1, :bt] = idx.masked_fill(invalid, -1).to(torch.int32)
    return out


def reference_sparse_attention_rows(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                                    cu: list[int], topk_idx: torch.Tensor, rows: list[int], *,
                                    block_size: int = 64) -> torch.Tensor:
    """Gather-based masked-softmax attention of the given query rows (prefill,
    causal, scale ``head_dim ** -0.5``) in float32: ``[len(rows), H, D]``.
    ``topk_idx`` is ``[G, total_q, take]``."""
    total_q, H, D = q.shape
    G = k.shape[1]
    gs = H // G
    scale = D ** -0.5
    out = torch.zeros((len(rows), H, D), dtype=torch.float32)
    offs = torch.arange(block_size)
    for i, r in enumerate(rows):
        b = next(j for j in range(len(cu) - 1) if cu[j] <= r < cu[j + 1])
        t = r - cu[b]
        for g in range(G):
            pages = topk_idx[g, r]
            pages = torch.unique(pages[(pages >= 0) & (pages <= t // block_size)])
            if pages.numel() == 0:
                continue
            j = (pages[:, None] * block_size + offs[None, :]).reshape(-1)
            j = j[j <= t] + cu[b]
            s = (q[r, g * gs : (g + 1) * gs].float() @ k[j, g].float().T) * scale
            p = torch.softmax(s, dim=-1)
            out[i, g * gs : (g + 1) * gs] = p @ v[j, g].float()
    return out
