"""CPU restatement of LeanSelect's prefill hot path (the oracle; test infrastructure).

Every function names the reference lines it restates.  Paths are relative to the
LeanSelect repository root.  The oracle follows the reference's rounding order:
the fused router weights are cast to the activation dtype, the projected queries
and keys are rounded to that dtype, the atom scores are rounded to that dtype,
and page scores are an exact max of the rounded atom scores.  Contractions are
accumulated in float64 and rounded once, which is the exact representative of
the reference's "float32-accumulated GEMM, one rounding" semantics.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
may use this module.
"""
from __future__ import annotations

import math
from typing import Sequence

import torch

__all__ = [
    "calc_chunks_with_stride",
    "compress_k",
    "compress_keys_mean",
    "fused_weights",
    "project_queries",
    "project_atom_keys",
    "atom_scores",
    "pool_atoms_to_pages",
    "forced_page_mask",
    "leanselect_take",
    "select_prefill",
    "sparse_attention",
    "attention_keys_for_row",
]


def _as_list(x) -> list[int]:
    if torch.is_tensor(x):
        return [int(v) for v in x.detach().cpu().tolist()]
    return [int(v) for v in x]


def _round(x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """One rounding from float64 to ``dtype`` (through float32 for 16-bit types)."""
    if dtype == torch.float64:
        return x
    if dtype == torch.float32:
        return x.to(torch.float32)
    return x.to(torch.float32).to(dtype)


# ----------------------------------------------------------------------------
# Compressed keys
# ----------------------------------------------------------------------------
def calc_chunks_with_stride(
    cu_seqlens: Sequence[int], kernel_size: int = 32, kernel_stride: int = 16
) -> tuple[list[list[int]], list[int]]:
    """Window starts per sequence and compressed cu_seqlens.

    Restates ``leanselect/models/minicpm.py:711-750``: windows of
    ``kernel_size`` tokens at stride ``kernel_stride`` that lie entirely inside
    one sequence.  A sequence shorter than ``kernel_size`` yields no window.
    """
    cu = _as_list(cu_seqlens)
    lengths = [cu[i + 1] - cu[i] for i in range(len(cu) - 1)]
    starts: list[list[int]] = []
    cu_c = [0]
    for length in lengths:
        n = (length - kernel_size) // kernel_stride + 1 if length >= kernel_size else 0
        starts.append([a * kernel_stride for a in range(n)])
        cu_c.append(cu_c[-1] + n)
    return starts, cu_c


def compress_k(
    k: torch.Tensor,
    cu_seqlens,
    kernel_size: int = 32,
    kernel_stride: int = 16,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Mean of ``kernel_size``-token windows per sequence.

    Restates ``CompressK.forward`` (``leanselect/models/minicpm.py:1158-1185``):
    ``k [total_k, G, D]`` -> ``([sum A, G, D], cu_seqlens_compressed int32)``.
    The mean is accumulated in float64 and rounded once to ``k.dtype``.
    """
    cu = _as_list(cu_seqlens)
    starts, cu_c = calc_chunks_with_stride(cu, kernel_size, kernel_stride)
    rows = []
    kd = k.detach().to(torch.float64)
    for b, seq_starts in enumerate(starts):
        if not seq_starts:
            continue
        base = cu[b]
        idx = torch.tensor(seq_starts, dtype=torch.long)[:, None] + torch.arange(
            kernel_size
        )
        rows.append(kd[base + idx].mean(dim=1))
    if rows:
        out = _round(torch.cat(rows, 0), k.dtype)
    else:
        out = k.new_empty((0,) + tuple(k.shape[1:]))
    return out, torch.tensor(cu_c, dtype=torch.int32)


def compress_keys_mean(
    k: torch.Tensor, *, kernel_size: int = 32, kernel_stride: int = 16
) -> torch.Tensor:
    """``[B, S, G, D] -> [B, C, G, D]`` window mean (``leanselect/pages.py:84-101``).

    Unlike ``CompressK`` a sequence shorter than the kernel yields one atom that
    is the mean of the whole sequence (``pages.py:99-100``).
    """
    if k.ndim != 4:
        raise ValueError("k must be [B, S, n_kv, D]")
    seq_len = int(k.shape[1])
    if min(seq_len, kernel_size, kernel_stride) <= 0:
        raise ValueError("sequence and compression geometry must be positive")
    kd = k.detach().to(torch.float64)
    if seq_len < kernel_size:
        return _round(kd.mean(dim=1, keepdim=True), k.dtype)
    n = (seq_len - kernel_size) // kernel_stride + 1
    idx = torch.arange(n)[:, None] * kernel_stride + torch.arange(kernel_size)
    return _round(kd[:, idx].mean(dim=2), k.dtype)


# ----------------------------------------------------------------------------
# Folded router weights, projections and atom scores
# ----------------------------------------------------------------------------
def fused_weights(
    head_mix: torch.Tensor,
    kv_head_mix: torch.Tensor,
    q_proj: torch.Tensor,
    k_proj: torch.Tensor,
    dtype: torch.dtype | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Fold mixing coefficients into the projections.

    Restates ``LeanSelectSelector.fused_weights`` (``leanselect/selector.py:144-158``):
    ``q_fused[h, d, r*F + j] = head_mix[h, r] * q_proj[r, d, j]`` (one float32
    product per element), likewise ``kv_fused`` with ``kv_head_mix``/``k_proj``,
    then a cast to ``dtype``.
    """
    h, r = head_mix.shape
    g = kv_head_mix.shape[0]
    _, d, f = q_proj.shape
    qf = (head_mix.float()[:, None, :, None] * q_proj.float().permute(1, 0, 2)[None])
    kf = (kv_head_mix.float()[:, None, :, None] * k_proj.float().permute(1, 0, 2)[None])
    qf = qf.reshape(h, d, r * f)
    kf = kf.reshape(g, d, r * f)
    if dtype is not None:
        qf, kf = qf.to(dtype), kf.to(dtype)
    return qf.contiguous(), kf.contiguous()


def project_queries(
    query: torch.Tensor, q_fused: torch.Tensor, num_kv_heads: int
) -> torch.Tensor:
    """GQA-group-summed query projection ``[N, H, D] -> [G, N, R*F]``.

    Restates ``LeanSelectSelector.project_queries`` (``leanselect/selector.py:160-177``):
    ``q~[g, n, f] = sum_{s<gs, d} Q[n, g*gs+s, d] * q_fused[g*gs+s, d, f]``.
    """
    n, h, d = query.shape
    g = int(num_kv_heads)
    gs = h // g
    qg = query.detach().to(torch.float64).reshape(n, g, gs * d).permute(1, 0, 2)
    wg = q_fused.to(torch.float64).reshape(g, gs * d, -1)
    return _round(torch.bmm(qg, wg), query.dtype)


def project_atom_keys(compressed_keys: torch.Tensor, kv_fused: torch.Tensor) -> torch.Tensor:
    """``[A, G, D] -> [G, A, R*F]`` (``leanselect/selector.py:179-190``)."""
    kc = compressed_keys.detach().to(torch.float64).permute(1, 0, 2)
    return _round(torch.bmm(kc, kv_fused.to(torch.float64)), compressed_keys.dtype)


def atom_scores(q_tilde: torch.Tensor, k_tilde: torch.Tensor) -> torch.Tensor:
    """Unscaled per-group atom dots ``[G, N, A]`` (``leanselect/selector.py:203-207``)."""
    s = torch.bmm(q_tilde.to(torch.float64), k_tilde.to(torch.float64).transpose(1, 2))
    return _round(s, q_tilde.dtype)


# ----------------------------------------------------------------------------
# Page pooling and forced pages
# ----------------------------------------------------------------------------
def pool_atoms_to_pages(
    atom_scores_: torch.Tensor,
    *,
    seq_len: int,
    block_size: int = 64,
    kernel_stride: int = 16,
) -> torch.Tensor:
    """Overlapping 5-atom page max ``[..., A] -> [..., ceil(seq_len/block_size)]``.

    Restates ``pool_atoms_to_pages(reduce="max")`` (``leanselect/pages.py:146-187``):
    page ``p`` is the max over atoms ``[p*s - 1, p*s + s)`` clipped to ``[0, A)``
    with ``s = block_size // kernel_stride``; a page whose window holds no atom
    scores ``-inf``.  Written as an explicit gather so that it does not reuse the
    reference's ``max_pool1d`` formulation.
    """
    if min(seq_len, block_size, kernel_stride) <= 0:
        raise ValueError("page geometry must be positive")
    if block_size % kernel_stride:
        raise ValueError("block_size must be divisible by kernel_stride")
    s = block_size // kernel_stride
    n_pages = (int(seq_len) + block_size - 1) // block_size
    n_atoms = int(atom_scores_.shape[-1])
    idx = torch.arange(n_pages)[:, None] * s - 1 + torch.arange(s + 1)[None, :]
    valid = (idx >= 0) & (idx < n_atoms)
    gathered = atom_scores_[..., idx.clamp(0, max(n_atoms - 1, 0))]
    gathered = gathered.masked_fill(~valid, float("-inf"))
    return gathered.amax(dim=-1)


def forced_page_mask(
    query_pos: torch.Tensor,
    *,
    num_pages: int,
    block_size: int = 64,
    init_blocks: int = 1,
    local_blocks: int = 32,
) -> torch.Tensor:
    """Sink + local forced pages (``leanselect/pages.py:222-240``), ``[B, Q, P]`` bool."""
    pos = query_pos.long()
    if pos.ndim == 1:
        pos = pos.view(1, -1)
    qp = (pos // int(block_size)).unsqueeze(-1)
    pages = torch.arange(int(num_pages)).view(1, 1, -1)
    local = (qp >= pages) & (qp <= pages + int(local_blocks))
    return (pages < int(init_blocks)) | local


def leanselect_take(cu_seqlens_q, topk: int, block_size: int = 64) -> int:
    """``take = min(topk, max_pages)`` (``leanselect/models/minicpm.py:3094-3104``)."""
    cu = _as_list(cu_seqlens_q)
    max_pages = max(
        ((cu[b + 1] - cu[b] + block_size - 1) // block_size for b in range(len(cu) - 1)),
        default=0,
    )
    return min(int(topk), max_pages)


# ----------------------------------------------------------------------------
# The LeanSelect prefill selection driver
# ----------------------------------------------------------------------------
def _stable_topk_desc(scores: torch.Tensor, k: int) -> torch.Tensor:
    """Indices of the ``k`` largest entries, ties to the lower index.

    The reference's deterministic top-k rule (``leanselect/pages.py:44``: stable
    descending argsort).  NaN sorts above +inf, as in ``torch.topk``.
    """
    key = torch.where(torch.isnan(scores), torch.full_like(scores, float("inf")), scores)
    nan_first = torch.isnan(scores).to(torch.float64)
    # Sort by (is_nan, value) descending, stable in index.
    order = torch.argsort(key, dim=-1, descending=True, stable=True)
    if bool(nan_first.any()):
        nan_sorted = torch.gather(nan_first, -1, order)
        order2 = torch.argsort(nan_sorted, dim=-1, descending=True, stable=True)
        order = torch.gather(order, -1, order2)
    return order[..., :k]


def select_prefill(
    q_unpad: torch.Tensor,
    k_compressed: torch.Tensor,
    cu_seqlens_q,
    cu_seqlens_k,
    q_fused: torch.Tensor,
    kv_fused: torch.Tensor,
    *,
    topk: int,
    block_size: int = 64,
    kernel_stride: int = 16,
    init_blocks: int = 1,
    local_blocks: int = 32,
    rows: Sequence[int] | None = None,
    return_scores: bool = False,
    chunk_rows: int = 2048,
):
    """Per-token, per-KV-group page plans ``[G, total_q, take]`` int32.

    Restates ``MiniCPMInfLLMv2Attention._lightweight_compressed_attention``
    (``leanselect/models/minicpm.py:3061-3142``) with
    ``LeanSelectSelector.score_pages`` (``leanselect/selector.py:192-214``):
    per sequence, atom scores are max-pooled to pages, pages after the query's
    page are ``-inf``, sink pages and the ``local_blocks + 1`` pages ending at
    the query's page are ``+inf``, and ``take = min(topk, max_pages)`` pages are
    chosen; ``-inf``/NaN choices become ``-1``.  A sequence with no query or no
    compressed key keeps ``-1`` everywhere (``minicpm.py:3114-3116``).

    The reference's ``torch.topk(sorted=False)`` leaves tie order and slot
    order unspecified; here ties go to the lower page index and each row lists
    its valid ids in ascending order followed by ``-1``.

    ``rows`` restricts the work to those global query rows (the returned ids and
    scores then have ``len(rows)`` in dim 1).  With ``return_scores`` the masked
    page scores (``+inf`` forced, ``-inf`` invisible, float64, padded with
    ``-inf`` to ``max_pages``) are returned as well.
    """
    cq = _as_list(cu_seqlens_q)
    ck = _as_list(cu_seqlens_k)
    total_q, num_heads, head_dim = q_unpad.shape
    G = kv_fused.shape[0]
    take = leanselect_take(cq, topk, block_size)
    max_pages = max(
        ((cq[b + 1] - cq[b] + block_size - 1) // block_size for b in range(len(cq) - 1)),
        default=0,
    )
    if rows is None:
        row_list = list(range(total_q))
    else:
        row_list = [int(r) for r in rows]
    pos_of = {r: i for i, r in enumerate(row_list)}
    out = torch.full((G, len(row_list), take), -1, dtype=torch.int32)
    scores_out = (
        torch.full((G, len(row_list), max_pages), float("-inf"), dtype=torch.float64)
        if return_scores
        else None
    )
    for b in range(len(cq) - 1):
        q_start, q_end = cq[b], cq[b + 1]
        k_start, k_end = ck[b], ck[b + 1]
        q_len = q_end - q_start
        if q_len <= 0 or k_end <= k_start:
            continue
        seq_rows = [r for r in row_list if q_start <= r < q_end]
        if not seq_rows:
            continue
        kt = project_atom_keys(k_compressed[k_start:k_end], kv_fused)
        n_pages = (q_len + block_size - 1) // block_size
        batch_take = min(take, n_pages)
        page_ids = torch.arange(n_pages)
        for c0 in range(0, len(seq_rows), chunk_rows):
            rr = torch.tensor(seq_rows[c0 : c0 + chunk_rows], dtype=torch.long)
            qt = project_queries(q_unpad[rr], q_fused, G)
            s = atom_scores(qt, kt)
            pages = pool_atoms_to_pages(
                s, seq_len=q_len, block_size=block_size, kernel_stride=kernel_stride
            ).to(torch.float64)
            qpage = (rr - q_start) // block_size
            visible = page_ids[None] <= qpage[:, None]
            local = visible & (page_ids[None] + local_blocks >= qpage[:, None])
            forced = (page_ids < init_blocks)[None] | local
            pages = pages.masked_fill(~visible[None], float("-inf"))
            pages = pages.masked_fill((forced & visible)[None], float("inf"))
            idx = _stable_topk_desc(pages, batch_take)
            vals = torch.gather(pages, -1, idx)
            invalid = torch.isnan(vals) | torch.isneginf(vals)
            idx = idx.masked_fill(invalid, n_pages + 1)
            idx = torch.sort(idx, dim=-1).values
            idx = idx.masked_fill(idx > n_pages, -1).to(torch.int32)
            dst = torch.tensor([pos_of[int(r)] for r in rr], dtype=torch.long)
            out[:, dst, :batch_take] = idx
            if scores_out is not None:
                scores_out[:, dst, :n_pages] = pages
    if return_scores:
        return out, scores_out
    return out


# ----------------------------------------------------------------------------
# Block-sparse causal attention over the selected pages
# ----------------------------------------------------------------------------
def attention_keys_for_row(
    row: int,
    ids: torch.Tensor,
    cq: list[int],
    ck: list[int],
    *,
    block_size: int = 64,
    causal: bool = True,
) -> torch.Tensor:
    """Global key rows attended by query ``row`` for one KV group's ``ids``.

    The per-token contract of ``infllmv2_attn_varlen_func(..., topk_idx=)``
    (``third_party/infllmv2/paper1.patch:1993-2100``; called at
    ``leanselect/models/minicpm.py:3229-3243``): keys of the selected pages
    (each valid id once) that satisfy the causal rule aligned to the end of
    the key sequence, ``j <= t + (len_k - len_q)``.
    """
    b = next(i for i in range(len(cq) - 1) if cq[i] <= row < cq[i + 1])
    t = row - cq[b]
    lq = cq[b + 1] - cq[b]
    lk = ck[b + 1] - ck[b]
    n_pages_k = (lk + block_size - 1) // block_size
    pages = sorted({int(p) for p in ids.tolist() if 0 <= int(p) < n_pages_k})
    if not pages:
        return torch.zeros(0, dtype=torch.long)
    j = (torch.tensor(pages)[:, None] * block_size + torch.arange(block_size)).reshape(-1)
    keep = j < lk
    if causal:
        keep &= j <= t + (lk - lq)
    return ck[b] + j[keep]


def sparse_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cu_seqlens_q,
    cu_seqlens_k,
    topk_idx: torch.Tensor,
    *,
    softmax_scale: float | None = None,
    causal: bool = True,
    block_size: int = 64,
    rows: Sequence[int] | None = None,
    ids_rows_aligned: bool = False,
    return_abs: bool = False,
):
    """Reference outputs ``(out [R, H, D] in q.dtype, lse [H, R] float32)``.

    With ``return_abs`` a third output ``[R, H, D]`` float64 holds
    ``sum_j p_j |v_j|`` with the same softmax weights: the magnitude an output
    element is summed from, which bounds the rounding error any 16-bit
    evaluation of the weights can make when the terms cancel.

    ``O[t, h] = softmax_j(scale * Q[t, h] . K[j, h // gs]) V[j, h // gs]`` over
    the keys of ``attention_keys_for_row``; ``scale = head_dim ** -0.5`` when
    ``softmax_scale`` is None (``paper1.patch:1993-2100``).  A row with no key
    gives a zero output and ``lse = +inf`` (flash-attention's convention for an
    empty row).  Accumulated in float64, rounded once.  ``topk_idx`` is
    ``[G, total_q, take]``, or ``[G, len(rows), take]`` with
    ``ids_rows_aligned``.
    """
    cq = _as_list(cu_seqlens_q)
    ck = _as_list(cu_seqlens_k)
    total_q, H, D = q.shape
    G = k.shape[1]
    gs = H // G
    scale = D ** -0.5 if softmax_scale is None else float(softmax_scale)
    row_list = list(range(total_q)) if rows is None else [int(r) for r in rows]
    out = torch.zeros((len(row_list), H, D), dtype=torch.float64)
    mass = torch.zeros((len(row_list), H, D), dtype=torch.float64) if return_abs else None
    lse = torch.full((H, len(row_list)), float("inf"), dtype=torch.float64)
    # Only the rows and keys each output reads are widened to float64.
    for i, r in enumerate(row_list):
        for g in range(G):
            ids = topk_idx[g, i if ids_rows_aligned else r]
            keys = attention_keys_for_row(r, ids, cq, ck, block_size=block_size, causal=causal)
            if keys.numel() == 0:
                continue
            qh = q[r, g * gs : (g + 1) * gs].detach().to(torch.float64)  # [gs, D]
            kk = k[keys, g].detach().to(torch.float64)
            vv = v[keys, g].detach().to(torch.float64)
            s = (qh @ kk.T) * scale  # [gs, nk]
            m = s.amax(dim=-1, keepdim=True)
            p = torch.exp(s - m)
            denom = p.sum(dim=-1, keepdim=True)
            out[i, g * gs : (g + 1) * gs] = (p @ vv) / denom
            if mass is not None:
                mass[i, g * gs : (g + 1) * gs] = (p @ vv.abs()) / denom
            lse[g * gs : (g + 1) * gs, i] = (m + torch.log(denom)).squeeze(-1)
    if mass is not None:
        return _round(out, q.dtype), lse.to(torch.float32), mass
    return _round(out, q.dtype), lse.to(torch.float32)


def attention_flops(
    cu_seqlens_q, cu_seqlens_k, topk_idx: torch.Tensor, num_heads: int, head_dim: int,
    *, block_size: int = 64, causal: bool = True,
) -> float:
    """Algorithmic attention FLOPs ``4 * H/G * D * sum_(t,g) keys(t, g)``."""
    cq = _as_list(cu_seqlens_q)
    ck = _as_list(cu_seqlens_k)
    G = topk_idx.shape[0]
    total = 0
    for r in range(cq[-1]):
        for g in range(G):
            total += attention_keys_for_row(
                r, topk_idx[g, r], cq, ck, block_size=block_size, causal=causal
            ).numel()
    return 4.0 * (num_heads // G) * head_dim * total
