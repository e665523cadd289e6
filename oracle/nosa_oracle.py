"""CPU restatement of the NOSA variant of the LeanSelect prefill path (the oracle;
test infrastructure).

Restated reference code (paths relative to the LeanSelect repository root):

* ``leanselect/ops/cis_pooling.py:8-72`` -- ``nosa_mean_pooling``: the CIS
  eviction scores averaged over 32-token windows at stride 16, broadcast to
  every query row of the sequence.
* ``third_party/infllmv2/paper1.patch:2664-2760`` -- ``max_pooling_1d_varlen``.
  Its kernel body is in the un-vendored ``infllm_v2`` upstream; the contract is
  the one the reference restates in ``leanselect/baselines/page_topk.py:4-26,
  94-117``: page ``p`` pools window ``[p*s - 1, p*s + s)`` (``s = block_size /
  stride``), sink pages and the ``local_blocks + 1`` pages ending at the row's
  page are ``+inf``.  Parity of that kernel is unpinned beyond this contract,
  and the contract leaves one choice open: whether a row pools only its own
  sequence's ``cu_seqlens_k`` columns or the whole padded row of
  ``max_seqlen_k`` columns.  Both are kept (``clip="sequence"`` / ``"row"``),
  each pinned against a brute-force loop.
* ``leanselect/models/nosa.py:1144-1307`` -- ``compressed_attention`` with
  ``precomputed_qk_score`` (the LeanSelect branch, ``nosa.py:2071-2098``), and
  ``nosa.py:1822-1853`` -- ``_leanselect_atom_scores``.
* ``leanselect/models/nosa.py:2211-2255`` -- the attention: ``V * exp(cis)``
  divided by the attention over ``exp(cis)``.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
may use this module.
"""
from __future__ import annotations

from typing import Sequence

import torch

from .leanselect_oracle import (
    _as_list,
    _round,
    _stable_topk_desc,
    attention_keys_for_row,
    atom_scores,
    project_atom_keys,
    project_queries,
)

__all__ = [
    "nosa_mean_pooling",
    "nosa_window_means",
    "page_maxpool_varlen",
    "nosa_atom_scores",
    "nosa_q_idx",
    "nosa_select_prefill",
    "nosa_two_stage",
    "nosa_pool_rows",
    "nosa_attention",
]


def nosa_mean_pooling(cis_score: torch.Tensor, cu_seqlens, max_seqlen: int,
                      kernel_size: int = 32, stride: int = 16) -> torch.Tensor:
    """``[N, H] -> [H, N, M]``, ``M = max_seqlen // stride - 1``.

    ``out[h, t, m]`` is the mean of ``cis_score[start_b + m*stride + i, h]`` over
    ``i < kernel_size`` for every row ``t`` of sequence ``b`` when that window
    lies inside the sequence, else 0 (``cis_pooling.py:41-52``: windows that
    reach past the sequence end are not written).  Summed in float64, rounded
    once to the input dtype.
    """
    if kernel_size != 32 or stride != 16:
        raise ValueError("nosa_mean_pooling supports kernel_size 32, stride 16")
    cu = _as_list(cu_seqlens)
    N, H = cis_score.shape
    M = int(max_seqlen) // stride - 1
    out = torch.zeros((H, N, max(M, 0)), dtype=torch.float64)
    c = cis_score.detach().to(torch.float64)
    for b in range(len(cu) - 1):
        s, e = cu[b], cu[b + 1]
        n = e - s
        for m in range(max(M, 0)):
            if m * stride + kernel_size > n:
                break
            val = c[s + m * stride : s + m * stride + kernel_size].mean(dim=0)  # [H]
            out[:, s:e, m] = val[:, None]
    return _round(out, cis_score.dtype)


def nosa_window_means(cis_score: torch.Tensor, start: int, end: int, max_seqlen: int,
                      kernel_size: int = 32, stride: int = 16) -> torch.Tensor:
    """``[H, M]``: the row vector ``nosa_mean_pooling`` broadcasts to every row of
    the sequence ``[start, end)`` (the same float64 mean rounded once; 0 past the
    sequence's last whole window)."""
    N, H = cis_score.shape
    M = max(int(max_seqlen) // stride - 1, 0)
    out = torch.zeros((H, M), dtype=torch.float64)
    n = end - start
    n_win = min(M, (n - kernel_size) // stride + 1) if n >= kernel_size else 0
    if n_win > 0:
        c = cis_score[start:end].detach().to(torch.float64)
        idx = torch.arange(n_win)[:, None] * stride + torch.arange(kernel_size)[None, :]
        out[:, :n_win] = c[idx].mean(dim=1).T
    return _round(out, cis_score.dtype)


def _pool_pages(x: torch.Tensor, lk: int, out_len: int, s: int) -> torch.Tensor:
    """Max of ``x[..., j]`` over ``j in [p*s - 1, p*s + s) ∩ [0, lk)`` for ``p < out_len``."""
    if x.shape[-1] == 0:  # no window at all: every page pools an empty range
        return torch.full((*x.shape[:-1], out_len), float("-inf"), dtype=x.dtype)
    idx = torch.arange(out_len)[:, None] * s - 1 + torch.arange(s + 1)[None, :]
    valid = (idx >= 0) & (idx < lk)
    g = x[..., idx.clamp(0, max(x.shape[-1] - 1, 0))]
    return g.masked_fill(~valid, float("-inf")).amax(dim=-1)


def _check_clip(clip: str) -> None:
    if clip not in ("sequence", "row"):
        raise ValueError(f"clip must be 'sequence' or 'row', got {clip!r}")


def _forced(off_bq: torch.Tensor, out_len: int, init_blocks: int, local_blocks: int) -> torch.Tensor:
    """Sink pages and the ``local_blocks + 1`` pages ending at ``off_bq``, ``[n, out_len]``."""
    pages = torch.arange(out_len)[None, :]
    return (pages < init_blocks) | ((off_bq[:, None] >= pages) & (off_bq[:, None] <= pages + local_blocks))


def page_maxpool_varlen(
    inp: torch.Tensor,
    cu_seqlens_q,
    cu_seqlens_k,
    cache_lens,
    max_seqlen_q: int,
    max_seqlen_k: int,
    *,
    local_blocks: int,
    init_blocks: int,
    block_size: int = 64,
    stride: int = 16,
    clip: str = "sequence",
) -> torch.Tensor:
    """``[Hk, total_q, max_k] -> [Hk, total_q, out_len]`` page max with the forced overlay.

    ``out_len = ceil((max_seqlen_q + max(cache_lens)) / block_size)``.  Row ``t``
    of sequence ``b`` has page ``off_bq = (t - cu_q[b] + cache_len[b]) //
    block_size``.  Page ``p`` is ``+inf`` when ``p < init_blocks`` or
    ``off_bq - local_blocks <= p <= off_bq``, else the max of
    ``inp[h, t, j]`` over ``j in [p*s - 1, p*s + s)`` clipped to the
    sequence's ``len_k(b)`` score columns (``clip="sequence"``) or to the row's
    ``max_k`` columns (``clip="row"``), ``-inf`` when empty.  Which of the two
    the upstream kernel applies is not fixed by the reference tree (its body is
    un-vendored); both are kept, and they differ only where a shorter
    sequence's padding columns hold values above ``-inf``.
    """
    _check_clip(clip)
    cq = _as_list(cu_seqlens_q)
    ck = _as_list(cu_seqlens_k)
    cl = _as_list(cache_lens)
    Hk, total_q, max_k = inp.shape
    s = block_size // stride
    out_len = (int(max_seqlen_q) + max(cl, default=0) + block_size - 1) // block_size
    x = inp.detach().to(torch.float64)
    out = torch.full((Hk, total_q, out_len), float("-inf"), dtype=torch.float64)
    for b in range(len(cq) - 1):
        q0, q1 = cq[b], cq[b + 1]
        if q1 <= q0:
            continue
        lk = max_k if clip == "row" else min(ck[b + 1] - ck[b], max_k)
        pooled = _pool_pages(x[:, q0:q1], lk, out_len, s)
        off_bq = (torch.arange(q1 - q0) + cl[b]) // block_size
        out[:, q0:q1] = pooled.masked_fill(_forced(off_bq, out_len, init_blocks, local_blocks)[None],
                                           float("inf"))
    return _round(out, inp.dtype) if inp.dtype != torch.float64 else out


def nosa_atom_scores(q_unpad, k_compressed, cu_seqlens_q, cu_seqlens_kc, q_fused, kv_fused,
                     rows: Sequence[int] | None = None) -> torch.Tensor:
    """``[G, R, max_k]`` atom scores, ``-inf`` past a sequence's atoms
    (``nosa.py:1822-1853``; no causal mask)."""
    cq = _as_list(cu_seqlens_q)
    ck = _as_list(cu_seqlens_kc)
    G = kv_fused.shape[0]
    max_k = max((ck[b + 1] - ck[b] for b in range(len(ck) - 1)), default=0)
    row_list = list(range(cq[-1])) if rows is None else [int(r) for r in rows]
    out = torch.full((G, len(row_list), max_k), float("-inf"), dtype=torch.float64)
    for b in range(len(cq) - 1):
        k0, k1 = ck[b], ck[b + 1]
        sel = [i for i, r in enumerate(row_list) if cq[b] <= r < cq[b + 1]]
        if not sel or k1 <= k0:
            continue
        kt = project_atom_keys(k_compressed[k0:k1], kv_fused)
        qt = project_queries(q_unpad[torch.tensor([row_list[i] for i in sel])], q_fused, G)
        s = atom_scores(qt, kt)
        out[:, torch.tensor(sel), : k1 - k0] = s.to(torch.float64)
    return out


def nosa_q_idx(cu_seqlens_q, max_seqlen_q: int, block_size: int = 64) -> torch.Tensor:
    """Each row's page index aligned to the end of the longest sequence
    (``nosa.py:1175-1189``): ``(t - cu_q[b] + max_seqlen_q - len_q(b)) // block_size``."""
    cq = _as_list(cu_seqlens_q)
    parts = [
        (torch.arange(cq[b + 1] - cq[b]) + int(max_seqlen_q) - (cq[b + 1] - cq[b])) // block_size
        for b in range(len(cq) - 1)
    ]
    return torch.cat(parts) if parts else torch.zeros(0, dtype=torch.long)


def nosa_select_prefill(
    atom_score: torch.Tensor,
    cis: torch.Tensor,
    cu_seqlens_q,
    cu_seqlens_kc,
    cu_seqlens_k,
    max_seqlen_q: int,
    max_seqlen_k: int,
    *,
    topk: int = 96,
    init_blocks: int = 1,
    local_blocks: int = 16,
    select_blocks: int = 24,
    block_size: int = 64,
    kernel_stride: int = 16,
    kernel_size: int = 32,
    rows: Sequence[int] | None = None,
    return_scores: bool = False,
    clip: str = "sequence",
):
    """NOSA page plans ``[G, R, min(topk, out_len)]`` int32 (prefill).

    Restates ``compressed_attention`` (``nosa.py:1144-1307``) on the LeanSelect
    branch: ``atom_score`` is ``[G, R, max_kc]`` (``nosa_atom_scores`` for the
    rows ``rows``), ``cis`` is ``[total_k, G]``.  The qk page scores and the CIS
    page scores are pooled by ``page_maxpool_varlen``; CIS pages after the row's
    page are ``-inf``; the ``min(init + local + select, out_len)`` best qk pages
    are set to ``+inf`` in the CIS scores; the ``min(topk, out_len)`` best CIS
    pages, sorted, with ids past the row's page replaced by ``-1``.  Ties go to
    the lower page (``torch.topk`` leaves them unspecified).  With
    ``return_scores`` the qk and (masked, overlaid) CIS page scores are returned.
    ``clip`` is the pooling's column range (``page_maxpool_varlen``): the
    sequence's ``len_kc(b)`` windows, or the rows' whole width (``max_kc``
    atom columns, ``max_seqlen_k // 16 - 1`` window means whose padding is 0).
    """
    _check_clip(clip)
    cq = _as_list(cu_seqlens_q)
    ckc = _as_list(cu_seqlens_kc)
    total_q = cq[-1]
    row_list = list(range(total_q)) if rows is None else [int(r) for r in rows]
    R = len(row_list)
    G = atom_score.shape[0]
    s = block_size // kernel_stride
    ck = _as_list(cu_seqlens_k)
    # Row t of sequence b reads the b-th sequence's window means in the
    # broadcast layout of nosa_mean_pooling; only those per-sequence vectors are
    # formed here (the broadcast copy would be [G, total_q, M]).
    means: dict[int, torch.Tensor] = {}
    out_len = (int(max_seqlen_q) + block_size - 1) // block_size
    block = torch.full((G, R, out_len), float("-inf"), dtype=torch.float64)
    block_cis = torch.full((G, R, out_len), float("-inf"), dtype=torch.float64)
    for i, r in enumerate(row_list):
        b = next(j for j in range(len(cq) - 1) if cq[j] <= r < cq[j + 1])
        lk = ckc[b + 1] - ckc[b]
        if b not in means:
            means[b] = nosa_window_means(cis, ck[b], ck[b + 1], max_seqlen_k, kernel_size,
                                         kernel_stride)
        forced = _forced(torch.tensor([(r - cq[b]) // block_size]), out_len, init_blocks,
                         local_blocks)[0]
        row_clip = clip == "row"
        pb = _pool_pages(atom_score[:, i].to(torch.float64),
                         atom_score.shape[-1] if row_clip else lk, out_len, s)
        pc = _pool_pages(means[b].to(torch.float64), means[b].shape[-1] if row_clip else lk,
                         out_len, s)
        block[:, i] = pb.masked_fill(forced[None], float("inf"))
        block_cis[:, i] = pc.masked_fill(forced[None], float("inf"))
    q_idx_all = nosa_q_idx(cq, max_seqlen_q, block_size)
    q_idx = q_idx_all[torch.tensor(row_list, dtype=torch.long)] if R else q_idx_all[:0]
    return nosa_two_stage(block, block_cis, q_idx, topk=topk,
                          qk_select=init_blocks + local_blocks + select_blocks,
                          return_scores=return_scores)


def nosa_two_stage(block: torch.Tensor, block_cis: torch.Tensor, q_idx: torch.Tensor, *,
                   topk: int, qk_select: int, return_scores: bool = False):
    """The selection tail of ``compressed_attention`` (``nosa.py:1288-1305``) on
    pooled page scores ``[G, R, out_len]`` (forced pages already ``+inf``):
    CIS pages after ``q_idx`` ``-inf``; the ``min(qk_select, out_len)`` best qk
    pages ``+inf`` in the CIS scores; the ``min(topk, out_len)`` best CIS pages
    sorted, ids after ``q_idx`` replaced by ``-1``.  Ties go to the lower page."""
    out_len = block.shape[-1]
    j_idx = torch.arange(out_len)[None, :]
    block_cis = block_cis.masked_fill((j_idx > q_idx[:, None])[None], float("-inf"))
    short = _stable_topk_desc(block, min(int(qk_select), out_len))
    over = block_cis.clone()
    over.scatter_(2, short, float("inf"))
    k = min(int(topk), out_len)
    idx = _stable_topk_desc(over, k)
    idx = torch.sort(idx, dim=-1).values
    idx = idx.masked_fill(idx > q_idx[None, :, None], -1).to(torch.int32)
    if return_scores:
        return idx, block, over
    return idx


def nosa_pool_rows(page_qk: torch.Tensor, cis_means: torch.Tensor, cu_seqlens_q,
                   cu_seqlens_kc, rows: Sequence[int], *, out_len: int, init_blocks: int,
                   local_blocks: int, block_size: int = 64, kernel_stride: int = 16,
                   clip: str = "sequence"):
    """Stage inputs of ``nosa_two_stage`` from given intermediate scores: qk page
    scores ``page_qk [G, R, >= out_len]`` (pages without atoms ``-inf``) and
    pooled CIS window means ``cis_means [G, total_q, M]`` (``nosa_mean_pooling``
    layout), with the forced overlay of ``max_pooling_1d_varlen`` and its
    ``clip`` (the CIS means pool the sequence's windows, or all ``M``).
    Returns ``(block, block_cis)`` ``[G, R, out_len]`` float64."""
    _check_clip(clip)
    cq = _as_list(cu_seqlens_q)
    ckc = _as_list(cu_seqlens_kc)
    s = block_size // kernel_stride
    G = page_qk.shape[0]
    R = len(rows)
    block = torch.full((G, R, out_len), float("-inf"), dtype=torch.float64)
    block_cis = torch.full((G, R, out_len), float("-inf"), dtype=torch.float64)
    for i, r in enumerate(rows):
        b = next(j for j in range(len(cq) - 1) if cq[j] <= r < cq[j + 1])
        lk = ckc[b + 1] - ckc[b]
        forced = _forced(torch.tensor([(r - cq[b]) // block_size]), out_len, init_blocks,
                         local_blocks)[0]
        n = min(out_len, page_qk.shape[-1])
        pb = torch.full((G, out_len), float("-inf"), dtype=torch.float64)
        pb[:, :n] = page_qk[:, i, :n].to(torch.float64)
        pc = _pool_pages(cis_means[:, r].to(torch.float64),
                         cis_means.shape[-1] if clip == "row" else lk, out_len, s)
        block[:, i] = pb.masked_fill(forced[None], float("inf"))
        block_cis[:, i] = pc.masked_fill(forced[None], float("inf"))
    return block, block_cis


def nosa_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cis: torch.Tensor,
    cu_seqlens_q,
    cu_seqlens_k,
    topk_idx: torch.Tensor,
    *,
    softmax_scale: float | None = None,
    block_size: int = 64,
    rows: Sequence[int] | None = None,
    ids_rows_aligned: bool = False,
    return_lse: bool = False,
):
    """NOSA output ``[R, H, D]``: ``attn(q, k, V*e^cis) / attn(q, k, e^cis)``
    (``nosa.py:2211-2255``), i.e. ``sum_j w_j v_j / sum_j w_j`` with
    ``w_j = exp(scale * q.k_j + cis_j)`` over the causal keys of the row's pages.
    Computed in float64 from that closed form and rounded once.  With
    ``return_lse`` also ``log sum_j w_j`` ``[H, R]`` (``+inf`` for rows without
    keys)."""
    cq = _as_list(cu_seqlens_q)
    ck = _as_list(cu_seqlens_k)
    total_q, H, D = q.shape
    G = k.shape[1]
    gs = H // G
    scale = D ** -0.5 if softmax_scale is None else float(softmax_scale)
    row_list = list(range(total_q)) if rows is None else [int(r) for r in rows]
    out = torch.zeros((len(row_list), H, D), dtype=torch.float64)
    lse = torch.full((H, len(row_list)), float("inf"), dtype=torch.float64)
    f64 = torch.float64  # only the rows and keys each output reads are widened
    for i, r in enumerate(row_list):
        for g in range(G):
            ids = topk_idx[g, i if ids_rows_aligned else r]
            keys = attention_keys_for_row(r, ids, cq, ck, block_size=block_size, causal=True)
            if keys.numel() == 0:
                continue
            qh = q[r, g * gs : (g + 1) * gs].detach().to(f64)
            s = (qh @ k[keys, g].detach().to(f64).T) * scale + cis[keys, g].detach().to(f64)[None, :]
            m = s.amax(dim=-1, keepdim=True)
            w = torch.exp(s - m)
            out[i, g * gs : (g + 1) * gs] = (w @ v[keys, g].detach().to(f64)) / w.sum(dim=-1, keepdim=True)
            lse[g * gs : (g + 1) * gs, i] = (m[:, 0] + torch.log(w.sum(dim=-1)))
    if return_lse:
        return _round(out, q.dtype), lse
    return _round(out, q.dtype)
