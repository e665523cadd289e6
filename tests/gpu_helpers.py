"""Shared helpers for the GPU parity tests (imports the oracle as the checker)."""
from __future__ import annotations

import torch

import oracle


def plan_structure_errors(ids: torch.Tensor, cu_host: list[int], take: int, init: int, local: int,
                          block_size: int = 64, kernel_size: int = 32) -> list[str]:
    """Size-independent checks of a page plan ``[G, total, take]`` (on its device).

    Per row: valid ids ascending and unique, ``-1`` only as a tail, exactly
    ``min(take_b, qp + 1)`` ids, every id visible and every forced page present;
    rows of a sequence without compressed key are all ``-1``.
    """
    errs = []
    G, total, T = ids.shape
    dev = ids.device
    if T != take:
        return [f"take {T} != {take}"]
    qpos = torch.empty(total, dtype=torch.long, device=dev)
    nval = torch.empty(total, dtype=torch.long, device=dev)
    for b in range(len(cu_host) - 1):
        s, e = cu_host[b], cu_host[b + 1]
        if e <= s:
            continue
        t = torch.arange(e - s, device=dev)
        qpos[s:e] = t // block_size
        n_pages = (e - s + block_size - 1) // block_size
        has_atoms = (e - s) >= kernel_size
        nval[s:e] = torch.minimum(torch.full_like(t, min(take, n_pages)), t // block_size + 1) if has_atoms else 0
    valid = ids >= 0
    cnt = valid.sum(-1)
    if not torch.equal(cnt, nval.expand(G, -1)):
        bad = (cnt != nval).nonzero()[:3].tolist()
        errs.append(f"count mismatch at {bad}")
    # -1 only as a tail: valid slots are a prefix.
    if T > 1 and bool((~valid[..., :-1] & valid[..., 1:]).any()):
        errs.append("-1 before a valid id")
    if T > 1:
        inc = (ids[..., 1:] > ids[..., :-1]) | ~valid[..., 1:]
        if not bool(inc.all()):
            errs.append("ids not strictly ascending")
    if bool((ids > qpos[None, :, None]).any()):
        errs.append("invisible page chosen")
    # Forced pages: sink pages and the local window ending at qp (all of them
    # whenever they fit in the row's budget).
    lo_end = torch.clamp(qpos + 1, max=init)
    hi_start = torch.maximum(qpos - local, lo_end)
    fits = (lo_end + (qpos + 1 - hi_start) <= nval) & (nval > 0)
    for p_rel in range(local + 1):
        p = qpos - p_rel
        need = (p >= 0) & fits
        present = (ids == p[None, :, None]).any(-1)
        if bool((need[None] & ~present).any()):
            errs.append(f"local page qp-{p_rel} missing")
    for p in range(init):
        need = (qpos >= p) & (nval > p)
        present = (ids == p).any(-1)
        if bool((need[None] & ~present).any()):
            errs.append(f"sink page {p} missing")
    return errs


def oracle_select_rows(case, kc_cpu, cu_c, rows, dtype):
    qf, kf = oracle.fused_weights(case.selector.head_mix.cpu(), case.selector.kv_head_mix.cpu(),
                                  case.selector.q_proj.cpu(), case.selector.k_proj.cpu(), dtype)
    return oracle.select_prefill(
        case.q.cpu(), kc_cpu, case.cu_host, cu_c, qf, kf, topk=case.topk,
        block_size=case.block_size, kernel_stride=case.kernel_stride,
        init_blocks=case.init_blocks, local_blocks=case.local_blocks, rows=rows,
        return_scores=True)


def spread_rows(cu_host: list[int], per_seq: int = 96) -> list[int]:
    """Deterministic sample: first/last rows, block edges and an even spread per sequence."""
    rows = set()
    for b in range(len(cu_host) - 1):
        s, e = cu_host[b], cu_host[b + 1]
        n = e - s
        if n <= 0:
            continue
        for r in (0, 1, 63, 64, 65, n - 1, n - 2, n - 64):
            if 0 <= r < n:
                rows.add(s + r)
        step = max(1, n // per_seq)
        rows.update(range(s, e, step))
    return sorted(rows)
