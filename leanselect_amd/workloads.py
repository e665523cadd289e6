"""Seeded synthetic inputs for the benchmark and tests.

Two families:

* ``head_space_layer`` -- the CPU-sized single-layer case: Q, K, V ~ N(0, 1) in
  head space plus a rank-4 per-page topic (amplitude 2.0) on K and on the
  queries of the block that "wants" those pages; router mixes ~ N(0, 0.1^2).
* ``hidden_space_layer`` -- the MiniCPM4.1-8B attention-layer shape: hidden
  states X ~ N(0, 1) [N, hidden], random projections W ~ N(0, 0.02^2), and
  rank-8 page topics planted in X (each query block and 8 of its earlier
  non-forced pages share a topic direction).  Topic directions are chosen among
  random candidates for a positive router-space alignment, so planted pages
  score high rather than at a random sign.

Generation uses ``torch.Generator`` on the target device; the oracle receives
the same bits by copying the generated tensors.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch

from .selector import LeanSelectSelector

__all__ = ["LayerCase", "head_space_layer", "hidden_space_layer", "planted_pages",
           "UNIT_SCALE"]


@dataclass
class LayerCase:
    q: torch.Tensor            # [total, H, D]
    k: torch.Tensor            # [total, G, D]
    v: torch.Tensor            # [total, G, D]
    cu_seqlens: torch.Tensor   # int32 [B + 1]
    cu_host: list[int]
    selector: LeanSelectSelector
    topk: int                  # total budget (incl. forced pages)
    init_blocks: int
    local_blocks: int
    block_size: int = 64
    kernel_size: int = 32
    kernel_stride: int = 16
    planted: dict = field(default_factory=dict)

    @property
    def max_seqlen(self) -> int:
        return max(self.cu_host[i + 1] - self.cu_host[i] for i in range(len(self.cu_host) - 1))


# Keyword arguments of ``hidden_space_layer`` for a unit-scale layer: plants
# that do not accumulate and values of std about 0.5 (hidden 4096).
UNIT_SCALE = {"accumulate_plants": False, "value_std": 0.4 / 64}


def planted_pages(n_blocks: int, init_blocks: int, local_blocks: int, per_block: int,
                  gen: torch.Generator) -> dict[int, list[int]]:
    """For each query block b, up to ``per_block`` distinct earlier non-forced pages."""
    out = {}
    for b in range(n_blocks):
        lo, hi = init_blocks, b - local_blocks - 1
        if hi < lo:
            continue
        n = hi - lo + 1
        k = min(per_block, n)
        perm = torch.randperm(n, generator=gen)[:k]
        out[b] = sorted(int(lo + x) for x in perm)
    return out


def _cu(seq_lens) -> list[int]:
    cu = [0]
    for n in seq_lens:
        cu.append(cu[-1] + int(n))
    return cu


def head_space_layer(
    seq_len: int = 4096,
    *,
    num_heads: int = 8,
    num_kv_heads: int = 2,
    head_dim: int = 128,
    dtype: torch.dtype = torch.float32,
    seed: int = 0,
    device: str | torch.device = "cpu",
    topk: int = 16,
    local_blocks: int = 2,
    init_blocks: int = 1,
    topic_rank: int = 4,
    topic_amp: float = 2.0,
    pages_per_block: int = 8,
    mix_std: float = 0.1,
    router_heads: int = 4,
    router_dim: int = 32,
) -> LayerCase:
    """CPU-runnable layer: seq 4096, 8q/2kv heads, budget 16 = 14 + 2 local pages."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    N, H, G, D = seq_len, num_heads, num_kv_heads, head_dim
    q = torch.randn(N, H, D, generator=g)
    k = torch.randn(N, G, D, generator=g)
    v = torch.randn(N, G, D, generator=g)
    U = torch.linalg.qr(torch.randn(D, topic_rank, generator=g)).Q.T  # [rank, D]
    n_blocks = (N + 63) // 64
    plan = planted_pages(n_blocks, init_blocks, local_blocks, pages_per_block, g)
    for b, pages in plan.items():
        w = torch.randn(topic_rank, generator=g) @ U
        w = w / w.norm()
        q[b * 64 : min(N, b * 64 + 64)] += topic_amp * w
        for p in pages:
            k[p * 64 : min(N, p * 64 + 64)] += topic_amp * w
    torch.manual_seed(seed)  # the selector's orthonormal frame
    sel = LeanSelectSelector(num_heads=H, num_kv_heads=G, head_dim=D,
                             router_heads=router_heads, router_dim=router_dim)
    with torch.no_grad():
        sel.head_mix.copy_(torch.randn(H, router_heads, generator=g) * mix_std)
        sel.kv_head_mix.copy_(torch.randn(G, router_heads, generator=g) * mix_std)
    sel.requires_grad_(False)
    dev = torch.device(device)
    cu_host = [0, N]
    return LayerCase(
        q=q.to(dtype).to(dev), k=k.to(dtype).to(dev), v=v.to(dtype).to(dev),
        cu_seqlens=torch.tensor(cu_host, dtype=torch.int32, device=dev), cu_host=cu_host,
        selector=sel.to(dev), topk=topk, init_blocks=init_blocks, local_blocks=local_blocks,
        planted=plan)


def hidden_space_layer(
    seq_lens=(32768,),
    *,
    hidden: int = 4096,
    num_heads: int = 32,
    num_kv_heads: int = 2,
    head_dim: int = 128,
    dtype: torch.dtype = torch.bfloat16,
    seed: int = 0,
    device: str | torch.device = "cpu",
    topk: int = 64,
    local_blocks: int = 4,
    init_blocks: int = 1,
    n_topics: int = 8,
    topic_amp: float = 48.0,
    pages_per_block: int = 8,
    weight_std: float = 0.02,
    router_heads: int = 4,
    router_dim: int = 32,
    accumulate_plants: bool = True,
    value_std: float | None = None,
) -> LayerCase:
    """MiniCPM4.1-8B attention-layer shape (hidden 4096, 32q/2kv, D 128), packed sequences.

    A page planted by several query blocks carries the sum of their topic
    directions (up to ~56 plants on early pages at 128K, so its keys and values
    grow with the count).  With ``accumulate_plants=False`` each planted row
    instead gets ``topic_amp`` times the unit vector of that sum: every row's
    plant has the same amplitude.  ``value_std`` (default ``weight_std``) is
    the value projection's std: ``0.4 / sqrt(hidden)`` keeps every value, and so
    every attention output, well inside (-4, 4)."""
    dev = torch.device(device)
    g = torch.Generator(device=dev).manual_seed(seed)
    gc = torch.Generator(device="cpu").manual_seed(seed + 1)
    H, G, D = num_heads, num_kv_heads, head_dim
    cu_host = _cu(seq_lens)
    N = cu_host[-1]
    torch.manual_seed(seed)
    sel = LeanSelectSelector(num_heads=H, num_kv_heads=G, head_dim=D,
                             router_heads=router_heads, router_dim=router_dim)
    sel.requires_grad_(False)
    wdt = torch.float32
    Wq = torch.randn(hidden, H * D, generator=g, device=dev, dtype=wdt) * weight_std
    Wk = torch.randn(hidden, G * D, generator=g, device=dev, dtype=wdt) * weight_std
    Wv = torch.randn(hidden, G * D, generator=g, device=dev, dtype=wdt) * (
        weight_std if value_std is None else value_std)

    # Topic directions: among random unit candidates keep those whose router
    # alignment q~(u) . k~(u) is largest in the worse of the KV groups.
    with torch.no_grad():
        cand = torch.randn(16 * n_topics, hidden, generator=g, device=dev, dtype=wdt)
        cand = cand / cand.norm(dim=1, keepdim=True)
        hm, khm = sel.head_mix.to(dev), sel.kv_head_mix.to(dev)
        qp, kp = sel.q_proj.to(dev), sel.k_proj.to(dev)
        qf = torch.einsum("hr,rdj->hdrj", hm, qp).reshape(H, D, -1)
        kf = torch.einsum("hr,rdj->hdrj", khm, kp).reshape(G, D, -1)
        qc = (cand @ Wq).reshape(-1, G, H // G, D)
        kc = (cand @ Wk).reshape(-1, G, D)
        qt = torch.einsum("cgsd,gsdf->cgf", qc, qf.reshape(G, H // G, D, -1))
        kt = torch.einsum("cgd,gdf->cgf", kc, kf)
        align = (qt * kt).sum(-1).min(dim=1).values
        topics = cand[torch.argsort(align, descending=True)[:n_topics]]

    X = torch.randn(N, hidden, generator=g, device=dev, dtype=wdt)
    planted = {}
    for b_idx in range(len(cu_host) - 1):
        start, length = cu_host[b_idx], cu_host[b_idx + 1] - cu_host[b_idx]
        n_blocks = (length + 63) // 64
        plan = planted_pages(n_blocks, init_blocks, local_blocks, pages_per_block, gc)
        if not plan:
            continue
        tau = torch.randint(0, n_topics, (n_blocks,), generator=gc)
        rows_q, rows_k, tq, tk = [], [], [], []
        for blk, pages in plan.items():
            r0, r1 = start + blk * 64, start + min(length, blk * 64 + 64)
            rows_q.append(torch.arange(r0, r1))
            tq.append(torch.full((r1 - r0,), int(tau[blk])))
            for p in pages:
                p0, p1 = start + p * 64, start + min(length, p * 64 + 64)
                rows_k.append(torch.arange(p0, p1))
                tk.append(torch.full((p1 - p0,), int(tau[blk])))
        planted[b_idx] = plan
        rq, rk = torch.cat(rows_q).to(dev), torch.cat(rows_k).to(dev)
        X.index_add_(0, rq, topic_amp * topics[torch.cat(tq).to(dev)])
        if accumulate_plants:
            X.index_add_(0, rk, topic_amp * topics[torch.cat(tk).to(dev)])
        else:
            urk, inv = torch.unique(rk, return_inverse=True)
            acc = torch.zeros(urk.numel(), hidden, device=dev, dtype=wdt)
            acc.index_add_(0, inv, topics[torch.cat(tk).to(dev)])
            acc = acc / acc.norm(dim=1, keepdim=True).clamp_min(1e-12)
            X.index_add_(0, urk, topic_amp * acc)
            del acc

    with torch.no_grad():
        q = (X @ Wq).to(dtype).reshape(N, H, D)
        k = (X @ Wk).to(dtype).reshape(N, G, D)
        v = (X @ Wv).to(dtype).reshape(N, G, D)
    del X
    return LayerCase(
        q=q, k=k, v=v, cu_seqlens=torch.tensor(cu_host, dtype=torch.int32, device=dev),
        cu_host=cu_host, selector=sel.to(dev), topk=topk, init_blocks=init_blocks,
        local_blocks=local_blocks, planted=planted)
