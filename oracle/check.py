"""Parity rules used by the tests (test infrastructure).

Page ids: the north-star rule is "bit-exact wherever the score gap at the k-th
boundary exceeds 1e-3 relative".  Page scores in the reference are rounded to
the activation dtype, so for a 16-bit dtype one quantisation step at the
boundary is already ``2**-8`` (bf16) relative, larger than 1e-3.  Two
conforming implementations that accumulate the same float32 GEMM in different
orders can round a score one step apart, which moves a page by at most two
steps relative to the boundary.  The band around the k-th score is therefore
``max(rel_tol * |s_k|, ulp_band * step(s_k))`` with ``step`` the dtype's
quantisation step (zero for float32, where the band is the plain 1e-3 rule).

Inside the band a page may be in or out; outside it the sets must agree, and
the count, the forced pages and visibility must agree exactly.  A row whose
boundary gap exceeds the band is therefore compared bit-exactly.

Attention: max abs <= 2e-2 (scaled by the output magnitude above 1) and mean relative error
``mean|a - b| / mean|b| <= 1e-3`` against the oracle on the same ids.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

__all__ = ["dtype_step", "TopkReport", "check_topk", "check_attention"]


def dtype_step(x: float, dtype: torch.dtype) -> float:
    """Quantisation step of ``dtype`` at magnitude ``|x|`` (0 for float32/64)."""
    if dtype in (torch.float32, torch.float64) or not math.isfinite(x) or x == 0.0:
        return 0.0 if dtype in (torch.float32, torch.float64) else 2.0 ** -133
    mant = {torch.bfloat16: 7, torch.float16: 10}[dtype]
    e = math.floor(math.log2(abs(x)))
    step = 2.0 ** (e - mant)
    # Within two steps of the top of the binade the next binade's (double)
    # step applies to the neighbours above.
    return 2.0 * step if abs(x) >= 2.0 ** (e + 1) - 2.0 * step else step


@dataclass
class TopkReport:
    rows: int = 0
    exact_rows: int = 0
    band_rows: int = 0
    failures: list = field(default_factory=list)

    @property
    def ok(self) -> bool:
        return not self.failures

    def __str__(self) -> str:
        return (
            f"rows={self.rows} exact={self.exact_rows} band_swaps={self.band_rows} "
            f"failures={len(self.failures)} first={self.failures[:3]}"
        )


def check_topk(
    ids_test: torch.Tensor,
    ids_oracle: torch.Tensor,
    scores: torch.Tensor,
    dtype: torch.dtype,
    *,
    rel_tol: float = 1e-3,
    ulp_band: float = 2.0,
    max_failures: int = 20,
) -> TopkReport:
    """Compare page plans ``[G, R, take]`` row by row.

    ``scores`` are the oracle's masked page scores ``[G, R, P]`` (``+inf``
    forced, ``-inf`` invisible, rounded values otherwise) for the same rows.
    """
    rep = TopkReport()
    G, R, _ = ids_test.shape
    it = ids_test.cpu().to(torch.int64)
    io = ids_oracle.cpu().to(torch.int64)
    sc = scores.cpu().to(torch.float64)
    for g in range(G):
        for r in range(R):
            rep.rows += 1
            t_ids = [int(x) for x in it[g, r] if x >= 0]
            o_ids = [int(x) for x in io[g, r] if x >= 0]
            T, O = set(t_ids), set(o_ids)
            row = sc[g, r]
            err = None
            if len(T) != len(t_ids):
                err = "duplicate ids"
            elif len(T) != len(O):
                err = f"count {len(T)} != {len(O)}"
            elif any(p >= row.numel() or row[p] == float("-inf") for p in T):
                err = "invisible id"
            if err is None and T == O:
                rep.exact_rows += 1
                continue
            if err is None:
                forced = {p for p in range(row.numel()) if row[p] == float("inf")}
                if len(forced) >= len(O):
                    err = "forced-only row differs"
                elif not forced <= T:
                    err = "missing forced page"
                else:
                    chosen = sorted((row[p].item() for p in O - forced), reverse=True)
                    s_k = chosen[-1]
                    band = max(rel_tol * abs(s_k), ulp_band * dtype_step(s_k, dtype))
                    cand = [
                        p for p in range(row.numel())
                        if p not in forced and math.isfinite(row[p].item())
                    ]
                    for p in cand:
                        v = row[p].item()
                        if v > s_k + band and p not in T:
                            err = f"page {p} ({v}) above band missing (s_k={s_k}, band={band})"
                            break
                        if v < s_k - band and p in T:
                            err = f"page {p} ({v}) below band chosen (s_k={s_k}, band={band})"
                            break
            if err is None:
                rep.band_rows += 1
            elif len(rep.failures) < max_failures:
                rep.failures.append((g, r, err))
            else:
                rep.failures.append((g, r, "..."))
    return rep


def check_attention(
    out_test: torch.Tensor,
    out_ref: torch.Tensor,
    *,
    max_abs: float = 2e-2,
    mean_rel: float = 1e-3,
) -> tuple[bool, float, float]:
    """``(ok, max scaled error, mean relative error)``.

    The max-abs bound applies to outputs of magnitude up to 1 and scales with
    the magnitude above it (``|a - b| <= max_abs * max(1, |b|)``): one bf16 step
    at |b| in [8, 16) is already 0.0625, so a fixed 2e-2 would be below the
    format's resolution for large outputs.
    """
    a = out_test.detach().cpu().to(torch.float64)
    b = out_ref.detach().cpu().to(torch.float64)
    diff = (a - b).abs()
    mx = float((diff / b.abs().clamp_min(1.0)).max()) if diff.numel() else 0.0
    denom = float(b.abs().mean()) if b.numel() else 1.0
    mr = float(diff.mean()) / max(denom, 1e-30) if diff.numel() else 0.0
    return (mx <= max_abs and mr <= mean_rel), mx, mr
