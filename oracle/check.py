"""Parity rules used by the tests (test infrastructure).

Page ids (the north-star rule): a row's selected set must be bit-exact
wherever the score gap at the k-th boundary exceeds 1e-3 relative.  Concretely,
with ``s_k`` the oracle's k-th chosen (non-forced) page score, a page whose
score lies more than ``1e-3 * |s_k|`` above ``s_k`` must be chosen and one more
than that below must not; only pages inside that band (ties and near-ties at
the boundary) may differ.  The count, the forced pages and visibility must
agree exactly.  Page scores are rounded to the activation dtype, so for bf16 /
fp16 the band holds exact ties only (one quantisation step is 2^-8 / 2^-11
relative).  ``TopkReport.band_rows`` counts rows that differ inside the band;
the tests assert it is zero wherever that is what was measured.

Attention (max abs 2e-2, mean relative 1e-3 against the
oracle on the same ids): every element must satisfy ``|a - b| <= 2e-2`` or,
where one quantisation step of the output dtype at ``|b|`` exceeds 2e-2
(bf16 outputs of magnitude 4 and above), ``|a - b| <= one step`` -- two
correct implementations can round one value to neighbouring representable
numbers, and no tighter bound exists in the format; and
``mean|a - b| / mean|b| <= 1e-3``.  The raw max-abs difference is reported.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

__all__ = ["dtype_step", "output_step", "TopkReport", "check_topk", "check_attention",
           "check_nosa_topk"]


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
    ulp_band: float = 0.0,
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


def output_step(b: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """One quantisation step of ``dtype`` at each ``|b|`` (0 for float32/64)."""
    if dtype not in (torch.bfloat16, torch.float16):
        return torch.zeros_like(b)
    mant = 7 if dtype == torch.bfloat16 else 10
    _, e = torch.frexp(b.abs())  # |b| = m * 2^e with m in [0.5, 1)
    return torch.ldexp(torch.ones_like(b), (e - 1 - mant).to(torch.int32))


def check_attention(
    out_test: torch.Tensor,
    out_ref: torch.Tensor,
    *,
    max_abs: float = 2e-2,
    mean_rel: float = 1e-3,
    literal: bool = False,
) -> tuple[bool, float, float]:
    """``(ok, raw max |a - b|, mean relative error)``.

    Element bound: ``|a - b| <= max(max_abs, one output-dtype step at |b|)``
    (the step exceeds 2e-2 only for bf16 outputs of magnitude 4 and above);
    with ``literal=True`` the bound is ``max_abs`` alone, with no allowance.
    Mean bound: ``mean|a - b| / mean|b| <= mean_rel``.
    """
    a = out_test.detach().cpu().to(torch.float64)
    b = out_ref.detach().cpu().to(torch.float64)
    diff = (a - b).abs()
    if not diff.numel():
        return True, 0.0, 0.0
    if literal:
        tol = torch.full_like(b, float(max_abs))
    else:
        tol = output_step(b, out_test.dtype).clamp_min(max_abs)
    elem_ok = bool((diff <= tol).all())
    mx = float(diff.max())
    denom = float(b.abs().mean())
    mr = float(diff.mean()) / max(denom, 1e-30)
    return (elem_ok and mr <= mean_rel), mx, mr


def _boundary_gap(row: torch.Tensor, k: int) -> tuple[float, float]:
    """(k-th largest, (k+1)-th largest) of a score row (``-inf`` past the end)."""
    vals = torch.sort(row, descending=True).values
    a = float(vals[k - 1]) if 0 < k <= vals.numel() else float("inf")
    b = float(vals[k]) if k < vals.numel() else float("-inf")
    return a, b


def _near_tie(a: float, b: float, rel_tol: float) -> bool:
    if a == b:
        return True
    if not (math.isfinite(a) and math.isfinite(b)):
        return False
    return a - b <= rel_tol * abs(a)


def check_nosa_topk(
    ids_test: torch.Tensor,
    ids_oracle: torch.Tensor,
    block: torch.Tensor,
    over: torch.Tensor,
    *,
    topk: int,
    qk_select: int,
    rel_tol: float = 1e-3,
    max_failures: int = 20,
) -> TopkReport:
    """Gap-aware comparison of NOSA page plans ``[G, R, take]``.

    ``block`` are the oracle's pooled qk page scores (forced pages ``+inf``) and
    ``over`` its stage-2 CIS scores (pages after ``q_idx`` ``-inf``, the qk
    shortlist ``+inf``), both ``[G, R, out_len]`` as ``nosa_two_stage`` returns
    them.  A row must equal the oracle's unless one of the two selection
    boundaries -- the ``qk_select``-th qk page (the shortlist) or the
    ``topk``-th stage-2 page -- is a tie or near-tie (gap within ``rel_tol``
    relative), where a different but equally valid choice exists; such a row
    counts as a band row and must still hold the same number of ids.
    """
    rep = TopkReport()
    G, R, _ = ids_test.shape
    it = ids_test.cpu().to(torch.int64)
    io = ids_oracle.cpu().to(torch.int64)
    out_len = block.shape[-1]
    k1 = min(int(qk_select), out_len)
    k2 = min(int(topk), out_len)
    for g in range(G):
        for r in range(R):
            rep.rows += 1
            if torch.equal(it[g, r], io[g, r]):
                rep.exact_rows += 1
                continue
            err = None
            if int((it[g, r] >= 0).sum()) != int((io[g, r] >= 0).sum()):
                err = "count differs"
            else:
                t1 = _near_tie(*_boundary_gap(block[g, r].double(), k1), rel_tol)
                t2 = _near_tie(*_boundary_gap(over[g, r].double(), k2), rel_tol)
                if not (t1 or t2):
                    err = "differs with no tie at either selection boundary"
            if err is None:
                rep.band_rows += 1
            elif len(rep.failures) < max_failures:
                rep.failures.append((g, r, err))
            else:
                rep.failures.append((g, r, "..."))
    return rep
