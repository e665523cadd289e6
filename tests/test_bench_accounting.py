"""The algorithmic work bench.py divides by kernel time (the roofline numerator)
equals a brute-force count on small ragged cases."""
from types import SimpleNamespace

import torch

import bench
import oracle
from oracle.leanselect_oracle import attention_flops


def _plans(cu, take, seed):
    """Valid page plans: unique visible pages per row, ascending, -1 tail."""
    g = torch.Generator().manual_seed(seed)
    N = cu[-1]
    ids = torch.full((2, N, take), -1, dtype=torch.int32)
    for b in range(len(cu) - 1):
        for t in range(cu[b], cu[b + 1]):
            qp = (t - cu[b]) // 64
            for grp in range(2):
                n = int(torch.randint(0, min(take, qp + 1) + 1, (1,), generator=g))
                pages = torch.randperm(qp + 1, generator=g)[:n].sort().values
                ids[grp, t, :n] = pages.to(torch.int32)
    return ids


def test_attention_keys_match_the_oracle_key_sets():
    cu = [0, 70, 70, 330, 521]
    ids = _plans(cu, take=5, seed=0)
    got = bench.attention_keys(ids, cu)
    want = sum(oracle.attention_keys_for_row(r, ids[g, r], cu, cu).numel()
               for r in range(cu[-1]) for g in range(2))
    assert got == want
    assert bench.attention_keys(ids, cu) * 4.0 * 16 * 128 == attention_flops(cu, cu, ids, 32, 128)


def test_selection_flops_brute_force():
    cu = [0, 31, 600, 1000, 1100]
    init, local, D, F, H, G = 1, 2, 128, 128, 32, 2
    case = SimpleNamespace(q=torch.empty(cu[-1], H, D), k=torch.empty(cu[-1], G, D), cu_host=cu,
                           local_blocks=local, init_blocks=init)
    dots = 0
    proj = 0.0
    for b in range(len(cu) - 1):
        n = cu[b + 1] - cu[b]
        A = (n - 32) // 16 + 1 if n >= 32 else 0
        proj += 2.0 * n * G * (H // G) * D * F + 2.0 * A * G * D * F
        for t in range(n):
            qp = t // 64
            atoms = set()
            for p in range(init, qp - local):  # non-forced visible pages
                atoms |= {a for a in range(4 * p - 1, 4 * p + 4) if 0 <= a < A}
            dots += len(atoms)
    assert bench.selection_flops(case) == proj + 2.0 * G * F * dots
