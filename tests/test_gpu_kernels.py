"""GPU parity of each HIP kernel against the CPU oracle (bit-level where the
reference's arithmetic is exact, one quantisation step otherwise)."""
import pytest
import torch

import oracle
from leanselect_amd import pages
from leanselect_amd.ops import compress_k
from leanselect_amd.selector import LeanSelectSelector

pytestmark = pytest.mark.gpu
DEV = "cuda"
DTYPES = [torch.float32, torch.bfloat16, torch.float16]


def _cu(lens):
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    return cu


def _ulp_diff(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """|a - b| in units of the dtype's step at |b| (16-bit dtypes)."""
    mant = 7 if a.dtype == torch.bfloat16 else 10
    af, bf = a.float(), b.float()
    e = torch.floor(torch.log2(bf.abs().clamp_min(1e-30)))
    return (af - bf).abs() / torch.exp2(e - mant)


def _step(x: torch.Tensor, dtype) -> torch.Tensor:
    """Quantisation step of ``dtype`` at |x| (elementwise)."""
    mant = 7 if dtype == torch.bfloat16 else 10
    e = torch.floor(torch.log2(x.float().abs().clamp_min(2.0 ** -126)))
    return torch.exp2(e - mant)


def _assert_rounded_gemm(got, want, absdot, K, dtype, max_mismatch):
    """One rounding of a float32-accumulated contraction: at most one step plus the
    float32 accumulation bound K * 2**-24 * sum|a*b|, and rare mismatches."""
    assert (got != want).float().mean().item() < max_mismatch
    bound = _step(want, dtype) + K * 2.0 ** -24 * absdot
    assert bool(((got.double() - want.double()).abs() <= bound).all())


def _selector(H=32, G=2, D=128, R=4, RD=32, seed=0):
    torch.manual_seed(seed)
    s = LeanSelectSelector(num_heads=H, num_kv_heads=G, head_dim=D, router_heads=R, router_dim=RD)
    with torch.no_grad():
        s.head_mix.normal_(0, 0.1)
        s.kv_head_mix.normal_(0, 0.1)
    return s.requires_grad_(False).to(DEV)


@pytest.mark.parametrize("geom", [(32, 16, 128), (32, 16, 64), (48, 16, 128), (32, 8, 128)])
def test_compress_k_geometries(geom):
    """Half-window sharing (windows of two strides, 16 or 32 windows per block) and
    the direct path for other geometries, across sequence and block boundaries."""
    ks, st, D = geom
    lens = [100, 31, ks, ks + st, 0, 77, 700, 16 * st + ks]
    cu = _cu(lens)
    torch.manual_seed(2)
    k = torch.randn(cu[-1], 2, D).to(torch.bfloat16)
    got, cu_c = compress_k(k.to(DEV), torch.tensor(cu, dtype=torch.int32, device=DEV),
                           kernel_size=ks, kernel_stride=st)
    want, cu_want = oracle.compress_k(k, cu, kernel_size=ks, kernel_stride=st)
    assert cu_c.cpu().tolist() == cu_want.tolist()
    got = got.cpu()
    assert (got != want).float().mean().item() < 1e-3
    assert _ulp_diff(got, want).max().item() <= 1.0


@pytest.mark.parametrize("dtype", DTYPES)
def test_compress_k_matches_oracle(dtype):
    lens = [100, 31, 32, 48, 0, 77, 5000]
    cu = _cu(lens)
    torch.manual_seed(1)
    k = torch.randn(cu[-1], 2, 128).to(dtype)
    got, cu_c = compress_k(k.to(DEV), torch.tensor(cu, dtype=torch.int32, device=DEV))
    want, cu_want = oracle.compress_k(k, cu)
    assert cu_c.cpu().tolist() == cu_want.tolist()
    got = got.cpu()
    if dtype == torch.float32:
        torch.testing.assert_close(got, want, rtol=2e-6, atol=1e-7)
    else:
        assert (got != want).float().mean().item() < 1e-3
        assert _ulp_diff(got, want).max().item() <= 1.0


@pytest.mark.parametrize("dtype", DTYPES)
def test_fused_weights_bit_exact(dtype):
    s = _selector()
    qf, kf = s.fused_weights(dtype=dtype)
    wq, wk = oracle.fused_weights(s.head_mix.cpu(), s.kv_head_mix.cpu(), s.q_proj.cpu(),
                                  s.k_proj.cpu(), dtype)
    assert torch.equal(qf.cpu(), wq) and torch.equal(kf.cpu(), wk)


@pytest.mark.parametrize("dtype", DTYPES)
def test_projections_match_oracle(dtype):
    s = _selector()
    torch.manual_seed(2)
    q = torch.randn(1000, 32, 128).to(dtype)
    kc = torch.randn(77, 2, 128).to(dtype)
    got_q = s.project_queries(q.to(DEV)).cpu()
    got_k = s.project_atom_keys(kc.to(DEV)).cpu()
    wq, wk = oracle.fused_weights(s.head_mix.cpu(), s.kv_head_mix.cpu(), s.q_proj.cpu(),
                                  s.k_proj.cpu(), dtype)
    want_q = oracle.project_queries(q, wq, 2)
    want_k = oracle.project_atom_keys(kc, wk)
    abs_q = oracle.project_queries(q.abs(), wq.abs(), 2).double()
    abs_k = oracle.project_atom_keys(kc.abs(), wk.abs()).double()
    for got, want, absdot, K in ((got_q, want_q, abs_q, 16 * 128), (got_k, want_k, abs_k, 128)):
        assert got.shape == want.shape and got.dtype == dtype
        if dtype == torch.float32:
            torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5)
        else:
            _assert_rounded_gemm(got, want, absdot, K, dtype, 2e-3)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n", [700, 64, 33])
def test_score_pages_matches_oracle(dtype, n):
    _check_score_pages(_selector(), dtype, n)


@pytest.mark.parametrize("router", [(8, 32), (2, 32), (1, 64)])
@pytest.mark.parametrize("n", [1000, 300])
def test_score_pages_router_widths(router, n):
    # Router widths 256 (shared-panel kernel, 8 k-slices) and 64 (per-wave kernel).
    _check_score_pages(_selector(R=router[0], RD=router[1]), torch.bfloat16, n)


def _check_score_pages(s, dtype, n):
    torch.manual_seed(3)
    q = torch.randn(n, 32, 128).to(dtype)
    k = torch.randn(n, 2, 128).to(dtype)
    kc, _ = oracle.compress_k(k, [0, n])
    got = s.score_pages(q.to(DEV), kc.to(DEV), seq_len=n, block_size=64, kernel_stride=16).cpu()
    wq, wk = oracle.fused_weights(s.head_mix.cpu(), s.kv_head_mix.cpu(), s.q_proj.cpu(),
                                  s.k_proj.cpu(), dtype)
    qt, kt = oracle.project_queries(q, wq, 2), oracle.project_atom_keys(kc, wk)
    want = oracle.pool_atoms_to_pages(oracle.atom_scores(qt, kt), seq_len=n)
    # Bound on one atom score when q~ and k~ may each sit one step off:
    # 2**-6 * sum_f |q~_f| |k~_f| (+ one step of the score itself), pooled by max.
    absdot = torch.bmm(qt.double().abs(), kt.double().abs().transpose(1, 2))
    page_bound = oracle.pool_atoms_to_pages(absdot, seq_len=n)
    assert got.shape == want.shape == (2, n, (n + 63) // 64)
    fin = torch.isfinite(want)
    assert torch.equal(torch.isfinite(got), fin)
    if dtype == torch.float32:
        torch.testing.assert_close(got[fin], want[fin], rtol=1e-4, atol=1e-4)
    else:
        assert (got[fin] != want[fin]).float().mean().item() < 0.05
        bound = 2 * _step(want[fin], dtype) + 2.0 ** -6 * page_bound[fin]
        assert bool(((got[fin].double() - want[fin].double()).abs() <= bound).all())


@pytest.mark.parametrize("dtype", DTYPES)
def test_pool_and_forced_mask_exact(dtype):
    torch.manual_seed(4)
    for n_atoms, seq_len in ((15, 256), (31, 512), (37, 3000), (1, 64)):
        x = torch.randn(3, 5, n_atoms).to(dtype)
        got = pages.pool_atoms_to_pages(x.to(DEV), seq_len=seq_len).cpu()
        assert torch.equal(got, oracle.pool_atoms_to_pages(x, seq_len=seq_len))
    pos = torch.tensor([[0, 5, 63, 64, 200, 1000], [7, 64, 128, 129, 640, 2047]])
    got = pages.forced_page_mask(pos.to(DEV), num_pages=40, init_blocks=2, local_blocks=3).cpu()
    assert torch.equal(got, oracle.forced_page_mask(pos, num_pages=40, init_blocks=2, local_blocks=3))


def test_compress_keys_mean_matches_oracle():
    torch.manual_seed(5)
    for S in (20, 32, 80, 1000):
        k = torch.randn(2, S, 2, 128, dtype=torch.float32)
        got = pages.compress_keys_mean(k.to(DEV)).cpu()
        torch.testing.assert_close(got, oracle.compress_keys_mean(k), rtol=2e-6, atol=1e-7)
