"""Pins of the MiniCPM decoder pieces of the oracle (CPU): closed forms in
float64, invariants of the rotary embedding and a planted mistake the checks
must catch.  Plus host-side argument checks of the matching C entry points."""
import math

import pytest
import torch

import oracle
from leanselect_amd import _hip


def test_rotary_tables_closed_form():
    D, P, base = 128, 300, 10000.0
    cos, sin = oracle.rotary_tables(D, P, base)
    assert cos.dtype == torch.float32 and cos.shape == (P, D)
    i = torch.arange(D // 2, dtype=torch.float64)
    theta = torch.arange(P, dtype=torch.float64)[:, None] * base ** (-2 * i / D)[None, :]
    # float32 argument rounding grows with the angle: |d cos| <= |d theta|.
    tol = 4 * torch.finfo(torch.float32).eps * (1 + theta)
    for half in (slice(0, D // 2), slice(D // 2, D)):
        assert bool(((cos[:, half].double() - theta.cos()).abs() <= tol).all())
        assert bool(((sin[:, half].double() - theta.sin()).abs() <= tol).all())
    assert torch.equal(cos[0], torch.ones(D)) and torch.equal(sin[0], torch.zeros(D))


def _rope64(x: torch.Tensor, pos: torch.Tensor, base=10000.0) -> torch.Tensor:
    """RoPE as a complex rotation of (x[d], x[d + D/2]) by pos * base^(-2d/D), float64."""
    D = x.shape[-1]
    i = torch.arange(D // 2, dtype=torch.float64)
    ang = pos.double()[:, None, None] * base ** (-2 * i / D)
    z = torch.complex(x[..., : D // 2].double(), x[..., D // 2:].double()) * torch.polar(
        torch.ones_like(ang), ang)
    return torch.cat((z.real, z.imag), dim=-1)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rope_is_a_complex_rotation(dtype):
    g = torch.Generator().manual_seed(0)
    n, H, D = 64, 3, 128
    x = torch.randn(n, H, D, generator=g).to(dtype)
    pos = torch.randint(0, 4000, (n,), generator=g)
    cos, sin = oracle.rotary_tables(D, 4000)
    got = oracle.apply_rotary_pos_emb(x, cos, sin, pos).double()
    want = _rope64(x, pos)
    step = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -20
    # float32 table error grows with pos (|d angle| ~ pos * 2^-24), then one rounding.
    tol = step * want.abs() + (pos.double()[:, None, None] * 2 ** -22 + 2 ** -20) * x.double().abs().max()
    assert bool(((got - want).abs() <= tol + 1e-30).all())
    # position 0 is the identity, exactly
    zero = torch.zeros(n, dtype=torch.long)
    assert torch.equal(oracle.apply_rotary_pos_emb(x, cos, sin, zero), x)


def test_rope_relative_position_and_norm():
    g = torch.Generator().manual_seed(1)
    D = 128
    q = torch.randn(1, 1, D, generator=g)
    k = torch.randn(1, 1, D, generator=g)
    cos, sin = oracle.rotary_tables(D, 2048)
    dots = []
    for m, nn in ((10, 3), (110, 103), (1500, 1493)):
        qm = oracle.apply_rotary_pos_emb(q, cos, sin, torch.tensor([m]))
        kn = oracle.apply_rotary_pos_emb(k, cos, sin, torch.tensor([nn]))
        dots.append(float((qm.double() * kn.double()).sum()))
        pair = lambda t: t[..., :64].double() ** 2 + t[..., 64:].double() ** 2  # noqa: E731
        assert torch.allclose(pair(qm), pair(q), rtol=1e-5, atol=1e-6)
    assert max(dots) - min(dots) < 1e-3 * max(1.0, abs(dots[0]))


def test_rope_planted_sign_mistake_is_caught():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(16, 2, 128, generator=g)
    pos = torch.randint(1, 500, (16,), generator=g)
    cos, sin = oracle.rotary_tables(128, 500)
    wrong = (x * cos[pos][:, None] - oracle.minicpm_oracle._rotate_half(x) * sin[pos][:, None])
    assert not torch.allclose(wrong.double(), _rope64(x, pos), atol=1e-3)
    assert torch.allclose(oracle.apply_rotary_pos_emb(x, cos, sin, pos).double(),
                          _rope64(x, pos), atol=1e-3)


@pytest.mark.parametrize("hidden", [512, 4096])
def test_rms_layernorm_closed_form(hidden):
    g = torch.Generator().manual_seed(hidden)
    x = (torch.randn(40, hidden, generator=g) * 3).bfloat16()
    w = (1 + 0.1 * torch.randn(hidden, generator=g)).bfloat16()
    got = oracle.rms_layernorm(x, w, 1e-6)
    assert got.dtype == torch.bfloat16
    xd = x.double()
    n = xd / torch.sqrt((xd ** 2).mean(-1, keepdim=True) + 1e-6)
    want = n * w.double()
    # two bf16 roundings (normalised value, then the weight product)
    assert bool(((got.double() - want).abs() <= 2 ** -7 * want.abs() + 1e-30).all())
    # a constant row normalises to +-1 before the weight
    c = torch.full((1, hidden), -2.5).bfloat16()
    assert torch.equal(oracle.rms_layernorm(c, torch.ones(hidden).bfloat16(), 0.0),
                       torch.full((1, hidden), -1.0).bfloat16())


def test_silu_mul_and_residual_closed_form():
    g = torch.Generator().manual_seed(3)
    a = (torch.randn(1000, generator=g) * 4).bfloat16()
    u = torch.randn(1000, generator=g).bfloat16()
    got = oracle.silu_mul(a, u).double()
    ad = a.double()
    want = ad / (1 + torch.exp(-ad)) * u.double()
    assert bool(((got - want).abs() <= 2 ** -7 * want.abs() + 1e-30).all())
    r = torch.randn(1000, generator=g).bfloat16()
    got = oracle.scaled_residual(r, u, 1.4, 32).double()
    want = r.double() + u.double() * 1.4 / math.sqrt(32)
    assert bool(((got - want).abs() <= 2 ** -7 * (want.abs() + (u.double() * 0.25).abs()) + 1e-30).all())


def test_embed_scale():
    table = torch.randn(50, 16).bfloat16()
    ids = torch.tensor([3, 0, 49, 3], dtype=torch.int32)
    got = oracle.embed_scale(ids, table, 12.0)
    assert torch.equal(got, (table[ids.long()].float() * 12.0).bfloat16())


def test_model_entry_points_validate_before_any_launch():
    lib = _hip.lib()
    B = _hip.LS_BF16
    assert lib.ls_rmsnorm(None, 4096, None, 4, 4100, 1e-6, B, None, 4100, None) == _hip.LS_ERR_UNSUPPORTED
    assert lib.ls_rmsnorm(None, 4096, None, 4, 4096, 1e-6, _hip.LS_F32, None, 4096, None) == _hip.LS_ERR_UNSUPPORTED
    assert lib.ls_rmsnorm(None, 100, None, 4, 4096, 1e-6, B, None, 4096, None) == _hip.LS_ERR_INVALID
    assert lib.ls_add_rmsnorm(None, 4096, None, 8, 1.0, None, 4, 4096, 1e-6, B, None, 4096,
                              None) == _hip.LS_ERR_INVALID
    rc = lib.ls_rope_inplace(None, 4608, None, 4, 32, 2, 4096, 64, None, None, 10, B, None)
    assert rc == _hip.LS_ERR_UNSUPPORTED and b"head_dim" in lib.ls_last_error()
    rc = lib.ls_rope_inplace(None, 4344, None, 4, 32, 2, 4096, 128, None, None, 10, B, None)
    assert rc == _hip.LS_ERR_INVALID  # key heads run past the row
    rc = lib.ls_rope_inplace(None, 4608, None, 4, 32, 2, 2048, 128, None, None, 10, B, None)
    assert rc == _hip.LS_ERR_INVALID  # key heads overlap the query heads
    assert lib.ls_silu_mul(None, 100, 4, 100, B, None, 100, None) == _hip.LS_ERR_UNSUPPORTED
    assert lib.ls_silu_mul(None, 100, 4, 64, B, None, 64, None) == _hip.LS_ERR_INVALID
    assert lib.ls_embed_scale(None, 4, None, 10, 12, 1.0, B, None, None) == _hip.LS_ERR_UNSUPPORTED
    # empty inputs are no-ops
    assert lib.ls_rmsnorm(None, 4096, None, 0, 4096, 1e-6, B, None, 4096, None) == _hip.LS_OK
    assert lib.ls_silu_mul(None, 128, 0, 64, B, None, 64, None) == _hip.LS_OK


def test_model_wrappers_refuse_cpu_tensors():
    from leanselect_amd import minicpm

    x = torch.zeros(4, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU"):
        minicpm.rms_layernorm(x, torch.ones(64, dtype=torch.bfloat16), 1e-6)
    with pytest.raises(RuntimeError, match="GPU"):
        minicpm.silu_mul(torch.zeros(4, 128, dtype=torch.bfloat16), 64)
    with pytest.raises(RuntimeError, match="GPU"):
        minicpm.MiniCPMLeanSelect(minicpm.MiniCPMConfig(num_hidden_layers=1), device="cpu")


def test_model_wrappers_check_outputs_and_views_before_any_launch(monkeypatch):
    """Shape checks run before the GPU is touched (the device check is bypassed here
    so the host-side validation is what raises)."""
    from leanselect_amd import _hip as hip
    from leanselect_amd import minicpm

    monkeypatch.setattr(hip, "require_gpu", lambda *t: t[0].device)
    monkeypatch.setattr(hip, "lib", lambda: (_ for _ in ()).throw(AssertionError("launched")))
    x = torch.zeros(4, 64, dtype=torch.bfloat16)
    w = torch.ones(64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="out must be"):
        minicpm.rms_layernorm(x, w, 1e-6, out=torch.zeros(3, 64, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="out must be"):
        minicpm.add_rms_layernorm(x, x.clone(), 1.0, w, 1e-6, out=torch.zeros(4, 64))
    with pytest.raises(ValueError, match="out must be"):
        minicpm.silu_mul(torch.zeros(4, 128, dtype=torch.bfloat16), 64,
                         out=torch.zeros(4, 32, dtype=torch.bfloat16))
    qkv = torch.zeros(4, 4608, dtype=torch.bfloat16)
    cos = torch.zeros(10, 128)
    with pytest.raises(ValueError, match="inside"):
        minicpm.rope_inplace(qkv[:, :4096], torch.zeros(4, dtype=torch.int32), cos, cos,
                             n_q_heads=32, n_k_heads=2, k_col_offset=4096)


def test_longrope_tables_closed_form():
    """LongRoPE tables (MiniCPMLongRoPE, minicpm.py:895-939) against float64:
    angle t / f_i * base^(-2i/D), both tables times the scale; t = 0 gives
    (scale, 0); unit factors and unit scale give the plain tables bit for bit."""
    from leanselect_amd.minicpm import MINICPM41_128K_LONGROPE_FACTOR as FAC
    D, P, base = 128, 3000, 10000.0
    sc = oracle.longrope_scale(131072, 65536)
    cos, sin = oracle.rotary_tables(D, P, base, ext_factors=FAC, scale=sc)
    i = torch.arange(D // 2, dtype=torch.float64)
    f = torch.tensor(FAC, dtype=torch.float64)
    theta = torch.arange(P, dtype=torch.float64)[:, None] / f[None, :] * base ** (-2 * i / D)[None, :]
    tol = 8 * torch.finfo(torch.float32).eps * (1 + theta) * sc
    for half in (slice(0, D // 2), slice(D // 2, D)):
        assert bool(((cos[:, half].double() - sc * theta.cos()).abs() <= tol).all())
        assert bool(((sin[:, half].double() - sc * theta.sin()).abs() <= tol).all())
    assert torch.allclose(cos[0].double(), torch.full((D,), sc, dtype=torch.float64), rtol=0, atol=1e-7)
    assert torch.equal(sin[0], torch.zeros(D))
    c1, s1 = oracle.rotary_tables(D, 500, base, ext_factors=[1.0] * (D // 2), scale=1.0)
    c0, s0 = oracle.rotary_tables(D, 500, base)
    assert torch.equal(c1, c0) and torch.equal(s1, s0)
    # A planted mistake (factor multiplied instead of divided) must fail the bound.
    bad = torch.cat([(torch.arange(P, dtype=torch.float64)[:, None] * f[None, :]
                      * base ** (-2 * i / D)[None, :]).cos() * sc] * 2, dim=-1)
    assert not bool(((bad - sc * torch.cat([theta.cos()] * 2, dim=-1)).abs() <= torch.cat([tol] * 2, dim=-1)).all())


def test_longrope_scale_and_factor_table():
    """sqrt(1 + log(s) / log(L)) at s = 1, 2 and 4 (L = 65536 = 2^16: 1, sqrt(17/16),
    sqrt(18/16)); the factor table holds 64 increasing values from 0.998 to 126.02
    (its sum pins every entry to the published table's)."""
    from leanselect_amd import minicpm
    assert minicpm.longrope_scale(65536, 65536) == 1.0
    assert math.isclose(minicpm.longrope_scale(131072, 65536), math.sqrt(17 / 16), rel_tol=1e-15)
    assert math.isclose(oracle.longrope_scale(262144, 65536), math.sqrt(18 / 16), rel_tol=1e-15)
    fac = minicpm.MINICPM41_128K_LONGROPE_FACTOR
    assert len(fac) == 64 and all(b > a for a, b in zip(fac, fac[1:]))
    assert math.isclose(fac[0], 0.9982316082870437) and math.isclose(fac[-1], 126.01712561287873)
    assert math.isclose(sum(fac), 3606.5291185034357, rel_tol=1e-15)


def test_model_longrope_tables_equal_the_oracle_on_cpu():
    """The model's table builder (torch on any device) run on the CPU equals the
    oracle's restatement bit for bit, LongRoPE and plain."""
    from leanselect_amd import minicpm
    fac = minicpm.MINICPM41_128K_LONGROPE_FACTOR
    sc = minicpm.longrope_scale(65536, 65536)
    c, s = minicpm.rotary_tables(128, 2000, 10000.0, "cpu", ext_factors=fac, scale=sc)
    co, so = oracle.rotary_tables(128, 2000, 10000.0, ext_factors=fac, scale=sc)
    assert torch.equal(c, co) and torch.equal(s, so)
    c, s = minicpm.rotary_tables(128, 2000, 10000.0, "cpu")
    co, so = oracle.rotary_tables(128, 2000, 10000.0)
    assert torch.equal(c, co) and torch.equal(s, so)
