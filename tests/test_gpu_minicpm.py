"""GPU parity of the MiniCPM decoder kernels (RMSNorm, residual + RMSNorm, RoPE,
SiLU-gated activation, embedding) against the oracle, and of one decoder layer
of the small MiniCPM-shaped model through its stages; properties of the
end-to-end prefill (determinism, packed = independent sequences)."""
import pytest
import torch

import oracle
from leanselect_amd import minicpm

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _ulps(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Distance in 16-bit steps (monotone integer image of the float order)."""
    def key(t):
        i = t.contiguous().view(torch.int16).to(torch.int32)
        return torch.where(i < 0, -(i & 0x7fff), i)
    return (key(a) - key(b)).abs()


def _close16(got: torch.Tensor, want: torch.Tensor, frac: float = 1e-3, steps: int = 1):
    """At most ``steps`` 16-bit steps apart everywhere, and equal except on a
    ``frac`` share (float32 reduction order and device exp/sqrt may move a value
    across a rounding boundary; a second rounding, as RMSNorm's weight product,
    can stretch one step of the first to two)."""
    u = _ulps(got.cpu(), want.cpu())
    assert int(u.max()) <= steps, f"max distance {int(u.max())} steps"
    assert float((u > 0).float().mean()) <= frac, f"{float((u > 0).float().mean()):.2e} differ"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("hidden", [4096, 1032])
def test_rmsnorm_matches_oracle(dtype, hidden):
    g = torch.Generator().manual_seed(hidden)
    n = 333
    x = (torch.randn(n, hidden + 16, generator=g) * 2).to(dtype)
    w = (1 + 0.1 * torch.randn(hidden, generator=g)).to(dtype)
    xv = x[:, :hidden]  # strided rows
    got = minicpm.rms_layernorm(xv.to(DEV), w.to(DEV), 1e-6)
    torch.cuda.synchronize()
    _close16(got, oracle.rms_layernorm(xv, w, 1e-6), steps=2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_add_rmsnorm_matches_oracle(dtype):
    g = torch.Generator().manual_seed(5)
    n, hidden = 257, 4096
    res = torch.randn(n, hidden, generator=g).to(dtype)
    h = (torch.randn(n, hidden, generator=g) * 3).to(dtype)
    w = (1 + 0.1 * torch.randn(hidden, generator=g)).to(dtype)
    res_d = res.to(DEV)
    out = minicpm.add_rms_layernorm(res_d, h.to(DEV), 1.4 / 32 ** 0.5, w.to(DEV), 1e-6)
    torch.cuda.synchronize()
    want_res = oracle.scaled_residual(res, h, 1.4, 32)
    assert torch.equal(res_d.cpu(), want_res)  # elementwise float32 ops: exact
    _close16(out, oracle.rms_layernorm(want_res, w, 1e-6), steps=2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_rope_inplace_matches_oracle_exactly(dtype):
    g = torch.Generator().manual_seed(7)
    H, G, D = 32, 2, 128
    n = 300
    width = H * D + 2 * G * D
    qkv = torch.randn(n, width, generator=g).to(dtype)
    pos = torch.randint(0, 5000, (n,), generator=g, dtype=torch.int32)
    cos, sin = oracle.rotary_tables(D, 5000)
    dev = qkv.to(DEV)
    minicpm.rope_inplace(dev, pos.to(DEV), cos.to(DEV), sin.to(DEV), n_q_heads=H, n_k_heads=G,
                         k_col_offset=H * D)
    torch.cuda.synchronize()
    got = dev.cpu()
    q_want = oracle.apply_rotary_pos_emb(qkv[:, :H * D].view(n, H, D), cos, sin, pos.long())
    k_want = oracle.apply_rotary_pos_emb(qkv[:, H * D:H * D + G * D].view(n, G, D), cos, sin, pos.long())
    assert torch.equal(got[:, :H * D].view(n, H, D), q_want)
    assert torch.equal(got[:, H * D:H * D + G * D].view(n, G, D), k_want)
    assert torch.equal(got[:, H * D + G * D:], qkv[:, H * D + G * D:])  # v untouched


def test_rope_tables_on_device_match_the_oracle():
    """The device builds its table from its own ``base ** x``; one float32 step of
    ``inv_freq`` moves angle t * inv_freq by up to t * inv_freq * 2^-23, so the
    bound grows with the angle."""
    cos, sin = minicpm.rotary_tables(128, 4096, 10000.0, DEV)
    ccpu, scpu = oracle.rotary_tables(128, 4096)
    inv = 1.0 / 10000.0 ** (torch.arange(0, 128, 2, dtype=torch.float64) / 128)
    ang = torch.arange(4096, dtype=torch.float64)[:, None] * torch.cat((inv, inv))[None, :]
    tol = 4 * 2.0 ** -23 * (1 + ang)
    assert bool(((cos.cpu().double() - ccpu.double()).abs() <= tol).all())
    assert bool(((sin.cpu().double() - scpu.double()).abs() <= tol).all())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_silu_mul_matches_oracle(dtype):
    g = torch.Generator().manual_seed(9)
    n, inter = 129, 2048
    gu = (torch.randn(n, 2 * inter, generator=g) * 3).to(dtype)
    got = minicpm.silu_mul(gu.to(DEV), inter)
    torch.cuda.synchronize()
    _close16(got, oracle.silu_mul(gu[:, :inter], gu[:, inter:]))


def test_embed_matches_oracle_and_checks_ids():
    g = torch.Generator().manual_seed(11)
    table = torch.randn(1000, 256, generator=g).bfloat16()
    ids = torch.randint(0, 1000, (777,), generator=g, dtype=torch.int32)
    got = minicpm.embed_scale(ids.to(DEV), table.to(DEV), 12.0)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), oracle.embed_scale(ids, table, 12.0))
    with pytest.raises(IndexError):
        minicpm.embed_scale(torch.tensor([0, 1000], dtype=torch.int32, device=DEV), table.to(DEV), 1.0)


SMALL = minicpm.MiniCPMConfig(hidden_size=1024, num_hidden_layers=2, num_attention_heads=8,
                              num_key_value_heads=2, intermediate_size=2048, vocab_size=1000,
                              topk=16, local_blocks=2)


def test_decoder_layer_stages_match_oracle():
    """One layer, stage by stage on the GPU's own library-GEMM outputs: RoPE exact,
    page plans and attention against the oracle, residual + norm kernels."""
    model = minicpm.MiniCPMLeanSelect(SMALL, device=DEV, seed=3)
    cu_host = [0, 700, 1536]
    N = cu_host[-1]
    gen = torch.Generator(device=DEV).manual_seed(4)
    ids = torch.randint(0, SMALL.vocab_size, (N,), generator=gen, device=DEV, dtype=torch.int32)
    cu = torch.tensor(cu_host, dtype=torch.int32, device=DEV)
    pos = model.positions(cu_host, DEV)
    x = minicpm.embed_scale(ids, model.embed, SMALL.scale_emb)
    h = minicpm.rms_layernorm(x, model.layers[0].input_norm, SMALL.rms_norm_eps)
    H, G, D = SMALL.num_attention_heads, SMALL.num_key_value_heads, SMALL.head_dim
    qkv_pre = torch.nn.functional.linear(h, model.layers[0].w_qkv).cpu()
    o, parts = model.attention(0, h, pos, cu, cu_host, return_parts=True)
    torch.cuda.synchronize()
    # RoPE on the projection output, exactly
    cos, sin = model.rope_tables(max(cu_host[1] - cu_host[0], cu_host[2] - cu_host[1]))
    qkv = parts["qkv"].cpu()
    want_q = oracle.apply_rotary_pos_emb(qkv_pre[:, :H * D].view(N, H, D), cos.cpu(), sin.cpu(), pos.long().cpu())
    assert torch.equal(qkv[:, :H * D].view(N, H, D), want_q)
    # selection and attention on the rotated q/k/v
    q = qkv[:, :H * D].view(N, H, D)
    k = qkv[:, H * D:H * D + G * D].view(N, G, D)
    v = qkv[:, H * D + G * D:].view(N, G, D)
    sel = model.layers[0].selector
    kc, cu_c = oracle.compress_k(k, cu_host)
    qf, kf = oracle.fused_weights(sel.head_mix.cpu(), sel.kv_head_mix.cpu(), sel.q_proj.cpu(),
                                  sel.k_proj.cpu(), q.dtype)
    rows = list(range(0, N, 7)) + [N - 1]
    want_ids, scores = oracle.select_prefill(
        q, kc, cu_host, cu_c.tolist(), qf, kf, topk=SMALL.topk, init_blocks=SMALL.init_blocks,
        local_blocks=SMALL.local_blocks, rows=rows, return_scores=True)
    got_ids = parts["topk_idx"].cpu()
    rep = oracle.check_topk(got_ids[:, rows], want_ids, scores, q.dtype)
    assert rep.ok, rep
    want, _ = oracle.sparse_attention(q, k, v, cu_host, cu_host, got_ids[:, rows], rows=rows,
                                      ids_rows_aligned=True)
    ok, mx, mr = oracle.check_attention(parts["attn"].cpu()[rows], want)
    assert ok, (mx, mr)
    # residual + post-attention norm on the GPU's o
    x_before = x.cpu()
    h2 = minicpm.add_rms_layernorm(x, o, model.residual_scale, model.layers[0].post_norm,
                                   SMALL.rms_norm_eps)
    torch.cuda.synchronize()
    want_x = oracle.scaled_residual(x_before, o.cpu(), SMALL.scale_depth, SMALL.num_hidden_layers)
    assert torch.equal(x.cpu(), want_x)
    _close16(h2, oracle.rms_layernorm(want_x, model.layers[0].post_norm.cpu(), SMALL.rms_norm_eps),
             steps=2)


def test_prefill_is_deterministic_and_packed_equals_independent():
    model = minicpm.MiniCPMLeanSelect(SMALL, device=DEV, seed=5)
    gen = torch.Generator(device=DEV).manual_seed(6)
    a = torch.randint(0, SMALL.vocab_size, (900,), generator=gen, device=DEV, dtype=torch.int32)
    b = torch.randint(0, SMALL.vocab_size, (1300,), generator=gen, device=DEV, dtype=torch.int32)
    packed = torch.cat([a, b])
    l1 = model.prefill(packed, [0, 900, 2200])
    l2 = model.prefill(packed, [0, 900, 2200])
    torch.cuda.synchronize()
    assert l1.shape == (2, SMALL.vocab_size) and bool(torch.isfinite(l1).all())
    assert torch.equal(l1, l2)
    la, lb = model.prefill(a), model.prefill(b)
    for got, want in ((l1[0], la[0]), (l1[1], lb[0])):
        cs = torch.nn.functional.cosine_similarity(got.double(), want.double(), dim=0)
        assert float(cs) > 0.999, float(cs)


def test_prefill_rejects_bad_offsets():
    model = minicpm.MiniCPMLeanSelect(
        minicpm.MiniCPMConfig(hidden_size=1024, num_hidden_layers=1, num_attention_heads=8,
                              num_key_value_heads=2, intermediate_size=1024, vocab_size=100),
        device=DEV)
    ids = torch.zeros(100, dtype=torch.int32, device=DEV)
    with pytest.raises(ValueError):
        model.prefill(ids, [0, 50])


def test_prefill_ragged_with_short_sequences_and_wide_local_window():
    """Sequences shorter than one compression window (no compressed key: plans of
    only the forced pages) beside longer ones, under a budget with a wide local
    window as in the reference's published setting (a third of the budget local)."""
    cfg = minicpm.MiniCPMConfig(hidden_size=1024, num_hidden_layers=2, num_attention_heads=8,
                                num_key_value_heads=2, intermediate_size=2048, vocab_size=1000,
                                topk=24, local_blocks=8)
    model = minicpm.MiniCPMLeanSelect(cfg, device=DEV, seed=7)
    gen = torch.Generator(device=DEV).manual_seed(8)
    lens = [20, 1300, 64, 1]
    seqs = [torch.randint(0, cfg.vocab_size, (n,), generator=gen, device=DEV, dtype=torch.int32)
            for n in lens]
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    packed = model.prefill(torch.cat(seqs), cu)
    torch.cuda.synchronize()
    assert packed.shape == (len(lens), cfg.vocab_size) and bool(torch.isfinite(packed).all())
    for i, s in enumerate(seqs):
        alone = model.prefill(s)[0]
        cs = torch.nn.functional.cosine_similarity(packed[i].double(), alone.double(), dim=0)
        assert float(cs) > 0.999, (i, float(cs))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_rope_k_compress_equals_rope_then_compress(dtype):
    """The fused pass (keys rotated while their compressed keys are formed) gives
    bit for bit the rotated keys of ls_rope_inplace and the compressed keys of
    ls_compress_k_varlen on them, on a ragged batch with sequences shorter than
    a window and lengths off the 16-row grid."""
    from leanselect_amd.ops import compress_k
    lens = [100, 31, 32, 47, 0, 1000, 16, 7]
    cu_host = [0]
    for n in lens:
        cu_host.append(cu_host[-1] + n)
    N, H, G, D = cu_host[-1], 4, 2, 128
    g = torch.Generator(device="cpu").manual_seed(9)
    x = (torch.randn(N, H * D + 2 * G * D, generator=g) * 2).to(dtype).to(DEV)
    pos = torch.cat([torch.arange(n, dtype=torch.int32) for n in lens]).to(DEV)
    cos, sin = minicpm.rotary_tables(D, 1024, 10000.0, DEV)
    cu = torch.tensor(cu_host, dtype=torch.int32, device=DEV)
    ref = x.clone()
    minicpm.rope_inplace(ref, pos, cos, sin, n_q_heads=0, n_k_heads=G, k_col_offset=H * D)
    want_kc, want_cu = compress_k(ref[:, H * D : H * D + G * D].view(N, G, D), cu,
                                  cu_seqlens_host=cu_host)
    got = x.clone()
    kc, cu_c = minicpm.rope_k_compress(got, pos, cos, sin, cu, cu_host, n_k_heads=G,
                                       k_col_offset=H * D)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)  # keys rotated in place, every other column untouched
    assert torch.equal(cu_c, want_cu)
    assert torch.equal(kc, want_kc)


@pytest.mark.parametrize("dtype,router", [(torch.bfloat16, (4, 32)), (torch.float16, (4, 32)),
                                          (torch.bfloat16, (2, 32))])
def test_rope_project_queries_equals_rope_then_project(dtype, router):
    """The fused pass (queries rotated while the selector's projection is formed)
    gives bit for bit the rotated queries of ls_rope_inplace and the q~ of
    ls_project_queries on them (router widths 128 and 64), with a row count off
    the 64-row workgroup grid, the positions of a ragged batch, and every other
    column untouched."""
    from leanselect_amd.selector import LeanSelectSelector
    lens = [1000, 77, 1, 300]
    N, H, G, D = sum(lens), 32, 2, 128
    g = torch.Generator(device="cpu").manual_seed(11)
    x = (torch.randn(N, H * D + 2 * G * D, generator=g) * 2).to(dtype).to(DEV)
    pos = torch.cat([torch.arange(n, dtype=torch.int32) for n in lens]).to(DEV)
    cos, sin = minicpm.rotary_tables(D, 2048, 10000.0, DEV)
    torch.manual_seed(3)
    sel = LeanSelectSelector(num_heads=H, num_kv_heads=G, head_dim=D, router_heads=router[0],
                             router_dim=router[1]).to(DEV).requires_grad_(False)
    ref = x.clone()
    minicpm.rope_inplace(ref, pos, cos, sin, n_q_heads=H, n_k_heads=0, k_col_offset=H * D)
    want = sel.project_queries(ref[:, : H * D].view(N, H, D))
    got = x.clone()
    qt = minicpm.rope_project_queries(got, pos, cos, sin, sel, n_q_heads=H)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)  # queries rotated in place, key/value columns untouched
    assert qt.shape == want.shape and torch.equal(qt, want)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_select_from_q_tilde_equals_select_from_queries(dtype):
    """ls_select_prefill_qt with the selector's projection of the queries gives
    the same plans as ls_select_prefill on the queries (ragged batch)."""
    from leanselect_amd import workloads
    from leanselect_amd.ops import compress_k, leanselect_prefill_topk_idx
    case = workloads.hidden_space_layer((3000, 64, 1500), device=DEV, dtype=dtype, seed=4)
    kc, cu_c = compress_k(case.k, case.cu_seqlens, cu_seqlens_host=case.cu_host)
    kw = dict(topk=case.topk, init_blocks=case.init_blocks, local_blocks=case.local_blocks,
              cu_seqlens_q_host=case.cu_host)
    want = leanselect_prefill_topk_idx(case.q, kc, case.cu_seqlens, cu_c, case.selector, **kw)
    qt = case.selector.project_queries(case.q)
    got = leanselect_prefill_topk_idx(case.q, kc, case.cu_seqlens, cu_c, case.selector,
                                      q_tilde=qt, **kw)
    assert torch.equal(got, want)
