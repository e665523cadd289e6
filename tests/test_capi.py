"""The C ABI library loads, exports what include/leanselect_hip.h declares and
rejects bad arguments before touching a GPU; host-side geometry (no GPU)."""
import ctypes
import re
from pathlib import Path

import pytest
import torch

from leanselect_amd import _hip, pages, selector as sel_mod
from leanselect_amd.ops import compress, select

HEADER = Path(__file__).resolve().parents[1] / "include" / "leanselect_hip.h"


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^[\w\s\*]*?\b(ls_\w+)\(", text, flags=re.M)))


def test_header_declares_the_boundary():
    names = declared_symbols()
    for must in ("ls_compress_k_varlen", "ls_select_prefill", "ls_sparse_attn_varlen",
                 "ls_fused_weights", "ls_project_queries", "ls_project_atom_keys",
                 "ls_score_pages", "ls_pool_atoms_to_pages", "ls_forced_page_mask"):
        assert must in names


def test_library_exports_every_declared_symbol():
    lib = _hip.lib()
    names = declared_symbols()
    assert set(names) == set(_hip.SIGNATURES), "ctypes table and header disagree"
    for name in names:
        assert hasattr(lib, name), name
    assert lib.ls_version() >= 100


def test_invalid_arguments_fail_before_any_launch():
    lib = _hip.lib()
    rc = lib.ls_compress_k_varlen(None, 0, None, -1, 2, 128, _hip.LS_BF16, 32, 16, None, 0,
                                  None, None)
    assert rc == _hip.LS_ERR_INVALID
    assert b"bad sizes" in lib.ls_last_error()
    rc = lib.ls_sparse_attn_varlen(None, 0, None, 0, None, 0, None, None, 1, 1, 1, 1, 1, 32, 2,
                                   64, _hip.LS_BF16, None, 1, 64, -1.0, 1, None, None, None, 0, None)
    assert rc == _hip.LS_ERR_UNSUPPORTED and b"head_dim" in lib.ls_last_error()
    rc = lib.ls_sparse_attn_varlen(None, 0, None, 0, None, 0, None, None, 1, 1, 1, 1, 1, 32, 2,
                                   128, _hip.LS_F32, None, 1, 64, -1.0, 1, None, None, None, 0, None)
    assert rc == _hip.LS_ERR_UNSUPPORTED
    rc = lib.ls_select_prefill(None, 0, 10, None, 0, 0, None, None, 1, 10, 32, 2, 128, None,
                               None, None, None, 4, 32, _hip.LS_BF16, 64, 64, 16, 1, 4, None,
                               5, None, 0, None)
    assert rc == _hip.LS_ERR_INVALID and b"take" in lib.ls_last_error()


def test_nosa_entry_points_validate_before_any_launch():
    lib = _hip.lib()
    B = _hip.LS_BF16
    # take must be min(topk, ceil(max_seqlen_q / 64)) = 2 for 100 tokens.
    rc = lib.ls_nosa_select_prefill(None, 0, 100, None, 0, 5, None, 0, B, None, None, None, 1,
                                    100, 32, 2, 128, None, None, None, None, 4, 32, B, 96, 64, 16,
                                    1, 16, 24, 0, None, 3, None, 0, None)
    assert rc == _hip.LS_ERR_INVALID and b"take" in lib.ls_last_error()
    rc = lib.ls_nosa_select_prefill(None, 0, 100, None, 0, 5, None, 0, B, None, None, None, 1,
                                    100, 32, 2, 128, None, None, None, None, 4, 32, B, 96, 32, 16,
                                    1, 16, 24, 0, None, 2, None, 0, None)
    assert rc == _hip.LS_ERR_UNSUPPORTED and b"block_size" in lib.ls_last_error()
    rc = lib.ls_nosa_select_prefill(None, 0, 100, None, 0, 5, None, 0, 7, None, None, None, 1,
                                    100, 32, 2, 128, None, None, None, None, 4, 32, B, 96, 64, 16,
                                    1, 16, 24, 0, None, 2, None, 0, None)
    assert rc == _hip.LS_ERR_INVALID and b"CIS dtype" in lib.ls_last_error()
    rc = lib.ls_nosa_select_prefill(None, 0, 100, None, 0, 5, None, 0, B, None, None, None, 1,
                                    100, 32, 2, 128, None, None, None, None, 4, 32, B, 96, 64, 16,
                                    1, 16, 24, 2, None, 2, None, 0, None)
    assert rc == _hip.LS_ERR_INVALID and b"pool_clip" in lib.ls_last_error()
    rc = lib.ls_nosa_attn_varlen(None, 0, None, 0, None, 0, None, 0, B, None, None, 1, 10, 10,
                                 10, 10, 32, 2, 128, B, None, 1, 64, -1.0, None, None, None, 0,
                                 None)
    assert rc == _hip.LS_ERR_INVALID and b"CIS" in lib.ls_last_error()
    rc = lib.ls_nosa_attn_varlen(None, 0, None, 0, None, 0, None, 0, B, None, None, 1, 10, 10,
                                 10, 10, 32, 2, 64, B, None, 1, 64, -1.0, None, None, None, 0,
                                 None)
    assert rc in (_hip.LS_ERR_INVALID, _hip.LS_ERR_UNSUPPORTED)
    rc = lib.ls_cis_mean_pool(None, 1, 10, 2, None, 1, 100, 16, 16, B, None, 5, None)
    assert rc == _hip.LS_ERR_UNSUPPORTED
    rc = lib.ls_cis_mean_pool(None, 1, 10, 2, None, 1, 100, 32, 16, B, None, 6, None)
    assert rc == _hip.LS_ERR_INVALID and b"columns" in lib.ls_last_error()
    rc = lib.ls_page_maxpool_varlen(None, None, None, None, 1, 2, 10, 10, 1, 2, 1, 64, 16, 0, 9,
                                    None, None)
    assert rc == _hip.LS_ERR_INVALID and b"dtype" in lib.ls_last_error()
    rc = lib.ls_page_maxpool_varlen(None, None, None, None, 1, 2, 10, 10, 1, 2, 1, 64, 48, 0, B,
                                    None, None)
    assert rc == _hip.LS_ERR_INVALID
    rc = lib.ls_page_maxpool_varlen(None, None, None, None, 1, 2, 10, 10, 1, 2, 1, 64, 16, 2, B,
                                    None, None)
    assert rc == _hip.LS_ERR_INVALID and b"clip" in lib.ls_last_error()
    assert (_hip.LS_POOL_CLIP_SEQUENCE, _hip.LS_POOL_CLIP_ROW) == (0, 1)
    with pytest.raises(ValueError, match="clip"):
        _hip.pool_clip_code("max_k")


def test_nosa_workspace_and_cpu_refusal():
    lib = _hip.lib()
    a = lib.ls_select_workspace_size(8192, 511, 1, 32, 2, 128, 4, 32, 128, _hip.LS_BF16)
    b = lib.ls_nosa_select_workspace_size(8192, 511, 1, 32, 2, 128, 4, 32, 128, _hip.LS_BF16)
    # + CIS page offsets and CIS page scores (2 groups x >= 511 / 4 + 1 floats).
    assert b >= a + 2 * (511 // 4 + 1) * 4
    assert (lib.ls_nosa_attn_workspace_size(131072, 1, 2, 128, 131072, _hip.LS_BF16)
            >= lib.ls_sparse_attn_workspace_size(131072, 1, 2, 128, 131072, _hip.LS_BF16)
            + 2 * 131072 * 4)
    from leanselect_amd.ops import max_pooling_1d_varlen, nosa_mean_pooling
    cu = torch.tensor([0, 64], dtype=torch.int32)
    with pytest.raises(RuntimeError, match="GPU"):
        nosa_mean_pooling(torch.randn(64, 2), cu, 64)
    with pytest.raises(RuntimeError, match="GPU"):
        max_pooling_1d_varlen(torch.randn(2, 64, 3), cu, torch.tensor([0, 3], dtype=torch.int32),
                              torch.zeros(1, dtype=torch.int32), 64, 3, 1, 1)


def test_workspace_sizes_are_host_only_and_grow():
    lib = _hip.lib()
    a = lib.ls_select_workspace_size(4096, 255, 1, 32, 2, 128, 4, 32, 64, _hip.LS_BF16)
    b = lib.ls_select_workspace_size(8192, 511, 1, 32, 2, 128, 4, 32, 128, _hip.LS_BF16)
    assert 0 < a < b
    # C3: 131072 tokens -> page-score scratch of 2 x 131072 x 2048 bf16 dominates.
    c3 = lib.ls_select_workspace_size(131072, 8191, 1, 32, 2, 128, 4, 32, 2048, _hip.LS_BF16)
    assert c3 >= 2 * 131072 * 2048 * 2
    assert lib.ls_sparse_attn_workspace_size(131072, 1, 2, 128, 131072, _hip.LS_BF16) >= 2 * 128 * 131072 * 2


def test_product_path_refuses_cpu_tensors():
    k = torch.randn(64, 2, 128)
    with pytest.raises(RuntimeError, match="GPU"):
        compress.compress_k(k, torch.tensor([0, 64], dtype=torch.int32))
    with pytest.raises(RuntimeError, match="GPU"):
        pages.pool_atoms_to_pages(torch.randn(4, 15), seq_len=256)
    s = sel_mod.LeanSelectSelector(num_heads=8, num_kv_heads=2, head_dim=128).requires_grad_(False)
    with pytest.raises(RuntimeError, match="GPU"):
        s.project_queries(torch.randn(4, 8, 128))


def test_selector_geometry_and_training_guard():
    for kwargs in ({"num_heads": 7}, {"router_heads": 9}, {"head_dim": 0}):
        cfg = dict(num_heads=8, num_kv_heads=2, head_dim=8)
        cfg.update(kwargs)
        with pytest.raises(ValueError):
            sel_mod.LeanSelectSelector(**cfg)
    s = sel_mod.LeanSelectSelector(num_heads=8, num_kv_heads=2, head_dim=8, router_heads=2, router_dim=4)
    assert all(getattr(p, "_is_indexer", False) for p in s.parameters())
    assert tuple(s.canonical_state()) == sel_mod.LEANSELECT_CANONICAL_TENSORS
    with pytest.raises(RuntimeError, match="forward-only"):
        s.project_queries(torch.randn(3, 8, 8))
    with pytest.raises(ValueError):
        with torch.no_grad():
            s.project_queries(torch.randn(2, 3, 8))


def test_supervision_windows_reference_property():
    # tests/test_core.py:183-188
    start = sel_mod.leanselect_informative_history_start(total_topk_blocks=96, block_size=64)
    windows = sel_mod.leanselect_supervision_windows(32768, 257, minimum_start=start)
    assert windows[0][0] == start and windows[-1][1] == 32768
    assert sum(e - b for b, e in windows) == 257
    assert all(l[1] <= r[0] for l, r in zip(windows, windows[1:]))
    assert len(windows) == 64


@pytest.mark.parametrize("n,rows,cap,lo", [(100, 10, 4, 0), (100, 100, 64, 0), (50, 7, 1, 3),
                                           (1000, 65, 64, 17), (9, 9, 3, 0)])
def test_supervision_windows_brute_force(n, rows, cap, lo):
    w = sel_mod.leanselect_supervision_windows(n, rows, max_windows=cap, minimum_start=lo)
    used = min(rows, n - lo)
    assert sum(e - b for b, e in w) == used
    assert w[-1][1] == n and (w[0][0] == lo or len(w) == 1)
    widths = [e - b for b, e in w]
    assert max(widths) - min(widths) <= 1 and widths == sorted(widths, reverse=True)
    gaps = [r[0] - l[1] for l, r in zip(w, w[1:])]
    assert all(g >= 0 for g in gaps) and gaps == sorted(gaps)
    assert len(w) == (1 if used == n - lo else min(cap, used))


def test_host_geometry():
    assert pages.group_size(32, 2) == 16
    with pytest.raises(ValueError):
        pages.group_size(30, 4)
    assert pages.infllm_atom_count(31) == 1 and pages.infllm_atom_count(32) == 1
    assert pages.infllm_atom_count(131072) == 8191
    assert pages.serve_dynamic_k(96, 10) == 10
    forced = torch.tensor([[True, False, True, False]])
    assert pages.serve_dynamic_k(3, 4, forced).tolist() == [1]
    assert select.select_take([0, 100, 4196], 64, 64) == 64
    assert select.select_take([0, 100, 300], 64, 64) == 4
    assert compress.compressed_lengths([0, 31, 63, 4159], 32, 16) == [0, 1, 255]


def test_variable_k_topk_mask_ties_to_lower_index():
    scores = torch.tensor([[1.0, 3.0, 3.0, float("-inf"), 2.0]])
    assert pages.variable_k_topk_mask(scores, 2).tolist() == [[False, True, True, False, False]]
    assert pages.variable_k_topk_mask(scores, 5).tolist() == [[True, True, True, False, True]]


def test_attention_spin_limit_hook_is_host_only():
    # Sets the bound for later launches and returns the previous one; no GPU call.
    lib = _hip.lib()
    default = lib.ls_attn_set_spin_limit(-1)
    assert default == 1 << 22
    assert lib.ls_attn_set_spin_limit(5) == default
    assert lib.ls_attn_set_spin_limit(-1) == 5
    assert lib.ls_attn_set_spin_limit(-1) == default


def test_fused_query_and_decode_entry_points_validate_before_any_launch():
    """The fused rotation + q~ projection, selection from a given q~ and the decode
    entry points reject unsupported geometry with an error code and message,
    without a GPU."""
    lib = _hip.lib()
    B = _hip.LS_BF16
    # ls_rope_project_queries: fp32 queries, head_dim 64, router width 96, bad stride.
    args = [None, 4096, None, 10, 32, 2, 128, None, None, 100, None, None, 4, 32]
    rc = lib.ls_rope_project_queries(*args, _hip.LS_F32, None, None, 0, None)
    assert rc == _hip.LS_ERR_UNSUPPORTED and b"bf16 or fp16" in lib.ls_last_error()
    rc = lib.ls_rope_project_queries(None, 4096, None, 10, 32, 2, 64, None, None, 100, None,
                                     None, 4, 32, B, None, None, 0, None)
    assert rc == _hip.LS_ERR_UNSUPPORTED and b"head_dim 128" in lib.ls_last_error()
    rc = lib.ls_rope_project_queries(None, 4096, None, 10, 32, 2, 128, None, None, 100, None,
                                     None, 3, 32, B, None, None, 0, None)
    assert rc == _hip.LS_ERR_UNSUPPORTED and b"router width" in lib.ls_last_error()
    rc = lib.ls_rope_project_queries(None, 4000, None, 10, 32, 2, 128, None, None, 100, None,
                                     None, 4, 32, B, None, None, 0, None)
    assert rc == _hip.LS_ERR_INVALID and b"stride" in lib.ls_last_error()
    rc = lib.ls_rope_project_queries(None, 4096, None, 10, 32, 2, 128, None, None, 100, None,
                                     None, 4, 32, B, None, None, 0, None)
    assert rc == _hip.LS_ERR_INVALID and b"null" in lib.ls_last_error()
    # ls_select_prefill_qt: take must be min(topk, pages) and q_tilde non-null.
    rc = lib.ls_select_prefill_qt(None, 10, None, 0, 0, None, None, 1, 10, 32, 2, 128, None,
                                  None, 4, 32, B, 64, 64, 16, 1, 4, None, 5, None, 0, None)
    assert rc == _hip.LS_ERR_INVALID and b"ls_select_prefill_qt" in lib.ls_last_error()
    rc = lib.ls_select_prefill_qt(None, 10, None, 0, 0, None, None, 1, 10, 32, 2, 128, None,
                                  None, 4, 32, B, 64, 64, 16, 1, 4, None, 1, None, 0, None)
    assert rc == _hip.LS_ERR_INVALID and b"null" in lib.ls_last_error()
    # ls_decode_select: out_len beyond the LDS key buffer, take above out_len.
    rc = lib.ls_decode_select(None, 4096, None, 1, None, 0, 256, None, 1, 10, 32, 2, 128, B,
                              0.088, 64, 64, 32, 16, 1, 4, 40000, 64, None, None, 0, None)
    assert rc == _hip.LS_ERR_UNSUPPORTED and b"pages per row" in lib.ls_last_error()
    rc = lib.ls_decode_select(None, 4096, None, 1, None, 0, 256, None, 1, 10, 32, 2, 128, B,
                              0.088, 64, 64, 32, 16, 1, 4, 10, 64, None, None, 0, None)
    assert rc == _hip.LS_ERR_INVALID and b"take" in lib.ls_last_error()
    # ls_sparse_attn_kvcache: more than 256 plan ids per row, too many splits.
    rc = lib.ls_sparse_attn_kvcache(None, 4096, None, 1, None, None, 0, 256, None, 1, 32, 2,
                                    128, B, None, 300, 0.088, 0, 4, None, None, None, 0, None)
    assert rc == _hip.LS_ERR_UNSUPPORTED and b"plan ids" in lib.ls_last_error()
    rc = lib.ls_sparse_attn_kvcache(None, 4096, None, 1, None, None, 0, 256, None, 1, 32, 2,
                                    128, B, None, 64, 0.088, 0, 65, None, None, None, 0, None)
    assert rc == _hip.LS_ERR_INVALID and b"n_splits" in lib.ls_last_error()
