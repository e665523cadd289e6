"""Host-side argument checks of the Python mirror that must fire before any
GPU call (CPU only): int32 prefix offsets of equal length, caller-given
outputs of the exact shape, and packed sequences that all hold a token."""
import types

import pytest
import torch

from leanselect_amd import minicpm
from leanselect_amd.ops import nosa_sparse_attention, sparse_attention


def _attn_args(total=96, H=4, G=2, D=128, take=2):
    q = torch.zeros(total, H, D, dtype=torch.bfloat16)
    k = torch.zeros(total, G, D, dtype=torch.bfloat16)
    v = torch.zeros_like(k)
    ids = torch.zeros(G, total, take, dtype=torch.int32)
    cu = torch.tensor([0, total], dtype=torch.int32)
    return q, k, v, cu, ids


@pytest.mark.parametrize("fn", ["plain", "nosa"])
def test_int64_offsets_rejected(fn):
    q, k, v, cu, ids = _attn_args()
    cu64 = cu.to(torch.int64)  # the dtype torch.cumsum returns
    with pytest.raises(ValueError, match="int32"):
        if fn == "plain":
            sparse_attention(q, k, v, cu64, cu64, 96, 96, ids)
        else:
            nosa_sparse_attention(q, k, v, torch.zeros(96, 2), cu64, cu64, 96, 96, ids)


@pytest.mark.parametrize("fn", ["plain", "nosa"])
def test_offsets_of_different_lengths_rejected(fn):
    q, k, v, cu, ids = _attn_args()
    cu_k = torch.tensor([0, 40, 96], dtype=torch.int32)
    with pytest.raises(ValueError, match="differ in length"):
        if fn == "plain":
            sparse_attention(q, k, v, cu, cu_k, 96, 56, ids)
        else:
            nosa_sparse_attention(q, k, v, torch.zeros(96, 2), cu, cu_k, 96, 56, ids)


@pytest.mark.parametrize("bad", ["shape", "dtype", "strided"])
def test_caller_output_must_match(bad):
    q, k, v, cu, ids = _attn_args()
    if bad == "shape":
        out = torch.empty(95, 4, 128, dtype=torch.bfloat16)
    elif bad == "dtype":
        out = torch.empty(96, 4, 128, dtype=torch.float16)
    else:
        out = torch.empty(96, 4, 256, dtype=torch.bfloat16)[..., ::2]
    with pytest.raises(ValueError, match="out must be"):
        sparse_attention(q, k, v, cu, cu, 96, 96, ids, out=out)
    with pytest.raises(ValueError, match="out must be"):
        nosa_sparse_attention(q, k, v, torch.zeros(96, 2), cu, cu, 96, 96, ids, out=out)


def test_valid_host_arguments_reach_the_device_check():
    # Well-formed CPU arguments pass every host check and then stop at the
    # device check (the product path never runs on the CPU).
    q, k, v, cu, ids = _attn_args()
    with pytest.raises(RuntimeError, match="GPU"):
        sparse_attention(q, k, v, cu, cu, 96, 96, ids, out=torch.empty_like(q))


@pytest.mark.parametrize("cu_host", [[0, 0, 10], [0, 5, 5, 10], [0, 10, 10]])
def test_prefill_rejects_empty_sequences(cu_host):
    # The logits of each sequence are read at its last token; an empty sequence
    # has none, so it is rejected before any device work.
    fake = types.SimpleNamespace(cfg=minicpm.MiniCPMConfig(num_hidden_layers=1))
    ids = torch.zeros(10, dtype=torch.int32)
    with pytest.raises(ValueError, match="at least one token"):
        minicpm.MiniCPMLeanSelect.prefill(fake, ids, cu_host)
