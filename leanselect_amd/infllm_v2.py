"""Drop-in for the native-op names the reference's model files import.

``leanselect/models/minicpm.py:78-98`` and ``nosa.py:1021-1039`` import these
names from ``infllm_v2``; ``load_model`` checks that they exist
(``leanselect/models/__init__.py:65-87``).  The LeanSelect prefill path uses
``infllmv2_attn_varlen_func(..., topk_idx=)``, and NOSA's selection
``max_pooling_1d_varlen``.  The native stage-1 selector, decode attention and
``max_pooling_1d`` belong to the non-LeanSelect paths and raise
``NotImplementedError``.
"""
from __future__ import annotations

from .ops.attention import infllmv2_attn_varlen_func
from .ops.nosa import max_pooling_1d_varlen

__all__ = [
    "infllmv2_attn_varlen_func",
    "infllmv2_attn_stage1",
    "infllmv2_attn_stage1_kl_teacher",
    "infllmv2_attn_with_kvcache",
    "max_pooling_1d",
    "max_pooling_1d_varlen",
]


def _not_provided(name: str):
    def fn(*args, **kwargs):
        raise NotImplementedError(f"{name} is outside the LeanSelect prefill hot path")

    fn.__name__ = name
    return fn


infllmv2_attn_stage1 = _not_provided("infllmv2_attn_stage1")
infllmv2_attn_stage1_kl_teacher = _not_provided("infllmv2_attn_stage1_kl_teacher")
infllmv2_attn_with_kvcache = _not_provided("infllmv2_attn_with_kvcache")
max_pooling_1d = _not_provided("max_pooling_1d")
