"""GPU operators of the LeanSelect prefill hot path (mirror of ``leanselect.ops``)."""
from .attention import infllmv2_attn_varlen_func, sparse_attention
from .compress import CompressK, compress_k
from .select import leanselect_prefill_topk_idx, select_take
from .cis_pooling import nosa_mean_pooling
from .nosa import max_pooling_1d_varlen, nosa_prefill_topk_idx, nosa_sparse_attention
from .decode import decode_topk_idx, kvcache_append, sparse_attention_kvcache
from . import profiling

__all__ = [
    "CompressK",
    "compress_k",
    "leanselect_prefill_topk_idx",
    "select_take",
    "infllmv2_attn_varlen_func",
    "sparse_attention",
    "nosa_mean_pooling",
    "max_pooling_1d_varlen",
    "nosa_prefill_topk_idx",
    "nosa_sparse_attention",
    "kvcache_append",
    "decode_topk_idx",
    "sparse_attention_kvcache",
    "profiling",
]
