"""The NOSA variant of the prefill hot path on the GPU.

NOSA (leanselect/models/nosa.py) keeps the LeanSelect router for its qk page
scores and adds a per-token eviction score (CIS) that ranks pages and biases
attention:

* ``max_pooling_1d_varlen`` -- the InfLLM-v2 varlen page max-pool with the
  forced overlay (third_party/infllmv2/paper1.patch:2664-2760, called at
  nosa.py:1263-1286), on ``ls_page_maxpool_varlen``;
* ``nosa_prefill_topk_idx`` -- ``compressed_attention`` on the LeanSelect
  branch (nosa.py:1144-1307 with ``_leanselect_atom_scores``,
  nosa.py:1822-1853), fused into ``ls_nosa_select_prefill``;
* ``nosa_sparse_attention`` -- ``attn(q, k, v e^cis) / attn(q, k, e^cis)``
  (nosa.py:2211-2255) as one biased pass, ``ls_nosa_attn_varlen``.
"""
from __future__ import annotations

import torch

from .. import _hip
from .select import _masters

__all__ = ["max_pooling_1d_varlen", "nosa_prefill_topk_idx", "nosa_sparse_attention"]


def max_pooling_1d_varlen(
    input: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    cu_seqlens_k: torch.Tensor,
    cache_lens: torch.Tensor,
    max_seqlen_q: int,
    max_seqlen_k: int,
    local_blocks: int,
    init_blocks: int,
    block_size: int = 64,
    stride: int = 16,
    buf: torch.Tensor | None = None,
    max_cache_len: int | None = None,
    clip: str = "sequence",
) -> torch.Tensor:
    """``[num_heads, total_q, max_k] -> [num_heads, total_q, out_len]``,
    ``out_len = ceil((max_seqlen_q + max_cache_len) / block_size)``.

    Page ``p`` of row ``t`` (sequence ``b``, page ``off = (t - cu_q[b] +
    cache_lens[b]) // block_size``) is ``+inf`` when ``p < init_blocks`` or
    ``off - local_blocks <= p <= off``, else the max of ``input[h, t, j]`` over
    ``j in [p*s - 1, p*s + s)`` (``-inf`` when empty), ``s = block_size //
    stride``, within the sequence's ``len_k`` columns (``clip="sequence"``) or
    the row's ``max_seqlen_k`` columns (``clip="row"``).  The upstream kernel
    body that fixes this choice is not in the reference tree; the two differ
    only where a shorter sequence's padding columns hold values above -inf.
    """
    if input.ndim != 3:
        raise ValueError(f"Expected 3D input, got {input.ndim}D")
    clip_code = _hip.pool_clip_code(clip)
    for name, t in (("cu_seqlens_q", cu_seqlens_q), ("cu_seqlens_k", cu_seqlens_k),
                    ("cache_lens", cache_lens)):
        if t.dtype != torch.int32:
            raise ValueError(f"{name} must be int32")
    if input.shape[2] != max_seqlen_k:
        raise ValueError(f"max_k mismatch: {input.shape[2]} vs {max_seqlen_k}")
    batch = cu_seqlens_q.numel() - 1
    if cache_lens.shape[0] != batch:
        raise ValueError(f"cache_lens batch size mismatch: {cache_lens.shape[0]} vs {batch}")
    dev = _hip.require_gpu(input, cu_seqlens_q, cu_seqlens_k, cache_lens)
    if max_cache_len is None:
        max_cache_len = int(cache_lens.max().item()) if batch else 0
    out_len = (int(max_seqlen_q) + int(max_cache_len) + block_size - 1) // block_size
    H, total_q, _ = input.shape
    if buf is None:
        out = torch.empty((H, total_q, out_len), dtype=input.dtype, device=dev)
    else:
        if tuple(buf.shape) != (H, total_q, out_len) or buf.dtype != input.dtype \
                or buf.device != input.device or not buf.is_contiguous():
            raise ValueError(f"buf must be a contiguous {input.dtype} tensor of shape "
                             f"{(H, total_q, out_len)} on {input.device}")
        out = buf
    if out.numel() == 0 or batch == 0:
        return out
    input = input.contiguous()
    rc = _hip.lib().ls_page_maxpool_varlen(
        input.data_ptr(), cu_seqlens_q.contiguous().data_ptr(),
        cu_seqlens_k.contiguous().data_ptr(), cache_lens.contiguous().data_ptr(), batch, H,
        total_q, int(max_seqlen_k), out_len, int(local_blocks), int(init_blocks), block_size,
        stride, clip_code, _hip.dtype_code(input.dtype), out.data_ptr(), _hip.stream_of(dev))
    _hip.check(rc, "ls_page_maxpool_varlen")
    return out


def _cis_2d(cis: torch.Tensor, G: int) -> torch.Tensor:
    if cis.ndim == 3 and cis.shape[-1] == 1:
        cis = cis.squeeze(-1)
    if cis.ndim != 2 or cis.shape[1] != G:
        raise ValueError(f"cis must be [total_k, {G}] (or [total_k, {G}, 1])")
    return cis if cis.stride(1) == 1 else cis.contiguous()


def nosa_prefill_topk_idx(
    q_unpad: torch.Tensor,
    k_compressed: torch.Tensor,
    cis: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    cu_seqlens_kc: torch.Tensor,
    cu_seqlens_k: torch.Tensor,
    selector,
    *,
    topk: int = 96,
    init_blocks: int = 1,
    local_blocks: int = 16,
    select_blocks: int = 24,
    block_size: int = 64,
    kernel_stride: int = 16,
    max_seqlen_q: int | None = None,
    cu_seqlens_q_host: list[int] | None = None,
    pool_clip: str = "sequence",
) -> torch.Tensor:
    """NOSA page plans ``[G, total_q, min(topk, ceil(max_seqlen_q / block_size))]`` int32.

    ``q_unpad [total_q, H, D]`` post-RoPE queries, ``k_compressed [A, G, D]``
    compressed keys (prefix offsets ``cu_seqlens_kc``), ``cis [total_k, G]``
    eviction scores of the original keys (prefix offsets ``cu_seqlens_k``),
    ``selector`` a ``LeanSelectSelector``.  Rows list their pages ascending;
    pages after the row's ``q_idx`` (aligned to the longest sequence) are -1.
    ``pool_clip`` is the column range of both page max-pools (see
    ``max_pooling_1d_varlen``): under ``"row"`` a shorter sequence's pages past
    its own windows pool the CIS means' zero padding, up to the longest
    sequence's window count.
    """
    if q_unpad.ndim != 3 or k_compressed.ndim != 3:
        raise ValueError("q_unpad must be [total_q, H, D] and k_compressed [A, G, D]")
    clip_code = _hip.pool_clip_code(pool_clip)
    dev = _hip.require_gpu(q_unpad, k_compressed, cis, cu_seqlens_q, cu_seqlens_kc, cu_seqlens_k)
    for t in (cu_seqlens_q, cu_seqlens_kc, cu_seqlens_k):
        if t.dtype != torch.int32:
            raise ValueError("cu_seqlens must be int32")
    if q_unpad.dtype != k_compressed.dtype:
        raise ValueError("q_unpad and k_compressed must share a dtype")
    total_q, H, D = q_unpad.shape
    G = k_compressed.shape[1]
    if (H, G, D) != (selector.num_heads, selector.num_kv_heads, selector.head_dim):
        raise ValueError("query / compressed-key shapes do not match the selector")
    cis = _cis_2d(cis, G)
    if q_unpad.stride(2) != 1 or q_unpad.stride(1) != D:
        q_unpad = q_unpad.contiguous()
    if k_compressed.stride(2) != 1 or k_compressed.stride(1) != D:
        k_compressed = k_compressed.contiguous()
    host = cu_seqlens_q_host if cu_seqlens_q_host is not None else cu_seqlens_q.tolist()
    batch = len(host) - 1
    if max_seqlen_q is None:
        max_seqlen_q = max((host[b + 1] - host[b] for b in range(batch)), default=0)
    out_len = (int(max_seqlen_q) + block_size - 1) // block_size
    take = min(int(topk), out_len)
    if take == 0 or total_q == 0:
        return torch.full((G, total_q, take), -1, dtype=torch.int32, device=dev)
    topk_idx = torch.empty((G, total_q, take), dtype=torch.int32, device=dev)
    dt = _hip.dtype_code(q_unpad.dtype)
    hm, khm, qp, kp = _masters(selector)
    L = _hip.lib()
    total_atoms = k_compressed.shape[0]
    nbytes = L.ls_nosa_select_workspace_size(
        total_q, total_atoms, batch, H, G, D, selector.router_heads, selector.router_dim,
        out_len, dt)
    ws = _hip.workspace(nbytes, dev)
    rc = L.ls_nosa_select_prefill(
        q_unpad.data_ptr(), q_unpad.stride(0), total_q,
        k_compressed.data_ptr() if total_atoms else None, k_compressed.stride(0), total_atoms,
        cis.data_ptr(), cis.stride(0), _hip.dtype_code(cis.dtype),
        cu_seqlens_q.contiguous().data_ptr(), cu_seqlens_kc.contiguous().data_ptr(),
        cu_seqlens_k.contiguous().data_ptr(), batch, int(max_seqlen_q), H, G, D,
        hm.data_ptr(), khm.data_ptr(), qp.data_ptr(), kp.data_ptr(), selector.router_heads,
        selector.router_dim, dt, int(topk), block_size, kernel_stride, int(init_blocks),
        int(local_blocks), int(select_blocks), clip_code, topk_idx.data_ptr(), take, ws.data_ptr(),
        ws.numel(), _hip.stream_of(dev))
    _hip.check(rc, "ls_nosa_select_prefill")
    return topk_idx


def nosa_sparse_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cis: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    cu_seqlens_k: torch.Tensor,
    max_seqlen_q: int,
    max_seqlen_k: int,
    topk_idx: torch.Tensor,
    *,
    softmax_scale: float | None = None,
    block_size: int = 64,
    return_lse: bool = False,
    out: torch.Tensor | None = None,
    sync_status: bool = False,
):
    """NOSA prefill attention ``out [total_q, H, D]``: for each head, the causal
    keys ``j`` of the row's pages weighted by ``exp(scale * q.k_j + cis[j, g])``
    (``cis [total_k, G]``, finite).  With ``return_lse`` also ``[H, total_q]``
    float32, the log of the summed weights.  The status word of the call is
    checked as ``sparse_attention`` checks it (deferred unless ``sync_status``)."""
    if q.ndim != 3 or k.ndim != 3 or v.ndim != 3:
        raise ValueError("q, k, v must be [tokens, heads, head_dim]")
    if topk_idx is None or topk_idx.ndim != 3:
        raise ValueError("topk_idx must be [num_kv_heads, total_q, k] int32")
    # Host-side checks first: no launch may see int64 offsets or a misshapen output.
    _hip.check_cu_seqlens(cu_seqlens_q, cu_seqlens_k)
    if out is not None:
        _hip.check_out(out, tuple(q.shape), q.dtype, q.device)
    dev = _hip.require_gpu(q, k, v, cis, cu_seqlens_q, cu_seqlens_k, topk_idx)
    total_q, H, D = q.shape
    total_k, G, Dk = k.shape
    if v.shape != k.shape or Dk != D:
        raise ValueError("k and v must be [total_k, num_kv_heads, head_dim] like q's head_dim")
    if H % G:
        raise ValueError("num_heads must be divisible by num_kv_heads")
    if topk_idx.shape[0] != G or topk_idx.shape[1] != total_q:
        raise ValueError(f"topk_idx must be [{G}, {total_q}, k], got {tuple(topk_idx.shape)}")
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError("q, k and v must share a dtype")
    if q.dtype not in (torch.bfloat16, torch.float16):
        raise RuntimeError("sparse attention supports fp16 and bf16 only")
    cis = _cis_2d(cis, G)
    if cis.shape[0] != total_k:
        raise ValueError(f"cis must have {total_k} rows, got {cis.shape[0]}")
    if topk_idx.dtype != torch.int32:
        topk_idx = topk_idx.to(torch.int32)
    q = q if (q.stride(2) == 1 and q.stride(1) == D) else q.contiguous()
    k = k if (k.stride(2) == 1 and k.stride(1) == D) else k.contiguous()
    v = v if (v.stride(2) == 1 and v.stride(1) == D) else v.contiguous()
    topk_idx = topk_idx.contiguous()
    batch = cu_seqlens_q.numel() - 1
    if out is None:
        out = torch.empty((total_q, H, D), dtype=q.dtype, device=dev)
    lse = torch.empty((H, total_q), dtype=torch.float32, device=dev) if return_lse else None
    L = _hip.lib()
    dt = _hip.dtype_code(q.dtype)
    ws = _hip.workspace(L.ls_nosa_attn_workspace_size(total_k, batch, G, D, int(max_seqlen_k), dt), dev)
    scale = -1.0 if softmax_scale is None else float(softmax_scale)
    rc = L.ls_nosa_attn_varlen(
        q.data_ptr(), q.stride(0), k.data_ptr(), k.stride(0), v.data_ptr(), v.stride(0),
        cis.data_ptr(), cis.stride(0), _hip.dtype_code(cis.dtype),
        cu_seqlens_q.contiguous().data_ptr(), cu_seqlens_k.contiguous().data_ptr(), batch,
        total_q, total_k, int(max_seqlen_q), int(max_seqlen_k), H, G, D, dt,
        topk_idx.data_ptr(), topk_idx.shape[2], block_size, scale, out.data_ptr(),
        _hip.ptr(lse), ws.data_ptr(), ws.numel(), _hip.stream_of(dev))
    _hip.check(rc, "ls_nosa_attn_varlen")
    if total_q > 0 and batch > 0:  # an empty call launches nothing and leaves no status
        _hip.check_attn_status(ws, "ls_nosa_attn_varlen", sync=sync_status)
    return (out, lse) if return_lse else out
