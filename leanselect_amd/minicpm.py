"""MiniCPM4.1-shaped prefill with LeanSelect attention at every layer (GPU only).

Follows ``MiniCPMForCausalLM``'s prefill with ``--method leanselect`` and
``dense_len = -1`` (every layer sparse): the decoder layer
(leanselect/models/minicpm.py:3562-3630), its attention
(``MiniCPMInfLLMv2Attention.forward``, 2146-2377, LeanSelect branch of
``_sparse_attention_forward``, 2389-2772), the model loop (3708-3837) and the
last-token LM head (3987-4090).  Projections are plain library GEMMs
(``torch.nn.functional.linear`` on hipBLASLt); RMSNorm, the scaled residual add,
rotary embedding, the SiLU-gated activation and the scaled embedding are HIP
kernels of ``libleanselect_hip.so``; attention is
:func:`leanselect_amd.prefill.leanselect_sparse_prefill`.

Layout choices: the q/k/v projections are one GEMM into a packed ``[N, H*D +
2*G*D]`` buffer; the rotary embedding runs in place on it, and the attention
layer reads q, k and v as strided views of that buffer (no copies).  The
residual stream is updated in place by the fused add + RMSNorm kernel, whose
normalised output feeds the next GEMM.

Decoding (``decode_step``) follows the reference's decode branch: each layer
appends its rotated keys and values to a :class:`LeanSelectKVCache` (with the
compressed keys they complete), selects pages with the stage-1 selector on the
compressed-key cache (LeanSelect hands decode selection to it,
minicpm.py:359-367, 2509-2512, 2718-2736) and attends the cache through those
pages (minicpm.py:3216-3244 with ``causal=False``).

Weights are random-initialised (no checkpoint is loaded here).  Nothing in this
module falls back to a non-HIP path: it raises when the library is missing or
the tensors are not on a GPU.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from . import _hip
from .cache import LeanSelectKVCache
from .ops.decode import decode_topk_idx, sparse_attention_kvcache
from .prefill import leanselect_sparse_prefill
from .selector import LeanSelectSelector

__all__ = [
    "MiniCPMConfig",
    "MiniCPMLeanSelect",
    "rotary_tables",
    "longrope_scale",
    "MINICPM41_128K_LONGROPE_FACTOR",
    "rms_layernorm",
    "add_rms_layernorm",
    "rope_inplace",
    "rope_k_compress",
    "rope_project_queries",
    "silu_mul",
    "embed_scale",
]


@dataclass
class MiniCPMConfig:
    """Architecture and LeanSelect geometry.

    Defaults are the MiniCPM4.1-8B shape (hidden 4096, 32 layers, 32 query / 2
    KV heads of 128, FFN 16384, vocabulary 73448) with its published
    ``scale_emb`` 12, ``scale_depth`` 1.4 and ``dim_model_base`` 256 (the
    reference's ``MiniCPMConfig`` defaults are 1, 1, 1:
    leanselect/models/configuration_minicpm.py:130-132), RoPE base 10000 with
    the LongRoPE scaling the reference installs for MiniCPM4.1 at 128K
    (``apply_minicpm41_128k_longrope``, leanselect/models/minicpm.py:1011-1023:
    the published per-frequency factors, original context 65536), and the
    LeanSelect geometry of configs/minicpm.json with a 64-page budget (1 sink
    page, 4 local blocks).  ``rope_scaling=None`` gives plain RoPE.
    """

    hidden_size: int = 4096
    num_hidden_layers: int = 32
    num_attention_heads: int = 32
    num_key_value_heads: int = 2
    intermediate_size: int = 16384
    vocab_size: int = 73448
    rms_norm_eps: float = 1e-6
    rope_theta: float = 10000.0
    rope_scaling: str | None = "longrope"
    max_position_embeddings: int = 65536
    original_max_position_embeddings: int = 65536
    scale_emb: float = 12.0
    scale_depth: float = 1.4
    dim_model_base: int = 256
    topk: int = 64             # total page budget, forced pages included
    init_blocks: int = 1
    local_blocks: int = 4
    block_size: int = 64
    kernel_size: int = 32
    kernel_stride: int = 16
    router_heads: int = 4
    router_dim: int = 32

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_attention_heads


# ---------------------------------------------------------------------------
# Kernel wrappers (HIP; 16-bit tensors on one GPU)
# ---------------------------------------------------------------------------
def _rows(t: torch.Tensor, name: str) -> torch.Tensor:
    if t.ndim != 2 or t.stride(1) != 1:
        raise ValueError(f"{name} must be a 2-D tensor with unit column stride")
    return t


def _out(out: torch.Tensor, shape: tuple, like: torch.Tensor) -> torch.Tensor:
    """A caller-given output must have exactly the output's shape, dtype and device."""
    _rows(out, "out")
    if tuple(out.shape) != tuple(shape) or out.dtype != like.dtype or out.device != like.device:
        raise ValueError(f"out must be {tuple(shape)} {like.dtype} on {like.device}, "
                         f"got {tuple(out.shape)} {out.dtype} on {out.device}")
    return out


# MiniCPM4.1-8B's LongRoPE factors for 128K contexts, one per rotary frequency
# (the same values serve as short and long factors): the model's published
# rope_scaling table, as leanselect/models/minicpm.py:942-1008 installs it.
MINICPM41_128K_LONGROPE_FACTOR = (
    0.9982316082870437, 1.033048153422584, 1.0749920956484724, 1.1255096879436193,
    1.1863348602111476, 1.259543828902579, 1.3476188888731149, 1.4535223827776373,
    1.5807816745852985, 1.7335856049489526, 1.9168922912975785, 2.1365471404135326,
    2.3994084200118646, 2.713475511863602, 3.0880118452194134, 3.533650295140154,
    4.062463396503134, 4.687974098908333, 5.425075306704039, 6.289818967956352,
    7.29902962722721, 8.6357018163639, 10.210822723989212, 12.053807765671676,
    14.193944598909404, 16.65780676784363, 19.463620727694074, 22.628311203524586,
    26.150106147261315, 30.02526691405111, 34.23183327975347, 38.73811934094828,
    43.502489489729555, 48.47627117965394, 53.61139491762471, 58.857366522037935,
    64.16798299215064, 69.51359464319125, 74.86555458220285, 80.21497790341579,
    85.55322183307433, 90.89611806932027, 96.26245306514224, 101.68269304046481,
    107.18619510219668, 112.82253283014026, 118.63764063163615, 119.88866203644656,
    120.9462882391725, 121.837565139014, 122.58663780572562, 123.2147719894291,
    123.74049454862576, 124.17980424685767, 124.54641761955492, 124.85202548028222,
    125.10654406389756, 125.31835105170659, 125.49450117164764, 125.64091910903052,
    125.76256945356558, 125.86360463815589, 125.94749252260765, 126.01712561287873,
)


def longrope_scale(max_position_embeddings: int, original_max_position_embeddings: int) -> float:
    """``MiniCPMLongRoPE``'s cos/sin scale (minicpm.py:908-914):
    sqrt(1 + log(max / original) / log(original))."""
    s = max_position_embeddings / original_max_position_embeddings
    return math.sqrt(1 + math.log(s) / math.log(original_max_position_embeddings))


def rotary_tables(head_dim: int, max_pos: int, base: float, device, *,
                  ext_factors=None, scale: float = 1.0) -> tuple[torch.Tensor, torch.Tensor]:
    """float32 ``(cos, sin)`` ``[max_pos, head_dim]`` built like
    ``MiniCPMRotaryEmbedding._set_cos_sin_cache`` (minicpm.py:804-838), or, with
    ``ext_factors`` (one per frequency), like ``MiniCPMLongRoPE._set_cos_sin_cache``
    (minicpm.py:917-939): ``freqs = outer(t, 1 / ext_factors) * inv_freq`` and both
    tables multiplied by ``scale``."""
    inv_freq = 1.0 / base ** (torch.arange(0, head_dim, 2, device=device).float() / head_dim)
    t = torch.arange(max_pos, device=device, dtype=inv_freq.dtype)
    if ext_factors is None:
        freqs = torch.outer(t, inv_freq)
    else:
        ext = torch.tensor(ext_factors, dtype=torch.float32, device=device)
        if ext.shape != inv_freq.shape:
            raise ValueError(f"need {inv_freq.numel()} LongRoPE factors, got {ext.numel()}")
        freqs = torch.mul(torch.outer(t, 1.0 / ext), inv_freq)
    emb = torch.cat((freqs, freqs), dim=-1)
    if ext_factors is None:
        return emb.cos().contiguous(), emb.sin().contiguous()
    return (emb.cos() * scale).contiguous(), (emb.sin() * scale).contiguous()


def rms_layernorm(x: torch.Tensor, weight: torch.Tensor, eps: float,
                  out: torch.Tensor | None = None) -> torch.Tensor:
    """``rms_layernorm`` (minicpm.py:772-788) of the rows of ``x [n, hidden]``."""
    _rows(x, "x")
    dev = _hip.require_gpu(x, weight)
    n, hidden = x.shape
    if weight.shape != (hidden,) or weight.dtype != x.dtype:
        raise ValueError("weight must be [hidden] in x's dtype")
    out = (torch.empty((n, hidden), dtype=x.dtype, device=dev) if out is None
           else _out(out, (n, hidden), x))
    _hip.check(_hip.lib().ls_rmsnorm(
        x.data_ptr(), x.stride(0), weight.contiguous().data_ptr(), n, hidden, float(eps),
        _hip.dtype_code(x.dtype), out.data_ptr(), out.stride(0), _hip.stream_of(dev)), "ls_rmsnorm")
    return out


def add_rms_layernorm(residual: torch.Tensor, h: torch.Tensor, h_scale: float,
                      weight: torch.Tensor, eps: float,
                      out: torch.Tensor | None = None) -> torch.Tensor:
    """``residual += h * h_scale`` (in place, rounded like minicpm.py:3616-3625),
    then the RMSNorm of the new residual (returned)."""
    _rows(residual, "residual")
    _rows(h, "h")
    dev = _hip.require_gpu(residual, h, weight)
    n, hidden = residual.shape
    if h.shape != residual.shape or h.dtype != residual.dtype:
        raise ValueError("h must match residual's shape and dtype")
    if weight.shape != (hidden,) or weight.dtype != residual.dtype:
        raise ValueError("weight must be [hidden] in residual's dtype")
    out = (torch.empty((n, hidden), dtype=residual.dtype, device=dev) if out is None
           else _out(out, (n, hidden), residual))
    _hip.check(_hip.lib().ls_add_rmsnorm(
        residual.data_ptr(), residual.stride(0), h.data_ptr(), h.stride(0), float(h_scale),
        weight.contiguous().data_ptr(), n, hidden, float(eps), _hip.dtype_code(residual.dtype),
        out.data_ptr(), out.stride(0), _hip.stream_of(dev)), "ls_add_rmsnorm")
    return out


def rope_inplace(x: torch.Tensor, positions: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                 *, n_q_heads: int, n_k_heads: int, k_col_offset: int, head_dim: int = 128,
                 check_positions: bool = True) -> torch.Tensor:
    """``apply_rotary_pos_emb`` (minicpm.py:1034-1070) in place on the query heads
    (columns ``[0, n_q_heads*head_dim)``) and key heads (from ``k_col_offset``) of
    each row of ``x [n, width]``; ``positions`` int32 ``[n]``."""
    _rows(x, "x")
    dev = _hip.require_gpu(x, positions, cos, sin)
    if positions.dtype != torch.int32 or positions.shape != (x.shape[0],):
        raise ValueError("positions must be int32 [n]")
    if cos.dtype != torch.float32 or sin.dtype != torch.float32 or cos.shape != sin.shape \
            or cos.ndim != 2 or cos.shape[1] != head_dim:
        raise ValueError("cos/sin must be float32 [table_rows, head_dim]")
    if x.shape[1] < max(n_q_heads * head_dim, k_col_offset + n_k_heads * head_dim):
        raise ValueError("the query and key heads must lie inside x's columns")
    if check_positions and positions.numel():
        lo, hi = int(positions.min()), int(positions.max())
        if lo < 0 or hi >= cos.shape[0]:
            raise ValueError(f"positions must lie in [0, {cos.shape[0]}) (got {lo}..{hi})")
    _hip.check(_hip.lib().ls_rope_inplace(
        x.data_ptr(), x.stride(0), positions.contiguous().data_ptr(), x.shape[0], n_q_heads,
        n_k_heads, k_col_offset, head_dim, cos.contiguous().data_ptr(), sin.contiguous().data_ptr(),
        cos.shape[0], _hip.dtype_code(x.dtype), _hip.stream_of(dev)), "ls_rope_inplace")
    return x


def rope_k_compress(x: torch.Tensor, positions: torch.Tensor, cos: torch.Tensor,
                    sin: torch.Tensor, cu_seqlens: torch.Tensor, cu_host: list[int], *,
                    n_k_heads: int, k_col_offset: int, head_dim: int = 128,
                    check_positions: bool = True):
    """Rotate the key heads of ``x [n, width]`` in place (as :func:`rope_inplace`)
    and return their compressed keys ``(kc [A, n_k_heads, D], cu_seqlens_compressed)``
    -- ``CompressK.forward`` (minicpm.py:1158-1185) of the rotated keys, formed
    while they are written (windows of 32 at stride 16)."""
    _rows(x, "x")
    dev = _hip.require_gpu(x, positions, cos, sin, cu_seqlens)
    if positions.dtype != torch.int32 or positions.shape != (x.shape[0],):
        raise ValueError("positions must be int32 [n]")
    if cu_seqlens.dtype != torch.int32 or cu_seqlens.numel() != len(cu_host):
        raise ValueError("cu_seqlens must be int32 [batch + 1] matching cu_host")
    if cos.dtype != torch.float32 or sin.dtype != torch.float32 or cos.shape != sin.shape \
            or cos.ndim != 2 or cos.shape[1] != head_dim:
        raise ValueError("cos/sin must be float32 [table_rows, head_dim]")
    if x.shape[1] < k_col_offset + n_k_heads * head_dim:
        raise ValueError("the key heads must lie inside x's columns")
    if check_positions and positions.numel():
        lo, hi = int(positions.min()), int(positions.max())
        if lo < 0 or hi >= cos.shape[0]:
            raise ValueError(f"positions must lie in [0, {cos.shape[0]}) (got {lo}..{hi})")
    batch = len(cu_host) - 1
    lens = [cu_host[i + 1] - cu_host[i] for i in range(batch)]
    total_atoms = sum((n - 32) // 16 + 1 for n in lens if n >= 32)
    kc = torch.empty((total_atoms, n_k_heads, head_dim), dtype=x.dtype, device=dev)
    cu_c = torch.empty((batch + 1,), dtype=torch.int32, device=dev)
    L = _hip.lib()
    ws = _hip.workspace(L.ls_rope_k_compress_workspace_size(x.shape[0], batch, n_k_heads,
                                                            head_dim), dev)
    _hip.check(L.ls_rope_k_compress(
        x.data_ptr(), x.stride(0), positions.contiguous().data_ptr(), cu_seqlens.data_ptr(), batch,
        x.shape[0], n_k_heads, k_col_offset, head_dim, cos.contiguous().data_ptr(),
        sin.contiguous().data_ptr(), cos.shape[0], _hip.dtype_code(x.dtype),
        kc.data_ptr() if total_atoms else None, total_atoms, cu_c.data_ptr(), ws.data_ptr(),
        ws.numel(), _hip.stream_of(dev)), "ls_rope_k_compress")
    return kc, cu_c


def rope_project_queries(x: torch.Tensor, positions: torch.Tensor, cos: torch.Tensor,
                         sin: torch.Tensor, selector, *, n_q_heads: int, head_dim: int = 128,
                         check_positions: bool = True) -> torch.Tensor:
    """Rotate the query heads of ``x [n, width]`` in place (as :func:`rope_inplace`)
    and return the selector's query projection of the rotated rows,
    ``q~ [G, n, R*F]`` -- ``LeanSelectSelector.project_queries`` (selector.py:160-177)
    formed in the same pass, so the selection does not read the queries again.
    bf16/fp16, ``head_dim`` 128, router width 64 or 128."""
    from .ops.select import _masters

    _rows(x, "x")
    dev = _hip.require_gpu(x, positions, cos, sin)
    if positions.dtype != torch.int32 or positions.shape != (x.shape[0],):
        raise ValueError("positions must be int32 [n]")
    if cos.dtype != torch.float32 or sin.dtype != torch.float32 or cos.shape != sin.shape \
            or cos.ndim != 2 or cos.shape[1] != head_dim:
        raise ValueError("cos/sin must be float32 [table_rows, head_dim]")
    if x.shape[1] < n_q_heads * head_dim:
        raise ValueError("the query heads must lie inside x's columns")
    if (n_q_heads, head_dim) != (selector.num_heads, selector.head_dim):
        raise ValueError("query heads do not match the selector")
    if check_positions and positions.numel():
        lo, hi = int(positions.min()), int(positions.max())
        if lo < 0 or hi >= cos.shape[0]:
            raise ValueError(f"positions must lie in [0, {cos.shape[0]}) (got {lo}..{hi})")
    G, n = selector.num_kv_heads, x.shape[0]
    F = selector.router_heads * selector.router_dim
    out = torch.empty((G, n, F), dtype=x.dtype, device=dev)
    hm, _, qp, _ = _masters(selector)
    L = _hip.lib()
    dt = _hip.dtype_code(x.dtype)
    ws = _hip.workspace(L.ls_select_workspace_size(0, 0, 0, n_q_heads, G, head_dim,
                                                   selector.router_heads, selector.router_dim,
                                                   0, dt), dev)
    _hip.check(L.ls_rope_project_queries(
        x.data_ptr(), x.stride(0), positions.contiguous().data_ptr(), n, n_q_heads, G, head_dim,
        cos.contiguous().data_ptr(), sin.contiguous().data_ptr(), cos.shape[0], hm.data_ptr(),
        qp.data_ptr(), selector.router_heads, selector.router_dim, dt, out.data_ptr(),
        ws.data_ptr(), ws.numel(), _hip.stream_of(dev)), "ls_rope_project_queries")
    return out


def silu_mul(gate_up: torch.Tensor, inter: int, out: torch.Tensor | None = None) -> torch.Tensor:
    """``silu(gate) * up`` for ``gate_up [n, 2*inter]`` = [gate | up] (minicpm.py:1098-1135)."""
    _rows(gate_up, "gate_up")
    dev = _hip.require_gpu(gate_up)
    n = gate_up.shape[0]
    if gate_up.shape[1] < 2 * inter:
        raise ValueError("gate_up must hold 2*inter columns")
    out = (torch.empty((n, inter), dtype=gate_up.dtype, device=dev) if out is None
           else _out(out, (n, inter), gate_up))
    _hip.check(_hip.lib().ls_silu_mul(
        gate_up.data_ptr(), gate_up.stride(0), n, inter, _hip.dtype_code(gate_up.dtype),
        out.data_ptr(), out.stride(0), _hip.stream_of(dev)), "ls_silu_mul")
    return out


def embed_scale(ids: torch.Tensor, table: torch.Tensor, scale: float,
                check_ids: bool = True) -> torch.Tensor:
    """``embed_tokens(ids) * scale_emb`` (minicpm.py:3773-3774); ``ids`` int32 [n]."""
    dev = _hip.require_gpu(ids, table)
    if ids.dtype != torch.int32 or ids.ndim != 1:
        raise ValueError("ids must be int32 [n]")
    if table.ndim != 2 or not table.is_contiguous():
        raise ValueError("table must be a contiguous [vocab, hidden] tensor")
    if check_ids and ids.numel():
        lo, hi = int(ids.min()), int(ids.max())
        if lo < 0 or hi >= table.shape[0]:
            raise IndexError(f"token ids must lie in [0, {table.shape[0]}) (got {lo}..{hi})")
    out = torch.empty((ids.numel(), table.shape[1]), dtype=table.dtype, device=dev)
    _hip.check(_hip.lib().ls_embed_scale(
        ids.contiguous().data_ptr(), ids.numel(), table.data_ptr(), table.shape[0], table.shape[1],
        float(scale), _hip.dtype_code(table.dtype), out.data_ptr(), _hip.stream_of(dev)),
        "ls_embed_scale")
    return out


# ---------------------------------------------------------------------------
# The model
# ---------------------------------------------------------------------------
class _Layer:
    __slots__ = ("input_norm", "w_qkv", "w_o", "post_norm", "w_gate_up", "w_down", "selector")


class MiniCPMLeanSelect:
    """Random-initialised MiniCPM4.1-shaped decoder with LeanSelect prefill attention.

    Linear weights ~ N(0, weight_std^2) in ``dtype``; norm weights 1 + N(0, 0.1^2);
    selectors use ``LeanSelectSelector.reset_parameters`` (torch's RNG seeded per
    layer).  ``prefill`` returns float32 last-token logits per sequence.
    """

    def __init__(self, cfg: MiniCPMConfig, *, device="cuda", dtype=torch.bfloat16,
                 seed: int = 0, weight_std: float = 0.02):
        if dtype not in (torch.bfloat16, torch.float16):
            raise ValueError("the model runs in bf16 or fp16")
        if cfg.head_dim != 128:
            raise ValueError("the attention kernels need head_dim 128")
        self.cfg, self.dtype = cfg, dtype
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise RuntimeError("MiniCPMLeanSelect runs on the GPU")
        g = torch.Generator(device=self.device).manual_seed(seed)
        H, G, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        hid, inter = cfg.hidden_size, cfg.intermediate_size

        def lin(out_f, in_f):
            return torch.empty(out_f, in_f, dtype=dtype, device=self.device).normal_(
                0.0, weight_std, generator=g)

        def norm_w():
            w = torch.empty(hid, dtype=torch.float32, device=self.device).normal_(0.0, 0.1, generator=g)
            return (1.0 + w).to(dtype)

        self.embed = lin(cfg.vocab_size, hid)
        self.layers = []
        for li in range(cfg.num_hidden_layers):
            L = _Layer()
            L.input_norm = norm_w()
            L.w_qkv = lin(H * D + 2 * G * D, hid)
            L.w_o = lin(hid, H * D)
            L.post_norm = norm_w()
            L.w_gate_up = lin(2 * inter, hid)
            L.w_down = lin(hid, inter)
            torch.manual_seed(seed * 1000 + li)
            sel = LeanSelectSelector(num_heads=H, num_kv_heads=G, head_dim=D,
                                     router_heads=cfg.router_heads, router_dim=cfg.router_dim)
            L.selector = sel.requires_grad_(False).to(self.device)
            self.layers.append(L)
        self.final_norm = norm_w()
        self.lm_head = lin(cfg.vocab_size, hid)
        self._rope = None

    # -- pieces ----------------------------------------------------------------
    def rope_tables(self, max_pos: int):
        """Tables covering positions ``< max_pos`` (grown geometrically, so a decode
        that adds one position per step rebuilds them rarely; a row's values do
        not depend on the table length)."""
        if self._rope is None or self._rope[0].shape[0] < max_pos:
            n = max(max_pos, 2 * self._rope[0].shape[0]) if self._rope is not None else max_pos
            cfg = self.cfg
            if cfg.rope_scaling == "longrope":
                self._rope = rotary_tables(
                    cfg.head_dim, n, cfg.rope_theta, self.device,
                    ext_factors=MINICPM41_128K_LONGROPE_FACTOR,
                    scale=longrope_scale(cfg.max_position_embeddings,
                                         cfg.original_max_position_embeddings))
            elif cfg.rope_scaling is None:
                self._rope = rotary_tables(cfg.head_dim, n, cfg.rope_theta, self.device)
            else:
                raise ValueError(f"unsupported rope_scaling {cfg.rope_scaling!r}")
        return self._rope

    @property
    def residual_scale(self) -> float:
        return self.cfg.scale_depth / math.sqrt(self.cfg.num_hidden_layers)

    def attention(self, li: int, h: torch.Tensor, positions: torch.Tensor, cu_seqlens: torch.Tensor,
                  cu_host: list[int], return_parts: bool = False,
                  cache: LeanSelectKVCache | None = None):
        """Attention block of layer ``li`` on the normalised input ``h [N, hidden]``.

        q/k/v projection (one GEMM), rotary embedding in place, LeanSelect sparse
        prefill on strided views of the projection output, output projection.
        With ``cache`` (a step open for these tokens) the rotated keys and the
        values are also written into it.
        """
        cfg, L = self.cfg, self.layers[li]
        H, G, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        N = h.shape[0]
        qkv = F.linear(h, L.w_qkv)
        cos, sin = self.rope_tables(max(cu_host[i + 1] - cu_host[i] for i in range(len(cu_host) - 1)))
        # Producer-side fusion: the queries rotate in the pass that also forms
        # the selector's query projection, the keys in the pass that also forms
        # their compressed keys (the selection then re-reads neither).
        fused_k = cfg.kernel_size == 32 and cfg.kernel_stride == 16
        F_router = L.selector.router_heads * L.selector.router_dim
        fused_q = D == 128 and F_router in (64, 128)
        q_tilde = None
        if fused_q:
            q_tilde = rope_project_queries(qkv, positions, cos, sin, L.selector, n_q_heads=H,
                                           head_dim=D, check_positions=False)
        if not (fused_q and fused_k):
            rope_inplace(qkv, positions, cos, sin, n_q_heads=0 if fused_q else H,
                         n_k_heads=0 if fused_k else G, k_col_offset=H * D, head_dim=D,
                         check_positions=False)
        compressed = None
        if fused_k:
            compressed = rope_k_compress(qkv, positions, cos, sin, cu_seqlens, cu_host,
                                         n_k_heads=G, k_col_offset=H * D, head_dim=D,
                                         check_positions=False)
        q = qkv[:, : H * D].view(N, H, D)
        k = qkv[:, H * D: H * D + G * D].view(N, G, D)
        v = qkv[:, H * D + G * D:].view(N, G, D)
        if cache is not None:
            cache.update(li, k, v)
        attn, ids = leanselect_sparse_prefill(
            q, k, v, cu_seqlens, L.selector, topk=cfg.topk, local_blocks=cfg.local_blocks,
            init_blocks=cfg.init_blocks, block_size=cfg.block_size, kernel_size=cfg.kernel_size,
            kernel_stride=cfg.kernel_stride, cu_seqlens_host=cu_host, return_topk_idx=True,
            compressed=compressed, q_tilde=q_tilde)
        o = F.linear(attn.view(N, H * D), L.w_o)
        if return_parts:
            return o, dict(qkv=qkv, attn=attn, topk_idx=ids)
        return o

    def mlp(self, li: int, h: torch.Tensor) -> torch.Tensor:
        """``down(silu(gate(h)) * up(h))`` with gate and up as one GEMM."""
        L = self.layers[li]
        return F.linear(silu_mul(F.linear(h, L.w_gate_up), self.cfg.intermediate_size), L.w_down)

    @staticmethod
    def positions(cu_host: list[int], device) -> torch.Tensor:
        """int32 position of each packed token inside its sequence."""
        parts = [torch.arange(cu_host[i + 1] - cu_host[i], dtype=torch.int32)
                 for i in range(len(cu_host) - 1)]
        return torch.cat(parts).to(device)

    # -- prefill -----------------------------------------------------------------
    def new_cache(self, batch: int, capacity: int) -> LeanSelectKVCache:
        """An empty decode cache for ``batch`` sequences of up to ``capacity`` tokens."""
        cfg = self.cfg
        return LeanSelectKVCache(cfg.num_hidden_layers, batch, capacity, cfg.num_key_value_heads,
                                 cfg.head_dim, dtype=self.dtype, device=self.device,
                                 kernel_size=cfg.kernel_size, kernel_stride=cfg.kernel_stride)

    @torch.no_grad()
    def prefill(self, input_ids: torch.Tensor, cu_seqlens_host: list[int] | None = None,
                *, layer_hook=None, cache: LeanSelectKVCache | None = None) -> torch.Tensor:
        """Last-token logits ``[B, vocab]`` (float32) of packed sequences.

        ``input_ids`` int32 ``[N]`` on the GPU; ``cu_seqlens_host`` the packed
        offsets (one sequence of N tokens when omitted).  ``layer_hook(li, x)``,
        if given, sees the residual stream after each layer.  With an empty
        ``cache`` (one slot per sequence) every layer's rotated keys, values and
        compressed keys are kept for ``decode_step``.
        """
        cfg = self.cfg
        N = input_ids.numel()
        cu_host = list(cu_seqlens_host) if cu_seqlens_host is not None else [0, N]
        if cu_host[0] != 0 or cu_host[-1] != N or any(b < a for a, b in zip(cu_host, cu_host[1:])):
            raise ValueError("cu_seqlens_host must be non-decreasing from 0 to the token count")
        if len(cu_host) < 2 or any(b == a for a, b in zip(cu_host, cu_host[1:])):
            # Each sequence's logits are read at its last token, which an empty
            # sequence does not have.
            raise ValueError("every packed sequence must hold at least one token")
        dev = _hip.require_gpu(input_ids)
        if cache is not None:
            if cache.batch != len(cu_host) - 1 or any(cache.lengths):
                raise ValueError("prefill fills an empty cache with one slot per sequence")
            cache.begin([b - a for a, b in zip(cu_host, cu_host[1:])])
        cu = torch.tensor(cu_host, dtype=torch.int32, device=dev)
        pos = self.positions(cu_host, dev)
        x = embed_scale(input_ids, self.embed, cfg.scale_emb)
        h = rms_layernorm(x, self.layers[0].input_norm, cfg.rms_norm_eps)
        c = self.residual_scale
        for li in range(cfg.num_hidden_layers):
            o = self.attention(li, h, pos, cu, cu_host, cache=cache)
            add_rms_layernorm(x, o, c, self.layers[li].post_norm, cfg.rms_norm_eps, out=h)
            d = self.mlp(li, h)
            nxt = self.layers[li + 1].input_norm if li + 1 < cfg.num_hidden_layers else self.final_norm
            add_rms_layernorm(x, d, c, nxt, cfg.rms_norm_eps, out=h)
            if layer_hook is not None:
                layer_hook(li, x)
        if cache is not None:
            cache.end()
        last = torch.tensor([b - 1 for b in cu_host[1:]], device=dev, dtype=torch.long)
        h_last = h.index_select(0, last) / (cfg.hidden_size / cfg.dim_model_base)
        return F.linear(h_last, self.lm_head).float()

    # -- decode ------------------------------------------------------------------
    def attention_decode(self, li: int, h: torch.Tensor, positions: torch.Tensor,
                         cache: LeanSelectKVCache, cu_q: torch.Tensor, cu_q_host: list[int]):
        """Attention block of layer ``li`` for one new token per sequence
        (``h [B, hidden]``): projection, rotary embedding at each sequence's
        position, append to the cache, stage-1 page plans on the compressed-key
        cache, block-sparse attention over the cache, output projection."""
        cfg, L = self.cfg, self.layers[li]
        H, G, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        B = h.shape[0]
        qkv = F.linear(h, L.w_qkv)
        cos, sin = self.rope_tables(max(cache.lengths_after))
        rope_inplace(qkv, positions, cos, sin, n_q_heads=H, n_k_heads=G, k_col_offset=H * D,
                     head_dim=D, check_positions=False)
        q = qkv[:, : H * D].view(B, H, D)
        k = qkv[:, H * D: H * D + G * D].view(B, G, D)
        v = qkv[:, H * D + G * D:].view(B, G, D)
        cache.update(li, k, v)
        after = cache.lengths_after
        ids = decode_topk_idx(q, cache.kc[li], cache.seqlens_after, cu_q, topk=cfg.topk,
                              init_blocks=cfg.init_blocks, local_blocks=cfg.local_blocks,
                              block_size=cfg.block_size, kernel_size=cfg.kernel_size,
                              kernel_stride=cfg.kernel_stride, cache_seqlens_host=after,
                              cu_seqlens_q_host=cu_q_host)
        attn = sparse_attention_kvcache(q, cache.k[li], cache.v[li], cache.seqlens_after, ids,
                                        cu_q, causal=False)
        return F.linear(attn.view(B, H * D), L.w_o)

    @torch.no_grad()
    def decode_step(self, input_ids: torch.Tensor, cache: LeanSelectKVCache) -> torch.Tensor:
        """Logits ``[B, vocab]`` (float32) of one new token per sequence
        (``input_ids`` int32 ``[B]``), appended to ``cache``."""
        cfg = self.cfg
        B = input_ids.numel()
        if B != cache.batch:
            raise ValueError(f"one token per cached sequence: {B} ids for {cache.batch} slots")
        if min(cache.lengths) < 1:
            raise ValueError("decode_step continues prefilled sequences")
        dev = _hip.require_gpu(input_ids)
        pos = torch.tensor(cache.lengths, dtype=torch.int32, device=dev)
        cu_q_host = list(range(B + 1))
        cu_q = torch.tensor(cu_q_host, dtype=torch.int32, device=dev)
        cache.begin([1] * B)
        x = embed_scale(input_ids, self.embed, cfg.scale_emb)
        h = rms_layernorm(x, self.layers[0].input_norm, cfg.rms_norm_eps)
        c = self.residual_scale
        for li in range(cfg.num_hidden_layers):
            o = self.attention_decode(li, h, pos, cache, cu_q, cu_q_host)
            add_rms_layernorm(x, o, c, self.layers[li].post_norm, cfg.rms_norm_eps, out=h)
            d = self.mlp(li, h)
            nxt = self.layers[li + 1].input_norm if li + 1 < cfg.num_hidden_layers else self.final_norm
            add_rms_layernorm(x, d, c, nxt, cfg.rms_norm_eps, out=h)
        cache.end()
        return F.linear(h / (cfg.hidden_size / cfg.dim_model_base), self.lm_head).float()
