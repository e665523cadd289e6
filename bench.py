"""LeanSelect prefill hot path benchmark on one MI355X.

One step = one MiniCPM4.1-8B attention layer of LeanSelect sparse prefill on a
128K-token sequence (bf16, 32 query / 2 KV heads, head_dim 128, page 64,
budget 64 pages = 1 sink + 5 local (4 local blocks and the query's own page)
+ 58 selected): compressed keys, page
selection and block-sparse attention, with inputs resident in HBM.

Prints one JSON line (metric: ms per layer, lower is better) with a roofline
object for the dominant kernel (block-sparse attention) measured with HIP
events on the launch stream, per-stage timings, and the CPU oracle timed on a
bounded row sample of the same workload on this host.

``--workload minicpm41_8b_prefill_64k`` times a whole random-init
MiniCPM4.1-8B-shaped prefill instead (32 layers, 65536 random token ids,
LeanSelect at every layer, last-token logits): library GEMMs for the
projections, HIP kernels for everything else.  Its line reports seconds per
prefill and a per-stage breakdown of one layer.

``--variant nosa`` times the NOSA layer instead (budget 96 pages = 1 sink +
16 local + 79 chosen, shortlist 41, CIS-biased attention) on the same shapes,
with the NOSA path restated on the host for its CPU baseline.

``--workload minicpm41_8b_decode_128k`` (and ``..._b16``) times one decode
step of one attention layer over a 128K-token KV cache per sequence: the
cache append with its compressed keys, stage-1 page plans and split-K
block-sparse attention over the cache (the reference's decode path), in
microseconds per layer; the roofline is the HBM rate of the attention's page
reads.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from leanselect_amd import workloads  # noqa: E402
from leanselect_amd.ops import (compress_k, leanselect_prefill_topk_idx,  # noqa: E402
                                nosa_prefill_topk_idx, nosa_sparse_attention, sparse_attention)
from leanselect_amd.ops.attention import attention_tile_rows  # noqa: E402

WORKLOADS = {
    "minicpm41_8b_layer_128k": dict(seq_lens=(131072,)),
    "minicpm41_8b_layer_32k": dict(seq_lens=(32768,)),
    "minicpm41_8b_layer_ragged_8k_24k_48k_96k": dict(seq_lens=(8192, 24576, 49152, 98304)),
    "minicpm41_8b_prefill_32k": dict(seq_lens=(32768,), model=True),
    "minicpm41_8b_prefill_64k": dict(seq_lens=(65536,), model=True),
    "minicpm41_8b_prefill_128k": dict(seq_lens=(131072,), model=True),
    "minicpm41_8b_decode_128k": dict(seq_lens=(131072,), decode=True, batch=1),
    "minicpm41_8b_decode_128k_b16": dict(seq_lens=(131072,), decode=True, batch=16),
}
# Published whole-model LeanSelect prefill times of the reference (H200, real
# weights, budget 96 pages with 32 local blocks, LongRoPE, median of 10 runs;
# results/minicpm_efficiency.json), for context beside the model workloads.
REFERENCE_PREFILL_S = {32768: 1.745, 65536: 3.603, 131072: 7.954}
HBM_PEAK_GBS = 8000.0
COPY_PROBE_BYTES = 1 << 30
# HBM bytes per launch of the attention kernel, from rocprofv3 FETCH_SIZE and
# WRITE_SIZE runs of `bench.py --traffic-probe`, each scaled by what the same
# counter reads for the probe's 1 GiB copy (see profiles/).
TRAFFIC_FILE = ROOT / "profiles" / "attention_traffic.json"
BF16_PEAK_TFLOPS = 2500.0


def attention_keys(ids: torch.Tensor, cu_host: list[int]) -> int:
    """Sum over (group, row) of the keys the row attends (causal, each page once)."""
    G, N, T = ids.shape
    dev = ids.device
    t_rel = torch.empty(N, dtype=torch.long, device=dev)
    lk = torch.empty(N, dtype=torch.long, device=dev)
    for b in range(len(cu_host) - 1):
        s, e = cu_host[b], cu_host[b + 1]
        t_rel[s:e] = torch.arange(e - s, device=dev)
        lk[s:e] = e - s
    jmax = torch.minimum(t_rel, lk - 1)  # prefill: len_q == len_k
    p = ids.long()
    valid = p >= 0
    keys = torch.clamp(jmax[None, :, None] - 64 * p + 1, min=0, max=64)
    return int((keys * valid).sum())


def plan_locality(ids: torch.Tensor, cu_host: list[int], tile: int | None = None) -> dict:
    """Mean distinct pages of a ``tile``-row query tile's plans (per KV group), and
    the mean number of the tile's rows that chose each of those pages: how much
    K/V one staged page serves. ``tile`` defaults to the attention kernel's."""
    G, N, T = ids.shape
    if tile is None:
        tile = attention_tile_rows(T)
    unions, chosen = 0.0, 0.0
    n_tiles = 0
    for b in range(len(cu_host) - 1):
        s, e = cu_host[b], cu_host[b + 1]
        n = (e - s) // tile
        if n == 0:
            continue
        x = ids[:, s : s + n * tile].reshape(G, n, tile * T)
        xs = x.sort(-1).values
        first = torch.ones_like(xs[..., :1], dtype=torch.bool)
        distinct = (xs >= 0) & torch.cat([first, xs[..., 1:] != xs[..., :-1]], -1)
        unions += float(distinct.sum())
        chosen += float((xs >= 0).sum())
        n_tiles += G * n
    return {"tile_rows": tile, "union_pages_per_tile": round(unions / max(n_tiles, 1), 1),
            "rows_per_union_page": round(chosen / max(unions, 1.0), 2)}


def selection_flops(case, D: int = 128, F: int = 128, all_pages: bool = False) -> float:
    """q~ projection + k~ projection + the atom dots of the non-forced visible pages
    (of every page with atoms when ``all_pages``: the NOSA shortlist ranks them all)."""
    H, G = case.q.shape[1], case.k.shape[1]
    N = case.cu_host[-1]
    total = 2.0 * N * G * (H // G) * D * F
    atom_dots = 0
    for b in range(len(case.cu_host) - 1):
        n = case.cu_host[b + 1] - case.cu_host[b]
        A = (n - 32) // 16 + 1 if n >= 32 else 0
        total += 2.0 * A * G * D * F
        if all_pages:
            atom_dots += n * A
            continue
        for qb in range((n + 63) // 64):
            if qb - case.local_blocks - 1 < case.init_blocks:
                continue  # no non-forced visible page yet
            hi = min(4 * (qb - case.local_blocks) - 1, A - 1)  # last atom of page qb-local-1
            lo = max(4 * case.init_blocks - 1, 0)
            rows = min(64, n - 64 * qb)
            atom_dots += rows * max(0, hi - lo + 1)
    return total + 2.0 * G * F * atom_dots


def _traffic(workload: str):
    """Measured HBM bytes per attention launch for this workload, if recorded."""
    try:
        rec = json.loads(TRAFFIC_FILE.read_text())
        return rec[workload]["hbm_bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def _event_ms(fn, iters: int) -> float:
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(iters):
        fn()
    end.record()
    end.synchronize()
    return start.elapsed_time(end) / iters


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _median_s(fn, runs: int, cap_s: float) -> tuple[float, int]:
    """Median wall time of ``runs`` calls (fewer when one call exceeds ``cap_s``)."""
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
        if times[-1] > cap_s:
            break
    times.sort()
    return times[len(times) // 2], len(times)


def cpu_baseline(case, attn_rows: int, threads: int, runs: int = 3) -> dict:
    """The reference's torch formulation of the path on the host CPU, ms per layer.

    Compressed keys and the whole selection (every query row) run in the
    activation dtype as the reference runs them (einsums, max_pool1d,
    torch.topk); attention is a gather-based float32 masked softmax timed on an
    even sample of query rows and scaled to the layer.  Each part is the median
    of ``runs`` warm runs.
    """
    import oracle

    torch.set_num_threads(threads)
    q, k, v = case.q.cpu(), case.k.cpu(), case.v.cpu()
    cu = case.cu_host
    N = cu[-1]
    sel = case.selector
    masters = [getattr(sel, n).detach().float().cpu()
               for n in ("head_mix", "kv_head_mix", "q_proj", "k_proj")]
    kw = dict(topk=case.topk, init_blocks=case.init_blocks, local_blocks=case.local_blocks)
    kc, cu_c = oracle.reference_compress_k(k, cu)  # warm-up, and the selection's input
    ids = oracle.reference_select_prefill(q, kc, cu, cu_c, masters, **kw)
    step = max(1, N // attn_rows)
    rows = list(range(step // 2, N, step))
    oracle.reference_sparse_attention_rows(q, k, v, cu, ids, rows[:64])
    t_c, n_c = _median_s(lambda: oracle.reference_compress_k(k, cu), runs, 60.0)
    t_s, n_s = _median_s(lambda: oracle.reference_select_prefill(q, kc, cu, cu_c, masters, **kw),
                         runs, 60.0)
    t_a, n_a = _median_s(lambda: oracle.reference_sparse_attention_rows(q, k, v, cu, ids, rows),
                         runs, 60.0)
    scale = N / len(rows)
    ms = 1e3 * (t_c + t_s + t_a * scale)
    return {
        "value": round(ms, 1),
        "unit": "ms/layer",
        "cores": threads,
        "kind": "port",
        "cpu_model": _cpu_model(),
        "stages_ms": {"compress_k": round(1e3 * t_c, 1), "select": round(1e3 * t_s, 1),
                      "sparse_attention": round(1e3 * t_a * scale, 1)},
        "sample": (f"the reference's torch formulation on the host CPU ({threads} threads), "
                   f"median of {min(n_c, n_s, n_a)}-{max(n_c, n_s, n_a)} warm runs: compressed "
                   f"keys and selection of all {N} query rows in {str(q.dtype).split('.')[-1]} "
                   f"(einsums, max_pool1d, torch.topk), attention (gather-based float32 masked "
                   f"softmax) on {len(rows)} evenly spaced rows ({1e3 * t_a:.0f} ms) scaled by "
                   f"{scale:.1f}"),
    }


def cpu_baseline_nosa(case, cis, n_rows: int, threads: int, runs: int = 3) -> dict:
    """The NOSA path restated on the host CPU (the oracle, float64), ms per layer.

    Compressed keys run in full; the atom scores, the two-stage page selection
    and the CIS-weighted attention run on an even sample of query rows and are
    scaled to the layer.  Each part is the median of ``runs`` warm runs.
    """
    import oracle

    torch.set_num_threads(threads)
    q, k, v, c = case.q.cpu(), case.k.cpu(), case.v.cpu(), cis.cpu()
    cu = case.cu_host
    N = cu[-1]
    max_len = max(cu[b + 1] - cu[b] for b in range(len(cu) - 1))
    sel = case.selector
    qf, kf = oracle.fused_weights(*[getattr(sel, n).detach().float().cpu()
                                    for n in ("head_mix", "kv_head_mix", "q_proj", "k_proj")],
                                  dtype=q.dtype)
    kc, cu_c = oracle.reference_compress_k(k, cu)
    step = max(1, N // n_rows)
    rows = list(range(step // 2, N, step))
    kw = dict(topk=case.topk, init_blocks=case.init_blocks, local_blocks=case.local_blocks,
              select_blocks=24, rows=rows)

    def select():
        atoms = oracle.nosa_atom_scores(q, kc, cu, cu_c, qf, kf, rows=rows)
        return oracle.nosa_select_prefill(atoms, c, cu, cu_c, cu, max_len, max_len, **kw)

    ids = select()
    t_c, n_c = _median_s(lambda: oracle.reference_compress_k(k, cu), runs, 60.0)
    t_s, n_s = _median_s(select, runs, 60.0)
    t_a, n_a = _median_s(lambda: oracle.nosa_attention(q, k, v, c, cu, cu, ids, rows=rows,
                                                       ids_rows_aligned=True), runs, 60.0)
    scale = N / len(rows)
    ms = 1e3 * (t_c + (t_s + t_a) * scale)
    return {
        "value": round(ms, 1),
        "unit": "ms/layer",
        "cores": threads,
        "kind": "port",
        "cpu_model": _cpu_model(),
        "stages_ms": {"compress_k": round(1e3 * t_c, 1), "select": round(1e3 * t_s * scale, 1),
                      "sparse_attention": round(1e3 * t_a * scale, 1)},
        "sample": (f"the NOSA path restated in float64 on the host CPU ({threads} threads), "
                   f"median of {min(n_c, n_s, n_a)}-{max(n_c, n_s, n_a)} warm runs: compressed "
                   f"keys of all {N} tokens, then atom scores, two-stage page selection and "
                   f"CIS-weighted attention on {len(rows)} evenly spaced query rows "
                   f"({1e3 * (t_s + t_a):.0f} ms) scaled by {scale:.1f}"),
    }


def decode_bench(args, dev) -> None:
    """One decode step of one MiniCPM4.1-8B attention layer over a KV cache."""
    from leanselect_amd.ops import decode_topk_idx, kvcache_append, sparse_attention_kvcache
    from leanselect_amd.ops.decode import n_windows

    wl = WORKLOADS[args.workload]
    B, ctx = wl["batch"], wl["seq_lens"][0]
    H, G, D, topk, local, init = 32, 2, 128, 64, 4, 1
    n_steps = args.warmup + args.steps
    cap = -(-(ctx + n_steps + 1) // 64) * 64
    bf = torch.bfloat16
    print(f"[bench] filling a {B} x {ctx}-token cache ...", file=sys.stderr, flush=True)
    g = torch.Generator(device=dev).manual_seed(0)
    k = torch.empty(B, cap, G, D, dtype=bf, device=dev)
    v = torch.empty_like(k)
    kc = torch.empty(B, n_windows(cap), G, D, dtype=bf, device=dev)
    zeros = torch.zeros(B, dtype=torch.int32, device=dev)
    for b in range(B):  # one sequence at a time keeps the fill's temporaries small
        kp = torch.randn(ctx, G, D, generator=g, device=dev).to(bf)
        vp = torch.randn(ctx, G, D, generator=g, device=dev).to(bf)
        one = torch.zeros(B + 1, dtype=torch.int32, device=dev)
        one[b + 1:] = ctx
        kvcache_append(k, v, zeros, kp, vp, one, kc_cache=kc, cache_seqlens_host=[0] * B,
                       cu_seqlens_new_host=[0] * (b + 1) + [ctx] * (B - b))
        del kp, vp
    q = torch.randn(n_steps, B, H, D, generator=g, device=dev).to(bf)
    kn = torch.randn(n_steps, B, G, D, generator=g, device=dev).to(bf)
    vn = torch.randn(n_steps, B, G, D, generator=g, device=dev).to(bf)
    cu_q_host = list(range(B + 1))
    cu_q = torch.tensor(cu_q_host, dtype=torch.int32, device=dev)
    lens = [ctx] * B

    def step(i, lens):
        after = [x + 1 for x in lens]
        before_t = torch.tensor(lens, dtype=torch.int32, device=dev)
        after_t = torch.tensor(after, dtype=torch.int32, device=dev)
        kvcache_append(k, v, before_t, kn[i], vn[i], cu_q, kc_cache=kc, cache_seqlens_host=lens,
                       cu_seqlens_new_host=cu_q_host)
        ids = decode_topk_idx(q[i], kc, after_t, cu_q, topk=topk, init_blocks=init,
                              local_blocks=local, cache_seqlens_host=after,
                              cu_seqlens_q_host=cu_q_host)
        out = sparse_attention_kvcache(q[i], k, v, after_t, ids, cu_q)
        return after, ids, out

    for i in range(args.warmup):
        lens, ids, out = step(i, lens)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.warmup, n_steps):
        lens, ids, out = step(i, lens)
    torch.cuda.synchronize()
    us_step = 1e6 * (time.perf_counter() - t0) / args.steps
    # Per-stage kernel time on the final lengths (HIP events on the launch stream).
    it = args.kernel_iters
    lens_t = torch.tensor(lens, dtype=torch.int32, device=dev)
    prev_t = lens_t - 1
    prev = [x - 1 for x in lens]
    us_append = 1e3 * _event_ms(lambda: kvcache_append(
        k, v, prev_t, kn[-1], vn[-1], cu_q, kc_cache=kc, cache_seqlens_host=prev,
        cu_seqlens_new_host=cu_q_host), it)
    us_select = 1e3 * _event_ms(lambda: decode_topk_idx(
        q[-1], kc, lens_t, cu_q, topk=topk, init_blocks=init, local_blocks=local,
        cache_seqlens_host=lens, cu_seqlens_q_host=cu_q_host), it)
    us_attn = 1e3 * _event_ms(lambda: sparse_attention_kvcache(q[-1], k, v, lens_t, ids, cu_q), it)
    # The same calls captured in HIP graphs and replayed: the GPU time of a step
    # without the host's per-call launch overhead (a serving loop would replay
    # the step the same way).  Each graph holds REPS back-to-back copies of its
    # calls, so the one launch per replay is spread over REPS steps; "step" is
    # the three calls in one graph, the stages are graphs of their own call.
    reps = 16
    graph_us = {}
    try:
        calls = {
            "append_and_compress": lambda: kvcache_append(
                k, v, prev_t, kn[-1], vn[-1], cu_q, kc_cache=kc, cache_seqlens_host=prev,
                cu_seqlens_new_host=cu_q_host),
            "select": lambda: decode_topk_idx(
                q[-1], kc, lens_t, cu_q, topk=topk, init_blocks=init, local_blocks=local,
                cache_seqlens_host=lens, cu_seqlens_q_host=cu_q_host),
            "sparse_attention": lambda: sparse_attention_kvcache(q[-1], k, v, lens_t, ids, cu_q),
        }
        calls["step"] = lambda: [fn() for name, fn in list(calls.items())[:3]]
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for fn in calls.values():
                fn()
        torch.cuda.current_stream().wait_stream(side)
        graphs = {}
        for name, fn in calls.items():
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr):
                for _ in range(reps):
                    fn()
            graphs[name] = gr
        for gr in graphs.values():
            gr.replay()
        torch.cuda.synchronize()
        for name, gr in graphs.items():
            graph_us[name] = round(1e3 * _event_ms(gr.replay, 10) / reps, 1)
    except Exception as exc:  # graph capture is an extra measurement only
        print(f"[bench] graph timing skipped: {exc}", file=sys.stderr, flush=True)
        graph_us = None
    us_attn_kernel = graph_us["sparse_attention"] if graph_us else us_attn
    # HBM bytes of the attention: K and V of every distinct visible page once per
    # row and group, plus q and out.
    pages = 0
    for row in ids.cpu().view(-1, ids.shape[2]).tolist():
        pages += len({p for p in row if p >= 0})
    attn_bytes = pages * 64 * D * 2 * 2 + 2 * B * H * D * 2
    gbs = attn_bytes / (us_attn_kernel * 1e-6) / 1e9
    result = {
        "metric": "decode step us/layer @128K context",
        "value": graph_us["step"] if graph_us else round(us_step, 1),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round((graph_us["step"] if graph_us else us_step) / 1e3, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": f"synthetic: {B} sequence(s) with {ctx} random N(0,1) bf16 keys/values in the cache, "
                "random queries and new tokens; value = the step's three calls captured 16 times "
                "in one HIP graph and replayed (GPU time per step, the graph launch spread over "
                "16 steps), stages_us = each call's own graph, eager_wall_us = the same step "
                "called from Python",
        "config": {"workload": args.workload, "batch": B, "context": ctx, "heads_q": H,
                   "heads_kv": G, "head_dim": D, "page": 64, "budget_pages": topk,
                   "sink_pages": init, "local_blocks": local, "selector": "stage-1 (decode)",
                   "parallelism": "single-gpu"},
        "eager_wall_us": round(us_step, 1),
        "stages_us": graph_us or {"append_and_compress": round(us_append, 1),
                                  "select": round(us_select, 1),
                                  "sparse_attention": round(us_attn, 1)},
        "stages_eager_us": {"append_and_compress": round(us_append, 1),
                            "select": round(us_select, 1), "sparse_attention": round(us_attn, 1)},
        "roofline": {"kernel": "ls_decode_attn_kernel + ls_decode_combine_kernel (split-K decode)",
                     "bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "algorithmic_bytes": attn_bytes},
    }
    if not args.no_cpu_baseline:
        import oracle
        threads = len(os.sched_getaffinity(0))
        if os.environ.get("OMP_NUM_THREADS", "").isdigit():
            threads = min(threads, int(os.environ["OMP_NUM_THREADS"]))
        torch.set_num_threads(threads)
        print(f"[bench] CPU baseline on {threads} threads ...", file=sys.stderr, flush=True)
        qc = q[-1].cpu()
        ncs = [n_windows(x) for x in lens]
        kcp = torch.cat([kc[b, :ncs[b]].cpu() for b in range(B)])
        kp = torch.cat([k[b, :lens[b]].cpu() for b in range(B)])
        vp = torch.cat([v[b, :lens[b]].cpu() for b in range(B)])
        cu_kc = [0]
        cu_k = [0]
        for b in range(B):
            cu_kc.append(cu_kc[-1] + ncs[b])
            cu_k.append(cu_k[-1] + lens[b])
        def cpu_step():
            ids_c = oracle.decode_select(qc, kcp, cu_q_host, cu_kc, lens, topk=topk,
                                         init_blocks=init, local_blocks=local)
            return oracle.sparse_attention(qc, kp, vp, cu_q_host, cu_k, ids_c, causal=False)
        cpu_step()
        t, n = _median_s(cpu_step, 3, 60.0)
        result["cpu_baseline"] = {
            "value": round(1e6 * t, 1), "unit": "us/layer", "cores": threads, "kind": "port",
            "cpu_model": _cpu_model(),
            "sample": (f"the oracle's decode step (stage-1 scores, page max-pool, top-k, then "
                       f"float64 attention over the plan) for all {B} row(s) on the host CPU, "
                       f"median of {n} warm runs"),
        }
    print(json.dumps(result), flush=True)


def model_bench(args, dev) -> None:
    """Whole-model prefill: seconds per prefill plus one layer's stage breakdown."""
    import torch.nn.functional as F

    from leanselect_amd import minicpm

    wl = WORKLOADS[args.workload]
    N = sum(wl["seq_lens"])
    cfg = minicpm.MiniCPMConfig(topk=args.budget_pages or 64, local_blocks=args.local_blocks or 4)
    print(f"[bench] building the random-init model ({cfg.num_hidden_layers} layers) ...",
          file=sys.stderr, flush=True)
    model = minicpm.MiniCPMLeanSelect(cfg, device=dev, seed=0)
    gen = torch.Generator(device=dev).manual_seed(1)
    ids = torch.randint(0, cfg.vocab_size, (N,), generator=gen, device=dev, dtype=torch.int32)
    cu_host = [0] + list(torch.tensor(wl["seq_lens"]).cumsum(0).tolist())
    for _ in range(args.warmup):
        model.prefill(ids, cu_host)
    torch.cuda.synchronize()
    print(f"[bench] warmup done, timing {args.steps} prefills", file=sys.stderr, flush=True)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        logits = model.prefill(ids, cu_host)
    torch.cuda.synchronize()
    s_step = (time.perf_counter() - t0) / args.steps
    assert bool(torch.isfinite(logits).all()), "non-finite logits"

    # Stage breakdown of layer 0 (HIP events on the launch stream).
    from leanselect_amd.ops import leanselect_prefill_topk_idx, sparse_attention

    it = args.kernel_iters
    H, G, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    L = model.layers[0]
    cu = torch.tensor(cu_host, dtype=torch.int32, device=dev)
    pos = model.positions(cu_host, dev)
    x = minicpm.embed_scale(ids, model.embed, cfg.scale_emb)
    h = minicpm.rms_layernorm(x, L.input_norm, cfg.rms_norm_eps)
    qkv = F.linear(h, L.w_qkv)
    cos, sin = model.rope_tables(max(wl["seq_lens"]))
    # As the model's attention runs it: the query heads rotate in the pass that
    # forms q~, the key heads in the pass that forms the compressed keys.
    qt = minicpm.rope_project_queries(qkv, pos, cos, sin, L.selector, n_q_heads=H, head_dim=D)
    kc, cu_c = minicpm.rope_k_compress(qkv, pos, cos, sin, cu, cu_host, n_k_heads=G,
                                       k_col_offset=H * D, head_dim=D)
    q = qkv[:, :H * D].view(N, H, D)
    k = qkv[:, H * D:H * D + G * D].view(N, G, D)
    v = qkv[:, H * D + G * D:].view(N, G, D)
    kw = dict(topk=cfg.topk, init_blocks=cfg.init_blocks, local_blocks=cfg.local_blocks,
              cu_seqlens_q_host=cu_host)
    sel_ids = leanselect_prefill_topk_idx(q, kc, cu, cu_c, L.selector, q_tilde=qt, **kw)
    attn = sparse_attention(q, k, v, cu, cu, N, N, sel_ids)
    o = F.linear(attn.view(N, H * D), L.w_o)
    gu = F.linear(h, L.w_gate_up)
    act = minicpm.silu_mul(gu, cfg.intermediate_size)
    xs = x.clone()
    stages = {
        "rmsnorm": lambda: minicpm.rms_layernorm(x, L.input_norm, cfg.rms_norm_eps, out=h),
        "qkv_gemm": lambda: F.linear(h, L.w_qkv),
        "rope_q_project": lambda: minicpm.rope_project_queries(
            qkv, pos, cos, sin, L.selector, n_q_heads=H, head_dim=D, check_positions=False),
        "rope_k_compress": lambda: minicpm.rope_k_compress(
            qkv, pos, cos, sin, cu, cu_host, n_k_heads=G, k_col_offset=H * D,
            check_positions=False),
        "select": lambda: leanselect_prefill_topk_idx(q, kc, cu, cu_c, L.selector, q_tilde=qt,
                                                      **kw),
        "sparse_attention": lambda: sparse_attention(q, k, v, cu, cu, N, N, sel_ids),
        "o_gemm": lambda: F.linear(attn.view(N, H * D), L.w_o),
        "add_rmsnorm": lambda: minicpm.add_rms_layernorm(xs, o, 0.0, L.post_norm, cfg.rms_norm_eps, out=h),
        "gate_up_gemm": lambda: F.linear(h, L.w_gate_up),
        "silu_mul": lambda: minicpm.silu_mul(gu, cfg.intermediate_size, out=act),
        "down_gemm": lambda: F.linear(act, L.w_down),
    }
    ms = {name: round(_event_ms(fn, it), 4) for name, fn in stages.items()}
    n_keys = attention_keys(sel_ids, cu_host)
    attn_flops = 4.0 * (H // G) * D * n_keys
    hid, inter = cfg.hidden_size, cfg.intermediate_size
    gemm_flops = 2.0 * N * hid * (H * D + 2 * G * D + H * D + 3 * inter)
    gemm_ms = ms["qkv_gemm"] + ms["o_gemm"] + ms["gate_up_gemm"] + ms["down_gemm"]
    result = {
        "metric": f"MiniCPM4.1-8B LeanSelect prefill seconds @{N // 1024}K (32 layers, B=1)",
        "value": round(s_step, 4),
        "unit": "s/prefill",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1e3 * s_step, 2),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (uniform random token ids, random-init weights)",
        "config": {
            "workload": args.workload, "seq_lens": list(wl["seq_lens"]),
            "layers": cfg.num_hidden_layers, "hidden": hid, "ffn": inter,
            "vocab": cfg.vocab_size, "heads_q": H, "heads_kv": G, "head_dim": D,
            "budget_pages": cfg.topk, "sink_pages": cfg.init_blocks,
            "local_blocks": cfg.local_blocks, "router": f"{cfg.router_heads}x{cfg.router_dim}",
            "rope": ("longrope: MiniCPM4.1 128K factors, base 10000, original context "
                     f"{cfg.original_max_position_embeddings}, scale "
                     f"{minicpm.longrope_scale(cfg.max_position_embeddings, cfg.original_max_position_embeddings):.4f}"
                     if cfg.rope_scaling == "longrope" else "plain, base 10000"),
            "parallelism": "single-gpu",
        },
        "layer0_stages_ms": ms,
        "layer0_gemm_tflops": round(gemm_flops / (gemm_ms * 1e-3) / 1e12, 1),
        "layer0_attention_tflops": round(attn_flops / (ms["sparse_attention"] * 1e-3) / 1e12, 1),
        "reference_published": (f"H200, real weights, budget 96 pages (32 local blocks), LongRoPE: "
                                f"{REFERENCE_PREFILL_S[N]} s (results/minicpm_efficiency.json)"
                                if N in REFERENCE_PREFILL_S and len(wl['seq_lens']) == 1 else None),
    }
    print(json.dumps(result), flush=True)


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="minicpm41_8b_layer_128k", choices=sorted(WORKLOADS))
    ap.add_argument("--variant", default="leanselect", choices=("leanselect", "nosa"))
    ap.add_argument("--kernel-iters", type=int, default=5)
    ap.add_argument("--cpu-attn-rows", type=int, default=1024,
                    help="query rows of the CPU baseline's attention sample")
    ap.add_argument("--cpu-nosa-rows", type=int, default=256,
                    help="query rows of the NOSA CPU baseline's selection and attention sample")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-secondary", action="store_true",
                    help="skip the secondary attention timing on plans without planted topics")
    ap.add_argument("--budget-pages", type=int, default=None,
                    help="model prefill only: total page budget (default 64)")
    ap.add_argument("--local-blocks", type=int, default=None,
                    help="model prefill only: local blocks (default 4)")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="run one plain copy of COPY_PROBE_BYTES and one step, untimed (for rocprofv3 --pmc)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this path runs on a single device "
              f"(--gpus {args.gpus} is not supported)", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    wl = WORKLOADS[args.workload]
    if wl.get("model"):
        model_bench(args, dev)
        return
    if wl.get("decode"):
        decode_bench(args, dev)
        return
    print(f"[bench] generating {args.workload} ...", file=sys.stderr, flush=True)
    nosa = args.variant == "nosa"
    if nosa:  # NOSA budget: topk 80 + 16 local, select_blocks 24 (nosa.py:643-676)
        case = workloads.hidden_space_layer(wl["seq_lens"], device=dev, seed=0, topk=96,
                                            local_blocks=16, init_blocks=1)
        g = torch.Generator(device="cpu").manual_seed(1)
        cis = torch.randn(case.cu_host[-1], case.k.shape[1], generator=g).to(torch.bfloat16).to(dev)
    else:
        case = workloads.hidden_space_layer(wl["seq_lens"], device=dev, seed=0)
    cu, cu_host = case.cu_seqlens, case.cu_host
    max_len = case.max_seqlen
    kw = dict(topk=case.topk, init_blocks=case.init_blocks, local_blocks=case.local_blocks,
              cu_seqlens_q_host=cu_host)

    def select(kc, cu_c):
        if nosa:
            return nosa_prefill_topk_idx(case.q, kc, cis, cu, cu_c, cu, case.selector,
                                         select_blocks=24, **kw)
        return leanselect_prefill_topk_idx(case.q, kc, cu, cu_c, case.selector, **kw)

    def attend(ids):
        if nosa:
            return nosa_sparse_attention(case.q, case.k, case.v, cis, cu, cu, max_len, max_len, ids)
        return sparse_attention(case.q, case.k, case.v, cu, cu, max_len, max_len, ids)

    def step():
        kc, cu_c = compress_k(case.k, cu, cu_seqlens_host=cu_host)
        ids = select(kc, cu_c)
        return attend(ids), ids

    if args.traffic_probe:
        # A plain device copy of known size calibrates the byte counters; then
        # one step of the workload.
        src = torch.empty(COPY_PROBE_BYTES // 2, dtype=torch.int16, device=dev).random_()
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        step()
        torch.cuda.synchronize()
        print(f"[bench] traffic probe done (copy of {COPY_PROBE_BYTES} bytes, one step)", file=sys.stderr)
        return

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    print(f"[bench] warmup done, timing {args.steps} steps", file=sys.stderr, flush=True)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        out, ids = step()
    torch.cuda.synchronize()
    ms_step = 1e3 * (time.perf_counter() - t0) / args.steps

    # Per-stage kernel time with HIP events on the launch stream.
    kc, cu_c = compress_k(case.k, cu, cu_seqlens_host=cu_host)
    it = args.kernel_iters
    ms_compress = _event_ms(lambda: compress_k(case.k, cu, cu_seqlens_host=cu_host), it)
    ms_select = _event_ms(lambda: select(kc, cu_c), it)
    ms_attn = _event_ms(lambda: attend(ids), it)

    H, G, D = case.q.shape[1], case.k.shape[1], case.q.shape[2]
    locality = plan_locality(ids, cu_host)
    secondary_plans = secondary_unit = None
    if not nosa and not args.no_secondary:
        # The same layer on hidden states without planted topics: plans that
        # share few pages between neighbouring rows, like the whole-model
        # prefill's on random token ids.
        print("[bench] secondary: attention on plans without planted topics ...",
              file=sys.stderr, flush=True)
        c0 = workloads.hidden_space_layer(wl["seq_lens"], device=dev, seed=0, topic_amp=0.0)
        kc0, cu_c0 = compress_k(c0.k, cu, cu_seqlens_host=cu_host)
        ids0 = leanselect_prefill_topk_idx(c0.q, kc0, cu, cu_c0, c0.selector, **kw)
        ms0 = _event_ms(lambda: sparse_attention(c0.q, c0.k, c0.v, cu, cu, max_len, max_len, ids0), it)
        fl0 = 4.0 * (H // G) * D * attention_keys(ids0, cu_host)
        secondary_plans = {
            "data": "same shapes and seed, no planted topics (topic amplitude 0)",
            "attention_ms": round(ms0, 4),
            "attention_tflops": round(fl0 / (ms0 * 1e-3) / 1e12, 2),
            "frac": round(fl0 / (ms0 * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
            "plan_locality": plan_locality(ids0, cu_host),
        }
        del c0, kc0, ids0
        print("[bench] secondary: attention on unit-scale plants ...", file=sys.stderr, flush=True)
        c1 = workloads.hidden_space_layer(wl["seq_lens"], device=dev, seed=0,
                                          **workloads.UNIT_SCALE)
        kc1, cu_c1 = compress_k(c1.k, cu, cu_seqlens_host=cu_host)
        ids1 = leanselect_prefill_topk_idx(c1.q, kc1, cu, cu_c1, c1.selector, **kw)
        ms1 = _event_ms(lambda: sparse_attention(c1.q, c1.k, c1.v, cu, cu, max_len, max_len, ids1), it)
        fl1 = 4.0 * (H // G) * D * attention_keys(ids1, cu_host)
        secondary_unit = {
            "data": ("same shapes and seed, each planted row given one topic-amplitude vector "
                     "(the unit vector of its plants' sum), so no page accumulates plants, and "
                     "value projection std 0.4/sqrt(4096) (values of std ~0.5)"),
            "attention_ms": round(ms1, 4),
            "attention_tflops": round(fl1 / (ms1 * 1e-3) / 1e12, 2),
            "frac": round(fl1 / (ms1 * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
            "plan_locality": plan_locality(ids1, cu_host),
        }
        del c1, kc1, ids1
    n_keys = attention_keys(ids, cu_host)
    attn_flops = 4.0 * (H // G) * D * n_keys
    sel_flops = selection_flops(case, all_pages=nosa)
    attn_tflops = attn_flops / (ms_attn * 1e-3) / 1e12
    N = cu_host[-1]
    result = {
        "metric": ("NOSA " if nosa else "") + "selector+sparse-attn prefill ms/layer @128K",
        "value": round(ms_step, 3),
        "unit": "ms/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 3),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": ("synthetic: seeded hidden states X ~ N(0,1) [N, 4096] with rank-8 page topics "
                 "planted at amplitude 48 (each 64-token query block and 8 of its earlier pages "
                 "share a topic direction; the amplitude is this benchmark's choice, the "
                 "reference fixes none; a page chosen by several blocks accumulates their "
                 "plants, up to ~56 on the earliest pages at 128K, so its keys and values "
                 "grow with the count), random-init projections (std 0.02); plan locality "
                 "in config.plan_locality, secondary.attention_without_topics for plans "
                 "that share few pages and secondary.attention_unit_scale_plants for plants "
                 "that do not accumulate"),
        "config": {
            "workload": args.workload,
            "seq_lens": list(wl["seq_lens"]),
            "heads_q": H, "heads_kv": G, "head_dim": D, "page": 64,
            "budget_pages": case.topk, "sink_pages": case.init_blocks,
            "local_blocks": case.local_blocks, "router": "4x32",
            **({"variant": "nosa", "select_blocks": 24, "cis": "bf16 N(0,1)"} if nosa else {}),
            "parallelism": "single-gpu",
            "plan_locality": locality,
        },
        "stages_ms": {"compress_k": round(ms_compress, 4), "select": round(ms_select, 4),
                      "sparse_attention": round(ms_attn, 4)},
        "roofline": {
            "kernel": ("ls_attn_tile_kernel (block-sparse attention"
                       + (", CIS key bias" if nosa else "") + "; timed with its K/V staging and plan kernels)"),
            "bound": "mfma",
            "achieved": round(attn_tflops, 2),
            "peak": BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(attn_tflops / BF16_PEAK_TFLOPS, 4),
            "traffic": _traffic(args.workload + (":nosa" if nosa else "")),
            "algorithmic_flops": attn_flops,
            "avg_keys_per_row": round(n_keys / (G * N), 1),
        },
        "secondary": {
            "select_tflops": round(sel_flops / (ms_select * 1e-3) / 1e12, 2),
            "select_flops": sel_flops,
            "attention_without_topics": secondary_plans,
            "attention_unit_scale_plants": secondary_unit,
        },
    }
    if not args.no_cpu_baseline:
        # The host cores of this GPU's share (OMP_NUM_THREADS on a shared box).
        threads = len(os.sched_getaffinity(0))
        if os.environ.get("OMP_NUM_THREADS", "").isdigit():
            threads = min(threads, int(os.environ["OMP_NUM_THREADS"]))
        print(f"[bench] CPU baseline on {threads} threads ...", file=sys.stderr, flush=True)
        if nosa:
            result["cpu_baseline"] = cpu_baseline_nosa(case, cis, args.cpu_nosa_rows, threads)
        else:
            result["cpu_baseline"] = cpu_baseline(case, args.cpu_attn_rows, threads)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
