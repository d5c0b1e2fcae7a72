"""Reuse TTFT on the reordered-RAG workload, with the re-rotate+assemble kernel's HBM roofline.

Default workload (the one the headline metric is quoted on): Qwen2.5-7B-shaped random-init decoder
in bf16 (28 layers, hidden 3584, 28 q / 4 kv heads, head_dim 128, theta 1e6, vocab 152064),
prompt = 64-token system prompt + 32 docs x 1000 tokens + 32-token query, uniform random ids
(seed 1), docs pre-cached in order, then the request uses a seeded permutation (seed 2) of the docs
with 20% deviation-guided recompute and the recompute loop replayed from a hipGraph.

One step = one warm reuse request (Engine.prefill) end to end: block lookups, fused assembly,
deviation pass + top-k, 27 recompute layers, query forward, first-token logits. Every block is
GPU-resident before the timed region. Printed: one JSON line (rank 0).
"""
import argparse
import json
import os
import statistics
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "reuse TTFT ms @32k ctx, 20% recompute; re-rotate+assemble GB/s (% HBM peak)"
HBM_PEAK_GBS = 8000.0
BF16_MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense bf16
# HBM bytes per assemble launch, from two rocprofv3 PMC passes on this workload (FETCH_SIZE x 2.0,
# WRITE_SIZE x 1.0: the factors a plain copy of known size reads on MI355X); the profiler cannot
# run inside this process, so the figure is carried here for the workload it was measured on, with
# the profile record it comes from (`traffic_source` of the line). Re-measure after a kernel change.
MEASURED_ASSEMBLE_TRAFFIC = {"qwen2.5-7b-32k": 3677757000}
ASSEMBLE_TRAFFIC_SOURCE = "profiles/rope_assemble_qwen2.5-7b-32k.md (PMC passes of the current kernel)"
# HBM bytes per recompute attention call (subset_attn_kernel + attn_halves_kernel), the same two
# passes and factors on the 6 400-row recompute shape of this workload
# (`python3 -m tread_amd.kernel_bench attention --shape recompute`): 473.7 + 49.1 MB read,
# 90.2 + 11.5 MB written
MEASURED_ATTENTION_TRAFFIC = {"qwen2.5-7b-32k": 624431360}
ATTENTION_TRAFFIC_SOURCE = "profiles/subset_attn_qwen2.5-7b-32k.md (PMC passes of the current kernel)"
# doc blocks the GPU tier holds (with the prefix block); the rest spill to the pinned-host tier
# and are copied back per request on the store's copy streams (None: everything stays on the GPU)
GPU_TIER_DOCS = {"qwen2.5-1.5b-16k": 8}
# docs per request that are not cached (fresh token ids every request): they go through the packed
# block-diagonal prefill inside the timed request
COLD_DOCS = {"llama3-70b-32k": 8}
# the request's doc order: a seeded permutation unless named here
ORDER = {"qwen2.5-0.5b-1k": "reversed"}
# recompute ratio when --ratio is not given (0.2 otherwise)
DEFAULT_RATIO = {"qwen2.5-0.5b-1k": 0.0}
# workloads whose CPU baseline runs the oracle's whole request end to end (the dtype it runs in);
# the others time its stages on the request's sizes
E2E_CPU = {"qwen2.5-0.5b-1k": torch.float32, "qwen2.5-0.5b-8k": torch.bfloat16,
           "qwen2.5-1.5b-16k": torch.bfloat16}
WORKLOADS = {
    # name: (preset, n_docs, doc_len, n_system, n_query)
    "qwen2.5-7b-32k": ("qwen2.5-7b", 32, 1000, 64, 32),
    "qwen2.5-0.5b-1k": ("qwen2.5-0.5b", 4, 256, 64, 32),
    "qwen2.5-1.5b-16k": ("qwen2.5-1.5b", 16, 1000, 64, 32),
    "qwen2.5-0.5b-8k": ("qwen2.5-0.5b", 8, 1000, 64, 32),
    "llama3-70b-32k": ("llama3-70b", 32, 1000, 64, 32),
}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_inputs(cfg, n_docs, doc_len, n_sys, n_query, device, order=None):
    g = torch.Generator().manual_seed(1)
    V = cfg.vocab_size
    system = torch.randint(0, V, (n_sys,), generator=g)
    docs = [torch.randint(0, V, (doc_len,), generator=g) for _ in range(n_docs)]
    query = torch.randint(0, V, (n_query,), generator=g)
    if order == "reversed":
        perm = list(range(n_docs))[::-1]
    else:
        perm = torch.randperm(n_docs, generator=torch.Generator().manual_seed(2)).tolist()
    to = lambda t: t.to(device)
    return to(system), [to(d) for d in docs], to(query), perm


def time_assemble(eng, system, docs, order, n_query, iters=20):
    """Launch the fused re-rotate+assemble kernel alone on the request's 33 sources, timed with HIP
    events on the stream it runs on. Returns (avg seconds per launch, algorithmic bytes)."""
    from tread_amd import _hip
    from tread_amd.forward import alloc_cache
    from tread_amd.store import block_key
    P = eng.P
    dev = system.device

    def on_gpu(key):  # blocks of any tier; host- and disk-tier ones are copied up for this measurement
        b = eng.store.blocks.get(key) or eng.store.cpu_blocks.get(key)
        if b is None:
            from types import SimpleNamespace
            from tread_amd import blockfile
            eng.store.drain()
            K, V, h = blockfile.read_block(eng.store.disk_blocks[key].path)
            return SimpleNamespace(n_tokens=h["n_tokens"], base=h["base"]), K.to(dev), V.to(dev)
        return b, b.K.to(dev), b.V.to(dev)

    pkey = block_key(*eng.sig, "", "prefix", system)
    pb, pK, pV = on_gpu(pkey)
    srcs = [(pK, pV, 0, 0)]
    off = pb.n_tokens
    for i in order:
        b, bK, bV = on_gpu(block_key(*eng.sig, pkey, docs[i]))
        srcs.append((bK, bV, off, off - b.base))
        off += b.n_tokens
    T = off
    K, V = alloc_cache(P, T + n_query, system.device)
    table = _hip.rope_assemble(srcs, K, V, P.inv_freq)  # warm
    torch.cuda.synchronize()
    s = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for _ in range(iters):
        _hip.rope_assemble(srcs, K, V, P.inv_freq, table=table)
    e1.record(s)
    e1.synchronize()
    sec = e0.elapsed_time(e1) / 1e3 / iters
    nbytes = 2 * 2 * (T * P.L * P.hkv * P.hd * 2)  # read + write, K and V
    return sec, nbytes


def time_recompute_attention(eng, S, T, n_query, iters=20):
    """The recompute attention of the request alone: the selected rows S and the query rows
    (positions T..T+n_query-1) over a cache of T + n_query rows, as one recompute layer launches
    it (subset_attn_kernel, plus attn_halves_kernel when the longest row tiles run as key halves),
    timed with HIP events on the stream it runs on. Inputs are random (the time does not depend on
    the values). Returns (avg seconds per call, FLOP per call: 4 hq hd sum(keys per row))."""
    from tread_amd import _hip
    P = eng.P
    dev = S.device
    rows = torch.cat([S.to(torch.int64), torch.arange(T, T + n_query, device=dev)])
    n, t_cap = rows.numel(), T + n_query
    g = torch.Generator(device=dev).manual_seed(5)
    q = torch.randn(n, P.hq, P.hd, device=dev, dtype=torch.bfloat16, generator=g)
    K = torch.randn(1, P.hkv, t_cap, P.hd, device=dev, dtype=torch.bfloat16, generator=g)
    V = torch.randn(1, P.hkv, t_cap, P.hd, device=dev, dtype=torch.bfloat16, generator=g)
    out = torch.empty(n, P.hq * P.hd, device=dev, dtype=torch.bfloat16)
    _hip.subset_attn(q, K, V, rows, P.hq, P.hkv, P.hd, P.scale, out=out)  # warm
    torch.cuda.synchronize()
    s = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for _ in range(iters):
        _hip.subset_attn(q, K, V, rows, P.hq, P.hkv, P.hd, P.scale, out=out)
    e1.record(s)
    e1.synchronize()
    sec = e0.elapsed_time(e1) / 1e3 / iters
    flop = 4 * P.hq * P.hd * float((rows.double() + 1).sum())
    return sec, flop


def time_decode(eng, system, docs, query, ratio, n):
    """n greedy decode steps after a reuse prefill, synchronising on every token as the reference
    server's loop does (tread/server.py:201-208). Bytes per step: every weight of the layers, the
    final norm and lm_head, plus the K and V rows each step attends to (one embedding row aside)."""
    P = eng.P
    wbytes = sum(t.numel() * t.element_size() for lw in P.layers for t in vars(lw).values()
                 if isinstance(t, torch.Tensor))
    wbytes += sum(t.numel() * t.element_size() for t in (P.norm, P.lm_head))
    logits, cache, _ = eng.prefill(system, docs, query, ratio=ratio, reserve=n)
    nxt = logits.argmax()
    int(nxt)
    for _ in range(2):  # first steps capture the decode graph
        nxt = eng.decode(cache, nxt.view(1)).argmax()
        int(nxt)
    T0 = cache.length
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(n):
        nxt = eng.decode(cache, nxt.view(1)).argmax()
        int(nxt)
    sec = (time.perf_counter() - t0) / n
    kv = 2 * P.L * P.hkv * P.hd * 2 * (T0 + (n + 1) / 2)  # mean keys attended per step
    step_bytes = wbytes + kv
    gbs = step_bytes / sec / 1e9
    log(f"[bench] decode: {sec * 1e3:.3f} ms/token over {n} tokens at {T0} context rows, "
        f"{step_bytes / 1e9:.2f} GB per step ({wbytes / 1e9:.2f} GB weights), {gbs:.0f} GB/s")
    return {"tokens": n, "context_rows": T0, "ms_per_token": round(sec * 1e3, 3), "bytes_per_token": int(step_bytes),
            "achieved_gbs": round(gbs, 1), "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
            "graph": cache.graph is not None}


def ratio_sweep(eng, system, order, query, ratios, steps, full_ms, full_logits, headline):
    """The reference's ratio sweep (bench/bench_scaling.py:68-72,88-91) on the timed request: for
    each recompute ratio, the median TTFT of `steps` warm requests (after one untimed request that
    captures the ratio's graph bucket), the speedup over full prefill, and the first-token KL and
    top-1 agreement against full prefill's logits. The headline ratio reuses its timed requests."""
    import torch.nn.functional as F
    out = []
    for r in ratios:
        if r == headline[0]:
            t = list(headline[1])
            logits, _, st = eng.prefill(system, order, query, ratio=r)
        else:
            eng.prefill(system, order, query, ratio=r)
            t = []
            for _ in range(steps):
                logits, _, st = eng.prefill(system, order, query, ratio=r)
                t.append(st.t["ttft"])
        ms = statistics.median(t) * 1e3
        row = {"ratio": r, "ttft_ms": round(ms, 2), "recompute_eff": round(st.recompute_eff, 4),
               "stages_ms": {k: round(v * 1e3, 2) for k, v in st.t.items()}}
        if full_logits is not None:
            a, b = full_logits.float(), logits.float()
            kl = F.kl_div(F.log_softmax(b, -1), F.log_softmax(a, -1), log_target=True, reduction="sum").item()
            row.update(speedup_vs_full_prefill=round(full_ms / ms, 2), kl_vs_full_prefill=float(f"{kl:.4g}"),
                       top1_matches_full_prefill=bool(int(a.argmax()) == int(b.argmax())))
        log(f"[bench] sweep r={r}: ttft {ms:.1f} ms" + (f", {row['speedup_vs_full_prefill']}x, KL {row['kl_vs_full_prefill']}, "
                                                        f"top-1 {'=' if row['top1_matches_full_prefill'] else '!='}"
                                                        if full_logits is not None else ""))
        out.append(row)
    return out


def cpu_baseline_e2e(model, cfg, system, docs, query, perm, ratio, dtype, threads, budget, cpu_budget):
    """The oracle's whole request (the reference's torch path restated, tread/engine.py:98-136) on
    this machine's host cores, on the same weights (copied from the GPU model, in `dtype`) and the
    same ids: a cold pass over the docs in order fills its store (untimed), then warm requests in
    the benchmark's doc order; TTFT = median of the timed ones (5 after 2 warm-ups; 3 after 1 when
    a request takes over 10 s)."""
    from oracle import tread_ref as R
    torch.set_num_threads(threads)
    ref = R.M.load(cfg, {k: v.detach().to("cpu") for k, v in model.state_dict().items()}, dtype)
    eng = R.Engine(ref, R.BlockStore(budget, cpu_budget))
    cpu = lambda t: t.to("cpu")
    sysc, docc, qc = cpu(system), [cpu(d) for d in docs], cpu(query)
    order = [docc[i] for i in perm]
    eng.prefill(sysc, docc, qc)
    t0 = time.perf_counter()
    _, _, st = eng.prefill(sysc, order, qc, ratio=ratio)
    first = time.perf_counter() - t0
    warm, reps = (1, 3) if first > 10 else (2, 5)
    for _ in range(warm - 1):
        eng.prefill(sysc, order, qc, ratio=ratio)
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        _, _, st = eng.prefill(sysc, order, qc, ratio=ratio)
        times.append(time.perf_counter() - t0)
    ms = statistics.median(times) * 1e3
    return {"value": round(ms, 1), "unit": "ms", "cores": threads, "kind": "port", "cpu": cpu_model(),
            "sample": (f"oracle (reference torch path restated, {str(dtype).split('.')[-1]}) end to end on {threads} "
                       f"host threads: the whole warm request (hits {st.hits}, misses {st.misses}), median of {reps} "
                       f"after {warm} warm-up(s); same weights and ids as the GPU run"),
            "reps_ms": [round(t * 1e3, 1) for t in times]}


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(preset_name, n_docs, doc_len, n_sys, n_query, ratio, threads):
    """The oracle (the reference's torch path restated on the CPU, bf16) timed on this machine's
    host cores, stage by stage on the request's own sizes:
      assemble: rotate_keys of every doc block by its shift + the per-layer cat (tread/engine.py:
        108-120), all n_docs blocks, in full;
      deviation: layer 0 over every candidate, layer-1 k/v, the score and the top-k
        (tread/blend.py:117-130,160), in full (attention in row chunks to bound memory);
      recompute: one recompute layer over all selected rows against the full cache, x (L - 1)
        (extrapolated: every recompute layer does the same work);
      query: one layer of the query forward over the blended cache, x L (extrapolated).
    Assemble and the two extrapolated layers are timed on their second run (the first builds the
    CPU kernels' primitives); the deviation pass, ~10 s, runs once.
    Random N(0, 0.02) weights for the two layers it runs; the embedding lookup (a gather) is not
    timed."""
    from oracle import model_ref as M
    from oracle import tread_ref as R
    from tread_amd.model import preset
    torch.set_num_threads(threads)
    cfg = preset(preset_name)
    L, hkv, hd, H = cfg.num_hidden_layers, cfg.num_key_value_heads, cfg.head_dim, cfg.hidden_size
    T = n_sys + n_docs * doc_len
    dt = torch.bfloat16
    g = torch.Generator().manual_seed(0)
    w = {}
    for l in (0, 1):
        pre = f"model.layers.{l}."
        q, k, I = cfg.num_attention_heads * hd, hkv * hd, cfg.intermediate_size
        shapes = {"self_attn.q_proj.weight": (q, H), "self_attn.k_proj.weight": (k, H), "self_attn.v_proj.weight": (k, H),
                  "self_attn.o_proj.weight": (H, q), "mlp.gate_proj.weight": (I, H), "mlp.up_proj.weight": (I, H),
                  "mlp.down_proj.weight": (H, I)}
        for n_, s_ in shapes.items():
            w[pre + n_] = (torch.randn(*s_, generator=g) * 0.02).to(dt)
        if cfg.attention_bias:
            for n_, s_ in (("q_proj", q), ("k_proj", k), ("v_proj", k)):
                w[pre + f"self_attn.{n_}.bias"] = torch.zeros(s_, dtype=dt)
        w[pre + "input_layernorm.weight"] = torch.ones(H, dtype=dt)
        w[pre + "post_attention_layernorm.weight"] = torch.ones(H, dtype=dt)
    m = M.RefModel(cfg=cfg, w=w, dtype=dt, inv_freq=M.inv_freq_of(cfg))
    mk = lambda n: torch.randn(1, hkv, n, hd, generator=g).to(dt)
    parts = {}
    # assemble: every doc block (four distinct random blocks, cycled; the work does not depend on
    # the values), rotated by its shift, then one cat per layer
    blocks = [(torch.randn(L, 1, hkv, doc_len, hd, generator=g).to(dt),
               torch.randn(L, 1, hkv, doc_len, hd, generator=g).to(dt)) for _ in range(4)]
    pref = (torch.randn(L, 1, hkv, n_sys, hd, generator=g).to(dt),) * 2
    perm = torch.randperm(n_docs, generator=g).tolist()
    for _ in range(2):  # the second run is timed (the first creates the kernels' primitives)
        t0 = time.perf_counter()
        Ks, Vs, off = [pref[0]], [pref[1]], n_sys
        for slot in range(n_docs):
            K, V = blocks[slot % 4]
            Ks.append(R.rotate_keys(m, K, off - (n_sys + perm[slot] * doc_len)))
            Vs.append(V)
            off += doc_len
        Kl = list(torch.cat(Ks, dim=-2).unbind(0))
        Vl = list(torch.cat(Vs, dim=-2).unbind(0))
        parts["assemble"] = time.perf_counter() - t0
        del Ks, Vs
    del blocks
    K0, V0 = Kl[0].clone(), Vl[0].clone()
    K1, V1 = Kl[1].clone(), Vl[1].clone()
    del Kl, Vl
    # deviation pass over every candidate, then the top-k
    n = n_docs * doc_len
    all_c = torch.arange(n_sys, T)
    h0 = (torch.randn(1, n, H, generator=g) * 0.02).to(dt)
    budget = int(round(ratio * n))
    t0 = time.perf_counter()
    ctx = R.subset_ctx(m, all_c, T, dt)
    h, _, _ = R.layer_subset_rows(m, 0, h0, all_c, K0, V0, ctx)
    _, k1, v1 = M.qkv(m, 1, M.norm(m, "model.layers.1.input_layernorm", h), *ctx[0])
    dev = R.deviation_score(k1, v1, K1[:, :, all_c], V1[:, :, all_c])[0]
    top = dev.topk(budget).indices
    S, order = all_c[top].sort()
    hS = h[:, top][:, order]
    parts["deviation"] = time.perf_counter() - t0
    del h0, ctx, k1, v1
    # one recompute layer over all selected rows against the full cache (timed on its second run)
    for _ in range(2):
        t0 = time.perf_counter()
        R.layer_subset_rows(m, 1, hS, S, K1, V1, R.subset_ctx(m, S, T, dt))
        t_layer = time.perf_counter() - t0
    parts["recompute"] = t_layer * (L - 1)
    # one layer of the query forward over the blended cache (T + n_query keys)
    Kq, Vq = torch.cat([K1, mk(n_query)], dim=2), torch.cat([V1, mk(n_query)], dim=2)
    Sq = torch.arange(T, T + n_query)
    hq = (torch.randn(1, n_query, H, generator=g) * 0.02).to(dt)
    for _ in range(2):
        t0 = time.perf_counter()
        R.layer_subset(m, 1, hq, Sq, Kq, Vq, inplace=True, ctx=R.subset_ctx(m, Sq, T + n_query, dt))
        parts["query"] = (time.perf_counter() - t0) * L
    total = sum(parts.values())
    return {"value": round(total * 1e3, 1), "unit": "ms", "cores": threads, "kind": "port", "cpu": cpu_model(),
            "sample": ("oracle (reference torch path restated, bf16) on %d host threads: assemble of all %d doc "
                       "blocks and the deviation pass + top-k over all %d candidates in full; one recompute "
                       "layer over all %d selected rows x%d layers and one query layer x%d extrapolated"
                       % (threads, n_docs, n, budget, L - 1, L)),
            "stages_ms": {k: round(v * 1e3, 1) for k, v in parts.items()},
            "extrapolated_ms": round((parts["recompute"] + parts["query"]) * 1e3, 1),
            "recompute_layer_ms": round(t_layer * 1e3, 1)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", default="qwen2.5-7b-32k", choices=list(WORKLOADS))
    ap.add_argument("--ratio", type=float, default=None,
                    help="recompute ratio (default: the workload's, 0.2 unless named in DEFAULT_RATIO)")
    ap.add_argument("--eager", action="store_true", help="recompute loop without the hipGraph")
    ap.add_argument("--no-fold", action="store_true",
                    help="run the query forward after the recompute instead of inside it")
    ap.add_argument("--full-reps", type=int, default=3, help="full-prefill reps for the TTFT denominator (0: skip)")
    ap.add_argument("--cpu-threads", type=int, default=os.cpu_count() or 1)
    ap.add_argument("--sweep", type=lambda v: [float(x) for x in v.split(",")] if v else [], default="0,0.2,0.5",
                    help="recompute ratios timed after the headline (comma list; empty: skip), each with the "
                         "first-token KL and top-1 against full prefill (bench/bench_scaling.py:68-72,88-91)")
    ap.add_argument("--sweep-steps", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--decode", type=int, default=32,
                    help="greedy decode steps timed after the TTFT loop on the last request's cache (0: skip)")
    ap.add_argument("--gpu-tier-docs", type=int, default=None,
                    help="doc blocks the GPU tier holds (default: the workload's setting; -1: all)")
    ap.add_argument("--disk-tier", default=None, metavar="DIR",
                    help="blocks outside the GPU tier live as files in DIR (no host tier): each request "
                         "reads them back (from the page cache once written)")
    ap.add_argument("--no-tune", action="store_true",
                    help="library-default GEMM solutions (default: the measured per-shape table in "
                         "tread_amd/tuning, applied through PyTorch TunableOp)")
    ap.add_argument("--retune", default=None, metavar="OUT_CSV",
                    help="benchmark GEMM solutions for every shape met (warm-up absorbs it) and write them here")
    ap.add_argument("--gemm-table", default=None, metavar="CSV",
                    help="GEMM solution table to apply instead of the model's table in tread_amd/tuning")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(f"bench.py measures one GPU: there is no multi-GPU path (asked for {args.gpus}); "
              "the KV-head sharding is designed but not built", file=sys.stderr)
        sys.exit(2)

    from tread_amd import BlockStore, Engine, prefill_full
    from tread_amd.model import preset, synthetic_model

    preset_name, n_docs, doc_len, n_sys, n_query = WORKLOADS[args.workload]
    gemm_tables = None
    if not args.no_tune:
        from tread_amd.tuning import table_for, use_tuned_gemms
        table = args.gemm_table or table_for(preset_name)
        if table is None:
            log(f"[bench] no GEMM solution table for {preset_name}: library defaults")
        tables = () if (args.retune or table is None) else (table,)
        gemm_tables = use_tuned_gemms(tables=tables, tune=bool(args.retune), out_file=args.retune)
        for t in gemm_tables:
            log(f"[bench] GEMM solution table {t['table']}: {'in effect' if t['loaded'] else 'NOT in effect'}, "
                f"{t['solutions']} solutions{'; stamps differ: ' + ', '.join(t['mismatched']) if t['mismatched'] else ''}")
    if args.ratio is None:
        args.ratio = DEFAULT_RATIO.get(args.workload, 0.2)
    cfg = preset(preset_name)
    dev = "cuda:0"
    torch.cuda.set_device(0)
    log(f"[bench] building {preset_name} (random init on the GPU)")
    model = synthetic_model(cfg, dev, torch.bfloat16, seed=0)
    system, docs, query, perm = make_inputs(cfg, n_docs, doc_len, n_sys, n_query, dev, ORDER.get(args.workload))
    T = n_sys + n_docs * doc_len
    tier_docs = GPU_TIER_DOCS.get(args.workload) if args.gpu_tier_docs is None else args.gpu_tier_docs
    if tier_docs is not None and tier_docs < 0:
        tier_docs = None
    budget = 1 << 40
    if tier_docs is not None:
        per_token = 2 * cfg.num_hidden_layers * cfg.num_key_value_heads * cfg.head_dim * 2
        budget = per_token * (n_sys + tier_docs * doc_len)
        log(f"[bench] GPU tier: prefix + {tier_docs} of {n_docs} doc blocks ({budget / 1e6:.0f} MB); "
            f"the rest live {'on disk' if args.disk_tier else 'in pinned host memory'}")
    if args.disk_tier:
        store = BlockStore(budget, 0, disk_dir=args.disk_tier, disk_budget_bytes=1 << 40)
    else:
        store = BlockStore(budget, 1 << 40)
    eng = Engine(model, store, graphs=not args.eager, fold_query=not args.no_fold)
    n_cold = COLD_DOCS.get(args.workload, 0)
    cold_gen = torch.Generator().manual_seed(3)

    def request_docs():
        """The request's docs in permuted order; the last n_cold slots of the permutation get
        fresh token ids (store misses)."""
        out = [docs[i] for i in perm]
        for j in range(n_docs - n_cold, n_docs):
            out[j] = torch.randint(0, cfg.vocab_size, (doc_len,), generator=cold_gen).to(dev)
        return out

    with torch.inference_mode():
        log("[bench] pass 1: cold prefill of every doc (packed block-diagonal)")
        _, _, st1 = eng.prefill(system, docs, query)
        for i in range(args.warmup):
            _, _, st = eng.prefill(system, request_docs(), query, ratio=args.ratio)
            log(f"[bench] warmup {i}: ttft {st.t['ttft'] * 1e3:.1f} ms hits {st.hits} misses {st.misses}")
        torch.cuda.synchronize()
        ttfts, stages = [], []
        c0 = store.stats.cpu_hits + store.stats.disk_hits
        reqs = [request_docs() for _ in range(args.steps)]
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(args.steps):
            _, _, st = eng.prefill(system, reqs[i], query, ratio=args.ratio)
            ttfts.append(st.t["ttft"])
            stages.append(st.t)
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) / args.steps
        assert st.hits == 1 + n_docs - n_cold and st.misses == n_cold
        order = reqs[-1]
        host_hits = (store.stats.cpu_hits + store.stats.disk_hits - c0) / args.steps
        if host_hits:
            log(f"[bench] {'disk' if args.disk_tier else 'host'}-tier hits per request: {host_hits:.1f} of "
                f"{1 + n_docs} blocks (promoted by H2D; evictions reuse the pinned copies"
                f"{', files are written once' if args.disk_tier else ''})")
        log(f"[bench] timed: median ttft {statistics.median(ttfts) * 1e3:.1f} ms, wall/step {wall * 1e3:.1f} ms")
        attn = None
        if eng.last_selected is not None:
            S = eng.last_selected.double()
            flop = 4 * cfg.num_attention_heads * cfg.head_dim * float((S + 1).sum())
            log(f"[bench] recompute: {S.numel()} rows, mean position {float(S.mean()):.0f}, "
                f"attention {flop:.3e} FLOP per layer")
            a_sec, a_flop = time_recompute_attention(eng, eng.last_selected, T, n_query)
            a_tf = a_flop / a_sec / 1e12
            log(f"[bench] recompute attention (selected + query rows): {a_sec * 1e6:.1f} us, {a_tf:.0f} TFLOP/s")
            attn = {"bound": "mfma", "kernel": "tread::subset_attn_kernel (+ attn_halves_kernel)",
                    "achieved": round(a_tf, 1), "peak": BF16_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                    "frac": round(a_tf / BF16_MFMA_PEAK_TFLOPS, 4),
                    "traffic": MEASURED_ATTENTION_TRAFFIC.get(args.workload),
                    "traffic_source": ATTENTION_TRAFFIC_SOURCE if args.workload in MEASURED_ATTENTION_TRAFFIC else None,
                    "avg_us": round(a_sec * 1e6, 2), "algorithmic_flop": a_flop}
        full_ms = full_logits = None
        if args.full_reps > 0:
            prefill_full(model, system, order, query)
            fr = []
            for _ in range(args.full_reps):
                full_logits, _, fst = prefill_full(model, system, order, query)
                fr.append(fst.t["ttft"])
            full_ms = statistics.median(fr) * 1e3
            log(f"[bench] full prefill: {full_ms:.1f} ms")
        sweep = None
        if args.sweep and n_cold == 0:
            sweep = ratio_sweep(eng, system, order, query, args.sweep, args.sweep_steps, full_ms, full_logits,
                                headline=(args.ratio, ttfts))
        sec, nbytes = time_assemble(eng, system, docs, perm, n_query)
        gbs = nbytes / sec / 1e9
        log(f"[bench] assemble: {sec * 1e6:.1f} us, {gbs:.0f} GB/s")
        decode = time_decode(eng, system, order, query, args.ratio, args.decode) if args.decode > 0 else None
    ttft_ms = statistics.median(ttfts) * 1e3
    med = {k: round(statistics.median(s[k] for s in stages) * 1e3, 2) for k in stages[0]}
    cpu = None
    if not args.no_cpu and args.workload in E2E_CPU and n_cold == 0:
        log("[bench] cpu baseline (oracle, the whole request)")
        cpu = cpu_baseline_e2e(model, cfg, system, docs, query, perm, args.ratio, E2E_CPU[args.workload],
                               args.cpu_threads, budget, 1 << 40)
        log(f"[bench] cpu baseline: {cpu['value']} ms")
    elif not args.no_cpu:
        log("[bench] cpu baseline (oracle, stage by stage)")
        cpu = cpu_baseline(preset_name, n_docs, doc_len, n_sys, n_query, args.ratio, args.cpu_threads)
        log(f"[bench] cpu baseline: {cpu['value']} ms (partly extrapolated)")
    out = {
        "metric": METRIC,
        "value": round(ttft_ms, 2),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3, 2),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (uniform random token ids, random-init N(0,0.02) weights)",
        "config": {"workload": args.workload, "model": preset_name, "context_tokens": T, "docs": n_docs,
                   "doc_len": doc_len, "system": n_sys, "query": n_query, "recompute_ratio": args.ratio,
                   "policy": "deviation", "hipgraph": not args.eager, "query_folded": not args.no_fold,
                   "gemm_tuning": not args.no_tune,
                   "gemm_table_in_effect": None if not gemm_tables else all(t["loaded"] for t in gemm_tables),
                   "gpu_tier_docs": n_docs if tier_docs is None else tier_docs, "cold_docs": n_cold,
                   "host_tier_hits_per_request": host_hits, "disk_tier": bool(args.disk_tier),
                   "parallelism": "single GPU"},
        "stages_ms": med,
        "ttft_full_prefill_ms": None if full_ms is None else round(full_ms, 2),
        "speedup_vs_full_prefill": None if full_ms is None else round(full_ms / ttft_ms, 2),
        "sweep": sweep,
        "gemm_tables": gemm_tables,
        "roofline": {"bound": "hbm", "kernel": "tread::rope_assemble_kernel", "achieved": round(gbs, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": MEASURED_ASSEMBLE_TRAFFIC.get(args.workload),
                     "traffic_source": ASSEMBLE_TRAFFIC_SOURCE if args.workload in MEASURED_ASSEMBLE_TRAFFIC else None,
                     "avg_us": round(sec * 1e6, 2),
                     "algorithmic_bytes": nbytes},
        "roofline_recompute_attention": attn,
        "cpu_baseline": cpu,
        "decode": decode,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
