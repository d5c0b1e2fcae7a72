"""Kernel micro-benchmarks on synthetic inputs of the reuse workloads' shapes.

    python -m tread_amd.kernel_bench assemble  [--workload qwen2.5-7b-32k] [--iters 20]
    python -m tread_amd.kernel_bench attention [--workload qwen2.5-7b-32k] [--shape recompute|prefill|query] [--sdpa]
    python -m tread_amd.kernel_bench copy      [--workload qwen2.5-7b-32k]
    python -m tread_amd.kernel_bench tiercopy  [--workload qwen2.5-1.5b-16k]
    python -m tread_amd.kernel_bench deviation [--workload qwen2.5-7b-32k]
    python -m tread_amd.kernel_bench skinny    [--workload qwen2.5-7b-32k]
    python -m tread_amd.kernel_bench request   [--workload qwen2.5-7b-32k] [--libs a.so,b.so]
    python -m tread_amd.kernel_bench tier      [--workload qwen2.5-1.5b-16k] [--gpu-docs 8]

`assemble` launches the fused re-rotate+assemble kernel on one request's blocks (prefix + every
doc, each doc shifted); `copy` copies the same number of bytes with torch (the calibration for
HBM traffic counters); `attention` runs the recompute attention kernel on a recompute-shaped row
set (20% of the doc positions, sorted), a full causal prefill, or the query rows (`--sdpa`: torch's
scaled_dot_product_attention on the same inputs beside it, the way the reference calls it). Each prints its
time per launch and achieved GB/s or TFLOP/s; under rocprofv3 every launch is one dispatch.
`tiercopy` moves every block of a request (prefix + docs) from pinned host memory to the GPU the
way a batch of host-tier promotions does (layer groups, one library call) and reports the DMA time.
`deviation` scores every doc position of a request (fresh layer-1 k/v rows of a qkv GEMM output
against the assembled layer-1 cache) and selects the top 20% of them, each launch timed alone.
`skinny` runs the projections of a decoding step (q|k|v with bias, o, gate|up, down, lm_head) for
1, 8 and 32 token rows through the skinny-linear kernel and through torch's GEMM, and reports the
weight-streaming bandwidth of each. `request` times whole reordered requests at 20 % recompute
(graph engines, every block on the GPU) under one or more builds of the library in one process,
alternating between them (A/B of a kernel change with the engine's own rows). `tier` runs
reordered requests whose blocks come from the pinned-host tier (the GPU tier holds the prefix and
`--gpu-docs` doc blocks, so under LRU every block of a request is promoted) and prints, per
request, when each copy schedule was queued, when each of its layer groups landed, and when the
compute stream reached each layer's assembly and how long it waited there.
"""
import argparse
import sys

import torch

from tread_amd import _hip
from tread_amd.model import inv_freq_of, preset

WORKLOADS = {
    "qwen2.5-7b-32k": ("qwen2.5-7b", 32, 1000, 64, 32),
    "qwen2.5-1.5b-16k": ("qwen2.5-1.5b", 16, 1000, 64, 32),
    "qwen2.5-0.5b-8k": ("qwen2.5-0.5b", 8, 1000, 64, 32),
    "llama3-70b-32k": ("llama3-70b", 32, 1000, 64, 32),
}


def _timed(fn, iters):
    fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(iters):
        fn()
    e1.record()
    e1.synchronize()
    return e0.elapsed_time(e1) / 1e3 / iters


def bench_assemble(cfg, n_docs, doc_len, n_sys, n_query, iters):
    L, kv, hd = cfg.num_hidden_layers, cfg.num_key_value_heads, cfg.head_dim
    mk = lambda n: torch.randn(L, 1, kv, n, hd, device="cuda", dtype=torch.bfloat16)
    srcs = [(mk(n_sys), mk(n_sys), 0, 0)]
    for i in range(n_docs):  # doc i cached at base n_sys, placed at a permuted slot
        off = n_sys + ((i * 7) % n_docs) * doc_len
        srcs.append((mk(doc_len), mk(doc_len), off, off - n_sys))
    T = n_sys + n_docs * doc_len
    K = torch.empty(L, 1, kv, T + n_query, hd, device="cuda", dtype=torch.bfloat16)
    V = torch.empty_like(K)
    table = _hip.rope_assemble(srcs, K, V, inv_freq_of(cfg))
    sec = _timed(lambda: _hip.rope_assemble(srcs, K, V, inv_freq_of(cfg), table=table), iters)
    nbytes = 4 * T * L * kv * hd * 2
    print(f"assemble: {sec * 1e6:.1f} us per launch, {nbytes} algorithmic bytes, {nbytes / sec / 1e9:.0f} GB/s")


def bench_copy(cfg, n_docs, doc_len, n_sys, n_query, iters):
    L, kv, hd = cfg.num_hidden_layers, cfg.num_key_value_heads, cfg.head_dim
    n = 2 * (n_sys + n_docs * doc_len) * L * kv * hd  # the assembled K + V element count
    src = torch.empty(n, device="cuda", dtype=torch.bfloat16)
    dst = torch.empty_like(src)
    sec = _timed(lambda: dst.copy_(src), iters)
    print(f"copy: {n * 2} bytes read + written, {sec * 1e6:.1f} us, {2 * n * 2 / sec / 1e9:.0f} GB/s")


def bench_tiercopy(cfg, n_docs, doc_len, n_sys, n_query, iters):
    L, kv, hd = cfg.num_hidden_layers, cfg.num_key_value_heads, cfg.head_dim
    lens = [n_sys] + [doc_len] * n_docs
    host = [torch.empty(L, 1, kv, n, hd, dtype=torch.bfloat16, pin_memory=True) for n in lens for _ in range(2)]
    dev = [torch.empty_like(t, device="cuda") for t in host]
    s = torch.cuda.Stream()
    groups = _hip.layer_groups(L)
    nbytes = sum(t.numel() * t.element_size() for t in host)
    times = []
    for _ in range(iters + 1):
        ev = [torch.cuda.Event() for _ in groups]
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        _hip.copy_layers(dev, host, s, groups, ev)
        e1.record(s)
        e1.synchronize()
        times.append(e0.elapsed_time(e1) / 1e3)
    sec = sorted(times[1:])[len(times[1:]) // 2]
    print(f"tiercopy: {len(lens)} blocks, {nbytes} bytes in {len(groups)} layer groups ({len(groups) * len(host)} DMAs): "
          f"{sec * 1e3:.2f} ms, {nbytes / sec / 1e9:.1f} GB/s")


def bench_attention(cfg, n_docs, doc_len, n_sys, n_query, iters, shape, ratio=0.2, sdpa=False):
    hq, hkv, hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    T = n_sys + n_docs * doc_len
    g = torch.Generator().manual_seed(0)
    if shape == "recompute":
        n = int(round(ratio * n_docs * doc_len))
        kend = torch.sort(torch.randperm(n_docs * doc_len, generator=g)[:n]).values + n_sys
        t_cap = T
    elif shape == "prefill":
        kend = torch.arange(T + n_query)
        t_cap = T + n_query
    else:
        kend = torch.arange(T, T + n_query)
        t_cap = T + n_query
    n = kend.numel()
    kend = kend.cuda()
    q = torch.randn(n, hq, hd, device="cuda", dtype=torch.bfloat16)
    K = torch.randn(1, hkv, t_cap, hd, device="cuda", dtype=torch.bfloat16)
    V = torch.randn_like(K)
    out = torch.empty(n, hq * hd, device="cuda", dtype=torch.bfloat16)
    sec = _timed(lambda: _hip.subset_attn(q, K, V, kend, hq, hkv, hd, hd ** -0.5, out=out), iters)
    flop = 4 * hq * hd * (kend + 1).double().sum().item()
    print(f"attention[{shape}]: rows {n} x {hq} heads over <= {t_cap} keys: {sec * 1e3:.3f} ms, "
          f"{flop / sec / 1e12:.1f} TFLOP/s")
    if sdpa:
        _against_sdpa(q, K, V, kend, out, hq, hkv, hd, t_cap, shape, flop, iters)


def _against_sdpa(q, K, V, kend, out, hq, hkv, hd, t_cap, shape, flop, iters):
    """torch's scaled_dot_product_attention on the same inputs, as the reference calls it
    (tread/blend.py:107-110: K/V expanded to the query heads, a boolean mask key <= row end; the
    causal prefill shape uses is_causal). Only the flash and memory-efficient backends are tried:
    the math backend would materialise [heads, rows, keys] scores in bf16."""
    from torch.nn.attention import SDPBackend, sdpa_kernel
    n = kend.numel()
    qh = q.view(1, n, hq, hd).transpose(1, 2).contiguous()
    kx = K.repeat_interleave(hq // hkv, dim=1).contiguous()
    vx = V.repeat_interleave(hq // hkv, dim=1).contiguous()
    causal = shape == "prefill"
    mask = None if causal else (torch.arange(t_cap, device=kend.device)[None, :] <= kend[:, None])[None, None]
    mine = out.view(n, hq, hd).transpose(0, 1)
    for name, backend in (("flash", SDPBackend.FLASH_ATTENTION), ("efficient", SDPBackend.EFFICIENT_ATTENTION)):
        try:
            with sdpa_kernel(backend):
                fn = lambda: torch.nn.functional.scaled_dot_product_attention(
                    qh, kx, vx, attn_mask=mask, is_causal=causal, scale=hd ** -0.5)
                o = fn()
                torch.cuda.synchronize()
                diff = (o[0].float() - mine.float()).abs().max().item()
                sec = _timed(fn, iters)
            print(f"  torch sdpa[{name}] on the same inputs: {sec * 1e3:.3f} ms, {flop / sec / 1e12:.1f} TFLOP/s, "
                  f"max |difference| {diff:.2e}")
        except RuntimeError as e:
            print(f"  torch sdpa[{name}]: not available ({str(e).splitlines()[0][:120]})")


def bench_deviation(cfg, n_docs, doc_len, n_sys, n_query, iters, ratio=0.2):
    hq, hkv, hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    T = n_sys + n_docs * doc_len
    n = n_docs * doc_len
    ld = (hq + 2 * hkv) * hd  # one row of the fused qkv projection output
    pos = torch.arange(n_sys, T, device="cuda")
    ang = pos[:, None].float() * inv_freq_of(cfg).cuda()[None, :]
    cos, sin = ang.cos().to(torch.bfloat16), ang.sin().to(torch.bfloat16)
    # four input sets (>= 1 GiB in all), used in turn, so that a launch reads HBM rather than the
    # 256 MB last-level cache that the previous launch filled
    sets = [(torch.randn(n, ld, device="cuda", dtype=torch.bfloat16),
             torch.randn(1, hkv, T + n_query, hd, device="cuda", dtype=torch.bfloat16),
             torch.randn(1, hkv, T + n_query, hd, device="cuda", dtype=torch.bfloat16)) for _ in range(4)]
    score = torch.empty(n, device="cuda", dtype=torch.bfloat16)
    k = int(round(ratio * n))
    sel = torch.empty(k, device="cuda", dtype=torch.int64)
    kc = hq * hd
    it = iter(range(1 << 30))

    def score_once():
        qkv, K, V = sets[next(it) % len(sets)]
        _hip.dev_score(qkv, cos, sin, pos, hkv, hd, K, V, k_col=kc, out=score)

    t_score = _timed(score_once, iters)
    t_sel = _timed(lambda: _hip.topk_select(score, k, out=sel), iters)
    nbytes = n * 4 * hkv * hd * 2  # fresh k, v + gathered cache rows
    print(f"dev_score: {n} candidates, {nbytes} algorithmic bytes, {t_score * 1e6:.1f} us, "
          f"{nbytes / t_score / 1e9:.0f} GB/s")
    print(f"topk_select: top {k} of {n}: {t_sel * 1e6:.1f} us")


def bench_skinny(cfg, iters):
    import torch.nn.functional as F
    H, I, hq, hkv, hd = (cfg.hidden_size, cfg.intermediate_size, cfg.num_attention_heads, cfg.num_key_value_heads,
                         cfg.head_dim)
    shapes = [("qkv", (hq + 2 * hkv) * hd, H, True), ("o", H, hq * hd, False), ("gate_up", 2 * I, H, False),
              ("down", H, I, False), ("lm_head", cfg.vocab_size, H, False)]
    for name, n, k, has_bias in shapes:
        # enough weight copies (>= 1 GiB) that each launch streams its weight from HBM, as in a
        # decoding step, not from the 256 MB last-level cache
        copies = max(2, -(-(1 << 30) // (n * k * 2)))
        Ws = [torch.randn(n, k, device="cuda", dtype=torch.bfloat16) * 0.02 for _ in range(copies)]
        b = torch.randn(n, device="cuda", dtype=torch.bfloat16) if has_bias else None
        for m in (1, 8, 32):
            x = torch.randn(m, k, device="cuda", dtype=torch.bfloat16)
            ok = _hip.skinny_ok(m, n, k)
            it = iter(range(1 << 30))
            t_s = _timed(lambda: _hip.skinny_linear(x, Ws[next(it) % copies], b), iters) if ok else float("nan")
            t_t = _timed(lambda: F.linear(x, Ws[next(it) % copies], b), iters)
            nbytes = n * k * 2
            print(f"skinny {name} [{m} x {k}] x [{n} x {k}]^T: kernel {t_s * 1e6:.1f} us "
                  f"({nbytes / t_s / 1e9:.0f} GB/s), torch {t_t * 1e6:.1f} us ({nbytes / t_t / 1e9:.0f} GB/s)")


def bench_request(cfg, name, n_docs, doc_len, n_sys, n_query, iters, libs, ratio=0.2):
    """Whole reordered requests (all blocks on the GPU, graph engines, `ratio` deviation recompute)
    under several builds of libtread_hip.so in one process: each build is loaded, an engine is
    captured with it, and timed requests alternate between the engines. Prints the median TTFT per
    build and the largest logits difference from the first build."""
    import statistics
    from pathlib import Path
    from tread_amd import BlockStore, Engine
    from tread_amd.model import synthetic_model
    from tread_amd.tuning import table_for, use_tuned_gemms
    table = table_for(name)
    if table is not None:
        use_tuned_gemms(tables=(table,))
    loaded = {}
    for p in libs:
        _hip._lib = None
        _hip.LIB_PATH = Path(p).resolve()
        loaded[p] = _hip.lib()
    model = synthetic_model(cfg, "cuda", torch.bfloat16, seed=0)
    g = torch.Generator().manual_seed(1)
    V = cfg.vocab_size
    system = torch.randint(0, V, (n_sys,), generator=g).cuda()
    docs = [torch.randint(0, V, (doc_len,), generator=g).cuda() for _ in range(n_docs)]
    query = torch.randint(0, V, (n_query,), generator=g).cuda()
    order = [docs[i] for i in torch.randperm(n_docs, generator=torch.Generator().manual_seed(2)).tolist()]
    store = BlockStore(1 << 40)
    engines, times, logits = {}, {p: [] for p in libs}, {}
    with torch.inference_mode():
        _hip._lib = loaded[libs[0]]
        Engine(model, store).prefill(system, docs, query)
        for p in libs:
            _hip._lib = loaded[p]
            engines[p] = Engine(model, store, graphs=True)
            for _ in range(2):  # capture, then one replay
                engines[p].prefill(system, order, query, ratio=ratio)
        for _ in range(iters):
            for p in libs:
                _hip._lib = loaded[p]
                out, _, st = engines[p].prefill(system, order, query, ratio=ratio)
                times[p].append(st.t["ttft"] * 1e3)
                logits[p] = out.float()
    for p in libs:
        d = (logits[p] - logits[libs[0]]).abs().max().item()
        print(f"request[{n_sys} + {n_docs} x {doc_len} + {n_query}, ratio {ratio}] {p}: median TTFT "
              f"{statistics.median(times[p]):.3f} ms (min {min(times[p]):.3f}), max |logits - first build| {d:.3e}")


def bench_tier(cfg, name, n_docs, doc_len, n_sys, n_query, iters, gpu_docs, ratio=0.2):
    """Timeline of host-tier requests (graph engine, `ratio` deviation recompute): GPU times from
    an event recorded as the request begins; host times from the same point."""
    import time
    from tread_amd import BlockStore, Engine
    from tread_amd import engine as E
    from tread_amd.model import synthetic_model
    from tread_amd.tuning import table_for, use_tuned_gemms
    table = table_for(name)
    if table is not None:
        use_tuned_gemms(tables=(table,))
    model = synthetic_model(cfg, "cuda", torch.bfloat16, seed=0)
    g = torch.Generator().manual_seed(1)
    V = cfg.vocab_size
    system = torch.randint(0, V, (n_sys,), generator=g).cuda()
    docs = [torch.randint(0, V, (doc_len,), generator=g).cuda() for _ in range(n_docs)]
    query = torch.randint(0, V, (n_query,), generator=g).cuda()
    order = [docs[i] for i in torch.randperm(n_docs, generator=torch.Generator().manual_seed(2)).tolist()]
    per_token = 2 * cfg.num_hidden_layers * cfg.num_key_value_heads * cfg.head_dim * 2
    store = BlockStore(per_token * (n_sys + gpu_docs * doc_len), 1 << 40)
    store.event_timing = True
    rec = {"sched": [], "layers": []}
    orig_copy, orig_ensure = _hip.copy_layers, E._Assembly.ensure

    def copy_layers(dsts, srcs, stream, groups, events):
        rec["sched"].append((groups, events, time.perf_counter(), len(dsts)))
        return orig_copy(dsts, srcs, stream, groups, events)

    def ensure(self, l):
        if self.done[l]:
            return
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        orig_ensure(self, l)
        b.record()
        rec["layers"].append((l, a, b))

    _hip.copy_layers, E._Assembly.ensure = copy_layers, ensure
    try:
        with torch.inference_mode():
            eng = Engine(model, store, graphs=True)
            eng.prefill(system, docs, query)
            for _ in range(2):
                eng.prefill(system, order, query, ratio=ratio)
            for it in range(iters):
                rec["sched"], rec["layers"] = [], []
                torch.cuda.synchronize()
                t0 = torch.cuda.Event(enable_timing=True)
                t0.record()
                h0 = time.perf_counter()
                _, _, st = eng.prefill(system, order, query, ratio=ratio)
                t1 = torch.cuda.Event(enable_timing=True)
                t1.record()
                t1.synchronize()
                print(f"request {it}: TTFT {st.t['ttft'] * 1e3:.2f} ms (stages " +
                      ", ".join(f"{k} {v * 1e3:.2f}" for k, v in st.t.items() if k != "ttft") +
                      f"), GPU span {t0.elapsed_time(t1):.2f} ms, {st.hits} hits")
                for groups, events, hq, n in rec["sched"]:
                    landed = ", ".join(f"{a}-{b - 1}: {t0.elapsed_time(e):.2f}" for (a, b), e in zip(groups, events))
                    print(f"  schedule of {n} tensors queued at host +{(hq - h0) * 1e3:.2f} ms; "
                          f"groups landed (ms): {landed}")
                print("  assembly of layer l (compute stream reaches it at ms, waits + assembles ms): " +
                      ", ".join(f"{l}: {t0.elapsed_time(a):.2f} +{a.elapsed_time(b):.3f}"
                                for l, a, b in rec["layers"]))
    finally:
        _hip.copy_layers, E._Assembly.ensure = orig_copy, orig_ensure


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("kernel", choices=["assemble", "copy", "attention", "tiercopy", "deviation", "skinny", "request",
                                       "tier"])
    ap.add_argument("--workload", default="qwen2.5-7b-32k", choices=list(WORKLOADS))
    ap.add_argument("--shape", default="recompute", choices=["recompute", "prefill", "query"])
    ap.add_argument("--iters", type=int, default=20)
    ap.add_argument("--sdpa", action="store_true", help="attention: also time torch's SDPA on the same inputs")
    ap.add_argument("--libs", default="", help="request: comma-separated builds of libtread_hip.so to compare")
    ap.add_argument("--gpu-docs", type=int, default=8, help="tier: doc blocks the GPU tier holds")
    args = ap.parse_args(argv)
    name, n_docs, doc_len, n_sys, n_query = WORKLOADS[args.workload]
    cfg = preset(name)
    torch.manual_seed(0)
    if args.kernel == "assemble":
        bench_assemble(cfg, n_docs, doc_len, n_sys, n_query, args.iters)
    elif args.kernel == "copy":
        bench_copy(cfg, n_docs, doc_len, n_sys, n_query, args.iters)
    elif args.kernel == "tiercopy":
        bench_tiercopy(cfg, n_docs, doc_len, n_sys, n_query, min(args.iters, 5))
    elif args.kernel == "skinny":
        bench_skinny(cfg, args.iters)
    elif args.kernel == "deviation":
        bench_deviation(cfg, n_docs, doc_len, n_sys, n_query, args.iters)
    elif args.kernel == "tier":
        bench_tier(cfg, name, n_docs, doc_len, n_sys, n_query, min(args.iters, 5), args.gpu_docs)
    elif args.kernel == "request":
        libs = [p for p in args.libs.split(",") if p] or [str(_hip.LIB_PATH)]
        bench_request(cfg, name, n_docs, doc_len, n_sys, n_query, args.iters, libs)
    else:
        bench_attention(cfg, n_docs, doc_len, n_sys, n_query, args.iters, args.shape, sdpa=args.sdpa)
    return 0


if __name__ == "__main__":
    sys.exit(main())
