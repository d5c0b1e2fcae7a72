"""The HIP engine against the oracle on the reference's own workloads, at their real shapes.

Two oracle backends: the oracle's torch code on the CPU (its home) and the same code run a second
time on the MI355X (hipBLASLt GEMMs, torch's memory-efficient attention kernel: the reference's own
path as it runs on a GPU). Measured on MI355X, the two backends of the reference's path are
themselves KL 1.3e-4 apart at the 0.5B 8k request and 4.8e-4 at the 1.5B 16k one (7.9e-5 at the
7B width with 3 layers), and each is 1e-4 to 5e-4 from the fp32 truth of the same weights: a KL
of 1e-4 to the reference is below what the reference reproduces across its own backends, so no
bf16 implementation with other kernels can be held to it. The logits bars, on one selection:
- KL(oracle on either backend, ours) <= max(1e-4, 2 x KL(oracle CPU, oracle GPU)): within twice
  the reference's own cross-backend distance (measured: 0.90-1.89x);
- KL(fp32 truth, ours) <= 1.25 x min(KL(fp32 truth, oracle CPU), KL(fp32 truth, oracle GPU)) +
  1e-5: about as accurate as the reference's bf16 path (measured: 0.96-1.24x of the oracle's);
- where only the GPU backend runs (the 70B width), KL(oracle GPU, ours) <= 0.5 x KL(fp32 truth,
  oracle GPU): ours differs from the reference by less than half the reference's own bf16 error
  (measured 0.26x).
Selections: equal to each oracle's except candidates whose oracle score lies within 2 bf16 ulps
of its selection threshold (printed: how many differ and the largest gap).

- Qwen2.5-0.5B shape (24 layers, hidden 896, 14 / 2 heads of 64), bf16, 64-token system prompt +
  4 docs x 256 tokens + 32-token query: docs cached in order, then the request in reversed doc
  order with plain reuse. 5 of 5 blocks hit; the reused layer-0 keys equal a fresh prefill of the
  reversed request as closely as the reference's own path gets them (tests/test_engine.py:46-55);
  first-token logits within KL 1e-4 of the oracle; the full prefill of the same request meets the
  bars below against both oracle backends.
- Same model, 64 + 8 docs x 1000 + 32, seeded permutation, 20 % deviation recompute through the
  hipGraph with the query rows folded in (the benchmark's composition).
- Qwen2.5-1.5B shape (28 layers, hidden 1536, 12 / 2 heads of 128), 64 + 16 docs x 1000 + 32,
  GPU tier holding the prefix and 8 doc blocks, pinned-host tier on: logits and the assembled cache
  bit-identical to the all-GPU store, on the first promotion and the next; store counters and LRU
  order equal the oracle store's on the same key sequence (tread/store.py:64-122); hits, selection
  and logits of the whole request against both oracle backends.
- The Qwen2.5-7B and Llama-3-70B widths over the full 64 + 32 x 1000 + 32 request, with few layers
  so that the oracle finishes (the 70B one with 8 cold docs packed into the request).
- A GPU budget smaller than one block (tread/engine.py:53,94; tread/store.py:84-85): the request is
  served from uncached blocks with the oracle's statistics and logits.
Weights are N(0, 0.02) random-init, generated on the GPU and copied to the oracle.
"""
import math

import pytest
import torch

from oracle import tread_ref as R
from tread_amd import BlockStore, Engine, prefill_full
from tread_amd.model import DecoderLM, ModelConfig, preset, synthetic_model
from tread_amd.store import block_key

pytestmark = pytest.mark.gpu
DEV = "cuda"


def kl(a, b):
    return R.kl(a.float().cpu(), b.float().cpu())


def models(cfg, std=0.02):
    gpu = synthetic_model(cfg, DEV, torch.bfloat16, seed=0, std=std)
    ref = R.M.load(cfg, gpu.state_dict(), torch.bfloat16)
    return gpu, ref


def inputs(cfg, n_docs, doc_len, n_sys=64, n_query=32):
    g = torch.Generator().manual_seed(1)
    V = cfg.vocab_size
    system = torch.randint(0, V, (n_sys,), generator=g)
    docs = [torch.randint(0, V, (doc_len,), generator=g) for _ in range(n_docs)]
    query = torch.randint(0, V, (n_query,), generator=g)
    perm = torch.randperm(n_docs, generator=torch.Generator().manual_seed(2)).tolist()
    return system, docs, query, perm


def on(x):
    return [t.to(DEV) for t in x] if isinstance(x, list) else x.to(DEV)


class Oracle:
    """The oracle engine on `device` with its store primed: the prefix and `warm` docs cached by
    one request (the packed cold prefill of tread/engine.py:59-96), or by one request per doc
    (`per_doc`: the same blocks up to rounding, without the dense [n, P + n] mask over every doc,
    which on the CPU costs as much as the rest of the test)."""

    def __init__(self, name, m, sig, system, warm, query, device="cpu", per_doc=False):
        self.name, self.m, self.dev = name, m, device
        self.eng = R.Engine(m, R.BlockStore(1 << 40), sig=sig)
        self.system, self.query = system.to(device), query.to(device)
        for group in ([[d] for d in warm] if per_doc else [warm]):
            self.eng.prefill(self.system, [d.to(device) for d in group], self.query)
        self.seen = []  # (selection, logits, cache) of the requests run so far

    def request(self, order, ratio, force_S=None):
        """(logits, stats, trace) of the request; `force_S` replaces the deviation top-k."""
        trace = {} if force_S is None else {"force_S": force_S}
        logits, cache, st = self.eng.prefill(self.system, [d.to(self.dev) for d in order], self.query, ratio=ratio,
                                             trace=trace)
        self.seen.append((trace["S"].cpu(), logits, cache))
        return logits, st, trace

    def _at(self, order, ratio, S):
        for seen in self.seen:
            if torch.equal(seen[0], S.cpu()):
                return seen
        self.request(order, ratio, force_S=S.cpu())
        return self.seen[-1]

    def at(self, order, ratio, S):
        """Logits of the request at the selection S (positions), run again only if no request so far
        selected exactly S."""
        return self._at(order, ratio, S)[1]

    def decode(self, order, ratio, S, toks):
        """Per-step logits of the reference server's greedy loop (tread/server.py:194-210) after the
        request at selection S, fed the tokens `toks`: [prompt logits, then one per token]."""
        _, logits, (K, V) = self._at(order, ratio, S)
        out, _, steps = R.generate_greedy(self.m, logits, list(K), list(V), len(toks), forced=toks)
        assert out == toks
        return steps


def fp32(cfg, gpu_model, device=DEV):
    """The fp32 truth of the same (bf16-valued) weights: the oracle's model in fp32."""
    return R.M.load(cfg, {n: w.float() for n, w in gpu_model.state_dict().items()}, torch.float32, device=device)


def selection_gap(S, trace):
    """Positions selected by exactly one of S (ours) and the oracle's trace, and the largest gap
    between such a position's oracle score and the oracle's selection threshold, in bf16 ulps of
    the threshold."""
    So = set(trace["S"].cpu().tolist())
    dev, all_c = trace["dev"].float().cpu(), trace["all_c"].cpu()
    thr = dev.topk(len(So)).values[-1].item()
    score = dict(zip(all_c.tolist(), dev.tolist()))
    ulp = 2.0 ** (math.floor(math.log2(abs(thr))) - 7)
    diff = set(S.cpu().tolist()) ^ So
    return diff, max((abs(score[p] - thr) / ulp for p in diff), default=0.0)


def check_selection(tag, S, *oracle_traces):
    for name, trace in oracle_traces:
        diff, gap = selection_gap(S, trace)
        print(f"[{tag}] |S xor S_{name}| = {len(diff)} of {len(trace['S'])}, largest gap to its threshold "
              f"{gap:.1f} ulp")
        assert len(trace["S"]) == len(S) and gap <= 2, (name, len(diff), gap)


def bars(tag, a, b, bg, c):
    """The logits bars of this module's docstring: ours a, oracle CPU b (or None), oracle GPU bg,
    fp32 truth c."""
    k_g = kl(bg, a)
    t_ours, t_g = kl(c, a), kl(c, bg)
    msg = f"[{tag}] KL(oracle GPU, ours) = {k_g:.3e}"
    if b is not None:
        k_c, k_cg, t_c = kl(b, a), kl(b, bg), kl(c, b)
        msg += f"; KL(oracle CPU, ours) = {k_c:.3e}, KL(oracle CPU, oracle GPU) = {k_cg:.3e}"
    msg += f"; from the fp32 truth: ours {t_ours:.3e}, oracle GPU {t_g:.3e}"
    if b is not None:
        msg += f", oracle CPU {t_c:.3e}"
    print(msg)
    if b is not None:
        floor = max(1e-4, 2 * k_cg)
        assert k_g <= floor and k_c <= floor, (k_g, k_c, floor)
        assert t_ours <= 1.25 * min(t_c, t_g) + 1e-5, (t_ours, t_c, t_g)
    else:
        assert k_g <= 0.5 * t_g, (k_g, t_g)
        assert t_ours <= 1.25 * t_g + 1e-5, (t_ours, t_g)


def check_logits(tag, a, S, order, ratio, cpu, gpu, truth):
    """The bars at our selection S."""
    bars(tag, a, cpu.at(order, ratio, S) if cpu is not None else None, gpu.at(order, ratio, S),
         truth.at(order, ratio, S))


def test_qwen05b_4x256_reversed_plain_reuse():
    cfg = preset("qwen2.5-0.5b")
    gpu, ref = models(cfg)
    system, docs, query, _ = inputs(cfg, 4, 256)
    eng = Engine(gpu, BlockStore(1 << 40))
    oeng = R.Engine(ref, R.BlockStore(1 << 40))
    eng.prefill(on(system), on(docs), on(query))
    oeng.prefill(system, docs, query)
    rev = docs[::-1]
    a, cache, st = eng.prefill(on(system), on(rev), on(query))
    b, (oK, _), ost = oeng.prefill(system, rev, query)
    want = (5, 0, 64 + 4 * 256, 0)
    assert (st.hits, st.misses, st.tokens_reused, st.tokens_prefilled) == want
    assert (ost.hits, ost.misses, ost.tokens_reused, ost.tokens_prefilled) == want
    assert list(eng.store.blocks) == list(oeng.store.blocks)
    k = kl(b, a)
    print(f"\n[0.5B 4x256 reversed] KL(oracle, ours) = {k:.3e}")
    assert k < 1e-4
    # layer 0 is context-free: the reused (re-rotated) layer-0 keys match a fresh prefill of the
    # reversed request. Ours must be no further from it than the reference's own bf16 path.
    T = 64 + 4 * 256
    full, fcache, _ = prefill_full(gpu, on(system), on(rev), on(query))
    ofull, (ofK, _), _ = R.prefill_full(ref, system, rev, query)
    ours = (cache.K[0, :, :, :T].float().cpu() - fcache.K[0, :, :, :T].float().cpu()).norm()
    theirs = (oK[0][:, :, :T].float() - ofK[0][:, :, :T].float()).norm()
    scale = ofK[0][:, :, :T].float().norm()
    print(f"[0.5B 4x256 reversed] layer-0 |reused - fresh| / |fresh|: ours {ours / scale:.3e}, "
          f"reference path {theirs / scale:.3e}")
    assert ours <= 1.1 * theirs + 1e-3 * scale
    # the full prefill of the reversed request against both oracle backends and the fp32 truth
    gfull, _, _ = R.prefill_full(R.M.load(cfg, gpu.state_dict(), torch.bfloat16, device=DEV), on(system), on(rev),
                                 on(query))
    tfull, _, _ = R.prefill_full(fp32(cfg, gpu), on(system), on(rev), on(query))
    bars("0.5B 4x256 reversed, full prefill", full, ofull, gfull, tfull)
    # the method's own quality figure (bench/bench_scaling.py:88-91): plain reuse against full prefill
    print(f"[0.5B 4x256 reversed] KL(full prefill, plain reuse) = {kl(full, a):.3e} "
          f"(oracle {kl(ofull, b):.3e}), top-1 {'equal' if int(full.argmax()) == int(a.argmax()) else 'differs'}")


def test_qwen05b_8k_deviation_graph_folded():
    """0.5B, 64 + 8 x 1000 + 32, 20 % deviation recompute through the hipGraph with the query rows
    folded in (the benchmark's composition): hits, misses and recompute_eff equal the oracle's
    (both backends); selections and logits meet the module's bars."""
    cfg = preset("qwen2.5-0.5b")
    gpu, ref = models(cfg)
    system, docs, query, perm = inputs(cfg, 8, 1000)
    eng = Engine(gpu, BlockStore(1 << 40), graphs=True)
    assert eng.fold_query
    eng.prefill(on(system), on(docs), on(query))
    order = [docs[i] for i in perm]
    for rep in range(2):  # capture, then replay
        a, cache, st = eng.prefill(on(system), on(order), on(query), ratio=0.2)
    assert eng.runner.captures == 1 and cache.graph is not None
    S = eng.last_selected
    sig = R.sig_of(cfg, torch.bfloat16)
    cpu = Oracle("CPU", ref, sig, system, docs, query)
    gref = R.M.load(cfg, gpu.state_dict(), torch.bfloat16, device=DEV)
    gorc = Oracle("GPU", gref, sig, system, docs, query, device=DEV)
    _, ost, trace = cpu.request(order, 0.2)
    _, gst, gtrace = gorc.request(order, 0.2)
    for o in (ost, gst):
        assert (st.hits, st.misses, st.tokens_prefilled) == (o.hits, o.misses, o.tokens_prefilled) == (9, 0, 0)
        assert st.recompute_eff == o.recompute_eff
    assert len(S) == 1600
    check_selection("0.5B 8k 20%", S, ("oracle CPU", trace), ("oracle GPU", gtrace))
    truth = Oracle("fp32", fp32(cfg, gpu), None, system, docs, query, device=DEV)
    check_logits("0.5B 8k 20%", a, S, order, 0.2, cpu, gorc, truth)


def test_qwen15b_16k_host_tier_is_bit_identical_to_gpu_tier():
    """1.5B, 64 + 16 x 1000 + 32 at 20 %, with half the doc blocks in the pinned-host tier: bit
    identity with the all-GPU store over two promotions, the oracle store's counters and LRUs on the
    same key sequence, and the request's hits, selection and logits against both oracle backends
    (tread/store.py:73-77; tread/blend.py:117-179)."""
    cfg = preset("qwen2.5-1.5b")
    gpu = synthetic_model(cfg, DEV, torch.bfloat16, seed=0)
    system, docs, query, perm = inputs(cfg, 16, 1000)
    L, kv, hd = cfg.num_hidden_layers, cfg.num_key_value_heads, cfg.head_dim
    per_token = 2 * L * kv * hd * 2
    budget = per_token * (64 + 8 * 1000)
    tiered = Engine(gpu, BlockStore(budget, 1 << 40), graphs=True)
    flat = Engine(gpu, BlockStore(1 << 40), graphs=True)
    order = [docs[i] for i in perm]
    for eng in (tiered, flat):
        eng.prefill(on(system), on(docs), on(query))
    for rnd in range(2):
        h0 = tiered.store.stats.cpu_hits
        a, ca, sa = tiered.prefill(on(system), on(order), on(query), ratio=0.2)
        Ka, Va = ca.K[..., :ca.length, :].clone(), ca.V[..., :ca.length, :].clone()
        b, cb, sb = flat.prefill(on(system), on(order), on(query), ratio=0.2)
        assert sa.misses == sb.misses == 0 and tiered.store.stats.cpu_hits - h0 >= 8
        assert torch.equal(a, b), rnd
        assert torch.equal(Ka, cb.K[..., :cb.length, :]) and torch.equal(Va, cb.V[..., :cb.length, :]), rnd
        assert torch.equal(tiered.last_selected, flat.last_selected)
    # the oracle store on the same key sequence: every counter of tread/store.py:44-53, both LRUs
    ostore = R.BlockStore(budget, 1 << 40)
    sig = tiered.sig
    pkey = R.block_key(*sig, "", "prefix", system)
    dkeys = [R.block_key(*sig, pkey, d) for d in docs]
    meta = lambda n: torch.empty(L, 1, kv, n, hd, dtype=torch.bfloat16, device="meta")
    assert ostore.get(pkey) is None
    ostore.put(pkey, meta(64), meta(64), 0)
    assert all(ostore.get(k) is None for k in dkeys)
    for k in dkeys:
        ostore.put(k, meta(1000), meta(1000), 64)
    for _ in range(2):
        ostore.get(pkey)
        for i in perm:
            assert ostore.get(dkeys[i]) is not None
    ours = vars(tiered.store.stats)
    assert {f: ours[f] for f in vars(ostore.stats)} == vars(ostore.stats)
    assert list(tiered.store.blocks) == list(ostore.blocks)
    assert list(tiered.store.cpu_blocks) == list(ostore.cpu_blocks)
    assert pkey == block_key(*sig, "", "prefix", system)
    # the whole request through both oracle backends
    S = tiered.last_selected
    osig = R.sig_of(cfg, torch.bfloat16)
    cpu = Oracle("CPU", R.M.load(cfg, gpu.state_dict(), torch.bfloat16), osig, system, docs, query, per_doc=True)
    gorc = Oracle("GPU", R.M.load(cfg, gpu.state_dict(), torch.bfloat16, device=DEV), osig, system, docs, query,
                  device=DEV)
    _, ost, trace = cpu.request(order, 0.2)
    _, gst, gtrace = gorc.request(order, 0.2)
    for o in (ost, gst):
        assert (sa.hits, sa.misses, sa.tokens_reused) == (o.hits, o.misses, o.tokens_reused) == (17, 0, 16064)
        assert sa.recompute_eff == o.recompute_eff
    assert len(S) == 3200
    check_selection("1.5B 16k 20%, host tier", S, ("oracle CPU", trace), ("oracle GPU", gtrace))
    truth = Oracle("fp32", fp32(cfg, gpu), None, system, docs, query, device=DEV)
    check_logits("1.5B 16k 20%, host tier", a, S, order, 0.2, cpu, gorc, truth)


SMALL = ModelConfig(512, 256, 4, 8, 2, 128, 512, rope_theta=1000000.0, attention_bias=True)


@pytest.mark.parametrize("prefix_fits", [False, True])
@pytest.mark.parametrize("ratio", [0.0, 0.2])
def test_blocks_larger_than_the_budget_are_served_uncached(prefix_fits, ratio):
    """tread/engine.py:53,94 and tread/store.py:84-85: put() refuses a block above the GPU budget and
    the engine serves it as an uncached _Tmp; every request then misses those blocks again."""
    gpu, ref = models(SMALL, std=0.02)
    g = torch.Generator().manual_seed(4)
    system = torch.randint(0, 512, (16,), generator=g)
    docs = [torch.randint(0, 512, (n,), generator=g) for n in (40, 25, 33)]
    query = torch.randint(0, 512, (7,), generator=g)
    prefix_bytes = 2 * SMALL.num_hidden_layers * SMALL.num_key_value_heads * 16 * SMALL.head_dim * 2
    budget = prefix_bytes if prefix_fits else prefix_bytes - 1
    eng = Engine(gpu, BlockStore(budget))
    oeng = R.Engine(ref, R.BlockStore(budget))
    for rep in range(2):
        order = docs if rep == 0 else docs[::-1]
        a, _, st = eng.prefill(on(system), on(order), on(query), ratio=ratio)
        b, _, ost = oeng.prefill(system, order, query, ratio=ratio)
        assert (st.hits, st.misses, st.tokens_reused, st.tokens_prefilled) == \
               (ost.hits, ost.misses, ost.tokens_reused, ost.tokens_prefilled)
        assert st.misses == len(docs) + (0 if prefix_fits and rep else 1)
        assert eng.store.stats.bytes_used == oeng.store.stats.bytes_used
        assert list(eng.store.blocks) == list(oeng.store.blocks)
        assert kl(b, a) < 1e-4, (rep, kl(b, a))


def test_qwen7b_width_32k_bench_composition():
    """The composition the benchmark times, at the Qwen2.5-7B width (hidden 3584, 28 / 4 heads of
    128, intermediate 18944, vocab 152064) over the full 64 + 32 x 1000 + 32-token request, with 3
    layers so the CPU oracle finishes: committed GEMM solution table on, hipGraph buckets, query
    rows folded into the recompute, the key-half attention of the 6 432 recompute rows, the split
    gate|up GEMM. Hits equal both oracles'; selections and logits meet the module's bars, and so do
    the logits of four decoding steps after the request against each oracle's greedy loop
    (tread/server.py:194-210) fed the same tokens."""
    from tread_amd.tuning import TABLE_7B, use_tuned_gemms
    status = use_tuned_gemms(tables=(TABLE_7B,))
    try:
        cfg = preset("qwen2.5-7b", num_hidden_layers=3)
        gpu, ref = models(cfg)
        system, docs, query, perm = inputs(cfg, 32, 1000)
        eng = Engine(gpu, BlockStore(1 << 40), graphs=True)
        eng.prefill(on(system), on(docs), on(query))
        order = [docs[i] for i in perm]
        for _ in range(2):  # capture, then replay
            a, cache, st = eng.prefill(on(system), on(order), on(query), ratio=0.2)
        assert cache.graph is not None
    finally:
        torch.cuda.tunable.enable(False)
    S = eng.last_selected
    print(f"\n[7B width 32k 20%, 3 layers] GEMM table {status}")
    sig = R.sig_of(cfg, torch.bfloat16)
    cpu = Oracle("CPU", ref, sig, system, docs, query, per_doc=True)
    gorc = Oracle("GPU", R.M.load(cfg, gpu.state_dict(), torch.bfloat16, device=DEV), sig, system, docs, query,
                  device=DEV)
    _, ost, trace = cpu.request(order, 0.2)
    _, gst, gtrace = gorc.request(order, 0.2)
    for o in (ost, gst):
        assert (st.hits, st.misses) == (o.hits, o.misses) == (33, 0)
        assert st.recompute_eff == o.recompute_eff
    assert len(S) == 6400
    check_selection("7B width 32k 20%, 3 layers", S, ("oracle CPU", trace), ("oracle GPU", gtrace))
    truth = Oracle("fp32", fp32(cfg, gpu), None, system, docs, query, device=DEV)
    check_logits("7B width 32k 20%, 3 layers", a, S, order, 0.2, cpu, gorc, truth)
    # decoding steps over the 32 096-row cache (graph-replayed; the decode attention splits each KV
    # head's keys into 63 slices merged by the combine kernel) against each oracle's greedy loop
    toks, ours = [], [a]
    for _ in range(4):
        toks.append(int(ours[-1].argmax()))
        ours.append(eng.decode(cache, torch.tensor([toks[-1]], device=DEV)))
    runs = [o.decode(order, 0.2, S, toks) for o in (cpu, gorc, truth)]
    for i in range(1, len(ours)):
        bars(f"7B width 32k, decode step {i}", ours[i], *(r[i] for r in runs))


def _rel(x, ref):
    return ((x.float() - ref.float()).norm() / ref.float().norm()).item()


def test_llama70b_width_32k_eight_cold_docs_packed_in_the_request():
    """The Llama-3-70B width (hidden 8192, 64 / 8 heads of 128, intermediate 28672, vocab 128256,
    theta 5e5, eps 1e-5, no biases) over the full 64 + 32 x 1000 + 32 request with 2 layers, 24
    docs cached beforehand and 8 cold: their misses go through the packed block-diagonal prefill
    inside the timed request (tread/engine.py:74-95), then 20 % deviation recompute through the
    graph. The oracle runs on the GPU here (at this width its CPU run of the dense-mask prefill and
    the deviation pass would take minutes; the tests above tie its GPU backend to the CPU one):
    stats equal; the 8 new blocks are no further from the fp32 truth's blocks than the oracle's
    bf16 blocks are (tests/test_engine.py:116-129 holds fp32 blocks to atol 1e-3; in bf16 the
    bar is the reference path's own error); selection and logits meet the module's bars."""
    cfg = preset("llama3-70b", num_hidden_layers=2)
    gpu = synthetic_model(cfg, DEV, torch.bfloat16, seed=0)
    system, docs, query, perm = inputs(cfg, 32, 1000)
    warm, cold = docs[:24], docs[24:]
    eng = Engine(gpu, BlockStore(1 << 40), graphs=True)
    eng.prefill(on(system), on(warm), on(query))
    order = [docs[i] for i in perm]
    a, cache, st = eng.prefill(on(system), on(order), on(query), ratio=0.2)
    assert cache.graph is not None
    S = eng.last_selected
    want = (25, 8, 64 + 24 * 1000, 8 * 1000)
    assert (st.hits, st.misses, st.tokens_reused, st.tokens_prefilled) == want
    sig = R.sig_of(cfg, torch.bfloat16)
    gorc = Oracle("GPU", R.M.load(cfg, gpu.state_dict(), torch.bfloat16, device=DEV), sig, system, warm, query,
                  device=DEV)
    truth = Oracle("fp32", fp32(cfg, gpu), sig, system, warm, query, device=DEV)
    _, gst, gtrace = gorc.request(order, 0.2)
    _, tst, _ = truth.request(order, 0.2, force_S=S.cpu())
    for o in (gst, tst):
        assert (o.hits, o.misses, o.tokens_reused, o.tokens_prefilled) == want
        assert st.recompute_eff == o.recompute_eff
    pkey = block_key(*eng.sig, "", "prefix", system)
    assert pkey == R.block_key(*sig, "", "prefix", system)
    worst = {}
    for d in cold:
        key = block_key(*eng.sig, pkey, d)
        ours, theirs, t = eng.store.blocks[key], gorc.eng.store.blocks[key], truth.eng.store.blocks[key]
        assert ours.base == theirs.base == 64 and ours.n_tokens == theirs.n_tokens == 1000
        for l in range(cfg.num_hidden_layers):
            for name in ("K", "V"):
                x, y, z = (getattr(b, name)[l] for b in (ours, theirs, t))
                e_ours, e_orc = _rel(x, z), _rel(y, z)
                worst[(l, name)] = max(worst.get((l, name), (0, 0)), (e_ours, e_orc))
                assert e_ours <= 1.25 * e_orc + 1e-3, (l, name, e_ours, e_orc)
    print("\n[70B width 32k, 8 cold] cold blocks, relative error to the fp32 truth (ours, oracle GPU): " +
          ", ".join(f"L{l} {n} {e[0]:.2e}/{e[1]:.2e}" for (l, n), e in sorted(worst.items())))
    assert len(S) == 6400
    check_selection("70B width 32k 20%, 8 cold", S, ("oracle GPU", gtrace))
    check_logits("70B width 32k 20%, 8 cold", a, S, order, 0.2, None, gorc, truth)
