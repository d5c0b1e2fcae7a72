"""The HIP engine against the oracle on the reference's own workloads, at their real shapes.

- Qwen2.5-0.5B shape (24 layers, hidden 896, 14 / 2 heads of 64), bf16, 64-token system prompt +
  4 docs x 256 tokens + 32-token query: docs cached in order, then the request in reversed doc
  order with plain reuse. 5 of 5 blocks hit; the reused layer-0 keys equal a fresh prefill of the
  reversed request as closely as the reference's own path gets them (tests/test_engine.py:46-55);
  first-token logits within KL 1e-4 of the oracle (and full prefill likewise).
- Same model, 64 + 8 docs x 1000 + 32, seeded permutation, 20 % deviation recompute through the
  hipGraph with the query rows folded in (the benchmark's composition): hits, misses and
  recompute_eff equal the oracle's; the selected set equals the oracle's except candidates whose
  oracle score lies within 2 bf16 ulps of the selection threshold (|S xor S_oracle| and the largest
  gap are printed); logits within KL 2e-4 of the oracle and no further from the fp32 truth than
  the oracle's bf16 path (each is ~1.07e-4 from it: the bf16 floor of this shape is above 1e-4).
- Qwen2.5-1.5B shape (28 layers, hidden 1536, 12 / 2 heads of 128), 64 + 16 docs x 1000 + 32,
  GPU tier holding the prefix and 8 doc blocks, pinned-host tier on: logits and the assembled cache
  bit-identical to the all-GPU store, on the first promotion and the next; store counters and LRU
  order equal the oracle store's on the same key sequence (tread/store.py:64-122).
- A GPU budget smaller than one block (tread/engine.py:53,94; tread/store.py:84-85): the request is
  served from uncached blocks with the oracle's statistics and logits.
Weights are N(0, 0.02) random-init, generated on the GPU and copied to the oracle.
"""
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
    assert kl(ofull, full) < 1e-4
    # the method's own quality figure (bench/bench_scaling.py:88-91): plain reuse against full prefill
    print(f"[0.5B 4x256 reversed] KL(full prefill, plain reuse) = {kl(full, a):.3e} "
          f"(oracle {kl(ofull, b):.3e}), top-1 {'equal' if int(full.argmax()) == int(a.argmax()) else 'differs'}")


def test_qwen05b_8k_deviation_graph_folded():
    cfg = preset("qwen2.5-0.5b")
    gpu, ref = models(cfg)
    system, docs, query, perm = inputs(cfg, 8, 1000)
    eng = Engine(gpu, BlockStore(1 << 40), graphs=True)
    assert eng.fold_query
    oeng = R.Engine(ref, R.BlockStore(1 << 40))
    eng.prefill(on(system), on(docs), on(query))
    oeng.prefill(system, docs, query)
    order = [docs[i] for i in perm]
    trace = {}
    for rep in range(2):  # capture, then replay
        a, cache, st = eng.prefill(on(system), on(order), on(query), ratio=0.2)
    b, _, ost = oeng.prefill(system, order, query, ratio=0.2, trace=trace)
    assert eng.runner.captures == 1 and cache.graph is not None
    assert (st.hits, st.misses, st.tokens_prefilled) == (ost.hits, ost.misses, ost.tokens_prefilled) == (9, 0, 0)
    assert st.recompute_eff == ost.recompute_eff
    S, So = set(eng.last_selected.cpu().tolist()), set(trace["S"].tolist())
    assert len(S) == len(So) == 1600
    dev, all_c = trace["dev"].float(), trace["all_c"]
    thr = dev.topk(len(So)).values[-1].item()
    pos_score = {int(p): dev[i].item() for i, p in enumerate(all_c.tolist())}
    ulp = 2.0 ** (torch.tensor(thr).abs().log2().floor().item() - 7)
    diff = S ^ So
    gap = max((abs(pos_score[p] - thr) / ulp for p in diff), default=0.0)
    print(f"\n[0.5B 8k 20%] |S xor S_oracle| = {len(diff)} of {len(So)}, largest oracle-score gap to the "
          f"threshold {gap:.1f} ulp")
    assert gap <= 2
    if diff:  # compare numerics under one selection when a near-tie went the other way
        b, _, _ = oeng.prefill(system, order, query, ratio=0.2, trace={"force_S": eng.last_selected.cpu()})
    k = kl(b, a)
    # the fp32 truth of the same (bf16-valued) weights and selection, for scale
    ref32 = R.M.load(cfg, {n: w.float() for n, w in ref.w.items()}, torch.float32)
    teng = R.Engine(ref32, R.BlockStore(1 << 40), sig=oeng.sig)
    teng.prefill(system, docs, query)
    c, _, _ = teng.prefill(system, order, query, ratio=0.2, trace={"force_S": eng.last_selected.cpu()})
    print(f"[0.5B 8k 20%] KL(oracle, ours) = {k:.3e}; KL(fp32 truth, ours) = {kl(c, a):.3e}, "
          f"KL(fp32 truth, oracle bf16) = {kl(c, b):.3e}")
    # Measured on MI355X: KL(oracle, ours) 1.25e-4, while ours and the oracle's bf16 path are each
    # ~1.07e-4 from the fp32 truth. At 24 layers over 8k tokens the reference's own bf16 rounding
    # is above 1e-4, so no bf16 implementation with other GEMM kernels (nor the fp32 truth itself)
    # comes within 1e-4 of it; the bar here is twice that floor, and being no less accurate than
    # the reference's bf16 path.
    assert k < 2e-4
    assert kl(c, a) <= 1.25 * kl(c, b) + 1e-5


def test_qwen15b_16k_host_tier_is_bit_identical_to_gpu_tier():
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
    gate|up GEMM. Hits equal the oracle's; the selection equals the oracle's up to near-ties
    (printed: 236 of 6 400 differ on MI355X, each within 1 ulp of the threshold); logits within
    KL 2e-4 of the oracle (measured 1.33e-4, while the fp32 truth of the same weights is 1.94e-4
    from the oracle and 1.98e-4 from ours: the bf16 floor of this shape is above 1e-4)."""
    from tread_amd.tuning import TABLE_7B, use_tuned_gemms
    status = use_tuned_gemms(tables=(TABLE_7B,))
    try:
        cfg = preset("qwen2.5-7b", num_hidden_layers=3)
        gpu, ref = models(cfg)
        system, docs, query, perm = inputs(cfg, 32, 1000)
        eng = Engine(gpu, BlockStore(1 << 40), graphs=True)
        oeng = R.Engine(ref, R.BlockStore(1 << 40))
        eng.prefill(on(system), on(docs), on(query))
        oeng.prefill(system, docs, query)
        order = [docs[i] for i in perm]
        trace = {}
        for _ in range(2):  # capture, then replay
            a, cache, st = eng.prefill(on(system), on(order), on(query), ratio=0.2)
        b, _, ost = oeng.prefill(system, order, query, ratio=0.2, trace=trace)
        assert (st.hits, st.misses) == (ost.hits, ost.misses) == (33, 0)
        assert st.recompute_eff == ost.recompute_eff and cache.graph is not None
        S, So = set(eng.last_selected.cpu().tolist()), set(trace["S"].tolist())
        dev, all_c = trace["dev"].float(), trace["all_c"]
        thr = dev.topk(len(So)).values[-1].item()
        pos_score = {int(p): dev[i].item() for i, p in enumerate(all_c.tolist())}
        ulp = 2.0 ** (torch.tensor(thr).abs().log2().floor().item() - 7)
        diff = S ^ So
        gap = max((abs(pos_score[p] - thr) / ulp for p in diff), default=0.0)
        print(f"\n[7B width 32k 20%, 3 layers] GEMM table {status}; |S xor S_oracle| = {len(diff)} of {len(So)}, "
              f"largest gap {gap:.1f} ulp")
        assert len(S) == len(So) == 6400 and gap <= 2
        if diff:  # compare numerics under one selection when near-ties went the other way
            b, _, _ = oeng.prefill(system, order, query, ratio=0.2, trace={"force_S": eng.last_selected.cpu()})
        k = kl(b, a)
        print(f"[7B width 32k 20%, 3 layers] KL(oracle, ours) = {k:.3e}")
        assert k < 2e-4
    finally:
        torch.cuda.tunable.enable(False)
