"""The drop-in boundary on the GPU: the reference's call forms of tread/blend.py's helpers, the
runner argument of blend(), the graph-bucket cache guard, the K-only re-rotation and the end of a
host-tier promotion.

- `_qkv(layer, model, x, pos)` (tread/blend.py:82-90, called as phase0/predictor.py:87 does) gives
  q, k, v equal to the same fused GEMM followed by transformers' apply_rotary_pos_emb in bf16;
- `_layer_subset(layer, model, h, S, K, V, ctx=_subset_ctx(...))` (tread/blend.py:93-114) equals the
  oracle's restatement within the first-token bar, leaves K, V alone unless inplace, and splices
  only the rows S;
- `blend(..., runner=SubsetRunner(model))` (tread/blend.py:170-172) replays the captured graph
  (one capture, reused) and gives the eager blend's selection and cache;
- `SubsetRunner.run(h, S, K, V, start)` in the reference's call form (tread/graphs.py:75-99)
  equals the eager layer loop;
- a cache that aliases a graph bucket raises once the next request claims the bucket, and a
  detached copy keeps its rows;
- rotate_keys moves K only and equals the K of the fused assemble launch;
- blocks promoted from the host tier stop being pending once their copies have landed, so the next
  request assembles them in the single fused launch.
"""
import pytest
import torch

from oracle import model_ref as M
from oracle import tread_ref as R
from tread_amd import BlockStore, Engine, KVCache, StaleCacheError
from tread_amd import _hip
from tread_amd.blend import _layer_subset, _qkv, _subset_ctx, blend, prefill_kv, rotate_keys
from tread_amd.graphs import SubsetRunner
from tread_amd.model import DecoderLM, ModelConfig, synthetic_model

pytestmark = pytest.mark.gpu
DEV = "cuda"
CFG = ModelConfig(512, 256, 4, 8, 2, 128, 512, rope_theta=1000000.0, attention_bias=True)


def kl(a, b):
    return R.kl(a.float().cpu(), b.float().cpu())


@pytest.fixture(scope="module")
def models():
    cpu = synthetic_model(CFG, "cpu", torch.bfloat16, seed=0, std=0.02, bias_std=0.05)
    sd = cpu.state_dict()
    gpu = DecoderLM(CFG, DEV, torch.bfloat16)
    gpu.load_state_dict(sd)
    return gpu, R.M.load(CFG, sd, torch.bfloat16)


def _request(seed, n_docs=4, n=60):
    g = torch.Generator().manual_seed(seed)
    prefix = torch.randint(0, CFG.vocab_size, (16,), generator=g)
    docs = [torch.randint(0, CFG.vocab_size, (n + 7 * i,), generator=g) for i in range(n_docs)]
    query = torch.randint(0, CFG.vocab_size, (9,), generator=g)
    return prefix, docs, query


def test_qkv_reference_call_form(models):
    gpu, _ = models
    layer = gpu.model.layers[2]
    g = torch.Generator(device=DEV).manual_seed(1)
    h = torch.randn(1, 37, CFG.hidden_size, device=DEV, dtype=torch.bfloat16, generator=g)
    pos = torch.arange(100, 137, device=DEV)
    x = layer.input_layernorm(h)
    q, k, v = _qkv(layer, gpu, x, pos)
    hq, hkv, hd = CFG.num_attention_heads, CFG.num_key_value_heads, CFG.head_dim
    assert q.shape == (1, hq, 37, hd) and k.shape == v.shape == (1, hkv, 37, hd)
    # the same fused GEMM, then the reference's op sequence (view, transpose, apply_rotary_pos_emb)
    at = layer.self_attn
    qkv = torch.nn.functional.linear(x[0], at.qkv_weight, at.qkv_bias)
    qr = qkv[:, :hq * hd].reshape(1, 37, hq, hd).transpose(1, 2)
    kr = qkv[:, hq * hd:(hq + hkv) * hd].reshape(1, 37, hkv, hd).transpose(1, 2)
    vr = qkv[:, (hq + hkv) * hd:].reshape(1, 37, hkv, hd).transpose(1, 2)
    cos, sin = gpu.model.rotary_emb(vr, pos[None])
    assert torch.equal(q, M.apply_rope(qr, cos, sin)) and torch.equal(k, M.apply_rope(kr, cos, sin))
    assert torch.equal(v, vr)
    # phase0/predictor.py:87: _qkv(layer, model, layer.input_layernorm(hidden[:, -1:]), pos)[0]
    q1 = _qkv(layer, gpu, layer.input_layernorm(h[:, -1:]), pos[-1:])[0]
    assert q1.shape == (1, hq, 1, hd) and torch.equal(q1, q[:, :, -1:])
    # rope passed in, as _layer_subset does with its context
    ctx = _subset_ctx(gpu, pos, 200, h)
    q2, k2, v2 = _qkv(layer, gpu, x, pos, ctx[0])
    assert torch.equal(q2, q) and torch.equal(k2, k) and torch.equal(v2, v)
    rope, mask = ctx
    assert mask.shape == (1, 1, 37, 200) and mask.dtype == torch.bool
    assert torch.equal(mask[0, 0], torch.arange(200, device=DEV)[None] <= pos[:, None])
    assert torch.equal(rope[0], cos) and torch.equal(rope[1], sin)


def test_layer_subset_reference_call_form(models):
    gpu, ref = models
    l = 1
    layer = gpu.model.layers[l]
    T = 300
    g = torch.Generator().manual_seed(2)
    S = torch.sort(torch.randperm(T, generator=g)[:40]).values
    h = (torch.randn(1, 40, CFG.hidden_size, generator=g) * 0.5).to(torch.bfloat16)
    K = torch.randn(1, CFG.num_key_value_heads, T, CFG.head_dim, generator=g).to(torch.bfloat16)
    V = torch.randn_like(K)
    Kg, Vg = K.to(DEV), V.to(DEV)
    ctx = _subset_ctx(gpu, S.to(DEV), T, h.to(DEV))
    h2, K2, V2 = _layer_subset(layer, gpu, h.to(DEV), S.to(DEV), Kg, Vg, inplace=False, ctx=ctx)
    assert torch.equal(Kg.cpu(), K) and torch.equal(Vg.cpu(), V)  # not inplace: inputs untouched
    keep = torch.ones(T, dtype=torch.bool)
    keep[S] = False
    assert torch.equal(K2.cpu()[:, :, keep], K[:, :, keep]) and torch.equal(V2.cpu()[:, :, keep], V[:, :, keep])
    ho, Ko, Vo = R.layer_subset(ref, l, h, S, K, V, inplace=False)
    err = (h2.float().cpu() - ho.float()).norm() / (ho.float() - h.float()).norm()
    assert err.item() < 2e-2, err.item()
    kerr = (K2.float().cpu()[:, :, S] - Ko.float()[:, :, S]).abs().max().item()
    assert kerr <= 2 ** -6 * Ko.float()[:, :, S].abs().max().item() + 1e-3, kerr
    # inplace splices into the caller's tensors; no ctx builds its own
    h3, K3, V3 = _layer_subset(l, gpu, h.to(DEV), S.to(DEV), Kg, Vg, inplace=True)
    assert K3 is Kg and torch.equal(Kg, K2) and torch.equal(h3, h2)


@pytest.mark.parametrize("policy,ratio", [("deviation", 0.2), ("boundary", 0.3)])
def test_blend_uses_the_runner(models, policy, ratio):
    gpu, _ = models
    prefix, docs, _ = _request(3)
    Ks, Vs = prefill_kv(gpu, torch.cat([prefix] + docs).to(DEV))
    ctx = torch.cat([prefix] + docs).to(DEV)
    cands, off = [], len(prefix)
    for d in docs:
        cands.append(torch.arange(off, off + len(d), device=DEV))
        off += len(d)
    Ke, Ve, Se, eff_e = blend(gpu, ctx, Ks, Vs, cands, ratio, policy)
    runner = SubsetRunner(gpu)
    for rep in range(2):
        Kr, Vr, Sr, eff_r = blend(gpu, ctx, Ks, Vs, cands, ratio, policy, runner=runner)
        assert runner.captures == 1, rep
        assert torch.equal(Sr, Se) and eff_r == eff_e
        for a, b in zip(Kr + Vr, Ke + Ve):
            assert ((a.float() - b.float()).norm() / b.float().norm()).item() < 1e-2
    assert all(torch.equal(k, k0) for k, k0 in zip(Ks, prefill_kv(gpu, ctx)[0]))  # not inplace


def test_runner_run_reference_call_form(models):
    """SubsetRunner.run(h, S, K, V, start) -> (h, K list, V list) as tread/graphs.py:75-99 defines it
    and tread/blend.py:170-172 calls it: layers start..L-1 of the sorted positions S replayed from
    one capture (reused by a second call of the same bucket), equal to the eager loop of
    _layer_subset over the same layers up to bf16 rounding (the hidden rows after the last layer
    included), K/V views of the bucket that change exactly the rows S; max_ctx defaults to the
    reference's 2048."""
    gpu, _ = models
    prefix, docs, _ = _request(5)
    ids = torch.cat([prefix] + docs).to(DEV)
    T = len(ids)
    Ks, Vs = prefill_kv(gpu, ids)
    g = torch.Generator().manual_seed(3)
    runner = SubsetRunner(gpu)
    assert runner.max_ctx == 2048 and runner.worth_it(T)
    for rep, start in enumerate((1, 1, 0)):
        S = torch.randperm(T - 16, generator=g)[:37].sort().values.to(DEV) + 16
        h = torch.randn(1, len(S), CFG.hidden_size, generator=g).to(DEV, torch.bfloat16)
        Kin, Vin = [k.clone() for k in Ks[start:]], [v.clone() for v in Vs[start:]]
        h_r, K_r, V_r = runner.run(h, S, Kin, Vin, start)
        assert runner.captures == (1 if rep < 2 else 2), rep
        assert h_r.shape == h.shape and len(K_r) == len(V_r) == CFG.num_hidden_layers - start
        assert all(torch.equal(a, b) for a, b in zip(Kin, Ks[start:]))  # the inputs are copied, not written
        ctx = _subset_ctx(gpu, S, T, h)
        he, Ke, Ve = h, [k.clone() for k in Ks[start:]], [v.clone() for v in Vs[start:]]
        for i, l in enumerate(range(start, CFG.num_hidden_layers)):
            he, Ke[i], Ve[i] = _layer_subset(l, gpu, he, S, Ke[i], Ve[i], inplace=True, ctx=ctx)
        # the graph runs the bucket's 64 padded rows, the eager loop 37: GEMMs over other row counts
        # may round differently, so the recomputed values agree to bf16 noise, the rest bit for bit
        rel = lambda a, b: ((a.float() - b.float()).norm() / b.float().norm()).item()
        assert rel(h_r, he) < 1e-2, (rep, rel(h_r, he))
        keep = torch.ones(T, dtype=torch.bool, device=DEV)
        keep[S] = False
        for a, b, k0 in zip(K_r + V_r, Ke + Ve, Ks[start:] + Vs[start:]):
            assert a.shape == b.shape and rel(a[:, :, S], b[:, :, S]) < 1e-2
            assert torch.equal(a[:, :, keep], k0[:, :, keep])


def test_graph_bucket_cache_guard(models):
    gpu, _ = models
    prefix, docs, query = _request(4)
    eng = Engine(gpu, BlockStore(1 << 30), graphs=True)
    on = lambda x: [t.to(DEV) for t in x] if isinstance(x, list) else x.to(DEV)
    eng.prefill(on(prefix), on(docs), on(query))
    _, c1, _ = eng.prefill(on(prefix), on(docs[::-1]), on(query), ratio=0.2, reserve=4)
    assert c1.graph is not None and c1.valid
    kept = KVCache(c1.K, c1.V, c1.length, graph=c1.graph).detach()
    KV = (c1.K[..., :c1.length, :].clone(), c1.V[..., :c1.length, :].clone())
    _, c2, _ = eng.prefill(on(prefix), on(docs[1:] + docs[:1]), on(query), ratio=0.2, reserve=4)
    assert c2.graph is c1.graph and c2.valid and not c1.valid
    with pytest.raises(StaleCacheError):
        c1.K
    with pytest.raises(StaleCacheError):
        eng.decode(c1, torch.tensor([5], device=DEV))
    assert torch.equal(kept.K[..., :kept.length, :], KV[0]) and torch.equal(kept.V[..., :kept.length, :], KV[1])
    eng.decode(kept, torch.tensor([5], device=DEV))  # a detached copy decodes
    eng.decode(c2, torch.tensor([5], device=DEV))
    assert kept.length == c2.length


def test_rotate_keys_moves_k_only(models):
    gpu, _ = models
    g = torch.Generator(device=DEV).manual_seed(5)
    K = torch.randn(CFG.num_hidden_layers, 1, 2, 77, CFG.head_dim, device=DEV, dtype=torch.bfloat16, generator=g)
    V = torch.randn_like(K)
    out = rotate_keys(gpu, K, 1234)
    dk = torch.empty_like(K)
    dv = torch.empty_like(V)
    _hip.rope_assemble([(K, V, 0, 1234)], dk, dv, gpu.model.rotary_emb.inv_freq)
    assert torch.equal(out, dk) and torch.equal(dv, V)
    assert rotate_keys(gpu, K, 0) is K
    # [1, kv, n, hd] per-layer tensors, as the reference's callers pass them
    assert torch.equal(rotate_keys(gpu, K[1], 1234), dk[1])


def test_promoted_blocks_stop_pending_and_take_the_fused_launch(models):
    gpu, _ = models
    prefix, docs, query = _request(6, n_docs=5)
    on = lambda x: [t.to(DEV) for t in x] if isinstance(x, list) else x.to(DEV)
    probe = BlockStore(1 << 30)
    Engine(gpu, probe).prefill(on(prefix), on(docs), on(query))
    one = max(b.nbytes for b in probe.blocks.values())
    store = BlockStore(8 * one, cpu_budget_bytes=1 << 30)
    eng = Engine(gpu, store)
    eng.prefill(on(prefix), on(docs), on(query))
    # a request over five other docs evicts three of ours to the host tier (LRU)
    _, _, st = eng.prefill(on(prefix), on([(d + 1) % CFG.vocab_size for d in docs]), on(query))
    assert store.stats.offloads > 0
    want, _, _ = Engine(gpu, probe).prefill(on(prefix), on(docs[::-1]), on(query))
    got, _, st = eng.prefill(on(prefix), on(docs[::-1]), on(query))
    assert st.misses == 0 and store.stats.cpu_hits > 0 and torch.equal(got, want)
    promoted = [b for b in store.blocks.values() if b.shadow is not None]
    assert promoted
    torch.cuda.synchronize()
    store.get(next(iter(store.blocks)))  # any lookup reaps landed copies
    assert all(b.ready is None and not b.pending for b in promoted)
    calls = []
    orig = _hip.rope_assemble

    def spy(*a, **k):
        calls.append(k.get("layer_lo", 0))
        return orig(*a, **k)

    _hip.rope_assemble = spy
    try:
        got2, _, _ = eng.prefill(on(prefix), on(docs[::-1]), on(query))
    finally:
        _hip.rope_assemble = orig
    assert calls == [0] and torch.equal(got2, want)  # one fused launch, no per-layer assembly


def test_plain_reuse_replays_the_query_forward_from_a_graph(models):
    """A request that recomputes nothing (ratio 0) replays its query forward from a graph captured
    over a query-only cache bucket: logits bit-identical to the eager forward, the cache decodes,
    and SubsetRunner.captures still counts only recompute-loop graphs (tests/test_engine.py:109
    expects 1 after a ratio-0 pass and two graphed requests)."""
    gpu, _ = models
    prefix, docs, query = _request(7)
    on = lambda x: [t.to(DEV) for t in x] if isinstance(x, list) else x.to(DEV)
    eager = Engine(gpu, BlockStore(1 << 30))
    graphed = Engine(gpu, BlockStore(1 << 30), graphs=True)
    for e in (eager, graphed):
        e.prefill(on(prefix), on(docs), on(query))
    a, ca, _ = eager.prefill(on(prefix), on(docs[::-1]), on(query), reserve=3)
    for _ in range(2):
        b, cb, _ = graphed.prefill(on(prefix), on(docs[::-1]), on(query), reserve=3)
    assert cb.graph is not None and graphed.runner.query_captures == 1 and graphed.runner.captures == 0
    assert torch.equal(a, b)
    n = ca.length
    assert torch.equal(ca.K[..., :n, :], cb.K[..., :n, :]) and torch.equal(ca.V[..., :n, :], cb.V[..., :n, :])
    nxt = torch.tensor([int(a.argmax())], device=DEV)
    assert torch.equal(eager.decode(ca, nxt), graphed.decode(cb, nxt))
    fresh = Engine(gpu, graphed.store, graphs=True)  # the reference test's sequence on a new runner
    fresh.prefill(on(prefix), on(docs), on(query))
    for _ in range(2):
        fresh.prefill(on(prefix), on(docs[::-1]), on(query), ratio=0.2)
    assert fresh.runner.captures == 1 and fresh.runner.query_captures == 1  # the reference's count
