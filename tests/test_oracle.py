"""Pins of the CPU oracle (oracle/) before it is trusted as the parity reference.

Each check is independent of the oracle's own formula: transformers' Qwen2/Llama models (library
routines), the RoPE group property, float64 fixtures written by tests/golden/make_golden.py with
the standard library only, brute-force sorts, an independent list-based LRU model, and the
reference's engine invariants (tests/test_engine.py:46-178) re-expressed with random-init models.
"""
import json
import random
from pathlib import Path

import pytest
import torch

from oracle import model_ref as M
from oracle import tread_ref as R
from tread_amd.model import ModelConfig, preset, synthetic_model

GOLDEN = Path(__file__).resolve().parent / "golden"


def tiny(family="qwen2", layers=2, hd=16, heads=4, kv=2, hidden=64, vocab=256, theta=10000.0):
    return ModelConfig(vocab, hidden, layers, heads, kv, hd, 96, rope_theta=theta,
                       attention_bias=(family == "qwen2"), tie_word_embeddings=(family == "qwen2"), family=family)


def oracle_model(cfg, seed=0, std=0.05, dtype=torch.float32):
    m = synthetic_model(cfg, "cpu", torch.float32, seed=seed, std=std, bias_std=0.05 if cfg.attention_bias else 0.0)
    return M.load(cfg, m.state_dict(), dtype), m.state_dict()


# ---------------------------------------------------------------------------- model math vs transformers

@pytest.mark.parametrize("family", ["qwen2", "llama"])
def test_model_matches_transformers(family):
    from transformers import LlamaConfig, LlamaForCausalLM, Qwen2Config, Qwen2ForCausalLM
    cfg = tiny(family)
    ref, sd = oracle_model(cfg, seed=3)
    kw = dict(vocab_size=256, hidden_size=64, num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
              intermediate_size=96, rope_theta=10000.0, rms_norm_eps=1e-6, max_position_embeddings=4096)
    if family == "qwen2":
        hf = Qwen2ForCausalLM(Qwen2Config(tie_word_embeddings=True, **kw))
    else:
        hf = LlamaForCausalLM(LlamaConfig(tie_word_embeddings=False, head_dim=16, **kw))
    hf.load_state_dict(sd, strict=True)
    hf.eval()
    ids = torch.randint(0, 256, (40,), generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        out = hf(ids[None], use_cache=True)
    h, K, V = M.forward(ref, ids)
    assert torch.allclose(M.logits_last(ref, h), out.logits[0, -1], atol=1e-5)
    for l in range(2):
        assert torch.equal(K[l], out.past_key_values.layers[l].keys)
        assert torch.equal(V[l], out.past_key_values.layers[l].values)


def test_rotary_tables_match_transformers():
    from transformers import Qwen2Config
    from transformers.models.qwen2.modeling_qwen2 import Qwen2RotaryEmbedding
    cfg = tiny(hd=16, theta=1000000.0)
    rot = Qwen2RotaryEmbedding(Qwen2Config(hidden_size=64, num_attention_heads=4, head_dim=16,
                                           rope_theta=1000000.0, max_position_embeddings=40000))
    ref, _ = oracle_model(cfg)
    pos = torch.tensor([0, 1, 63, 1064, 31999, 32063])
    c, s = rot(torch.zeros(1, dtype=torch.bfloat16), pos[None])
    oc, os_ = M.rope_cos_sin(ref, pos, torch.bfloat16)
    assert torch.equal(c, oc) and torch.equal(s, os_)


# ---------------------------------------------------------------------------- RoPE re-rotation

def test_rotation_group_property_and_identity():
    cfg = tiny(hd=16, theta=1000000.0)
    ref, _ = oracle_model(cfg)
    K = torch.randn(2, 1, 2, 50, 16, generator=torch.Generator().manual_seed(2))
    assert R.rotate_keys(ref, K, 0) is K
    for a, b in [(3, 5), (1000, -1000), (31000, 64), (-7, 7)]:
        two = R.rotate_keys(ref, R.rotate_keys(ref, K, a), b)
        one = R.rotate_keys(ref, K, a + b)
        # angles are fp32 products pos * inv_freq (inv_freq <= 1): each carries up to half an fp32
        # ulp of |pos| radians of rounding, which bounds the difference of the two paths
        tol = 1e-5 + 4 * K.abs().max().item() * 2.0 ** -24 * (abs(a) + abs(b) + abs(a + b))
        assert (two - one).abs().max().item() <= tol, (a, b, (two - one).abs().max().item(), tol)
    # norms are preserved per (i, i + d/2) pair
    r = R.rotate_keys(ref, K, 777)
    pair = lambda x: x[..., :8] ** 2 + x[..., 8:] ** 2
    assert torch.allclose(pair(r), pair(K), rtol=1e-5, atol=1e-5)


def test_rotation_matches_float64_fixture():
    for case in json.loads((GOLDEN / "rotate.json").read_text()):
        cfg = tiny(hd=case["d"], theta=case["theta"])
        m = M.RefModel(cfg=cfg, w={}, dtype=torch.float32, inv_freq=M.inv_freq_of(cfg))
        K = torch.tensor(case["K"], dtype=torch.float32)[None, None]
        exp = torch.tensor(case["expected"], dtype=torch.float64)
        for fn in (R.rotate_keys, R.rotate_keys_fp32):
            got = fn(m, K, case["delta"])[0, 0].double()
            assert torch.allclose(got, exp, atol=2e-5, rtol=0), (case["theta"], case["delta"], (got - exp).abs().max())


def test_rotation_composes_with_fresh_prefill():
    """tests/test_engine.py:46-55: layer-0 keys prefilled at 0 and shifted by d equal keys
    prefilled at +d."""
    cfg = tiny(hd=16, theta=1000000.0)
    ref, _ = oracle_model(cfg)
    doc = torch.randint(0, 256, (30,), generator=torch.Generator().manual_seed(4))
    d = 37
    K0, _ = R.prefill_kv(ref, doc)
    Kd, _ = R.prefill_kv(ref, torch.cat([torch.zeros(d, dtype=torch.long), doc]))
    assert torch.allclose(R.rotate_keys(ref, K0[0], d), Kd[0][:, :, d:], atol=1e-5)


# ---------------------------------------------------------------------------- block keys

def _decode(p):
    if "ids" in p:
        return torch.tensor(p["ids"], dtype=torch.int64)
    if "none" in p:
        return None
    if "float" in p:
        return p["float"]
    return p["str"]


def test_block_key_golden_digests():
    from tread_amd.store import block_key as product_key
    cases = json.loads((GOLDEN / "block_keys.json").read_text())
    assert len(cases) > 30
    for c in cases:
        parts = [_decode(p) for p in c["parts"]]
        assert R.block_key(*parts) == c["digest"]
        assert product_key(*parts) == c["digest"]
        # int32 / GPU-style id tensors hash the same (converted to int64 first)
        if isinstance(parts[-1], torch.Tensor) and parts[-1].numel() and parts[-1].abs().max() < 2 ** 31:
            alt = parts[:-1] + [parts[-1].to(torch.int32)]
            assert R.block_key(*alt) == c["digest"]


def test_sha256_known_answers():
    import hashlib
    assert hashlib.sha256(b"abc").hexdigest() == \
        "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad"
    assert hashlib.sha256(b"").hexdigest() == \
        "e3b0c44298fc1c149afbf4c8996fb92427ae41e4649b934ca495991b7852b855"


# ---------------------------------------------------------------------------- deviation + top-k

def test_deviation_score_and_topk_match_fixture():
    for case in json.loads((GOLDEN / "deviation.json").read_text()):
        k1 = torch.tensor(case["k1"])[None]
        v1 = torch.tensor(case["v1"])[None]
        K1 = torch.tensor(case["K1"])[None]
        V1 = torch.tensor(case["V1"])[None]
        score = R.deviation_score(k1, v1, K1, V1)[0]
        exp = torch.tensor(case["score"], dtype=torch.float64)
        assert torch.allclose(score.double(), exp, rtol=1e-5, atol=1e-6)
        for k, want in case["topk"].items():
            k = int(k)
            got = set(score.topk(k).indices.tolist()) if k else set()
            if not k:
                assert not want
                continue
            thr = exp[want].min()
            # equal sets except for exact ties at the threshold (torch.topk's tie order is unspecified)
            assert all(abs(exp[i] - thr) < 1e-6 for i in got ^ set(want)), (k, got, want)


def test_bucket_matches_brute_force_fixture():
    from tread_amd.graphs import _bucket
    for row in json.loads((GOLDEN / "buckets.json").read_text()):
        assert R.bucket(row["n"], row["T"]) == (row["nb"], row["Tb"])
        assert _bucket(row["n"], row["T"]) == (row["nb"], row["Tb"])


# ---------------------------------------------------------------------------- block store

class ListLRU:
    """Independent model of the two-tier store: plain lists, least recent first."""

    def __init__(self, budget, cpu_budget):
        self.budget, self.cpu_budget = budget, cpu_budget
        self.gpu, self.cpu = [], []  # (key, nbytes)
        self.st = dict(hits=0, misses=0, evictions=0, cpu_hits=0, offloads=0, cpu_evictions=0)

    def used(self, tier):
        return sum(n for _, n in tier)

    def _find(self, tier, key):
        return next((i for i, (k, _) in enumerate(tier) if k == key), None)

    def _insert(self, key, nb):
        while self.used(self.gpu) + nb > self.budget:
            k, n = self.gpu.pop(0)
            self.st["evictions"] += 1
            if n <= self.cpu_budget:
                while self.used(self.cpu) + n > self.cpu_budget:
                    self.cpu.pop(0)
                    self.st["cpu_evictions"] += 1
                self.cpu.append((k, n))
                self.st["offloads"] += 1
        self.gpu.append((key, nb))

    def get(self, key):
        i = self._find(self.gpu, key)
        if i is not None:
            self.gpu.append(self.gpu.pop(i))
        else:
            j = self._find(self.cpu, key)
            if j is None:
                self.st["misses"] += 1
                return False
            _, n = self.cpu.pop(j)
            self.st["cpu_hits"] += 1
            self._insert(key, n)
        self.st["hits"] += 1
        return True

    def put(self, key, nb):
        if nb > self.budget:
            return False
        for tier in (self.gpu, self.cpu):
            i = self._find(tier, key)
            if i is not None:
                tier.pop(i)
        self._insert(key, nb)
        return True


def _trace(seed, n_ops=400):
    rnd = random.Random(seed)
    keys = [f"k{i}" for i in range(12)]
    sizes = {k: rnd.choice([1, 2, 3, 5]) for k in keys}
    return [(rnd.choice(["get", "get", "put"]), rnd.choice(keys)) for _ in range(n_ops)], sizes


@pytest.mark.parametrize("seed,budget,cpu_budget", [(0, 8, 0), (1, 8, 10), (2, 5, 3), (3, 12, 12), (4, 4, 100)])
def test_block_store_matches_list_model(seed, budget, cpu_budget):
    from tread_amd.store import BlockStore as ProductStore
    ops, sizes = _trace(seed)
    unit = 16  # bytes per size unit: K and V of 2 fp32 elements each
    model = ListLRU(budget * unit, cpu_budget * unit)
    stores = [R.BlockStore(budget * unit, cpu_budget * unit), ProductStore(budget * unit, cpu_budget * unit)]
    for op, k in ops:
        if op == "get":
            want = model.get(k)
            for s in stores:
                assert (s.get(k) is not None) == want
        else:
            n = sizes[k]
            want = model.put(k, n * unit)
            for s in stores:
                K = torch.zeros(1, 1, 1, n, 2)
                assert (s.put(k, K, K.clone(), 0) is not None) == want
        for s in stores:
            assert [k for k, _ in model.gpu] == list(s.blocks)
            assert [k for k, _ in model.cpu] == list(s.cpu_blocks)
            assert s.stats.bytes_used == model.used(model.gpu) <= s.budget
            assert s.stats.cpu_bytes_used == model.used(model.cpu) <= s.cpu_budget
            for name, v in model.st.items():
                assert getattr(s.stats, name) == v, name
            assert len(s) == len(model.gpu) + len(model.cpu)


# ---------------------------------------------------------------------------- engine invariants (oracle)

def kl(a, b):
    return R.kl(a, b)


def _req(cfg, seed=1, lens=(20, 13, 27)):
    g = torch.Generator().manual_seed(seed)
    V = cfg.vocab_size
    prefix = torch.randint(0, V, (8,), generator=g)
    docs = [torch.randint(0, V, (n,), generator=g) for n in lens]
    query = torch.randint(0, V, (5,), generator=g)
    return prefix, docs, query


@pytest.fixture(scope="module")
def om():
    cfg = tiny(layers=3, hd=16, theta=1000000.0)
    return cfg, oracle_model(cfg, seed=5)[0]


def test_full_recompute_matches_full_prefill(om):
    cfg, m = om
    prefix, docs, query = _req(cfg)
    ref, _, _ = R.prefill_full(m, prefix, docs, query)
    out, _, _ = R.Engine(m, R.BlockStore(1 << 30)).prefill(prefix, docs, query, ratio=1.0, policy="boundary")
    assert kl(ref, out) < 1e-5
    out2, _, st = R.Engine(m, R.BlockStore(1 << 30)).prefill_prefix_only(prefix, docs, query)
    assert kl(ref, out2) < 1e-5 and st.tokens_prefilled == len(prefix) + sum(map(len, docs))


def test_greedy_generation_steps_equal_full_forward_of_the_extended_sequence(om):
    """tread/server.py:194-210 restated: every step's logits (incremental, on the cache) equal a
    fresh full forward over the prompt plus the tokens emitted so far; the stop rules (eos id,
    max_tokens) cut the token list where the reference's loop does."""
    cfg, m = om
    prefix, docs, query = _req(cfg)
    logits, (K, V), _ = R.prefill_full(m, prefix, docs, query)
    toks, reason, steps = R.generate_greedy(m, logits, K, V, max_tokens=5)
    assert reason == "length" and len(toks) == 5 and len(steps) == 6
    for i in range(6):
        ext = torch.cat([query, torch.tensor(toks[:i], dtype=torch.long)])
        full, _, _ = R.prefill_full(m, prefix, docs, ext)
        assert kl(full, steps[i]) < 1e-6
        if i < 5:
            assert toks[i] == int(full.argmax())
    j = toks.index(toks[2])
    t2, r2, _ = R.generate_greedy(m, logits, K, V, max_tokens=5, eos_ids={toks[2]})
    assert (t2, r2) == (toks[:j], "stop")
    assert R.generate_greedy(m, logits, K, V, max_tokens=0)[:2] == ([], "length")
    forced = [(t + 1) % cfg.vocab_size for t in toks[:3]]
    t4, r4, s4 = R.generate_greedy(m, logits, K, V, max_tokens=5, forced=forced)
    assert t4 == forced and len(s4) == 4


def test_reordered_request_hits_and_equals_cold_assembly(om):
    cfg, m = om
    prefix, docs, query = _req(cfg)
    eng = R.Engine(m, R.BlockStore(1 << 30))
    _, _, st1 = eng.prefill(prefix, docs, query)
    assert (st1.hits, st1.misses) == (0, 1 + len(docs))
    warm, _, st2 = eng.prefill(prefix, docs[::-1], query)
    assert (st2.hits, st2.misses, st2.tokens_prefilled) == (1 + len(docs), 0, 0)
    cold, _, _ = R.Engine(m, R.BlockStore(1 << 30)).prefill(prefix, docs[::-1], query)
    assert kl(cold, warm) < 1e-5


def test_packed_cold_path_equals_per_doc_prefill(om):
    cfg, m = om
    prefix, docs, query = _req(cfg)
    Kr, Vr = R.assemble(m, prefix, docs, "shared")
    eng = R.Engine(m, R.BlockStore(1 << 30))
    out, (K, V), st = eng.prefill(prefix, docs, query)
    T = len(prefix) + sum(map(len, docs))
    for l in range(cfg.num_hidden_layers):
        assert torch.allclose(K[l][:, :, :T], Kr[l], atol=1e-5)
        assert torch.allclose(V[l][:, :, :T], Vr[l], atol=1e-5)
    ref = M.logits_last(m, M.forward(m, query, past=(Kr, Vr))[0])
    assert kl(ref, out) < 1e-5


def test_cpu_tier_and_eviction_stay_exact(om):
    cfg, m = om
    prefix, docs, query = _req(cfg)
    probe = R.BlockStore(1 << 30)
    R.Engine(m, probe).prefill(prefix, docs, query)
    one = max(b.nbytes for b in probe.blocks.values())
    store = R.BlockStore(2 * one, cpu_budget_bytes=1 << 30)
    eng = R.Engine(m, store)
    eng.prefill(prefix, docs, query)
    assert store.stats.offloads > 0 and store.stats.bytes_used <= store.budget and store.stats.cpu_evictions == 0
    warm, _, st = eng.prefill(prefix, docs[::-1], query)
    assert st.misses == 0 and store.stats.cpu_hits > 0
    cold, _, _ = R.Engine(m, R.BlockStore(1 << 30)).prefill(prefix, docs[::-1], query)
    assert kl(cold, warm) < 1e-5
    small = R.BlockStore(2 * one)
    e2 = R.Engine(m, small)
    e2.prefill(prefix, docs, query)
    assert small.stats.bytes_used <= small.budget and small.stats.evictions > 0
    full, _, _ = R.prefill_full(m, prefix, docs, query)
    out, _, _ = e2.prefill(prefix, docs, query, ratio=1.0, policy="boundary")
    assert kl(full, out) < 1e-5


def test_block_key_depends_on_prefix_and_namespace(om):
    cfg, m = om
    prefix, docs, query = _req(cfg)
    eng = R.Engine(m, R.BlockStore(1 << 30))
    eng.prefill(prefix, docs, query)
    _, _, st = eng.prefill((prefix + 1) % cfg.vocab_size, docs, query)
    assert st.hits == 0
    _, _, st = eng.prefill(prefix, docs, query, namespace="other-tenant")
    assert st.hits == 0


def test_deviation_blend_selection_and_eff(om):
    cfg, m = om
    prefix, docs, query = _req(cfg)
    eng = R.Engine(m, R.BlockStore(1 << 30))
    eng.prefill(prefix, docs, query)
    trace = {}
    _, _, st = eng.prefill(prefix, docs[::-1], query, ratio=0.25, trace=trace)
    n = sum(map(len, docs))
    budget = int(round(0.25 * n))
    assert len(trace["S"]) == budget and torch.equal(trace["S"], trace["S"].sort().values)
    L = cfg.num_hidden_layers
    assert st.recompute_eff == pytest.approx((budget * (L - 1) + n) / (n * L))
    # the selected positions are the top-`budget` scores (brute force, ties at the threshold aside)
    dev, all_c = trace["dev"], trace["all_c"]
    order = sorted(range(n), key=lambda i: (-float(dev[i]), i))
    want = set(all_c[order[:budget]].tolist())
    thr = float(dev[order[budget - 1]])
    got = set(trace["S"].tolist())
    pos = {int(p): float(dev[i]) for i, p in enumerate(all_c.tolist())}
    assert all(pos[p] == thr for p in got ^ want)


def test_forced_selection_hook(om):
    """The test hook that hands the oracle a selection: its own selection reproduces the natural
    run exactly; another one is used as given (sorted) with the same budget."""
    cfg, m = om
    prefix, docs, query = _req(cfg)
    eng = R.Engine(m, R.BlockStore(1 << 30))
    eng.prefill(prefix, docs, query)
    t0 = {}
    a, _, _ = eng.prefill(prefix, docs[::-1], query, ratio=0.25, trace=t0)
    t1 = {"force_S": t0["S"].flip(0)}
    b, _, _ = eng.prefill(prefix, docs[::-1], query, ratio=0.25, trace=t1)
    assert torch.equal(a, b) and torch.equal(t1["S"], t0["S"])
    other = t0["all_c"][torch.randperm(len(t0["all_c"]), generator=torch.Generator().manual_seed(3))[:len(t0["S"])]]
    t2 = {"force_S": other}
    c, _, _ = eng.prefill(prefix, docs[::-1], query, ratio=0.25, trace=t2)
    assert torch.equal(t2["S"], other.sort().values) and not torch.equal(a, c)


def test_blend_with_no_docs_and_zero_budget(om):
    cfg, m = om
    K = [torch.zeros(1, 2, 5, 16)] * cfg.num_hidden_layers
    _, _, S, eff = R.blend(m, torch.zeros(5, dtype=torch.long), K, K, [], 0.5, "deviation")
    assert S.numel() == 0 and eff == 0.0
    _, _, S, eff = R.blend(m, torch.zeros(5, dtype=torch.long), K, K, [torch.arange(1, 3)], 0.2, "deviation")
    assert S.numel() == 0 and eff == 0.0  # round(0.4) == 0


# ---------------------------------------------------------------------------- the reference's CPU case

def test_small_model_cpu_fp32_reversed_reuse_of_4_docs():
    """Qwen2.5-0.5B-shaped fp32 model (24 layers, hidden 896, 14/2 heads, head_dim 64, theta 1e6,
    vocab 151936), 64-token system prompt + 4 docs x 256 + 32-token query; docs cached in order
    1..4, then reassembled in reversed order with plain reuse: all 5 blocks hit, and every doc's
    re-rotated layer-0 keys equal an in-place fresh prefill of the same request."""
    torch.manual_seed(0)
    cfg = preset("qwen2.5-0.5b")
    m = synthetic_model(cfg, "cpu", torch.float32, seed=0)
    ref = M.load(cfg, m.state_dict(), torch.float32)
    del m
    g = torch.Generator().manual_seed(1)
    system = torch.randint(0, cfg.vocab_size, (64,), generator=g)
    docs = [torch.randint(0, cfg.vocab_size, (256,), generator=g) for _ in range(4)]
    query = torch.randint(0, cfg.vocab_size, (32,), generator=g)
    eng = R.Engine(ref, R.BlockStore(1 << 32))
    _, _, st1 = eng.prefill(system, docs, query)
    assert (st1.hits, st1.misses) == (0, 5)
    rev = docs[::-1]
    _, (K, _), st2 = eng.prefill(system, rev, query)
    assert (st2.hits, st2.misses, st2.tokens_reused, st2.tokens_prefilled) == (5, 0, 64 + 1024, 0)
    # layer 0 depends only on token + position: the reused, re-rotated keys equal a fresh prefill
    # of the reversed request at every doc position
    Kf, _ = R.prefill_kv(ref, torch.cat([system] + rev))
    assert torch.allclose(K[0][:, :, :64 + 1024], Kf[0], atol=1e-3)


def test_row_chunked_layer_equals_layer_subset():
    """The row-chunked recompute layer the CPU baseline times gives layer_subset's bits."""
    from tread_amd.model import ModelConfig, synthetic_model
    cfg = ModelConfig(512, 256, 2, 8, 2, 64, 384)
    m = M.load(cfg, synthetic_model(cfg, "cpu", torch.bfloat16, seed=3).state_dict(), torch.bfloat16)
    g = torch.Generator().manual_seed(5)
    T = 700
    S = torch.sort(torch.randperm(T, generator=g)[:300]).values
    h = (torch.randn(1, 300, 256, generator=g) * 0.3).to(torch.bfloat16)
    K = torch.randn(1, 2, T, 64, generator=g).to(torch.bfloat16)
    V = torch.randn_like(K)
    ctx = R.subset_ctx(m, S, T, torch.bfloat16)
    want, Kw, Vw = R.layer_subset(m, 1, h, S, K.clone(), V.clone(), inplace=True, ctx=ctx)
    got, Kg, Vg = R.layer_subset_rows(m, 1, h, S, K.clone(), V.clone(), ctx, chunk=64)
    assert torch.equal(got, want) and torch.equal(Kg, Kw) and torch.equal(Vg, Vw)
