"""Reuse engine: build a request's KV cache from content-addressed blocks (tread/engine.py).

Request = [prefix][doc_1]...[doc_N][query] as separate segments (tread/engine.py:1-7). The prefix
is an exact-prefix block; every doc block is computed once on top of the prefix at base position
P, cached under a key chained on the prefix key, and re-rotated to wherever it lands later.

Same API, keys, hit/miss accounting and stage timings as the reference; what runs underneath:
  - assembly: ONE fused HIP launch rotates every doc block by (offset - base) and gathers it,
    with the prefix block, into a preallocated [L, 1, kv, T + Nq, hd] cache (kernel (a)).
    Blocks still arriving from the host tier are assembled per layer group, right before the
    group is first read, after waiting that group's copy event (overlap of DMA and compute); with
    the deviation pass, the docs' layer 0 is recomputed rather than assembled, so their copies
    move layer 0 last and are queued once the pass's layer 0 is launched;
  - blend: deviation pass + top-k (kernel (b)) and the recompute loop with the MFMA attention
    (kernel (c)), eager or replayed from a hipGraph whose static buffer is the cache itself;
  - query: the query rows are appended in place at rows T.. of the same cache (no cat/copy).
  - cold path: all missed docs in one packed forward whose attention is block-diagonal in-kernel
    (each doc sees the prefix and itself), no [n, P + n] mask tensor.
Stage boundaries synchronise the current stream only, so copies on the store's copy stream keep
overlapping compute across them.
"""
import time
from dataclasses import dataclass, field

import torch

from tread_amd import _hip
from tread_amd.blend import blend_cache, blend_query, forward_into, prepared, select
from tread_amd.cache import KVCache
from tread_amd.forward import alloc_cache, embed, final_logits, make_rows, run_layers
from tread_amd.graphs import SubsetRunner
from tread_amd.model import rope_theta_of
from tread_amd.store import BlockStore, block_key


@dataclass
class RequestStats:
    """tread/engine.py:19-26."""
    hits: int = 0
    misses: int = 0
    tokens_reused: int = 0
    tokens_prefilled: int = 0
    recompute_eff: float = 0.0
    t: dict = field(default_factory=dict)  # stage -> seconds


class _Tmp:
    """tread/engine.py:169-173: an uncached block (store budget too small): Block's fields."""

    def __init__(self, K, V, base):
        self.K, self.V, self.base, self.n_tokens = K, V, base, K.shape[-2]
        self.ready = None

    def wait(self, layers=None, stream=None):
        pass


def model_sig(model):
    """tread/engine.py:36-38: (name_or_path, str(dtype), rope_theta, rope_scaling). The theta is
    read from rope_parameters when the config keeps it there, so keys match a config that carries
    it as rope_theta; default RoPE counts as no scaling."""
    cfg = model.config
    scaling = getattr(cfg, "rope_scaling", None)
    if isinstance(scaling, dict) and scaling.get("rope_type", scaling.get("type")) == "default":
        scaling = None
    return (getattr(cfg, "_name_or_path", ""), str(model.dtype), rope_theta_of(cfg), scaling)


class _Assembly:
    """Rotate+gather of the request's blocks into the cache; per-layer for in-flight blocks.

    `store`: flushed before a layer of an in-flight block is read (its DMAs may have been left
    unqueued, see BlockStore.batch). `skip0`: indices of sources whose layer 0 the request
    recomputes in place (the deviation pass splices fresh k/v into every doc row of layer 0), so
    layer 0 of those in flight is not assembled and their layer-0 DMAs are not waited for."""

    def __init__(self, P, K, V, sources, store=None, skip0=()):
        self.P, self.K, self.V = P, K, V
        self.store = store
        ready = [(b.K, b.V, off, delta) for b, off, delta in sources if getattr(b, "ready", None) is None]
        self.pending = [(b, off, delta) for b, off, delta in sources if getattr(b, "ready", None) is not None]
        skip = set(skip0)
        self.pending0 = self.pending if not skip else [
            (b, off, delta) for i, (b, off, delta) in enumerate(sources)
            if getattr(b, "ready", None) is not None and i not in skip]
        self.done = [False] * P.L
        self.tables = {}
        self.waited = set()  # ids of copy events the current stream already waits on
        if ready:
            _hip.rope_assemble(ready, K, V, P.inv_freq)
        if not self.pending:
            self.done = [True] * P.L

    def ensure(self, l):
        if self.done[l]:
            return
        pend = self.pending0 if l == 0 else self.pending
        if self.store is not None and any(b.ready is not None and not b.ready for b, _, _ in pend):
            self.store.flush()  # their DMAs were left unqueued: queue them now
        # blocks promoted in one batch share their layer-group events: one stream wait per event
        # (each wait is a barrier packet the GPU processes in order)
        cur = torch.cuda.current_stream()
        for b, _, _ in pend:
            e = b.ready[l] if b.ready is not None else None
            if e is not None and id(e) not in self.waited:
                cur.wait_event(e)
                self.waited.add(id(e))
        # the following layers whose copies landed with layer l's (the same event for every pending
        # block) are assembled by the same launch
        hi = l + 1
        if pend is self.pending:  # (layer 0 of a skipping request is assembled alone)
            while hi < self.P.L and not self.done[hi] and all(
                    b.ready is None or (b.ready[hi] is b.ready[l]) for b, _, _ in pend):
                hi += 1
        if pend:
            key = id(pend)
            self.tables[key] = _hip.rope_assemble([(b.K, b.V, off, delta) for b, off, delta in pend], self.K,
                                                  self.V, self.P.inv_freq, layer_lo=l, layer_hi=hi,
                                                  table=self.tables.get(key))
        for x in range(l, hi):
            self.done[x] = True

    def finish(self):
        for l in range(self.P.L):
            self.ensure(l)


class Engine:
    def __init__(self, model, store: BlockStore, graphs=False, fold_query=True):
        self.model = model
        self.store = store
        self.P = prepared(model)
        # hipGraph replay of the recompute loop (tread/graphs.py); off by default as in the
        # reference, since each new size bucket pays a one-off capture. Requests assemble straight
        # into a bucket's cache (no copy in or out), so graphs serve every context length.
        self.runner = SubsetRunner(model, max_ctx=None) if graphs else None
        # with recompute, the query forward rides in the recompute loop (blend_query) instead of
        # running after it: same per-layer inputs, one weight pass less
        self.fold_query = fold_query
        self.sig = model_sig(model)
        self.last_selected = None  # positions recomputed by the last prefill (diagnostics)

    def _sync(self):
        torch.cuda.current_stream().synchronize()

    @torch.inference_mode()
    def prefix_block(self, prefix_ids, st, namespace="", host_ids=None, key=None):
        """tread/engine.py:44-57. `host_ids`: the same ids already in host memory (hashed instead of
        prefix_ids, which saves a device-to-host copy per key); `key`: the key, if already known."""
        if key is None:
            key = block_key(*self.sig, namespace, "prefix", prefix_ids if host_ids is None else host_ids)
        b = self.store.get(key)
        if b is None:
            st.misses += 1
            st.tokens_prefilled += len(prefix_ids)
            K, V = alloc_cache(self.P, len(prefix_ids), prefix_ids.device)
            forward_into(self.model, prefix_ids, K, V, want_logits=False)
            b = self.store.put(key, K, V, 0) or _Tmp(K, V, 0)
        else:
            st.hits += 1
            st.tokens_reused += len(prefix_ids)
        return key, b

    @torch.inference_mode()
    def doc_blocks(self, prefix_key, pb, docs, st, host_docs=None, keys=None):
        """tread/engine.py:59-96: look up every doc; prefill all misses in one packed forward.

        The packed sequence sits on top of the prefix rows of a temporary cache; token j of doc i
        has RoPE position P + j, writes cache row P + off_i + j, and sees rows [0, P) plus
        [P + off_i, P + off_i + j]: the reference's block-diagonal mask, evaluated in-kernel.
        `host_docs`: the docs' ids already in host memory, hashed instead of `docs`; `keys`: the
        docs' keys, if already known."""
        if keys is None:
            keys = [block_key(*self.sig, prefix_key, d) for d in (docs if host_docs is None else host_docs)]
        blocks = [self.store.get(k) for k in keys]
        miss = [i for i, b in enumerate(blocks) if b is None]
        st.hits += len(docs) - len(miss)
        st.tokens_reused += sum(len(d) for d, b in zip(docs, blocks) if b is not None)
        if not miss:
            return blocks
        st.misses += len(miss)
        self.store.flush()  # the packed prefill reads the prefix block
        P = pb.n_tokens
        ids = torch.cat([docs[i] for i in miss])
        n, dev = len(ids), ids.device
        st.tokens_prefilled += n
        lens = [len(docs[i]) for i in miss]
        offs = [0]
        for Ld in lens[:-1]:
            offs.append(offs[-1] + Ld)
        local = torch.cat([torch.arange(Ld, device=dev) for Ld in lens])
        seg0 = torch.cat([torch.full((Ld,), P + o, device=dev, dtype=torch.int64) for Ld, o in zip(lens, offs)])
        K, V = alloc_cache(self.P, P + n, dev)
        pb.wait()
        _hip.rope_assemble([(pb.K, pb.V, 0, 0)], K, V, self.P.inv_freq)
        forward_into(self.model, ids, K, V, start_row=P, pos=P + local, kseg=seg0, n_shared=P, want_logits=False)
        for i, o, Ld in zip(miss, offs, lens):
            Kd = K[..., P + o:P + o + Ld, :].contiguous()
            Vd = V[..., P + o:P + o + Ld, :].contiguous()
            blocks[i] = self.store.put(keys[i], Kd, Vd, P) or _Tmp(Kd, Vd, P)
        return blocks

    @torch.inference_mode()
    def prefill(self, prefix_ids, docs, query_ids, ratio=0.0, policy="deviation", namespace="", gen=None, reserve=0):
        """tread/engine.py:98-136. Returns (logits [vocab], KVCache, RequestStats). `reserve`: rows
        kept free after the query for `decode` (an addition; the reference's cache grows by
        concatenation)."""
        st = RequestStats()
        self._sync()
        t0 = time.perf_counter()

        hp = hd = None
        if prefix_ids.device.type != "cpu":  # one device-to-host copy for every key's ids
            hp, *hd = torch.cat([prefix_ids] + list(docs)).to("cpu", torch.int64).split(
                [len(prefix_ids)] + [len(d) for d in docs])
        budget = select(ratio, docs)[1] if (ratio > 0 and docs) else 0
        # With the deviation pass, layer 0 of every doc row is recomputed in place: the docs'
        # host-tier copies move layer 0 last, and their DMAs are queued once the deviation pass's
        # layer 0 is launched (the first assembly of a later layer flushes the store), so that
        # the host time of queueing them runs beside GPU work instead of before it.
        recompute0 = budget > 0 and policy == "deviation"
        with self.store.batch():  # host-tier hits share one layer-major H2D schedule
            pkey = block_key(*self.sig, namespace, "prefix", prefix_ids if hp is None else hp)
            dkeys = [block_key(*self.sig, pkey, d) for d in (docs if hd is None else hd)]
            self.store.prefetch([pkey] + dkeys)  # disk-tier files: read and verified in parallel
            pkey, pb = self.prefix_block(prefix_ids, st, namespace, host_ids=hp, key=pkey)
        with self.store.batch(flush=not recompute0, layer0_last=recompute0):
            blocks = self.doc_blocks(pkey, pb, docs, st, host_docs=hd, keys=dkeys)
        Pn = pb.n_tokens
        T = Pn + sum(len(d) for d in docs)
        Nq = len(query_ids)
        dev = prefix_ids.device
        graph = None
        if self.runner is not None and self.runner.worth_it(T):
            if budget > 0:
                start = 1 if policy == "deviation" else 0
                graph = self.runner.cache_for(start, budget, T, Nq, dev, room=Nq + reserve,
                                              fold=self.fold_query and Nq > 0)
            elif Nq > 0:  # nothing to recompute: the query forward alone is replayed
                graph = self.runner.query_cache_for(T, Nq, dev, room=Nq + reserve)
        if graph is not None:
            K, V = graph.K, graph.V
        else:
            K, V = alloc_cache(self.P, T + Nq + reserve, dev)
        sources = [(pb, 0, 0)]
        offset = Pn
        for d, b in zip(docs, blocks):
            sources.append((b, offset, offset - b.base))
            offset += len(d)
        cands = list(torch.arange(Pn, T, device=dev).split([len(d) for d in docs])) if docs else []
        asm = _Assembly(self.P, K, V, sources, store=self.store,
                        skip0=range(1, len(sources)) if recompute0 else ())
        hook = asm.ensure if asm.pending else None  # None: nothing to wait for between layers
        Kl, Vl = K.unbind(0), V.unbind(0)
        self._sync()
        t1 = time.perf_counter()

        self.last_selected = None
        logits = None
        if ratio > 0:
            ctx = torch.cat([prefix_ids] + list(docs))
            if self.fold_query and Nq > 0:  # the query rows ride in the recompute (blend_query)
                self.last_selected, st.recompute_eff, logits = blend_query(
                    self.model, ctx, Kl, Vl, cands, ratio, policy, query_ids, T, gen=gen, runner=self.runner,
                    graph=graph, hook=hook)
            else:
                self.last_selected, st.recompute_eff = blend_cache(
                    self.model, ctx, Kl, Vl, cands, ratio, policy, gen=gen, runner=self.runner, graph=graph, T=T,
                    hook=hook)
        self._sync()
        t2 = time.perf_counter()

        if logits is not None:
            logits = logits.clone()  # a graph's output is static
        elif graph is not None and Nq > 0:
            logits = self.runner.query(graph, query_ids, T, hook=hook).clone()  # the graph's output is static
        else:
            R = make_rows(self.P, torch.arange(T, T + Nq, device=dev))
            h, d = run_layers(self.P, embed(self.P, query_ids), None, R, Kl, Vl, range(self.P.L), hook=hook)
            logits = final_logits(self.P, h, d)
        self.store.flush()  # nothing is left unqueued past the request (a no-op after any later layer)
        self._sync()
        t3 = time.perf_counter()
        st.t = dict(assemble=t1 - t0, blend=t2 - t1, query=t3 - t2, ttft=t3 - t0)
        return logits, KVCache(K, V, T + Nq, graph=graph), st

    @torch.inference_mode()
    def decode(self, cache, ids):
        """One step of the reference server's generation loop (tread/server.py:201-208:
        `model(nxt.view(1, 1), past_key_values=cache, use_cache=True, num_logits_to_keep=1)`) on
        this engine's cache: the token ids' k/v are written in place at rows cache.length.. (no
        per-layer concatenation) and the last one's logits [vocab] are returned. Replayed from a
        graph when the cache is a graph bucket with room for the padded rows; a cache without
        room grows first. A bucket's cache is valid until the next request claims that bucket
        (then this raises StaleCacheError; `cache.detach()` keeps a copy that stays valid)."""
        cache.check()
        n = ids.numel()
        T = cache.length
        if T + n > cache.capacity:
            cache.grow(T + n + 256)
        g = cache.graph
        if g is not None and self.runner is not None and self.runner.fits(g, n, T):
            logits = self.runner.decode(g, ids, T).clone()
        else:
            R = make_rows(self.P, torch.arange(T, T + n, device=ids.device))
            h, d = run_layers(self.P, embed(self.P, ids), None, R, cache.K.unbind(0), cache.V.unbind(0),
                              range(self.P.L))
            logits = final_logits(self.P, h, d)
        cache.length = T + n
        return logits

    @torch.inference_mode()
    def generate(self, prefix_ids, docs, query_ids, max_tokens=16, eos_ids=(), ratio=0.0, policy="deviation",
                 namespace="", max_seconds=None):
        """The reference server's greedy loop around prefill (tread/server.py:194-210): the next
        token is the argmax; stop on an eos id ("stop"), after max_tokens tokens ("length") or
        past max_seconds ("time"); every emitted token goes through `decode`. Returns
        (tokens, finish_reason, RequestStats, KVCache)."""
        t0 = time.perf_counter()
        logits, cache, st = self.prefill(prefix_ids, docs, query_ids, ratio=ratio, policy=policy,
                                         namespace=namespace, reserve=max_tokens)
        out, reason = [], "stop"
        nxt = logits.argmax()
        eos = set(int(e) for e in eos_ids)
        while int(nxt) not in eos:
            if len(out) >= max_tokens:
                reason = "length"
                break
            if max_seconds is not None and time.perf_counter() - t0 > max_seconds:
                reason = "time"
                break
            out.append(int(nxt))
            nxt = self.decode(cache, nxt.view(1)).argmax()
        return out, reason, st, cache

    @torch.inference_mode()
    def prefill_prefix_only(self, prefix_ids, docs, query_ids):
        """tread/engine.py:138-152: exact-prefix caching only; every doc is prefilled again."""
        st = RequestStats()
        self._sync()
        t0 = time.perf_counter()
        _, pb = self.prefix_block(prefix_ids, st)
        rest = torch.cat(list(docs) + [query_ids])
        st.tokens_prefilled += len(rest) - len(query_ids)
        Pn = pb.n_tokens
        K, V = alloc_cache(self.P, Pn + len(rest), prefix_ids.device)
        pb.wait()
        _hip.rope_assemble([(pb.K, pb.V, 0, 0)], K, V, self.P.inv_freq)
        logits = forward_into(self.model, rest, K, V, start_row=Pn)
        self._sync()
        st.t = dict(ttft=time.perf_counter() - t0)
        return logits, KVCache(K, V, Pn + len(rest)), st


@torch.inference_mode()
def prefill_full(model, prefix_ids, docs, query_ids):
    """tread/engine.py:155-166: no caching at all (the TTFT denominator)."""
    torch.cuda.current_stream().synchronize()
    t0 = time.perf_counter()
    ids = torch.cat([prefix_ids] + list(docs) + [query_ids])
    P = prepared(model)
    K, V = alloc_cache(P, len(ids), ids.device)
    logits = forward_into(model, ids, K, V)
    torch.cuda.current_stream().synchronize()
    st = RequestStats(tokens_prefilled=len(ids) - len(query_ids), t=dict(ttft=time.perf_counter() - t0))
    return logits, KVCache(K, V, len(ids)), st
