"""hipGraph replay of the selective-recompute layer loop (tread/graphs.py, redesigned).

The reference captures layers start..L-1 per padded size bucket, but copies the whole cache into
the graph's static buffers before each replay and back out after, which made graphs lose above
2k tokens (tread/graphs.py:64-67,92-99). Here the static buffer of a bucket IS the assembled
cache: the engine asks the runner for it before assembly (`cache_for`), the fused assemble kernel
writes the request's blocks straight into it, and a replay only needs the selected positions S
and their hidden rows copied in (a few MB). Padding follows the reference's buckets: padded
rows sit in the bucket's spare rows after the context (and after the query slots when the query
rows ride along), where no real row looks, and see no key themselves (key end -1), so they cost
the GEMMs their rows but no attention.

Each bucket holds one [L, 1, kv, t_cap, hd] K/V pair; the cache returned by the engine aliases
it and stays valid until the next request claims the same bucket (the bucket's generation counter
then moves on and the old cache raises on access; `KVCache.detach()` keeps a copy). The loop is captured as one
graph per layer group of the block store's host-tier copies (chained through static hidden-state
tensors), so a replay waits for a group's copies only right before that group: the block-tier
DMAs overlap the recompute. With no copy in flight the same loop replays as one graph.
"""
from collections import OrderedDict

import torch

from tread_amd import _hip
from tread_amd.forward import alloc_cache, embed, make_rows, norm_logits, run_layers


def _bucket(n, T, n_min=64, n_step=256, t_step=1024):
    """tread/graphs.py:22-27: rows padded to a power of two >= n_min up to n_step, then to a
    multiple of n_step; cache length padded so the padded slots fit, to a multiple of t_step."""
    if n <= n_step:
        nb = max(n_min, 1 << (n - 1).bit_length())
    else:
        nb = -(-n // n_step) * n_step
    Tb = -(-(T + nb - n) // t_step) * t_step
    return nb, Tb


def _q_room(n_query):
    return 256 * max(1, -(-n_query // 256))


def _q_bucket(n_query):
    """Query rows of a captured query forward: a power of two up to 256 (one row for a decode
    step: padded rows cost attention work), then multiples of 256."""
    if n_query <= 256:
        return 1 << (n_query - 1).bit_length()
    return -(-n_query // 256) * 256


def _capture(body, device, pool=None):
    """Warm `body` up twice on a side stream (default priority), then capture it."""
    s = torch.cuda.Stream(device=device)
    s.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(s):
        for _ in range(2):
            body()
    torch.cuda.current_stream(device).wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, pool=pool):
        out = body()
    return graph, out


class _QueryGraph:
    """The query forward (all layers, then the final norm and lm_head on the last real row) over
    a bucket's cache for nq padded query rows at positions T, T+1, ...; padded rows sit after the
    real ones, in the bucket's spare rows, and no real row can see them."""

    def __init__(self, P, g, nq, device):
        self.nq = nq
        self.ids = torch.zeros(nq, dtype=torch.int64, device=device)
        # capture-time positions: the top rows of the bucket, never part of an assembled context
        self.pos = torch.arange(g.t_cap - nq, g.t_cap, dtype=torch.int64, device=device)
        self.last = torch.zeros(1, dtype=torch.int64, device=device)
        self.last_n = 1  # the query rows `last` was set for (index 0: one row); only `query` writes it

        def body():
            R = make_rows(P, self.pos)
            h, d = run_layers(P, embed(P, self.ids), None, R, g.Kl, g.Vl, range(P.L))
            if nq == 1:  # a decoding step: the one row is the last (a view, no gather launches)
                return norm_logits(P, h[:1], None if d is None else d[:1])[0]
            return norm_logits(P, h.index_select(0, self.last), d.index_select(0, self.last))[0]

        self.graph, self.out = _capture(body, device)


class _Graph:
    """The recompute loop of one bucket, captured as one graph per segment of layers, the segments
    chaining through static hidden-state tensors: a replay can then wait for each segment's
    host-tier copies (and assemble them) right before it, instead of before the whole loop. The
    segments are the layer groups the store's host-tier copies arrive in (`seg=None`), so a replay
    with copies in flight waits once per group; `seg=k` cuts every k layers instead.

    Rows of a replay: the n recomputed positions, then (with nq > 0) nq query slots at T, T+1, ...
    whose forward rides along (the last segment ends with the final norm + lm_head of query slot
    `last`), then padding. Padded rows see no key (key end -1) and write their k/v to spare rows
    no real row reads."""

    def __init__(self, P, start, nb, Tb, t_cap, device, trim_last, seg=None, nq=0):
        self.t_cap = t_cap
        self.generation = 0  # bumped whenever a request claims this bucket's cache
        self.queries = {}  # nq -> _QueryGraph over this bucket's cache
        self.K, self.V = alloc_cache(P, t_cap, device)
        self.K.zero_()
        self.V.zero_()
        self.Kl, self.Vl = self.K.unbind(0), self.V.unbind(0)
        self.h = torch.zeros(nb, P.H, dtype=P.embed.dtype, device=device)
        self.S = torch.arange(nb, dtype=torch.int64, device=device)
        self.kend = self.S.clone()
        self.nq = nq
        self.q_idx = torch.arange(nb - nq, nb, dtype=torch.int64, device=device)
        self.last = torch.zeros(1, dtype=torch.int64, device=device)
        self.nb, self.Tb, self.start = nb, Tb, start
        self.pool = torch.cuda.graph_pool_handle()
        layers = list(range(start, P.L))
        if seg is None:
            groups = [list(range(max(a, start), b)) for a, b in _hip.layer_groups(P.L) if b > start]
        else:
            groups = [layers[i:i + seg] for i in range(0, len(layers), seg)]

        def loop(ls, first, last, prev, carry):
            """Layers ls of the loop; the first group builds the row tables, later ones continue
            from the previous group's static (h, delta)."""
            if first:
                R = make_rows(P, self.S)
                R.kend = self.kend
                if nq and (nb - nq) % 256 == 0:  # the query slots would add a row of GEMM tiles
                    R.gemm_split = nb - nq
                carry["R"] = R
                h, delta = self.h, None
            else:
                h, delta = prev
            keep = self.q_idx if (nq and last and trim_last) else None
            h, delta = run_layers(P, h, delta, carry["R"], self.Kl, self.Vl, ls,
                                  kv_only_last=trim_last and last, keep=keep)
            if not (nq and last):
                return h, delta
            if keep is None:  # every row ran the last layer: pick the query slots
                h, delta = h.index_select(0, self.q_idx), delta.index_select(0, self.q_idx)
            return norm_logits(P, h.index_select(0, self.last), delta.index_select(0, self.last))[0]

        self.segs = []
        carry = {"out": []}
        for gi, ls in enumerate(groups):
            last = gi == len(groups) - 1

            def body(ls=ls, gi=gi, last=last):
                return loop(ls, gi == 0, last, carry["out"][gi - 1] if gi else None, carry)

            graph, out = _capture(body, device, self.pool)
            carry["out"].append(out)
            self.segs.append((ls, graph))
        self._carry = carry  # keeps the chained static tensors alive
        self.out = carry["out"][-1]
        # The same loop as one graph, replayed when nothing has to wait between layers (no
        # host-tier copies in flight): each graph launch leaves the GPU idle for a few microseconds
        # before its first kernel (measured ~8 us per layer boundary of a 0.5B-shaped loop).
        self.whole = None
        if len(groups) > 1:
            wcarry = {}
            self.whole, self.whole_out = _capture(lambda: loop(layers, True, True, None, wcarry), device, self.pool)
            self._wcarry = wcarry


class _QueryBucket:
    """A cache bucket without a recompute loop: a request that recomputes nothing (ratio 0, or a
    budget that rounds to 0) only replays the query forward captured over this bucket's cache."""

    def __init__(self, P, Tb, t_cap, device):
        self.t_cap, self.Tb, self.nb, self.nq = t_cap, Tb, 0, 0
        self.generation = 0
        self.queries = {}
        self.K, self.V = alloc_cache(P, t_cap, device)
        self.K.zero_()
        self.V.zero_()
        self.Kl, self.Vl = self.K.unbind(0), self.V.unbind(0)


class SubsetRunner:
    """One captured graph per (start layer, rows bucket, cache bucket, query room); LRU of
    `max_graphs`. `max_ctx`: contexts above it run eagerly (None: always graph). The default is
    the reference's 2048 (tread/graphs.py:66-70), chosen there because `run` copies the cache into
    the bucket and back; the engine assembles into its buckets instead, copies nothing, and
    constructs its runner with max_ctx=None."""

    def __init__(self, model, max_graphs=4, max_ctx=2048, trim_last=True, seg=None, max_query_buckets=2):
        from tread_amd.blend import prepared
        self.model = model
        self.P = prepared(model)
        self.max_graphs = max_graphs
        self.max_ctx = max_ctx
        self.trim_last = trim_last
        self.seg = seg
        self.graphs: "OrderedDict[tuple, _Graph]" = OrderedDict()
        # buckets of requests that recompute nothing, in an LRU of their own, so that traffic mixing
        # plain reuse with recompute does not evict (and recapture) recompute buckets; each holds a
        # full [L, 1, kv, Tb + room, hd] K/V pair (10.8 GB at a 70B shape over 32k tokens)
        self.max_query_buckets = max_query_buckets
        self.query_graphs: "OrderedDict[tuple, _QueryBucket]" = OrderedDict()
        self.captures = 0  # graphs of the recompute loop (tread/graphs.py's count, tests/test_engine.py:109)
        self.query_captures = 0  # query forwards and decoding steps captured over a bucket's cache

    def worth_it(self, T):
        return self.max_ctx is None or T <= self.max_ctx

    def _graph(self, start, n, T, n_query, device, nq=0, trim=None):
        nb, Tb = _bucket(n, T)  # the reference's bucket for the recomputed rows, plus the query slots
        nb += nq
        trim = self.trim_last if trim is None else trim
        key = (start, nb, Tb, _q_room(n_query), nq, trim)
        g = self.graphs.get(key)
        if g is None:
            while len(self.graphs) >= self.max_graphs:
                self.graphs.popitem(last=False)
            g = _Graph(self.P, start, nb, Tb, Tb + key[3], device, trim, self.seg, nq)
            self.graphs[key] = g
            self.captures += 1
        self.graphs.move_to_end(key)
        return g

    @torch.inference_mode()
    def cache_for(self, start, n, T, n_query, device, room=None, fold=False):
        """The bucket graph serving a request that recomputes n rows from layer `start` over a
        T-row context followed by n_query query rows (and `room` >= n_query rows in all after the
        context, for decoding); its .K/.V are the cache to assemble into. With fold, the query rows
        ride in the recompute graph (`run(..., hq=...)` returns the logits); otherwise the query
        forward for n_query rows is captured beside it (before anything is assembled)."""
        nq = _q_bucket(n_query) if (fold and n_query > 0) else 0
        g = self._graph(start, n, T, max(n_query, room or 0), device, nq)
        g.generation += 1  # a cache handed out for this bucket earlier is about to be overwritten
        if n_query > 0 and not nq:
            nqb = _q_bucket(n_query)
            if nqb not in g.queries:
                g.queries[nqb] = _QueryGraph(self.P, g, nqb, device)
                self.query_captures += 1
        return g

    @torch.inference_mode()
    def query_cache_for(self, T, n_query, device, room=None, t_step=1024):
        """The bucket serving a request that recomputes nothing over a T-row context: its .K/.V
        are the cache to assemble into, and the query forward for n_query rows is captured over it
        (before anything is assembled); rows after the context: room >= n_query (for decoding)."""
        Tb = -(-T // t_step) * t_step
        key = (Tb, _q_room(max(n_query, room or 0)))
        g = self.query_graphs.get(key)
        if g is None:
            while len(self.query_graphs) >= self.max_query_buckets:
                self.query_graphs.popitem(last=False)
            g = _QueryBucket(self.P, Tb, Tb + key[1], device)
            self.query_graphs[key] = g
        self.query_graphs.move_to_end(key)
        g.generation += 1  # a cache handed out for this bucket earlier is about to be overwritten
        nqb = _q_bucket(n_query)
        if nqb not in g.queries:
            g.queries[nqb] = _QueryGraph(self.P, g, nqb, device)
            self.query_captures += 1
        return g

    @torch.inference_mode()
    def query(self, g, ids, T, hook=None):
        """Replay the captured query forward of bucket `g` for query token ids at rows T.. of its
        cache; returns the last query row's logits [vocab]. `hook(l)` runs for every layer first."""
        n = ids.numel()
        q = g.queries.get(_q_bucket(n))
        if q is None or T + q.nq > g.t_cap:
            raise ValueError(f"no captured query forward for {n} rows at T={T} in this bucket")
        if hook is not None:
            for l in range(self.P.L):
                hook(l)
        q.ids[:n].copy_(ids)
        if n < q.nq:
            q.ids[n:].zero_()
        torch.arange(T, T + q.nq, out=q.pos)
        if q.last_n != n:  # a decoding step keeps n: no fill launch per token
            q.last.fill_(n - 1)
            q.last_n = n
        q.graph.replay()
        return q.out

    def fits(self, g, n, T):
        """Whether n rows appended at row T fit the padded query forward of bucket g."""
        return T + _q_bucket(n) <= g.t_cap

    @torch.inference_mode()
    def decode(self, g, ids, T):
        """One decoding step on bucket g's cache: the query forward for the token ids at rows
        T.., replayed from a graph (captured on first use for this row bucket; its capture-time
        rows are the bucket's top rows, which hold no valid cache rows yet or are rewritten
        before they are read). Returns the last row's logits [vocab]."""
        nq = _q_bucket(ids.numel())
        if nq not in g.queries:
            g.queries[nq] = _QueryGraph(self.P, g, nq, ids.device)
            self.query_captures += 1
        return self.query(g, ids, T)

    @torch.inference_mode()
    def run(self, h, S, K, V, start):
        """tread/graphs.py:75-99, the reference's call form: recompute layers start..L-1 for sorted
        positions S (len n) with hidden rows h [1, n, H]; K, V are per-layer lists [1, kv, T, hd] for
        those layers. The layers are copied into the bucket's static cache, its captured loop is
        replayed (every layer complete, the last one's hidden rows included), and (h [1, n, H] after
        layer L-1, K list, V list) is returned, K/V being views of the bucket's buffers, valid until
        the next replay of the same bucket. The engine skips both copies by assembling straight into
        a bucket (`cache_for`) and replaying it with `replay`."""
        n, T = len(S), K[0].shape[2]
        if len(K) != self.P.L - start or len(V) != len(K):
            raise ValueError(f"run: K/V must hold layers {start}..{self.P.L - 1}")
        g = self._graph(start, n, T, 0, S.device, trim=False)
        g.generation += 1  # a cache handed out for this bucket earlier is about to be overwritten
        for i, (k, v) in enumerate(zip(K, V)):
            g.K[start + i, :, :, :T].copy_(k)
            g.V[start + i, :, :, :T].copy_(v)
        hh, d = self.replay(g, h.reshape(n, -1), S, T)
        out = (hh[:n] + d[:n])[None]  # the residual add the last layer's output defers
        return out, list(g.K[start:, :, :, :T].unbind(0)), list(g.V[start:, :, :, :T].unbind(0))

    @torch.inference_mode()
    def replay(self, g, h, S, T, hook=None, hq=None):
        """Replay layers start..L-1 of bucket graph `g` for sorted positions S (len n) with hidden
        rows h [n, H] over a T-row context, and, for a bucket with query slots, the query rows hq
        [m, H] (m <= g.nq) at positions T, T+1, ...; returns the last query row's logits then
        (static), else the last segment's static (h, delta). `hook(l)` runs before the graph
        segment holding layer l (lazy assembly must complete before the replay reads that layer)."""
        n, m = len(S), (0 if hq is None else hq.shape[0])
        rows = n + g.nq
        pad = g.nb - rows
        if rows > g.nb or T + pad > g.Tb or m > g.nq or (g.nq > 0) != (m > 0):
            raise ValueError(f"request (n={n}, queries={m}, T={T}) does not fit bucket "
                             f"(nb={g.nb}, Tb={g.Tb}, query slots={g.nq})")
        dev = S.device
        g.S[:n].copy_(S)
        g.h[:n].copy_(h)
        if g.nq:
            torch.arange(T, T + g.nq, out=g.S[n:rows])
            g.h[n:n + m].copy_(hq)
            torch.arange(n, rows, out=g.q_idx)
            g.last.fill_(m - 1)
        if pad:
            # padded rows: spare cache rows after the query slots, no visible key
            torch.arange(T + g.nq, T + g.nq + pad, out=g.S[rows:])
        g.kend[:rows].copy_(g.S[:rows])
        g.kend[rows:].fill_(-1)
        if g.nb > n + m:
            g.h[n + m:].zero_()
        if hook is None and g.whole is not None:
            g.whole.replay()
            return g.whole_out
        for ls, graph in g.segs:
            if hook is not None:
                for l in ls:
                    hook(l)
            graph.replay()
        return g.out
