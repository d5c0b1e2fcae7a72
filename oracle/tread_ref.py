"""tread's store / engine / blend path restated on the CPU. TEST INFRASTRUCTURE ONLY.

Every function follows the reference op for op (cited file:line under the reference tree), with
the model math from oracle.model_ref. Runs in fp32 or bf16; in bf16 every torch op rounds where
the reference's does (e.g. rotate_keys casts cos/sin to bf16 and rounds each product and sum).
It runs where its model's weights are (oracle.model_ref.load's device; inputs on that device):
on the CPU as the oracle, or on a GPU as a second backend of the same torch code, whose roundings
(GEMM kernels, attention kernel, libm) differ from the CPU's.
"""
import hashlib
from collections import OrderedDict
from dataclasses import dataclass, field

import torch

from oracle import model_ref as M


# ----------------------------------------------------------------------------- store (tread/store.py)

def block_key(*parts) -> str:
    """tread/store.py:21-30: sha256 over parts; tensors as native int64 bytes, others as str(p)
    in UTF-8; a NUL byte after every part."""
    h = hashlib.sha256()
    for p in parts:
        if isinstance(p, torch.Tensor):
            h.update(p.detach().to("cpu", torch.int64).numpy().tobytes())
        else:
            h.update(str(p).encode())
        h.update(b"\x00")
    return h.hexdigest()


@dataclass
class Block:
    """tread/store.py:33-41."""
    K: torch.Tensor
    V: torch.Tensor
    base: int
    n_tokens: int
    nbytes: int
    device: torch.device
    hits: int = 0


@dataclass
class StoreStats:
    """tread/store.py:44-53."""
    hits: int = 0
    misses: int = 0
    evictions: int = 0
    bytes_used: int = 0
    cpu_hits: int = 0
    offloads: int = 0
    cpu_evictions: int = 0
    cpu_bytes_used: int = 0


class BlockStore:
    """tread/store.py:56-125: GPU-tier LRU under `budget`, spilling to a CPU-tier LRU under
    `cpu_budget`. On the CPU oracle both tiers hold CPU tensors; the tier move is a clone."""

    def __init__(self, budget_bytes, cpu_budget_bytes=0):
        self.budget = budget_bytes
        self.cpu_budget = cpu_budget_bytes
        self.blocks = OrderedDict()
        self.cpu_blocks = OrderedDict()
        self.stats = StoreStats()

    def get(self, key):  # store.py:64-80
        b = self.blocks.get(key)
        if b is not None:
            self.blocks.move_to_end(key)
        else:
            b = self.cpu_blocks.pop(key, None)
            if b is None:
                self.stats.misses += 1
                return None
            self.stats.cpu_bytes_used -= b.nbytes
            self.stats.cpu_hits += 1
            b.K, b.V = b.K.clone(), b.V.clone()
            self._insert(key, b)
        b.hits += 1
        self.stats.hits += 1
        return b

    def put(self, key, K, V, base):  # store.py:82-91
        nbytes = K.numel() * K.element_size() + V.numel() * V.element_size()
        if nbytes > self.budget:
            return None
        for tier in (self.blocks, self.cpu_blocks):
            if key in tier:
                self._remove(tier, key)
        b = Block(K=K, V=V, base=base, n_tokens=K.shape[-2], nbytes=nbytes, device=K.device)
        self._insert(key, b)
        return b

    def _insert(self, key, b):  # store.py:93-97
        while self.stats.bytes_used + b.nbytes > self.budget:
            self._evict_gpu()
        self.blocks[key] = b
        self.stats.bytes_used += b.nbytes

    def _evict_gpu(self):  # store.py:99-115
        key, b = self.blocks.popitem(last=False)
        self.stats.bytes_used -= b.nbytes
        self.stats.evictions += 1
        if b.nbytes > self.cpu_budget:
            return
        while self.stats.cpu_bytes_used + b.nbytes > self.cpu_budget:
            _, old = self.cpu_blocks.popitem(last=False)
            self.stats.cpu_bytes_used -= old.nbytes
            self.stats.cpu_evictions += 1
        nb = Block(K=b.K.clone(), V=b.V.clone(), base=b.base, n_tokens=b.n_tokens, nbytes=b.nbytes,
                   device=b.device, hits=b.hits)
        self.cpu_blocks[key] = nb
        self.stats.cpu_bytes_used += nb.nbytes
        self.stats.offloads += 1

    def _remove(self, tier, key):  # store.py:117-122
        b = tier.pop(key)
        if tier is self.blocks:
            self.stats.bytes_used -= b.nbytes
        else:
            self.stats.cpu_bytes_used -= b.nbytes

    def __len__(self):
        return len(self.blocks) + len(self.cpu_blocks)


# ----------------------------------------------------------------------------- blend (tread/blend.py)

def prefill_kv(m, ids):
    """tread/blend.py:12-19: forward over ids from an empty cache; per-layer K, V lists."""
    _, K, V = M.forward(m, ids)
    return K, V


def _delta_cos_sin(m, delta, dtype):
    """cos/sin of the one position `delta` as [1, hd], broadcast over a block's rows. The reference
    builds rotary_emb(K, full((1, n), delta)), n identical rows (tread/blend.py:34-36); computing
    the row once keeps every row's fp32 cos/sin identical, as they are in the reference, where
    torch's CPU threading would otherwise split a large [n, hd] table into chunks whose ragged
    tails go through a second cos/sin routine."""
    cos, sin = M.rope_cos_sin(m, torch.full((1,), delta, dtype=torch.long), dtype)
    return cos[0], sin[0]


def rotate_keys(m, K, delta):
    """tread/blend.py:22-39: delta 0 returns K itself; otherwise cos/sin of delta in K.dtype and
    K*cos + rotate_half(K)*sin (attention_scaling is 1 for default RoPE)."""
    if delta == 0:
        return K
    cos, sin = _delta_cos_sin(m, delta, K.dtype)
    return K * cos + M.rotate_half(K) * sin


def rotate_keys_fp32(m, K, delta):
    """The fp32 reference for a re-rotation: fp32 K, unrounded fp32 cos/sin, one rounding to K.dtype."""
    if delta == 0:
        return K.clone()
    cos, sin = _delta_cos_sin(m, delta, torch.float32)
    K32 = K.float()
    return (K32 * cos + M.rotate_half(K32) * sin).to(K.dtype)


def chunk_kv(m, prefix_ids, doc_ids, mode):
    """tread/blend.py:42-54."""
    if mode == "shared":
        K, V = prefill_kv(m, torch.cat([prefix_ids, doc_ids]))
        P = len(prefix_ids)
        return [k[:, :, P:] for k in K], [v[:, :, P:] for v in V], P
    K, V = prefill_kv(m, doc_ids)
    return K, V, 0


def assemble(m, prefix_ids, docs_ids, mode):
    """tread/blend.py:57-68: exact prefix KV + per-doc KV rotated to its offset, concatenated."""
    Kp, Vp = prefill_kv(m, prefix_ids)
    Ks, Vs = [[k] for k in Kp], [[v] for v in Vp]
    offset = len(prefix_ids)
    for d in docs_ids:
        Kd, Vd, base = chunk_kv(m, prefix_ids, d, mode)
        for l in range(len(Ks)):
            Ks[l].append(rotate_keys(m, Kd[l], offset - base))
            Vs[l].append(Vd[l])
        offset += len(d)
    return [torch.cat(x, dim=2) for x in Ks], [torch.cat(x, dim=2) for x in Vs]


def subset_ctx(m, S, T, dtype):
    """tread/blend.py:71-79: RoPE for positions S and the bool mask key <= S[i] over T keys."""
    rope = M.rope_cos_sin(m, S, dtype)
    mask = (torch.arange(T, device=S.device)[None, :] <= S[:, None])[None, None]
    return rope, mask


def layer_subset(m, l, h, S, K, V, inplace=False, ctx=None):
    """tread/blend.py:93-114: recompute layer l for rows S; splice fresh k/v at S before attention."""
    (cos, sin), mask = ctx if ctx is not None else subset_ctx(m, S, K.shape[2], h.dtype)
    x = M.norm(m, f"model.layers.{l}.input_layernorm", h)
    q, k, v = M.qkv(m, l, x, cos, sin)
    if not inplace:
        K, V = K.clone(), V.clone()
    K[:, :, S], V[:, :, S] = k, v
    o = M.o_proj(m, l, M.attend(m, q, K, V, mask))
    h = h + o
    h = h + M.mlp(m, l, M.norm(m, f"model.layers.{l}.post_attention_layernorm", h))
    return h, K, V


def layer_subset_rows(m, l, h, S, K, V, ctx, chunk=4096):
    """layer_subset with the attention and the MLP evaluated over chunks of `chunk` rows, so a
    32 000-row deviation pass over a 32k cache stays within host memory; every fresh k/v is spliced
    before any row attends, as in layer_subset (inplace). Row i's result depends on row i only
    once the cache is spliced, so the chunking changes nothing (pinned against layer_subset)."""
    (cos, sin), mask = ctx
    x = M.norm(m, f"model.layers.{l}.input_layernorm", h)
    q, k, v = M.qkv(m, l, x, cos, sin)
    K[:, :, S], V[:, :, S] = k, v
    out = torch.empty_like(h)
    for a in range(0, h.shape[1], chunk):
        b = min(a + chunk, h.shape[1])
        o = M.o_proj(m, l, M.attend(m, q[:, :, a:b], K, V, mask[:, :, a:b]))
        hc = h[:, a:b] + o
        out[:, a:b] = hc + M.mlp(m, l, M.norm(m, f"model.layers.{l}.post_attention_layernorm", hc))
    return out, K, V


def deviation_score(k1, v1, K1c, V1c):
    """The score expression of tread/blend.py:129 on gathered cache rows: per-head L2 norm of the
    k and v differences, summed over heads, k part + v part (each op in the input dtype)."""
    return (k1 - K1c).norm(dim=-1).sum(dim=1) + (v1 - V1c).norm(dim=-1).sum(dim=1)


def layer1_deviation(m, ctx_ids, K, V, all_c, inplace=False):
    """tread/blend.py:117-130."""
    h0 = M.embed(m, ctx_ids[all_c])[None]
    ctx = subset_ctx(m, all_c, K[0].shape[2], h0.dtype)
    h, K0, V0 = layer_subset(m, 0, h0, all_c, K[0], V[0], inplace=inplace, ctx=ctx)
    x1 = M.norm(m, "model.layers.1.input_layernorm", h)
    _, k1, v1 = M.qkv(m, 1, x1, *ctx[0])
    dev = deviation_score(k1, v1, K[1][:, :, all_c], V[1][:, :, all_c])
    return dev[0], h, K0, V0, (k1, v1)


def blend(m, ctx_ids, K, V, candidates, ratio, policy, gen=None, inplace=False, trace=None):
    """tread/blend.py:133-179. `trace` (a dict, optional) receives dev, top and S for the checks.

    Test hook (not reference behaviour): trace["force_S"], a tensor of candidate positions, replaces
    the deviation top-k selection, so that a test can compare numerics under one shared selection
    when two implementations split a near-tie differently."""
    K, V = list(K), list(V)
    if not candidates:
        return K, V, torch.empty(0, dtype=torch.long), 0.0
    all_c = torch.cat(candidates)
    budget = int(round(ratio * len(all_c)))
    if budget == 0:
        return K, V, all_c[:0], 0.0
    start = 0
    if policy == "boundary":
        rank = torch.cat([torch.arange(len(c), device=c.device) for c in candidates])
        S = all_c[rank.argsort(stable=True)[:budget]]
    elif policy == "random":
        S = all_c[torch.randperm(len(all_c), generator=gen).to(all_c.device)[:budget]]
    elif policy == "deviation":
        dev, h, K[0], V[0], kv1 = layer1_deviation(m, ctx_ids, K, V, all_c, inplace=inplace)
        top = dev.topk(budget).indices
        if trace is not None and trace.get("force_S") is not None:
            where = {int(p): i for i, p in enumerate(all_c.tolist())}
            top = torch.tensor([where[int(p)] for p in trace["force_S"].tolist()], dtype=torch.long,
                               device=all_c.device)
        if trace is not None:
            trace.update(dev=dev, top=top, all_c=all_c, kv1=kv1)
        S, h, start = all_c[top], h[:, top], 1
    else:
        raise ValueError(policy)
    S, order = S.sort()
    if start == 0:
        h = M.embed(m, ctx_ids[S])[None]
    else:
        h = h[:, order]
    if trace is not None:
        trace["S"] = S
    ctx = subset_ctx(m, S, K[0].shape[2], h.dtype)
    for l in range(start, m.L):
        h, K[l], V[l] = layer_subset(m, l, h, S, K[l], V[l], inplace=inplace, ctx=ctx)
    L, n = m.L, len(all_c)
    eff = (len(S) * (L - start) + start * n) / (n * L)
    return K, V, S, eff


def bucket(n, T, n_min=64, n_step=256, t_step=1024):
    """tread/graphs.py:22-27: padded (rows, cache length) bucket for a graphed recompute."""
    nb = max(n_min, 1 << (n - 1).bit_length()) if n <= n_step else -(-n // n_step) * n_step
    Tb = -(-(T + nb - n) // t_step) * t_step
    return nb, Tb


# ----------------------------------------------------------------------------- engine (tread/engine.py)

@dataclass
class RequestStats:
    """tread/engine.py:19-26."""
    hits: int = 0
    misses: int = 0
    tokens_reused: int = 0
    tokens_prefilled: int = 0
    recompute_eff: float = 0.0
    t: dict = field(default_factory=dict)


class _Tmp:
    """tread/engine.py:169-173."""

    def __init__(self, K, V, base):
        self.K, self.V, self.base, self.n_tokens = K, V, base, K.shape[-2]


def sig_of(cfg, dtype):
    """tread/engine.py:36-38 for a config-constructed model: (name_or_path, str(dtype), theta, scaling)."""
    return (getattr(cfg, "_name_or_path", ""), str(dtype), getattr(cfg, "rope_theta", None),
            getattr(cfg, "rope_scaling", None))


class Engine:
    """tread/engine.py:29-152 on the oracle model."""

    def __init__(self, m, store, sig=None):
        self.m = m
        self.store = store
        self.sig = sig if sig is not None else sig_of(m.cfg, m.dtype)

    def prefix_block(self, prefix_ids, st, namespace=""):  # engine.py:44-57
        key = block_key(*self.sig, namespace, "prefix", prefix_ids)
        b = self.store.get(key)
        if b is None:
            st.misses += 1
            st.tokens_prefilled += len(prefix_ids)
            K, V = (torch.stack(x) for x in prefill_kv(self.m, prefix_ids))
            b = self.store.put(key, K, V, 0) or _Tmp(K, V, 0)
        else:
            st.hits += 1
            st.tokens_reused += len(prefix_ids)
        return key, b

    def doc_keys(self, prefix_key, docs):
        return [block_key(*self.sig, prefix_key, d) for d in docs]

    def doc_blocks(self, prefix_key, pb, docs, st):  # engine.py:59-96
        keys = self.doc_keys(prefix_key, docs)
        blocks = [self.store.get(k) for k in keys]
        miss = [i for i, b in enumerate(blocks) if b is None]
        st.hits += len(docs) - len(miss)
        st.tokens_reused += sum(len(d) for d, b in zip(docs, blocks) if b is not None)
        if not miss:
            return blocks
        st.misses += len(miss)
        P = pb.n_tokens
        ids = torch.cat([docs[i] for i in miss])
        n, dev = len(ids), ids.device
        seg = torch.cat([torch.full((len(docs[i]),), j, device=dev) for j, i in enumerate(miss)])
        local = torch.cat([torch.arange(len(docs[i]), device=dev) for i in miss])
        st.tokens_prefilled += n
        allowed = torch.ones(n, P + n, dtype=torch.bool, device=dev)
        allowed[:, P:] = (seg[:, None] == seg[None, :]) & (local[:, None] >= local[None, :])
        mask = torch.zeros(1, 1, n, P + n, dtype=self.m.dtype, device=dev)
        mask.masked_fill_(~allowed, torch.finfo(self.m.dtype).min)
        _, Kl, Vl = M.forward(self.m, ids, past=(list(pb.K.unbind(0)), list(pb.V.unbind(0))),
                              position_ids=P + local, mask4d=mask)
        Kall, Vall = torch.stack(Kl)[..., P:, :], torch.stack(Vl)[..., P:, :]
        off = 0
        for i in miss:
            Ld = len(docs[i])
            K, V = Kall[..., off:off + Ld, :].contiguous(), Vall[..., off:off + Ld, :].contiguous()
            blocks[i] = self.store.put(keys[i], K, V, P) or _Tmp(K, V, P)
            off += Ld
        return blocks

    def assemble_blocks(self, prefix_ids, docs, st, namespace=""):
        """engine.py:107-120: returns per-layer K, V lists and the candidate ranges."""
        pkey, pb = self.prefix_block(prefix_ids, st, namespace)
        Ks, Vs = [pb.K], [pb.V]
        offset = pb.n_tokens
        cands = []
        for d, b in zip(docs, self.doc_blocks(pkey, pb, docs, st)):
            Ks.append(rotate_keys(self.m, b.K, offset - b.base))
            Vs.append(b.V)
            cands.append(torch.arange(offset, offset + len(d), device=prefix_ids.device))
            offset += len(d)
        K = list(torch.cat(Ks, dim=-2).unbind(0))
        V = list(torch.cat(Vs, dim=-2).unbind(0))
        return K, V, cands

    def prefill(self, prefix_ids, docs, query_ids, ratio=0.0, policy="deviation", namespace="",
                gen=None, trace=None):  # engine.py:98-136
        st = RequestStats()
        K, V, cands = self.assemble_blocks(prefix_ids, docs, st, namespace)
        if ratio > 0:
            ctx = torch.cat([prefix_ids] + list(docs))
            K, V, _, st.recompute_eff = blend(self.m, ctx, K, V, cands, ratio, policy, gen=gen, inplace=True,
                                              trace=trace)
        h, Kq, Vq = M.forward(self.m, query_ids, past=(K, V))
        return M.logits_last(self.m, h), (Kq, Vq), st

    def prefill_prefix_only(self, prefix_ids, docs, query_ids):  # engine.py:138-152
        st = RequestStats()
        _, pb = self.prefix_block(prefix_ids, st)
        rest = torch.cat(list(docs) + [query_ids])
        st.tokens_prefilled += len(rest) - len(query_ids)
        h, K, V = M.forward(self.m, rest, past=(list(pb.K.unbind(0)), list(pb.V.unbind(0))))
        return M.logits_last(self.m, h), (K, V), st


def prefill_full(m, prefix_ids, docs, query_ids):
    """tread/engine.py:155-166: no caching at all."""
    ids = torch.cat([prefix_ids] + list(docs) + [query_ids])
    h, K, V = M.forward(m, ids)
    st = RequestStats(tokens_prefilled=len(ids) - len(query_ids))
    return M.logits_last(m, h), (K, V), st


def generate_greedy(m, logits, K, V, max_tokens, eos_ids=(), forced=None):
    """tread/server.py:194-210, the greedy loop after `engine.prefill`: next = argmax(logits); stop
    on an eos id or after max_tokens tokens; every emitted token is run through the model on top
    of the cache (the reference's DynamicCache path, concatenating K/V) to give the next logits.
    `forced` (a token list) replaces the argmax picks, so another implementation's tokens can be
    replayed step by step (test hook, not reference behaviour).
    Returns (tokens, finish_reason, per-step logits [logits of the prompt, then one per token])."""
    out, steps = [], [logits]
    reason = "stop"
    while True:
        nxt = int(logits.argmax()) if forced is None else forced[len(out)] if len(out) < len(forced) else None
        if nxt is None or nxt in eos_ids:
            break
        if len(out) >= max_tokens:
            reason = "length"
            break
        out.append(nxt)
        h, K, V = M.forward(m, torch.tensor([nxt], device=m.device), past=(K, V))
        logits = M.logits_last(m, h)
        steps.append(logits)
    return out, reason, steps


def kl(a, b):
    """tests/test_engine.py:42-43."""
    import torch.nn.functional as F
    return F.kl_div(F.log_softmax(a.float(), -1), F.log_softmax(b.float(), -1), log_target=True,
                    reduction="sum").item()
