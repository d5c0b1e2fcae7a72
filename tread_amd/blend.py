"""KV ops of the reuse path: re-rotation, assembly, deviation scoring and selective recompute.

Public names and signatures follow tread/blend.py (prefill_kv, rotate_keys, chunk_kv, assemble,
_subset_ctx, _qkv, _layer_subset, layer1_deviation, blend, to_cache), including the private
helpers phase0/blend.py re-exports, so callers written against the reference keep working; the
engine itself runs the fused forms underneath (forward.layer_forward, blend_cache, blend_query).
KV tensors are [1, kv_heads, T, head_dim] per layer (post-RoPE keys), blocks are stacked
[L, 1, kv_heads, n, head_dim]. All arithmetic runs in the HIP kernels of
libtread_hip.so (tread_amd._hip) plus torch GEMMs; bf16 on the GPU only.
"""
import weakref

import torch
import torch.nn.functional as F

from tread_amd import _hip
from tread_amd.cache import KVCache
from tread_amd.forward import Rows, alloc_cache, embed, final_logits, make_rows, run_layers, layer_forward
from tread_amd.model import prepare

_PREPARED = weakref.WeakKeyDictionary()


def prepared(model):
    """Fused-weight view of `model` (built once per model object)."""
    P = _PREPARED.get(model)
    if P is None:
        if model.dtype != torch.bfloat16:
            raise TypeError(f"the HIP path computes in bf16; model dtype is {model.dtype}")
        P = prepare(model)
        _PREPARED[model] = P
    return P


def forward_into(model, ids, K, V, start_row=0, pos=None, kseg=None, n_shared=0, want_logits=True):
    """Forward `ids` whose k/v land in cache rows start_row.. of K, V ([L, 1, kv, t_cap, hd]),
    attending causally to every earlier row (or block-diagonally with kseg / n_shared)."""
    P = prepared(model)
    n = len(ids)
    rows = torch.arange(start_row, start_row + n, device=ids.device)
    R = make_rows(P, rows, pos=pos, kseg=kseg, n_shared=n_shared)
    Kl, Vl = K.unbind(0), V.unbind(0)
    h, d = run_layers(P, embed(P, ids), None, R, Kl, Vl, range(P.L))
    return final_logits(P, h, d) if want_logits else None


def prefill_kv(model, ids):
    """tread/blend.py:12-19: per-layer (K, V) lists of a forward over `ids` from position 0."""
    P = prepared(model)
    K, V = alloc_cache(P, len(ids), ids.device)
    forward_into(model, ids, K, V, want_logits=False)
    return list(K.unbind(0)), list(V.unbind(0))


def rotate_keys(model, K, delta):
    """tread/blend.py:22-39: shift post-RoPE keys by `delta` positions, R(p + delta) = R(delta) R(p).

    delta 0 returns K itself. Otherwise one K-only pass of the fused re-rotation kernel with fp32
    cos/sin and one rounding to bf16 (the fp32 reference rotation, op for op). K: [..., n, hd] with
    any leading dims (e.g. [L, 1, kv, n, hd])."""
    if delta == 0:
        return K
    P = prepared(model)
    shape = K.shape
    Kc = K.contiguous().reshape(-1, 1, 1, shape[-2], shape[-1])
    out = torch.empty_like(Kc)
    _hip.rope_assemble([(Kc, None, 0, delta)], out, None, P.inv_freq)
    return out.reshape(shape)


def chunk_kv(model, prefix_ids, doc_ids, mode):
    """tread/blend.py:42-54."""
    if mode == "shared":
        K, V = prefill_kv(model, torch.cat([prefix_ids, doc_ids]))
        P = len(prefix_ids)
        return [k[:, :, P:] for k in K], [v[:, :, P:] for v in V], P
    K, V = prefill_kv(model, doc_ids)
    return K, V, 0


def assemble(model, prefix_ids, docs_ids, mode):
    """tread/blend.py:57-68: exact prefix KV + independently computed doc KV, re-rotated and
    gathered into one cache by the fused kernel. Returns per-layer K, V lists [1, kv, T, hd]."""
    P_ = prepared(model)
    Kp, Vp = prefill_kv(model, prefix_ids)
    srcs = [(torch.stack(Kp), torch.stack(Vp), 0, 0)]
    offset = len(prefix_ids)
    for d in docs_ids:
        Kd, Vd, base = chunk_kv(model, prefix_ids, d, mode)
        srcs.append((torch.stack(Kd).contiguous(), torch.stack(Vd).contiguous(), offset, offset - base))
        offset += len(d)
    K, V = alloc_cache(P_, offset, prefix_ids.device)
    _hip.rope_assemble(srcs, K, V, P_.inv_freq)
    return list(K.unbind(0)), list(V.unbind(0))


class SubsetCtx(tuple):
    """What tread/blend.py:71-79 returns, (rope, mask): rope = (cos, sin) [1, n, hd] in the dtype
    of `ref` (the reference's rotary_emb rounding), mask [1, 1, n, T] bool, key <= S[i]. It also
    carries `rows`, the per-row RoPE tables and key ends the HIP layer consumes, so a context built
    once serves every layer of a blend without rebuilding either."""

    def __new__(cls, rope, mask, rows):
        obj = super().__new__(cls, (rope, mask))
        obj.rows = rows
        return obj


def _layer_index(model, layer):
    """Index of `layer` (a decoder layer module of `model`, or an int) in model.model.layers."""
    if isinstance(layer, int):
        return layer
    for i, lyr in enumerate(model.model.layers):
        if lyr is layer:
            return i
    raise ValueError("layer is not a decoder layer of this model")


def _rows_of(model, S, ctx=None):
    """Rows for positions S: from a SubsetCtx, from a (rope, mask) pair built elsewhere (its
    tables are taken as given; the reference's mask is always key <= S[i]), or built here."""
    P = prepared(model)
    if isinstance(ctx, SubsetCtx):
        return ctx.rows
    if ctx is not None:
        (cos, sin), _ = ctx
        half = P.hd // 2
        rows = S.to(torch.int64).contiguous()
        return Rows(rows=rows, kend=rows, cos=cos.reshape(-1, P.hd)[:, :half].contiguous(),
                    sin=sin.reshape(-1, P.hd)[:, :half].contiguous())
    return make_rows(P, S)


def _subset_ctx(model, S, T, ref):
    """tread/blend.py:71-79: per-blend constants for positions S against a T-row cache: RoPE
    (cos, sin) [1, n, hd] in ref.dtype and the bool mask arange(T)[None] <= S[:, None] as
    [1, 1, n, T]. The tables come from the HIP rope-table kernel (the reference's rotary_emb
    rounding); the attention kernel itself evaluates key <= S[i] and never reads the mask."""
    P = prepared(model)
    R = make_rows(P, S)
    dt = ref.dtype
    cos = torch.cat([R.cos, R.cos], dim=-1).to(dt)[None]
    sin = torch.cat([R.sin, R.sin], dim=-1).to(dt)[None]
    mask = (torch.arange(T, device=S.device)[None, :] <= S[:, None])[None, None]
    return SubsetCtx((cos, sin), mask, R)


def _qkv(layer, model, x, pos, rope=None):
    """tread/blend.py:82-90: q/k/v projections of x [1, n, H] (already normed) and RoPE at
    positions pos. Returns q [1, hq, n, hd], k and v [1, hkv, n, hd] (q and k rotated). `layer` is
    the decoder layer module (or its index); `rope` an optional (cos, sin) as _subset_ctx gives.
    One fused q|k|v GEMM, then the HIP RoPE kernel writes rotated q, k and v in head-major order."""
    P = prepared(model)
    l = _layer_index(model, layer)
    lw = P.layers[l]
    n = x.shape[-2]
    R = _rows_of(model, pos, None if rope is None else (rope, None))
    qkv = F.linear(x.reshape(n, P.H), lw.wqkv, lw.bqkv)
    q = torch.empty(n, P.hq, P.hd, dtype=x.dtype, device=x.device)
    k = torch.empty(1, P.hkv, n, P.hd, dtype=x.dtype, device=x.device)
    v = torch.empty_like(k)
    local = torch.arange(n, device=x.device)
    _hip.qkv_rope_splice(qkv, R.cos, R.sin, local, P.hq, P.hkv, P.hd, k, v, q_out=q)
    return q.transpose(0, 1)[None], k, v


def _layer_subset(layer, model, h, S, K, V, inplace=False, ctx=None):
    """tread/blend.py:93-114: recompute decoder layer `layer` (module or index) for positions S
    against the full layer cache K, V [1, kv, T, hd]; fresh k/v are spliced at S before attention
    (in place when `inplace`, else into copies). h: [1, n, H]; ctx: _subset_ctx(...), built once
    per blend. Returns (h, K, V)."""
    P = prepared(model)
    l = _layer_index(model, layer)
    R = _rows_of(model, S, ctx)
    if not inplace:
        K, V = K.clone(), V.clone()
    Kl, Vl = {l: K}, {l: V}
    h2, d = layer_forward(P, l, h[0].contiguous(), None, R, Kl, Vl)
    return (h2 + d)[None], K, V


def _deviation(P, ctx_ids, Kl, Vl, all_c, hook=None):
    """Layer 0 for all candidates (k/v spliced into layer 0 in place), then layer-1 k/v and the
    fused deviation score. Returns (score bf16 [n], hidden entering layer 1 [n, H], rows).
    `hook(1)` runs right before the score reads layer 1 of the cache (its copy may still fly
    during layer 0)."""
    R = make_rows(P, all_c)
    h, d = layer_forward(P, 0, embed(P, ctx_ids[all_c]), None, R, Kl, Vl)
    lw = P.layers[1]
    h, x = _hip.add_rmsnorm(h, lw.ln1, P.eps, delta=d)
    q_rows = P.hq * P.hd
    kv = F.linear(x, lw.wqkv[q_rows:], None if lw.bqkv is None else lw.bqkv[q_rows:])
    if hook is not None:
        hook(1)
    score = _hip.dev_score(kv, R.cos, R.sin, R.rows, P.hkv, P.hd, Kl[1], Vl[1])
    return score, h, R


def layer1_deviation(model, ctx_ids, K, V, all_c, inplace=False):
    """tread/blend.py:117-130. Returns (dev [n] bf16, layer-0 hidden [1, n, H], K0, V0)."""
    P = prepared(model)
    K, V = list(K), list(V)
    if not inplace:
        K[0], V[0] = K[0].clone(), V[0].clone()
    score, h, _ = _deviation(P, ctx_ids, K, V, all_c)
    return score, h[None], K[0], V[0]


def select(ratio, candidates):
    """Selection budget of tread/blend.py:144-145 (Python round-half-even)."""
    n = sum(len(c) for c in candidates)
    return n, int(round(ratio * n))


def blend_cache(model, ctx_ids, K, V, candidates, ratio, policy, gen=None, runner=None, graph=None, T=None,
                hook=None, trim_last=True):
    """Selective recompute in place on per-layer cache lists K, V (tread/blend.py:133-179).

    With `graph` (a SubsetRunner bucket whose buffers K, V are) the layer loop is replayed from
    the captured hipGraph; T is then the context length (rows before the query).
    `hook(l)`, if given, runs before layer l is first read (lazy assembly of in-flight blocks).
    With trim_last, the last layer only splices its k/v: its hidden output is discarded by the
    reference as well, so K/V are unchanged. Returns (S, eff)."""
    S, eff, _ = _blend(model, ctx_ids, K, V, candidates, ratio, policy, gen, runner, graph, T, hook, trim_last, None)
    return S, eff


def blend_query(model, ctx_ids, K, V, candidates, ratio, policy, query_ids, T, gen=None, runner=None, graph=None,
                hook=None, trim_last=True):
    """blend_cache with the query forward of tread/engine.py:131-132 folded into the recompute: the
    query rows (positions T, T+1, ...) join the recomputed rows from the first recomputed layer on
    (with the deviation policy their layer 0 runs right after the deviation pass, on its own: 32
    000 + 32 rows would cost the layer's GEMMs an extra row of tiles), so their projections ride
    in the recompute's GEMMs.
    Layer by layer they see what the reference's query forward sees afterwards: the layer's
    recomputed rows are spliced before its attention, and a layer's cache does not change once
    it is recomputed. At the last layer every row splices its k/v and only the query rows run the
    rest. Returns (S, eff, logits of the last query row [vocab]); logits is None when nothing is
    recomputed (the caller then runs the query forward itself). With `graph` the logits are the
    graph's static output."""
    return _blend(model, ctx_ids, K, V, candidates, ratio, policy, gen, runner, graph, T, hook, trim_last, query_ids)


def _select(P, ctx_ids, K, V, candidates, all_c, budget, policy, gen, hook=None):
    """The selection of tread/blend.py:144-162: sorted positions S [budget], their hidden rows
    h [budget, H] entering layer `start` and `start` (1 after the deviation pass, which has
    recomputed layer 0 of every candidate in place in K[0], V[0])."""
    dev = all_c.device
    if policy == "boundary":
        rank = torch.cat([torch.arange(len(c), device=c.device) for c in candidates])
        S = all_c[rank.argsort(stable=True)[:budget]].sort().values
        return S, embed(P, ctx_ids[S]), 0
    if policy == "random":
        S = all_c[torch.randperm(len(all_c), generator=gen, device="cpu").to(dev)[:budget]].sort().values
        return S, embed(P, ctx_ids[S]), 0
    if policy == "deviation":
        if hook is not None:
            hook(0)  # the prefix rows layer 0 attends to (the doc rows are recomputed in place)
        score, h_all, _ = _deviation(P, ctx_ids, K, V, all_c, hook=hook)
        sel = _hip.topk_select(score, budget)  # ascending candidate indices => S sorted
        return all_c[sel], h_all.index_select(0, sel), 1
    raise ValueError(policy)


def _blend(model, ctx_ids, K, V, candidates, ratio, policy, gen, runner, graph, T, hook, trim_last, query_ids):
    P = prepared(model)
    dev = K[0].device
    if not candidates:
        return torch.empty(0, dtype=torch.long, device=dev), 0.0, None
    all_c = torch.cat(candidates)
    n, budget = select(ratio, candidates)
    if budget == 0:
        return all_c[:0], 0.0, None
    nq = 0 if query_ids is None else query_ids.numel()
    q_pos = torch.arange(T, T + nq, device=dev) if nq else None
    hq = None
    S, h, start = _select(P, ctx_ids, K, V, candidates, all_c, budget, policy, gen, hook)
    if nq and start == 1:  # the query rows' layer 0 (after every candidate's layer-0 k/v is in place)
        hq, dq = layer_forward(P, 0, embed(P, query_ids), None, make_rows(P, q_pos), K, V)
        hq = hq + dq  # the hidden entering layer 1, as the deviation pass returns it
    if nq and hq is None:
        hq = embed(P, query_ids)
    logits = None
    if graph is not None:
        out = runner.replay(graph, h, S, T, hook=hook, hq=hq)
        logits = out if nq else None
    elif nq:
        R = make_rows(P, torch.cat([S, q_pos]))
        keep = torch.arange(budget, budget + nq, device=dev) if trim_last else None
        hk, dk = run_layers(P, torch.cat([h, hq]), None, R, K, V, range(start, P.L), kv_only_last=trim_last,
                            hook=hook, keep=keep)
        logits = final_logits(P, hk, dk)  # the query rows are last either way
    else:
        R = make_rows(P, S)
        run_layers(P, h, None, R, K, V, range(start, P.L), kv_only_last=trim_last, hook=hook)
    L = P.L
    eff = (len(S) * (L - start) + start * n) / (n * L)
    return S, eff, logits


def blend(model, ctx_ids, K, V, candidates, ratio, policy, gen=None, inplace=False, runner=None):
    """tread/blend.py:133-179 signature: returns (K list, V list, S, eff).

    With a SubsetRunner whose worth_it(T) holds, the selection runs eagerly and the recompute
    layers go through `runner.run(h, S, K[start:], V[start:], start)`, the reference's call
    (tread/blend.py:170-172): the layers are copied into the runner's bucket and the returned
    K[start:], V[start:] are views of it, valid until its next replay, as in the reference. The
    engine avoids both copies by assembling straight into the bucket (Engine(graphs=True))."""
    K, V = list(K), list(V)
    if not inplace:
        K, V = [k.clone() for k in K], [v.clone() for v in V]
    T = K[0].shape[2] if K else 0
    n, budget = select(ratio, candidates)
    if runner is None or not candidates or budget == 0 or not runner.worth_it(T):
        S, eff = blend_cache(model, ctx_ids, K, V, candidates, ratio, policy, gen=gen)
        return K, V, S, eff
    P = prepared(model)
    with torch.inference_mode():  # the bucket's buffers are inference tensors
        S, h, start = _select(P, ctx_ids, K, V, candidates, torch.cat(candidates), budget, policy, gen)
        _, K[start:], V[start:] = runner.run(h[None], S, K[start:], V[start:], start)
        S = S.clone()
    eff = (len(S) * (P.L - start) + start * n) / (n * P.L)
    return K, V, S, eff


def to_cache(K, V):
    """tread/blend.py:182-186: a cache object over per-layer K/V (views, no copy)."""
    return KVCache.from_layers(K, V)
