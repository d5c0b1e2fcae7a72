"""Attention inputs with planted high-score keys, and the reference that checks them.

With N(0, 1) q and K at scale hd^-1/2 the scores of a long row are ~N(0, 1), its softmax is nearly
flat and the output is a mean of thousands of V rows (RMS ~ sqrt(e / n): 0.009 at 32k keys), so
an error bar on absolute outputs cannot see a key range that a kernel dropped or counted twice.
Here each checked (row, head) pair gets `per_pair` keys whose scaled scores are set to
LEVELS[0], LEVELS[1], ... (14, 13.5, 13 in natural-log units, i.e. softmax weights 1 : 0.61 :
0.37 against a background of total weight ~0.04 at 32k keys). The keys of one row are spread
over the row's visible range in equal strata, so across the checked pairs every key slice, key
half and split-K range of the kernels' plans holds planted keys. The output of such a pair is
~(V1 + 0.61 V2 + 0.37 V3) / 1.98: dropping the range that holds one planted key, or counting it
twice, moves the output by about 0.2 |V_i - V_j| or more (max over a row of 128 N(0, 1) elements:
~0.4 or more), where a correct kernel stays within the bound of `check` (~0.02 at these
magnitudes); the tests compute, per pair, the change that removing each planted key makes
(`reference`) and assert that it is at least 10x that pair's bound.
"""
import math

import torch

LEVELS = (14.0, 13.5, 13.0)


def scale_log2(scale):
    """fp32(scale) * fp32(log2 e), rounded to fp32, as the kernels form it."""
    return (torch.tensor(scale, dtype=torch.float32) * torch.tensor(1.4426950408889634, dtype=torch.float32)).item()


def visible(i, t_cap, kend, kseg=None, n_shared=0):
    """Key indices row i sees: [0, kend[i]], or [0, n_shared) and [kseg[i], kend[i]]."""
    e = int(kend[i])
    if kseg is None:
        return torch.arange(0, e + 1)
    return torch.cat([torch.arange(0, n_shared), torch.arange(int(kseg[i]), e + 1)])


def plant(q, K, kend, pairs, gen, kseg=None, n_shared=0, per_pair=2, rounds=1, rnd=0):
    """Overwrite rows of K (bf16 [hkv, t_cap, hd], any device; q and kend on the CPU) so that
    each (row i, head h) of `pairs` has `per_pair` keys with scaled scores LEVELS[:per_pair] (in
    natural-log units, before the kernel's bf16 roundings); a key is planted for one pair only
    (rows that see the fewest keys choose first). The visible keys of a row are cut, per KV head,
    into m = (the row's pairs in that head) x per_pair x rounds equal strata; call `rnd` of `rounds`
    plants one key in each of its m / rounds strata (assigned to the pairs at random), so that
    `rounds` calls with fresh K put a planted key in every stratum. Returns {pair: [keys]}."""
    n, hq, hd = q.shape
    hkv, t_cap, _ = K.shape
    G = hq // hkv
    scale = hd ** -0.5
    used = set()
    out = {}
    groups = {}
    for i, h in pairs:
        groups.setdefault((i, h // G), []).append(h)
    seen = lambda i: int(kend[i]) + 1 - (0 if kseg is None else int(kseg[i]) - n_shared)
    for (i, kh), heads in sorted(groups.items(), key=lambda x: seen(x[0][0])):
        vis = visible(i, t_cap, kend, kseg, n_shared)
        per_round = len(heads) * per_pair
        m = per_round * rounds
        if len(vis) < 2 * m:
            raise ValueError(f"row {i} sees {len(vis)} keys, too few for {m} strata")
        strata = (rnd * per_round + torch.randperm(per_round, generator=gen)).tolist()
        for a, h in enumerate(heads):
            qv = q[i, h].float()
            keys = []
            for j in range(per_pair):
                s = strata[a * per_pair + j]
                lo, hi = len(vis) * s // m, len(vis) * (s + 1) // m
                key = int(vis[lo + int(torch.randint(hi - lo, (1,), generator=gen))])
                if (kh, key) in used:  # taken by another pair: the first free key of the stratum,
                    free = [int(k) for k in vis[lo:hi] if (kh, int(k)) not in used]
                    if not free:  # else of the row
                        free = [int(k) for k in vis if (kh, int(k)) not in used]
                    if not free:
                        raise RuntimeError(f"row {i} has no free key left in KV head {kh}")
                    key = free[0]
                used.add((kh, key))
                # score = scale * q . k = LEVELS[j]  <=>  k = LEVELS[j] / scale * q / |q|^2
                K[kh, key] = (LEVELS[j] / scale * qv / qv.dot(qv)).to(K.device, K.dtype)
                keys.append(key)
            out[(i, h)] = keys
    return out


def rounds_for(pairs_per_group, per_pair, n_keys, unit=128):
    """Calls of `plant` after which every `unit`-key range of n_keys holds a planted key: strata of
    at most unit / 2 keys (each range then contains a whole stratum)."""
    return max(1, -(-2 * n_keys // unit // (pairs_per_group * per_pair)))


def reference(q, K, V, kend, pairs, scale, kseg=None, n_shared=0, planted=None, device="cuda"):
    """For each (row, head) pair: the attention output in float64 with the kernels' one input
    rounding (q multiplied by scale * log2 e in fp32 and rounded to bf16, softmax in base 2), and
    the same weights applied to |V| (the scale of the P-rounding error). With `planted` (what
    `plant` returned) also, per pair, the smallest over its planted keys of the largest output
    change when that key's weight is removed, (out - p_j v_j) / (1 - p_j) - out: what dropping the
    key range that holds it would do at the least (inf for a pair without planted keys). Returns
    ([len(pairs), hd] float64 outputs, the |V| outputs, [len(pairs)] changes)."""
    n, hq, hd = q.shape
    hkv, t_cap, _ = K.shape
    G = hq // hkv
    c = scale_log2(scale)
    Kd, Vd = K.to(device, torch.float64), V.to(device, torch.float64)
    ref = torch.empty(len(pairs), hd, dtype=torch.float64, device=device)
    mag = torch.empty_like(ref)
    drop = torch.full((len(pairs),), math.inf, dtype=torch.float64, device=device)
    groups = {}
    for idx, (i, h) in enumerate(pairs):
        groups.setdefault((i, h // G), []).append((idx, h))
    for (i, kh), items in groups.items():
        vis = visible(i, t_cap, kend, kseg, n_shared).to(device)
        idx = torch.tensor([x for x, _ in items], device=device)
        qs = (q[i, [h for _, h in items]].float() * c).to(torch.bfloat16).to(device, torch.float64)
        kk, vv = Kd[kh, vis], Vd[kh, vis]
        s = kk @ qs.T  # [keys, heads]
        p = torch.exp2(s - s.max(0).values)
        p = p / p.sum(0)
        out = p.T @ vv
        ref[idx] = out
        mag[idx] = p.T @ vv.abs()
        if planted:
            rows, keys = [], []
            for col, (_, h) in enumerate(items):
                for key in planted.get((i, h), ()):
                    rows.append(col)
                    keys.append(key)
            if keys:
                cols = torch.tensor(rows, device=device)
                pos = torch.searchsorted(vis, torch.tensor(keys, device=device))
                pj = p[pos, cols][:, None]
                d = ((out[cols] - pj * vv[pos]) / (1 - pj) - out[cols]).abs().max(1).values
                drop.scatter_reduce_(0, idx[cols], d, reduce="amin")
    return ref, mag, drop


def check(got, ref, mag, drop, what=""):
    """got: [len(pairs), hd] kernel outputs (bf16). Bound per element: the bf16 rounding of the
    output (half an ulp, at most 2^-8 of it) plus the bf16 rounding of every weight in P V (at most
    2^-8 each relative, doubled for the fp32 score and sum roundings: 2^-7 of sum p |v|) plus 2e-4.
    Asserts the bound, and that each pair's drop effect (from `reference`) is at least 10x the
    largest bound of its row; returns (largest bound, smallest drop effect / bound ratio)."""
    got = got.to(ref.device, torch.float64)
    err = (got - ref).abs()
    bound = 2.0 ** -8 * ref.abs() + 2.0 ** -7 * mag + 2e-4
    worst = (err / bound).max().item()
    assert worst <= 1.0, (what, worst, err.max().item())
    ratio = (drop.to(bound.device) / bound.max(dim=1).values).min().item()
    assert ratio >= 10, (what, ratio)
    return bound.max().item(), ratio
