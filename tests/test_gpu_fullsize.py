"""Kernels at the full shapes of the reference's large workloads, checked through properties that
need no CPU oracle run of the whole request:

- assembly at the Qwen2.5-7B shape (64 + 32 x 1000 context tokens, 28 layers, 4 KV heads of 128)
  and the Llama-3-70B shape (80 layers, 8 KV heads): V rows and the delta-0 prefix are bit copies
  in torch.cat order; re-rotated K equals the oracle's fp32 rotation bit for bit on three sampled
  layers (every head and row); rotating back by -delta returns the cached keys up to two bf16
  roundings of each rotated pair;
- deviation score on the oracle's own inputs for all 32 000 candidates equals the reference
  expression evaluated by the oracle on the CPU bit for bit, and the selection equals torch.topk
  on those scores except the choice among exact ties at the threshold; the top-k is sorted,
  distinct, of size k and breaks threshold ties towards the lowest indices;
- attention on the full recompute shapes (6 400 and 16 000 rows x 28 heads over 32 064 keys)
  equals float64 attention on sampled rows with planted dominant keys (tests/planted.py);
- the packed cold prefill of 8 docs at the 70B shape (8 000 rows x 64 heads over 8 064 keys, 8
  query heads per KV head, block-diagonal visibility) equals per-doc float64 attention on sampled
  rows with planted keys (tread/engine.py:74-95);
- the skinny linear kernel on the vocab-sized lm_head equals the fp32 product.
"""
import math

import pytest
import torch

from oracle import model_ref as M
from oracle import tread_ref as R
from tread_amd import _hip
from tread_amd.model import inv_freq_of, preset

pytestmark = pytest.mark.gpu
DEV = "cuda"
N_SYS, N_DOCS, DOC_LEN = 64, 32, 1000


def bf16_ulps(a, b):
    def ordered(t):
        i = t.contiguous().view(torch.int16).to(torch.int32)
        return torch.where(i >= 0, i, -(i + 32768))
    return (ordered(a) - ordered(b)).abs()


@pytest.fixture(scope="module")
def cfg():
    return preset("qwen2.5-7b")


@pytest.mark.parametrize("shape", ["qwen2.5-7b", "llama3-70b"])
def test_full_request_assembly(shape):
    cfg = preset(shape)
    L, kv, hd = cfg.num_hidden_layers, cfg.num_key_value_heads, cfg.head_dim
    g = torch.Generator(device=DEV).manual_seed(3)
    mk = lambda n: torch.randn(L, 1, kv, n, hd, device=DEV, dtype=torch.bfloat16, generator=g)
    inv = inv_freq_of(cfg)
    m = M.RefModel(cfg=cfg, w={}, dtype=torch.bfloat16, inv_freq=M.inv_freq_of(cfg))
    srcs = [(mk(N_SYS), mk(N_SYS), 0, 0)]
    order = [(i * 7) % N_DOCS for i in range(N_DOCS)]
    for slot in range(N_DOCS):
        off = N_SYS + slot * DOC_LEN
        base_slot = order[slot]  # the block was cached at the position of another slot
        srcs.append((mk(DOC_LEN), mk(DOC_LEN), off, off - (N_SYS + base_slot * DOC_LEN)))
    T = N_SYS + N_DOCS * DOC_LEN
    K = torch.empty(L, 1, kv, T + 32, hd, device=DEV, dtype=torch.bfloat16)
    V = torch.empty_like(K)
    _hip.rope_assemble(srcs, K, V, inv)
    torch.cuda.synchronize()
    assert torch.equal(K[..., :N_SYS, :], srcs[0][0]) and torch.equal(V[..., :N_SYS, :], srcs[0][1])
    worst = 0
    for sK, sV, off, delta in srcs[1:]:
        n = sK.shape[-2]
        assert torch.equal(V[..., off:off + n, :], sV)
        got = K[..., off:off + n, :]
        # the oracle's fp32 rotation (on the CPU) for three sampled layers, every head and row
        for l in (0, L // 2, L - 1):
            want = R.rotate_keys_fp32(m, sK[l:l + 1].cpu(), delta)
            worst = max(worst, bf16_ulps(got[l:l + 1].cpu(), want).max().item())
    assert worst == 0, worst
    # R(-delta) R(delta) = identity: rotating the assembled docs back recovers the cached keys
    back = torch.empty_like(K)
    _hip.rope_assemble([(K[..., off:off + sK.shape[-2], :].contiguous(), None, off, -delta)
                        for sK, _, off, delta in srcs[1:]], back, None, inv)
    torch.cuda.synchronize()
    for sK, _, off, _ in srcs[1:]:
        # rotations preserve each (i, i + hd/2) pair's norm r; two bf16 roundings of the pair move
        # each component by at most about r * 2^-8
        b, k = back[..., off:off + sK.shape[-2], :].float(), sK.float()
        h = hd // 2
        r = torch.sqrt(k[..., :h] ** 2 + k[..., h:] ** 2).repeat(1, 1, 1, 1, 2)
        assert bool(((b - k).abs() <= r * 2.0 ** -7).all())


def test_full_deviation_score_and_topk(cfg):
    hq, hkv, hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    T = N_SYS + N_DOCS * DOC_LEN
    n = N_DOCS * DOC_LEN
    g = torch.Generator(device=DEV).manual_seed(5)
    ld = (hq + 2 * hkv) * hd
    qkv = torch.randn(n, ld, device=DEV, dtype=torch.bfloat16, generator=g)
    rows = torch.arange(N_SYS, T, device=DEV)
    inv = inv_freq_of(cfg).to(DEV)
    ang = rows[:, None].float() * inv[None, :]
    cos, sin = ang.cos().to(torch.bfloat16), ang.sin().to(torch.bfloat16)
    K1 = torch.randn(1, hkv, T + 32, hd, device=DEV, dtype=torch.bfloat16, generator=g)
    V1 = torch.randn_like(K1)
    score = _hip.dev_score(qkv, cos, sin, rows, hkv, hd, K1, V1, k_col=hq * hd)
    sample = torch.randperm(n, device=DEV)[:512].sort().values
    k = qkv[sample, hq * hd:(hq + hkv) * hd].view(1, -1, hkv, hd).transpose(1, 2)
    v = qkv[sample, (hq + hkv) * hd:].view(1, -1, hkv, hd).transpose(1, 2)
    c = torch.cat([cos[sample], cos[sample]], -1)[None, None]
    s = torch.cat([sin[sample], sin[sample]], -1)[None, None]
    rot = torch.cat([-k[..., hd // 2:], k[..., :hd // 2]], dim=-1)
    k1 = k * c + rot * s  # bf16 ops, rounded like the reference's apply_rotary_pos_emb
    ref = R.deviation_score(k1, v, K1[:, :, rows[sample]], V1[:, :, rows[sample]])[0]
    u = bf16_ulps(score[sample], ref)
    assert u.max().item() <= 1 and (u == 0).float().mean().item() > 0.98
    budget = int(round(0.2 * n))
    sel = _hip.topk_select(score, budget)
    assert sel.numel() == budget
    assert bool((sel[1:] > sel[:-1]).all())  # ascending, hence distinct
    sf = score.float()
    thr = sf[sel].min()
    mask = torch.zeros(n, dtype=torch.bool, device=DEV)
    mask[sel] = True
    assert bool((sf[~mask] <= thr).all()) and bool((sf[sf > thr] > thr).all())
    assert int((sf > thr).sum()) <= budget and bool(mask[sf > thr].all())
    ties = torch.nonzero(sf == thr).flatten()
    taken = mask[ties]
    # ties at the threshold: a prefix of the tied indices is taken
    assert bool((taken[:-1].int() >= taken[1:].int()).all())


@pytest.mark.parametrize("ratio", [0.2, 0.5])
def test_full_recompute_attention_on_sampled_rows(cfg, ratio):
    """The recompute rows of the 7B request (6 400 or 16 000 rows x 28 heads over 32 064 keys:
    key-half work groups for the longest row tiles, merged by attn_halves_kernel). 64 sampled rows
    (among them the shortest and the longest) get two planted dominant keys per head
    (tests/planted.py), so that a dropped or double-counted key half or key tile moves their
    outputs by O(1), at least 10x the error bound (asserted on the inputs); every sampled row and
    head is checked against the float64 reference (tread/blend.py:107-110)."""
    import planted as PL
    hq, hkv, hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    T = N_SYS + N_DOCS * DOC_LEN
    g = torch.Generator().manual_seed(7)
    gd = torch.Generator(device=DEV).manual_seed(7)
    n = int(round(ratio * N_DOCS * DOC_LEN))
    kend = torch.randperm(N_DOCS * DOC_LEN, generator=g)[:n].sort().values + N_SYS
    q = torch.randn(n, hq, hd, generator=g).to(torch.bfloat16)
    K = torch.randn(hkv, T, hd, device=DEV, generator=gd).to(torch.bfloat16)
    V = torch.randn(hkv, T, hd, device=DEV, generator=gd).to(torch.bfloat16)
    rows = torch.randperm(n, generator=g)[:62].tolist() + [0, n - 1]
    pairs = [(i, h) for i in rows for h in range(hq)]
    keys = PL.plant(q, K, kend, pairs, g, per_pair=2)
    scale = hd ** -0.5
    out = _hip.subset_attn(q.to(DEV), K[None], V[None], kend.to(DEV), hq, hkv, hd, scale).view(n, hq, hd)
    ref, mag, drop = PL.reference(q, K, V, kend, pairs, scale, planted=keys)
    bound, margin = PL.check(torch.stack([out[i, h] for i, h in pairs]), ref, mag, drop, ratio)
    print(f"\n[7B recompute {n} rows] error bound <= {bound:.3e}; one-key drop effect >= {margin:.1f}x the bound")


def test_packed_cold_prefill_attention_at_the_70b_shape():
    """8 cold docs of 1 000 tokens packed on top of a 64-token prefix: row t of doc j sits at cache
    row P + 1000 j + t and sees the prefix rows [0, P) and its own doc's rows up to itself
    (tread/engine.py:74-95). 44 sampled rows (the first and last of the first two docs among them),
    every head, two planted dominant keys each within what the row sees (tests/planted.py): a
    leaked or dropped segment moves their outputs by O(1), at least 10x the error bound."""
    import planted as PL
    cfg = preset("llama3-70b")
    hq, hkv, hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    P, nd, dl = N_SYS, 8, DOC_LEN
    n = nd * dl
    g = torch.Generator().manual_seed(11)
    gd = torch.Generator(device=DEV).manual_seed(11)
    rows = torch.arange(P, P + n)
    kseg = P + (torch.arange(n) // dl) * dl
    q = torch.randn(n, hq, hd, generator=g).to(torch.bfloat16)
    K = torch.randn(hkv, P + n, hd, device=DEV, generator=gd).to(torch.bfloat16)
    V = torch.randn(hkv, P + n, hd, device=DEV, generator=gd).to(torch.bfloat16)
    pick = torch.randperm(n, generator=g)[:40].tolist() + [0, dl - 1, dl, n - 1]
    pairs = [(i, h) for i in pick for h in range(hq)]
    keys = PL.plant(q, K, rows, pairs, g, kseg=kseg, n_shared=P, per_pair=2)
    scale = hd ** -0.5
    out = _hip.subset_attn(q.to(DEV), K[None], V[None], rows.to(DEV), hq, hkv, hd, scale, kseg=kseg.to(DEV),
                           n_shared=P).view(n, hq, hd)
    ref, mag, drop = PL.reference(q, K, V, rows, pairs, scale, kseg=kseg, n_shared=P, planted=keys)
    bound, margin = PL.check(torch.stack([out[i, h] for i, h in pairs]), ref, mag, drop)
    print(f"\n[70B packed prefill] error bound <= {bound:.3e}; one-key drop effect >= {margin:.1f}x the bound")


@pytest.mark.parametrize("ratio", [0.2, 0.5])
def test_full_selection_on_shared_inputs_equals_torch_topk(cfg, ratio):
    """The layer-1 deviation score and top-k on the oracle's inputs: raw k/v rows of all 32 000
    candidates with the RoPE tables of their positions, and cache rows that drift from them by
    candidate-dependent amounts (many bf16 scores tie). The oracle evaluates tread/blend.py:129
    and :160 on the CPU; the kernels must give the same scores bit for bit and a selection that
    differs from torch.topk's only among candidates whose score equals the threshold."""
    hkv, hd = cfg.num_key_value_heads, cfg.head_dim
    n, T = N_DOCS * DOC_LEN, N_SYS + N_DOCS * DOC_LEN
    m = M.RefModel(cfg=cfg, w={}, dtype=torch.bfloat16, inv_freq=M.inv_freq_of(cfg))
    g = torch.Generator().manual_seed(13)
    rows = torch.arange(N_SYS, T)
    k_raw = torch.randn(n, hkv * hd, generator=g).to(torch.bfloat16)
    v_raw = torch.randn(n, hkv * hd, generator=g).to(torch.bfloat16)
    cos, sin = M.rope_cos_sin(m, rows, torch.bfloat16)
    k = k_raw.view(1, n, hkv, hd).transpose(1, 2)
    v = v_raw.view(1, n, hkv, hd).transpose(1, 2)
    k1 = M.apply_rope(k, cos, sin)
    eps = (torch.rand(1, 1, n, 1, generator=g) * 0.4 + 0.01)
    K1 = torch.randn(1, hkv, T + 32, hd, generator=g).to(torch.bfloat16)
    V1 = torch.randn_like(K1)
    K1[:, :, rows] = (k1.float() + eps * torch.randn(1, hkv, n, hd, generator=g)).to(torch.bfloat16)
    V1[:, :, rows] = (v.float() + eps * torch.randn(1, hkv, n, hd, generator=g)).to(torch.bfloat16)
    want = R.deviation_score(k1, v, K1[:, :, rows], V1[:, :, rows])[0]
    half = hd // 2
    got = _hip.dev_score(torch.cat([k_raw, v_raw], 1).to(DEV), cos[0, :, :half].contiguous().to(DEV),
                         sin[0, :, :half].contiguous().to(DEV), rows.to(DEV), hkv, hd, K1.to(DEV), V1.to(DEV))
    got_c = got.cpu()
    print(f"\n[7B 32k shared inputs] scores differing from the oracle: {int((got_c != want).sum())} of {n}; "
          f"distinct bf16 scores: {want.unique().numel()}")
    assert torch.equal(got_c, want)
    budget = int(round(ratio * n))
    sel = _hip.topk_select(got, budget).cpu()
    assert sel.numel() == budget and bool((sel[1:] > sel[:-1]).all())
    wf = want.float()
    top = wf.topk(budget)
    thr = top.values[-1].item()
    diff = set(sel.tolist()) ^ set(top.indices.tolist())
    assert all(wf[i].item() == thr for i in diff)
    ties = torch.nonzero(wf == thr).flatten()
    taken = torch.zeros(n, dtype=torch.bool)
    taken[sel] = True
    print(f"[7B 32k shared inputs] {ratio:.0%}: |S xor S_torch.topk| = {len(diff)}, all at the threshold "
          f"({ties.numel()} candidates tie there)")
    assert bool((taken[ties][:-1].int() >= taken[ties][1:].int()).all())  # lowest tied indices first


def test_full_lm_head_skinny(cfg):
    H, Vsz = cfg.hidden_size, cfg.vocab_size
    g = torch.Generator(device=DEV).manual_seed(9)
    W = (torch.randn(Vsz, H, device=DEV, generator=g) * 0.02).to(torch.bfloat16)
    x = torch.randn(1, H, device=DEV, generator=g).to(torch.bfloat16)
    got = _hip.skinny_linear(x, W).float()
    ref = x.float() @ W.float().T
    terms = x.float().abs() @ W.float().abs().T
    ulp = 2.0 ** (ref.abs().clamp_min(1e-30).log2().floor() - 7)
    assert bool(((got - ref).abs() <= ulp + 1e-5 * terms).all())
    assert math.isfinite(got.sum().item())
