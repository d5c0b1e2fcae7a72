"""Kernels at the full Qwen2.5-7B-shaped 32k workload (64 + 32 x 1000 context tokens, 28 layers,
4 KV heads of 128), checked through properties that do not need a CPU oracle run at that size:

- assembly: V rows and the delta-0 prefix are bit copies in torch.cat order; re-rotated K is
  within 1 bf16 ulp of the oracle's fp32 rotation on two sampled layers (every head and row), and
  rotating back by -delta returns the cached keys up to two bf16 roundings of each rotated pair;
- deviation score on sampled candidates equals the reference expression; the top-k is sorted,
  distinct, of size k, takes every score above its threshold, and breaks threshold ties towards
  the lowest indices;
- attention on the full recompute shape (6 400 rows x 28 heads over 32 064 keys) equals fp32
  textbook attention on sampled rows;
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


def test_full_request_assembly(cfg):
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
    for sK, sV, off, delta in srcs[1:]:
        n = sK.shape[-2]
        assert torch.equal(V[..., off:off + n, :], sV)
        got = K[..., off:off + n, :]
        # the oracle's fp32 rotation (on the CPU) for two sampled layers, every head and row
        for l in (0, L - 1):
            want = R.rotate_keys_fp32(m, sK[l:l + 1].cpu(), delta)
            assert bf16_ulps(got[l:l + 1].cpu(), want).max().item() <= 1
    # R(-delta) R(delta) = identity: rotating the assembled docs back recovers the cached keys
    back = torch.empty_like(K)
    _hip.rope_assemble([(K[..., off:off + sK.shape[-2], :].contiguous(), V[..., off:off + sK.shape[-2], :].contiguous(),
                         off, -delta) for sK, _, off, delta in srcs[1:]], back, torch.empty_like(V), inv)
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


def test_full_recompute_attention_on_sampled_rows(cfg):
    hq, hkv, hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    T = N_SYS + N_DOCS * DOC_LEN
    g = torch.Generator(device=DEV).manual_seed(7)
    n = int(round(0.2 * N_DOCS * DOC_LEN))
    kend = (torch.randperm(N_DOCS * DOC_LEN, device=DEV, generator=g)[:n].sort().values + N_SYS)
    q = torch.randn(n, hq, hd, device=DEV, dtype=torch.bfloat16, generator=g)
    K = torch.randn(1, hkv, T, hd, device=DEV, dtype=torch.bfloat16, generator=g)
    V = torch.randn_like(K)
    out = _hip.subset_attn(q, K, V, kend, hq, hkv, hd, hd ** -0.5).view(n, hq, hd)
    G = hq // hkv
    rows = torch.randperm(n, device=DEV, generator=g)[:48]
    for r in rows.tolist():
        e = int(kend[r]) + 1
        for h in (0, 13, hq - 1):
            kh = K[0, h // G, :e].float()
            vh = V[0, h // G, :e].float()
            p = torch.softmax((kh @ q[r, h].float()) * hd ** -0.5, 0)
            ref = p @ vh
            err = (out[r, h].float() - ref).abs().max().item()
            assert err < 3e-2, (r, h, err)


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
