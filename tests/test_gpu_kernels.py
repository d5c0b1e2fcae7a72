"""Kernel-level parity of libtread_hip.so against the CPU oracle (and fp32 textbook formulas).

Every test builds seeded inputs on the CPU, runs the HIP kernel through tread_amd._hip (the C-ABI)
and compares with the oracle's restatement of the reference op on the same inputs.
"""
import pytest
import torch

from oracle import model_ref as M
from oracle import tread_ref as R
from tread_amd import _hip
from tread_amd.model import ModelConfig

pytestmark = pytest.mark.gpu
DEV = "cuda"


def bf16_ulps(a, b):
    """Distance in bf16 units in the last place between two bf16 tensors (same shape)."""
    def ordered(t):
        i = t.contiguous().view(torch.int16).to(torch.int32)
        return torch.where(i >= 0, i, -(i + 32768))
    return (ordered(a.cpu()) - ordered(b.cpu())).abs()


def _cfg(hd, theta=1000000.0):
    return ModelConfig(64, 64, 2, 2, 1, hd, 64, rope_theta=theta)


def _ref_model(hd, theta=1000000.0):
    cfg = _cfg(hd, theta)
    return M.RefModel(cfg=cfg, w={}, dtype=torch.bfloat16, inv_freq=M.inv_freq_of(cfg))


# ------------------------------------------------------------------------------------------- (a)

@pytest.mark.parametrize("hd,kv,L", [(128, 4, 3), (64, 2, 2)])
def test_rope_assemble_matches_fp32_rotation_and_cat_layout(hd, kv, L):
    g = torch.Generator().manual_seed(11)
    m = _ref_model(hd)
    P = 64
    lens = [1, 127, 128, 129, 300, 1000]
    t_cap = P + sum(lens) + 40
    prefK = torch.randn(L, 1, kv, P, hd, generator=g).to(torch.bfloat16)
    prefV = torch.randn(L, 1, kv, P, hd, generator=g).to(torch.bfloat16)
    srcs, exp_K, exp_V, exp_Kbf = [(prefK, prefV, 0, 0)], [prefK], [prefV], [prefK]
    off = P
    for i, n in enumerate(lens):
        K = (3 * torch.randn(L, 1, kv, n, hd, generator=g)).to(torch.bfloat16)
        V = torch.randn(L, 1, kv, n, hd, generator=g).to(torch.bfloat16)
        delta = off - P if i != 2 else -(i + 5)  # one negative shift for generality
        srcs.append((K, V, off, delta))
        exp_K.append(R.rotate_keys_fp32(m, K, delta))
        exp_Kbf.append(R.rotate_keys(m, K, delta))
        exp_V.append(V)
        off += n
    T = off
    sentinel = torch.tensor(-7.0, dtype=torch.bfloat16)
    dK = torch.full((L, 1, kv, t_cap, hd), -7.0, dtype=torch.bfloat16, device=DEV)
    dV = torch.full_like(dK, -7.0)
    dsrcs = [(K.to(DEV), V.to(DEV), o, d) for K, V, o, d in srcs]
    _hip.rope_assemble(dsrcs, dK, dV, m.inv_freq)
    torch.cuda.synchronize()
    gK, gV = dK.cpu(), dV.cpu()
    eK, eV = torch.cat(exp_K, dim=-2), torch.cat(exp_V, dim=-2)
    # V and the delta-0 prefix: bit copies; layout equals torch.cat
    assert torch.equal(gV[..., :T, :], eV)
    assert torch.equal(gK[..., :P, :], prefK)
    # K: the fp32 reference rotation op for op, so bit-exact (the bar is 1 bf16 ulp)
    u = bf16_ulps(gK[..., :T, :], eK)
    assert u.max().item() == 0, (u.max(), (u > 0).sum())
    # rows past T untouched
    assert (gK[..., T:, :] == sentinel).all() and (gV[..., T:, :] == sentinel).all()
    # against the exact rotation (fp64 arithmetic on the same fp32 angles): the kernel stays within
    # 1 bf16 ulp everywhere, closer than the reference's own bf16 torch path (bf16 cos/sin, every
    # op rounded to bf16)
    exact = torch.cat([prefK.double()] + [_rotate_fp64(m, K, d) for K, _, _, d in srcs[1:]], dim=-2)
    ex_bf = exact.to(torch.bfloat16)
    ours = bf16_ulps(gK[..., :T, :], ex_bf)
    theirs = bf16_ulps(torch.cat(exp_Kbf, dim=-2), ex_bf)
    assert ours.max().item() <= 1
    assert ours.float().mean().item() < theirs.float().mean().item()


@pytest.mark.parametrize("hd", [128, 64])
def test_rope_assemble_more_sources_than_one_launch_holds(hd):
    """More sources than one launch carries (48): the library splits the list into launches, each
    with its own slice of the cos/sin table; every source lands rotated, in cat order."""
    g = torch.Generator().manual_seed(12)
    m = _ref_model(hd)
    L, kv, n_src = 2, 2, 61
    lens = [1 + (7 * i) % 40 for i in range(n_src)]
    t_cap = sum(lens) + 16
    srcs, exp_K, exp_V, off = [], [], [], 0
    for i, n in enumerate(lens):
        K = (2 * torch.randn(L, 1, kv, n, hd, generator=g)).to(torch.bfloat16)
        V = torch.randn(L, 1, kv, n, hd, generator=g).to(torch.bfloat16)
        delta = off - 3 * i  # a different shift per source
        srcs.append((K, V, off, delta))
        exp_K.append(R.rotate_keys_fp32(m, K, delta))
        exp_V.append(V)
        off += n
    dK = torch.zeros(L, 1, kv, t_cap, hd, dtype=torch.bfloat16, device=DEV)
    dV = torch.zeros_like(dK)
    _hip.rope_assemble([(K.to(DEV), V.to(DEV), o, d) for K, V, o, d in srcs], dK, dV, m.inv_freq)
    torch.cuda.synchronize()
    assert torch.equal(dV[..., :off, :].cpu(), torch.cat(exp_V, dim=-2))
    u = bf16_ulps(dK[..., :off, :].cpu(), torch.cat(exp_K, dim=-2))
    assert u.max().item() == 0, (u.max(), (u > 0).sum())


@pytest.mark.parametrize("hd,with_v", [(128, True), (64, True), (128, False), (64, False)])
def test_rope_assemble_empty_and_uneven_sources(hd, with_v):
    """Empty, one-token and long sources in one launch: a work group finds its source through the
    launch's bucket table, and here buckets hold several sources (and empty ones) as well as runs
    inside one long source. Every source lands rotated in cat order; with no V (rotate_keys' form)
    only K moves."""
    g = torch.Generator().manual_seed(13)
    m = _ref_model(hd)
    L, kv = 3, 2
    lens = [0, 1, 0, 3000, 1, 1, 0, 17, 2000, 0, 5, 1, 33, 0]
    t_cap = sum(lens) + 8
    srcs, exp_K, exp_V, off = [], [], [], 0
    for i, n in enumerate(lens):
        K = (2 * torch.randn(L, 1, kv, n, hd, generator=g)).to(torch.bfloat16)
        V = torch.randn(L, 1, kv, n, hd, generator=g).to(torch.bfloat16)
        delta = off + 11 * i - 20
        srcs.append((K, V, off, delta))
        exp_K.append(R.rotate_keys_fp32(m, K, delta))
        exp_V.append(V)
        off += n
    dK = torch.zeros(L, 1, kv, t_cap, hd, dtype=torch.bfloat16, device=DEV)
    dV = torch.zeros_like(dK) if with_v else None
    _hip.rope_assemble([(K.to(DEV), V.to(DEV) if with_v else None, o, d) for K, V, o, d in srcs], dK, dV,
                       m.inv_freq)
    torch.cuda.synchronize()
    u = bf16_ulps(dK[..., :off, :].cpu(), torch.cat(exp_K, dim=-2))
    assert u.max().item() == 0, (u.max(), (u > 0).sum())
    assert (dK[..., off:, :] == 0).all()
    if with_v:
        assert torch.equal(dV[..., :off, :].cpu(), torch.cat(exp_V, dim=-2))
        assert (dV[..., off:, :] == 0).all()


def _rotate_fp64(m, K, delta):
    n = K.shape[-2]
    freqs = (m.inv_freq[:, None].float() @ torch.full((1, n), float(delta))).transpose(0, 1).double()
    c, s = torch.cat((freqs, freqs), -1).cos(), torch.cat((freqs, freqs), -1).sin()
    K64 = K.double()
    return K64 * c + M.rotate_half(K64) * s


def test_rope_assemble_layer_range_and_rejects_bad_rows():
    m = _ref_model(128)
    L, kv, hd, n = 4, 2, 128, 50
    K = torch.randn(L, 1, kv, n, hd).to(torch.bfloat16).to(DEV)
    V = torch.randn(L, 1, kv, n, hd).to(torch.bfloat16).to(DEV)
    dK = torch.zeros(L, 1, kv, 80, hd, dtype=torch.bfloat16, device=DEV)
    dV = torch.zeros_like(dK)
    _hip.rope_assemble([(K, V, 10, 5)], dK, dV, m.inv_freq, layer_lo=1, layer_hi=3)
    torch.cuda.synchronize()
    assert (dV[0] == 0).all() and (dV[3] == 0).all()
    assert torch.equal(dV[1:3, :, :, 10:60].cpu(), V[1:3].cpu())
    with pytest.raises(RuntimeError, match="outside the cache"):
        _hip.rope_assemble([(K, V, 40, 0)], dK, dV, m.inv_freq)


# ------------------------------------------------------------------------------------ RoPE / glue

@pytest.mark.parametrize("hd,theta", [(128, 1000000.0), (64, 10000.0), (128, 500000.0)])
def test_rope_table_matches_reference_rotary_emb(hd, theta):
    m = _ref_model(hd, theta)
    pos = torch.cat([torch.arange(0, 70), torch.randint(0, 40000, (500,), generator=torch.Generator().manual_seed(1))])
    cos, sin = _hip.rope_table(pos.to(DEV), m.inv_freq, hd)
    rc, rs = M.rope_cos_sin(m, pos, torch.bfloat16)  # [1, n, hd]
    for got, ref in ((cos, rc[0, :, :hd // 2]), (sin, rs[0, :, :hd // 2])):
        u = bf16_ulps(got, ref)
        assert u.max().item() <= 1
        assert (u == 0).float().mean().item() > 0.995


@pytest.mark.parametrize("hd,hq,hkv", [(128, 7, 1), (64, 14, 2), (128, 8, 8)])
def test_qkv_rope_splice_bit_exact_vs_apply_rotary(hd, hq, hkv):
    g = torch.Generator().manual_seed(5)
    m = _ref_model(hd)
    n, t_cap = 37, 200
    qkv = torch.randn(n, (hq + 2 * hkv) * hd, generator=g).to(torch.bfloat16)
    rows = torch.randperm(t_cap, generator=g)[:n]
    pos = torch.randint(0, 33000, (n,), generator=g)
    cos, sin = M.rope_cos_sin(m, pos, torch.bfloat16)
    Kc = torch.zeros(1, hkv, t_cap, hd, dtype=torch.bfloat16, device=DEV)
    Vc = torch.zeros_like(Kc)
    q_out = torch.empty(n, hq, hd, dtype=torch.bfloat16, device=DEV)
    _hip.qkv_rope_splice(qkv.to(DEV), cos[0, :, :hd // 2].contiguous().to(DEV), sin[0, :, :hd // 2].contiguous().to(DEV),
                         rows.to(DEV), hq, hkv, hd, Kc, Vc, q_out=q_out)
    torch.cuda.synchronize()
    q = qkv[:, :hq * hd].view(1, n, hq, hd).transpose(1, 2)
    k = qkv[:, hq * hd:(hq + hkv) * hd].view(1, n, hkv, hd).transpose(1, 2)
    v = qkv[:, (hq + hkv) * hd:].view(1, n, hkv, hd).transpose(1, 2)
    qr, kr = M.apply_rope(q, cos, sin), M.apply_rope(k, cos, sin)
    assert torch.equal(q_out.cpu(), qr[0].transpose(0, 1))
    assert torch.equal(Kc.cpu()[0][:, rows], kr[0])
    assert torch.equal(Vc.cpu()[0][:, rows], v[0])
    mask = torch.ones(t_cap, dtype=torch.bool)
    mask[rows] = False
    assert (Kc.cpu()[0][:, mask] == 0).all()


@pytest.mark.parametrize("H", [896, 1536, 3584, 8192])
def test_add_rmsnorm_vs_hf_rmsnorm(H):
    g = torch.Generator().manual_seed(2)
    n = 33
    x = torch.randn(n, H, generator=g).to(torch.bfloat16)
    d = torch.randn(n, H, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16)
    s, y = _hip.add_rmsnorm(x.to(DEV), w.to(DEV), 1e-6, delta=d.to(DEV))
    rs = x + d
    ry = M.rms_norm(rs, w, 1e-6)
    assert torch.equal(s.cpu(), rs)
    u = bf16_ulps(y, ry)
    assert u.max().item() <= 1 and (u == 0).float().mean().item() > 0.99
    _, y2 = _hip.add_rmsnorm(x.to(DEV), w.to(DEV), 1e-6)
    assert bf16_ulps(y2, M.rms_norm(x, w, 1e-6)).max().item() <= 1


def test_silu_mul_vs_torch():
    g = torch.Generator().manual_seed(3)
    n, I = 19, 4864
    gu = (2 * torch.randn(n, 2 * I, generator=g)).to(torch.bfloat16)
    out = _hip.silu_mul(gu.to(DEV))
    ref = torch.nn.functional.silu(gu[:, :I]) * gu[:, I:]
    u = bf16_ulps(out, ref)
    assert u.max().item() <= 1 and (u == 0).float().mean().item() > 0.99


@pytest.mark.parametrize("m,n,k,bias,ldx", [(1, 32, 256, False, 256), (8, 4608, 3584, True, 3584),
                                             (3, 96, 512, True, 640), (32, 3584, 4608, False, 4608),
                                             (17, 1024, 4096, False, 4096), (8, 3584, 18944, False, 18944),
                                             (1, 37888, 3584, False, 3584), (5, 32, 16384, True, 16384),
                                             (2, 2048, 2048, True, 2056), (2, 96, 16384, False, 16384),
                                             (1, 3584, 18944, True, 18944),
                                             # one row over 16 388 groups of 8 features: 8 passes per
                                             # work group, the last one partial; K of one chunk per lane
                                             (1, 131104, 128, True, 128),
                                             # rows shorter than 2 048 over more than 1 024 groups:
                                             # 2 passes per work group
                                             (1, 8224, 896, True, 896)])
def test_skinny_linear_matches_fp32_reference(m, n, k, bias, ldx):
    """y = x W^T (+ b) of a few rows against the fp32 product of the same bf16 values: within one
    bf16 ulp of it plus the fp32 reordering error (1e-5 of the sum of |terms|, which matters only
    where the terms cancel to near zero), and mostly equal to it rounded once."""
    g = torch.Generator().manual_seed(m * 7 + n)
    xs = torch.randn(m, ldx, generator=g).to(torch.bfloat16)
    W = (torch.randn(n, k, generator=g) * 0.05).to(torch.bfloat16)
    b = torch.randn(n, generator=g).to(torch.bfloat16) if bias else None
    x = xs[:, :k]
    ref = x.float() @ W.float().T
    if bias:
        ref = ref + b.float()
    got = _hip.skinny_linear(xs.to(DEV)[:, :k], W.to(DEV), None if b is None else b.to(DEV)).cpu()
    terms = x.float().abs() @ W.float().abs().T + (b.float().abs() if bias else 0)
    ulp = 2.0 ** (ref.abs().clamp_min(1e-30).log2().floor() - 7)
    assert ((got.float() - ref).abs() <= ulp + 1e-5 * terms).all()
    assert (bf16_ulps(got, ref.to(torch.bfloat16)) == 0).float().mean().item() > 0.95


@pytest.mark.parametrize("k", [128, 896, 1536, 2048, 2560, 2816, 3456, 3712, 8960, 13824])
def test_skinny_row_tail_has_the_bits_of_zero_padding(k):
    """One row streams each weight row in batches of 7 16-byte chunks per lane (448 per batch); a
    row of k / 8 chunks that leaves a partial last batch (here 1 .. 7 load steps, some with only
    part of the lanes in the row) must give the bits of the same row zero-padded to whole batches:
    the padded products are +0, and a sum that starts at +0 never holds -0, so adding them changes
    nothing. A dropped chunk or a chunk taken twice in the last batch changes the bits."""
    g = torch.Generator().manual_seed(k)
    kp = -(-k // 3584) * 3584
    n = 96
    x = torch.randn(1, k, generator=g).to(torch.bfloat16)
    W = (torch.randn(n, k, generator=g) * 0.05).to(torch.bfloat16)
    b = torch.randn(n, generator=g).to(torch.bfloat16)
    xp = torch.zeros(1, kp, dtype=torch.bfloat16)
    xp[:, :k] = x
    Wp = torch.zeros(n, kp, dtype=torch.bfloat16)
    Wp[:, :k] = W
    got = _hip.skinny_linear(x.to(DEV), W.to(DEV), b.to(DEV))
    assert torch.equal(got, _hip.skinny_linear(xp.to(DEV), Wp.to(DEV), b.to(DEV)))
    # the SiLU prologue stages silu(gate) * up, 0 in the padding
    gu, gup = torch.randn(1, 2 * k, generator=g).to(torch.bfloat16), torch.zeros(1, 2 * kp, dtype=torch.bfloat16)
    gup[:, :k], gup[:, kp:kp + k] = gu[:, :k], gu[:, k:]
    assert torch.equal(_hip.skinny_silu_linear(gu.to(DEV), W.to(DEV)), _hip.skinny_silu_linear(gup.to(DEV), Wp.to(DEV)))
    ref = x.float() @ W.float().T + b.float()  # and the bound of the fp32 reference test above
    terms = x.float().abs() @ W.float().abs().T + b.float().abs()
    ulp = 2.0 ** (ref.abs().clamp_min(1e-30).log2().floor() - 7)
    assert ((got.cpu().float() - ref).abs() <= ulp + 1e-5 * terms).all()


def test_skinny_linear_splits_k_for_few_features():
    """Few output features split K over work groups (fp32 partials + a reduce kernel); many do not."""
    assert _hip.lib().tread_skinny_workspace_bytes(8, 3584, 18944) == 4 * 8 * 3584 * 4
    assert _hip.lib().tread_skinny_workspace_bytes(1, 37888, 3584) == 0  # many features
    assert _hip.lib().tread_skinny_workspace_bytes(8, 3584, 3584) == 0  # short K
    assert _hip.lib().tread_skinny_workspace_bytes(5, 32, 16384) == 4 * 5 * 32 * 4
    # one or two rows take 16-feature tiles below 128 tiles of 32: twice the work groups, fewer splits
    assert _hip.lib().tread_skinny_workspace_bytes(1, 3584, 18944) == 0  # 224 groups: unsplit
    assert _hip.lib().tread_skinny_workspace_bytes(2, 96, 16384) == 4 * 2 * 96 * 4


@pytest.mark.parametrize("m,H,n,with_delta,bias", [(1, 3584, 4608, True, True), (8, 512, 1536, True, False),
                                                     (3, 256, 96, False, False), (2, 3584, 3584, True, True),
                                                     (1, 896, 1152, False, True)])
def test_skinny_norm_linear_equals_norm_then_linear(m, H, n, with_delta, bias):
    """The fused norm prologue gives add_rmsnorm's bits: its output equals skinny_linear applied
    to add_rmsnorm's output bit for bit, and h_out equals add_rmsnorm's sum."""
    g = torch.Generator().manual_seed(m + H)
    h = torch.randn(m, H, generator=g).to(torch.bfloat16).to(DEV)
    d = torch.randn(m, H, generator=g).to(torch.bfloat16).to(DEV) if with_delta else None
    lnw = (1 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16).to(DEV)
    W = (0.05 * torch.randn(n, H, generator=g)).to(torch.bfloat16).to(DEV)
    b = torch.randn(n, generator=g).to(torch.bfloat16).to(DEV) if bias else None
    y, hs = _hip.skinny_norm_linear(h, d, lnw, 1e-6, W, b)
    s, x = _hip.add_rmsnorm(h, lnw, 1e-6, delta=d)
    assert torch.equal(hs, s)
    assert torch.equal(y, _hip.skinny_linear(x, W, b))


@pytest.mark.parametrize("m,H,hq,hkv,hd,bias,oob", [
    (1, 3584, 28, 4, 128, True, False),    # 7B decoding step (one row: one weight row per wave)
    (2, 3584, 28, 4, 128, True, False),    # two rows: 32-feature MFMA tiles
    (1, 896, 14, 2, 64, True, False),      # 0.5B
    (1, 8192, 64, 8, 128, False, False),   # 70B, no q|k|v bias
    (1, 512, 8, 2, 64, True, True),        # one row whose cache row is outside the cache, no delta
    (3, 512, 8, 2, 64, False, True),
])
def test_skinny_norm_qkv_rope_equals_norm_linear_then_rope_splice(m, H, hq, hkv, hd, bias, oob):
    """The fused q|k|v epilogue (paired features, RoPE, cache splice) gives the bits of
    skinny_norm_linear followed by qkv_rope_splice: q, both cache layers (including the untouched
    rows and a row index outside the cache, which splices nothing) and h + delta."""
    g = torch.Generator().manual_seed(m * 31 + H + hq)
    n = (hq + 2 * hkv) * hd
    t_cap = 64
    h = torch.randn(m, H, generator=g).to(torch.bfloat16).to(DEV)
    d = None if (oob and m == 1) else torch.randn(m, H, generator=g).to(torch.bfloat16).to(DEV)
    lnw = (1 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16).to(DEV)
    W = (0.05 * torch.randn(n, H, generator=g)).to(torch.bfloat16).to(DEV)
    b = torch.randn(n, generator=g).to(torch.bfloat16).to(DEV) if bias else None
    pos = torch.tensor([5, 40, 63][:m], dtype=torch.int64, device=DEV)
    rows = pos.clone()
    if oob:
        rows[m // 2] = t_cap + 7  # outside the cache: its k/v are not written
    inv_freq = (1.0 / (1e6 ** (torch.arange(0, hd, 2, dtype=torch.float32) / hd))).to(DEV)
    cos, sin = _hip.rope_table(pos, inv_freq, hd)
    K0 = torch.randn(1, hkv, t_cap, hd, generator=g).to(torch.bfloat16).to(DEV)
    V0 = torch.randn(1, hkv, t_cap, hd, generator=g).to(torch.bfloat16).to(DEV)
    # two steps
    qkv, hs_ref = _hip.skinny_norm_linear(h, d, lnw, 1e-6, W, b)
    q_ref = torch.empty(m, hq, hd, dtype=torch.bfloat16, device=DEV)
    K_ref, V_ref = K0.clone(), V0.clone()
    _hip.qkv_rope_splice(qkv, cos, sin, rows, hq, hkv, hd, K_ref, V_ref, q_out=q_ref)
    # one launch
    q = torch.full((m, hq, hd), 9.0, dtype=torch.bfloat16, device=DEV)
    K, V = K0.clone(), V0.clone()
    hs = _hip.skinny_norm_qkv_rope(h, d, lnw, 1e-6, W, b, hq, hkv, hd, cos, sin, rows, q, K, V)
    torch.cuda.synchronize()
    assert torch.equal(hs, hs_ref)
    assert torch.equal(q, q_ref)
    assert torch.equal(K, K_ref) and torch.equal(V, V_ref)
    assert torch.equal(K, K0) == (oob and m == 1)  # in-range rows were written, none otherwise


@pytest.mark.parametrize("m,H,inter,with_delta", [(1, 3584, 18944, True), (2, 3584, 18944, True),
                                                 (1, 896, 4864, False), (1, 8192, 28672, True),
                                                 (3, 512, 1024, True), (8, 256, 272, False)])
def test_skinny_norm_swiglu_equals_norm_linear_then_silu_mul(m, H, inter, with_delta):
    """The fused gate|up epilogue (gate and up rows paired in one tile or pass) gives the bits of
    skinny_norm_linear followed by silu_mul, and h + delta."""
    g = torch.Generator().manual_seed(m * 13 + H + inter)
    h = torch.randn(m, H, generator=g).to(torch.bfloat16).to(DEV)
    d = torch.randn(m, H, generator=g).to(torch.bfloat16).to(DEV) if with_delta else None
    lnw = (1 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16).to(DEV)
    W = (0.05 * torch.randn(2 * inter, H, generator=g)).to(torch.bfloat16).to(DEV)
    act, hs = _hip.skinny_norm_swiglu(h, d, lnw, 1e-6, W)
    gu, hs_ref = _hip.skinny_norm_linear(h, d, lnw, 1e-6, W)
    assert torch.equal(hs, hs_ref)
    assert torch.equal(act, _hip.silu_mul(gu))


@pytest.mark.parametrize("m,inter,n", [(1, 18944, 3584), (8, 512, 256), (2, 4096, 64)])
def test_skinny_silu_linear_equals_silu_mul_then_linear(m, inter, n):
    g = torch.Generator().manual_seed(m + inter)
    gu = torch.randn(m, 2 * inter, generator=g).to(torch.bfloat16).to(DEV)
    W = (0.05 * torch.randn(n, inter, generator=g)).to(torch.bfloat16).to(DEV)
    y = _hip.skinny_silu_linear(gu, W)
    assert torch.equal(y, _hip.skinny_linear(_hip.silu_mul(gu), W))


def test_fused_skinny_kernels_keep_their_staged_rows_in_lds():
    """Rows that would overflow LDS: the norm-fused kernel refuses them (the layer then runs
    unfused); the SiLU-fused kernel splits K further (here 8 rows of a 28 672-wide gate|up)."""
    g = torch.Generator().manual_seed(3)
    h = torch.randn(8, 8192, generator=g).to(torch.bfloat16).to(DEV)
    lnw = torch.ones(8192, dtype=torch.bfloat16, device=DEV)
    W = (0.02 * torch.randn(64, 8192, generator=g)).to(torch.bfloat16).to(DEV)
    assert not _hip.norm_fused_ok(8, 64, 8192) and _hip.norm_fused_ok(7, 64, 8192)
    with pytest.raises(ValueError):
        _hip.skinny_norm_linear(h, None, lnw, 1e-5, W)
    y, _ = _hip.skinny_norm_linear(h[:7].contiguous(), None, lnw, 1e-5, W)
    _, x = _hip.add_rmsnorm(h[:7].contiguous(), lnw, 1e-5)
    assert torch.equal(y, _hip.skinny_linear(x, W))
    inter, n = 28672, 512
    gu = torch.randn(8, 2 * inter, generator=g).to(torch.bfloat16).to(DEV)
    Wd = (0.02 * torch.randn(n, inter, generator=g)).to(torch.bfloat16).to(DEV)
    assert _hip.lib().tread_skinny_silu_workspace_bytes(8, n, inter) > 0
    got = _hip.skinny_silu_linear(gu, Wd).float().cpu()
    act = _hip.silu_mul(gu).float().cpu()
    ref = act @ Wd.float().cpu().T
    terms = act.abs() @ Wd.float().cpu().abs().T
    ulp = 2.0 ** (ref.abs().clamp_min(1e-30).log2().floor() - 7)
    assert bool(((got - ref).abs() <= ulp + 1e-5 * terms).all())


def test_skinny_linear_rejects_unsupported_shapes():
    x = torch.zeros(33, 256, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        _hip.skinny_linear(x, torch.zeros(32, 256, device=DEV, dtype=torch.bfloat16))
    with pytest.raises(ValueError):
        _hip.skinny_linear(x[:4], torch.zeros(48, 256, device=DEV, dtype=torch.bfloat16))


# ------------------------------------------------------------------------------------------- (b)

@pytest.mark.parametrize("hd,hkv", [(128, 4), (64, 2), (128, 8)])
def test_dev_score_matches_reference_expression(hd, hkv):
    g = torch.Generator().manual_seed(7)
    m = _ref_model(hd)
    n, t_cap = 301, 1200
    kv_raw = torch.randn(n, 2 * hkv * hd, generator=g).to(torch.bfloat16)
    rows = torch.sort(torch.randperm(t_cap, generator=g)[:n]).values
    K1 = torch.randn(1, hkv, t_cap, hd, generator=g).to(torch.bfloat16)
    V1 = torch.randn(1, hkv, t_cap, hd, generator=g).to(torch.bfloat16)
    cos, sin = M.rope_cos_sin(m, rows, torch.bfloat16)
    # make some candidates drift little: copy the cache row (planted near-ties / zeros)
    k = kv_raw[:, :hkv * hd].view(1, n, hkv, hd).transpose(1, 2)
    v = kv_raw[:, hkv * hd:].view(1, n, hkv, hd).transpose(1, 2)
    k1 = M.apply_rope(k, cos, sin)
    ref = R.deviation_score(k1, v, K1[:, :, rows], V1[:, :, rows])[0]
    got = _hip.dev_score(kv_raw.to(DEV), cos[0, :, :hd // 2].contiguous().to(DEV),
                         sin[0, :, :hd // 2].contiguous().to(DEV), rows.to(DEV), hkv, hd, K1.to(DEV), V1.to(DEV))
    # the reference expression as the oracle evaluates it on the CPU (fp32 sums, bf16 roundings)
    assert torch.equal(got.cpu(), ref), bf16_ulps(got, ref).max()


def _brute_topk(score, k):
    s = score.float().tolist()
    order = sorted(range(len(s)), key=lambda i: (-s[i], i))
    return sorted(order[:k])


@pytest.mark.parametrize("n,k", [(1, 1), (10, 0), (10, 10), (1000, 200), (32000, 6400), (32000, 16000), (40000, 1),
                                 (65536, 13107), (65537, 13107), (100000, 20000)])
def test_topk_select_equals_brute_force(n, k):
    g = torch.Generator().manual_seed(n + k)
    # few distinct bf16 values => many ties at the threshold
    score = (torch.randint(0, 50, (n,), generator=g).float() / 8 + 3).to(torch.bfloat16)
    sel = _hip.topk_select(score.to(DEV), k).cpu().tolist()
    assert sel == _brute_topk(score, k)
    if k:
        # same as torch.topk up to the tie order at the threshold
        thr = score.float().topk(k).values[-1]
        ref = set(score.float().topk(k).indices.tolist())
        got = set(sel)
        assert all(score[i].float() == thr for i in got ^ ref)


def test_topk_select_handles_negative_and_distinct_scores():
    g = torch.Generator().manual_seed(9)
    score = torch.randn(5000, generator=g).to(torch.bfloat16)
    sel = _hip.topk_select(score.to(DEV), 777).cpu().tolist()
    assert sel == _brute_topk(score, 777)


# ------------------------------------------------------------------------------------------- (c)

def ref_attention_rounded(q, K, V, kend, scale):
    """The causal attention with the kernel's rounding points: q scaled by scale * log2(e) and
    rounded to bf16, fp32 scores, P = exp2(s - row max) rounded to bf16 for P V, fp32 sum."""
    n, hq, hd = q.shape
    hkv, t_cap, _ = K.shape
    G = hq // hkv
    vis = torch.arange(t_cap)[None, :] <= kend[:, None]
    out = torch.empty(n, hq, hd)
    for h in range(hq):
        qs = (q[:, h].float() * (scale * 1.4426950408889634)).to(torch.bfloat16).float()
        s = (qs @ K[h // G].float().T).masked_fill(~vis, -float("inf"))
        p = torch.exp2(s - s.max(-1, keepdim=True).values)
        out[:, h] = (p.to(torch.bfloat16).float() @ V[h // G].float()) / p.sum(-1, keepdim=True)
    return out


def ref_attention(q, K, V, kend, scale, kseg=None, n_shared=0):
    """Textbook masked GQA softmax attention in fp32 on the CPU. q [n, hq, hd], K/V [hkv, T, hd]."""
    n, hq, hd = q.shape
    hkv, T, _ = K.shape
    G = hq // hkv
    Kf = K.float().repeat_interleave(G, 0)
    Vf = V.float().repeat_interleave(G, 0)
    s = torch.einsum("nhd,htd->nht", q.float(), Kf) * scale
    keys = torch.arange(T)
    vis = keys[None, :] <= kend[:, None]
    if kseg is not None:
        vis &= (keys[None, :] < n_shared) | (keys[None, :] >= kseg[:, None])
    s = s.masked_fill(~vis[:, None, :], float("-inf"))
    return torch.einsum("nht,htd->nhd", torch.softmax(s, -1), Vf)


CASES = [
    # hq, hkv, hd, t_cap, n, kind
    (8, 2, 128, 700, 137, "subset"),
    (14, 2, 64, 1030, 300, "subset"),
    (28, 4, 128, 2100, 1, "subset"),
    (28, 4, 128, 3000, 600, "subset"),
    (12, 2, 128, 513, 513, "prefill"),
    (7, 1, 64, 200, 64, "prefill"),
    (6, 3, 64, 900, 250, "subset"),
    (64, 8, 128, 1500, 90, "subset"),
    (8, 2, 128, 700, 337, "segments"),
    (14, 2, 64, 500, 230, "segments"),
    # >= 8 row tiles per KV head and no key split: the longest quarter of the row tiles runs as
    # two key-half work groups merged by attn_halves_kernel
    (28, 4, 128, 1000, 1000, "subset"),
    (28, 4, 128, 1000, 1000, "prefill"),
    (14, 2, 64, 1000, 900, "segments"),
    # the same with a few late keys scaled up: row maxima move by far more than 2^8 in later key
    # tiles, so the lazy rescale fires inside the key halves and the merge sees different maxima
    (28, 4, 128, 1000, 1000, "spikes"),
    # few rows over a long cache: split-K + combine
    (28, 4, 128, 20000, 32, "query"),
    (14, 2, 64, 9000, 5, "query"),
    (28, 4, 128, 6000, 40, "subset"),
    (64, 8, 128, 33000, 17, "query"),
    # at most 32 rows per KV head (decoding steps): decode_attn_kernel, the keys split between the
    # waves of a work group and across work groups (slices merged by the combine kernels), or one
    # slice written directly
    (28, 4, 128, 32098, 1, "query"),   # 7B step over a 32k cache: 63 slices
    (14, 2, 64, 8100, 1, "query"),     # 0.5B step: 64 slices of 4 tiles (half the waves idle)
    (12, 2, 128, 16100, 1, "query"),   # 1.5B step: 126 slices, two rounds of the merge's loads
    (64, 8, 128, 33000, 4, "query"),   # 70B, 4 tokens x 8 heads = 32 rows
    (28, 4, 128, 300, 2, "query"),     # 3 slices, the last one of 44 keys
    (28, 4, 128, 100, 2, "query"),     # one slice: normalised output written directly
    (6, 3, 64, 900, 5, "subset"),      # rows scattered over the cache: per-row key ends mid-tile
    (8, 2, 128, 2000, 4, "segfew"),    # block-diagonal visibility on a few rows
    # key ends (and segment starts) on every side of every 32-key boundary, so of every key tile
    # the kernels use (96 keys at head_dim 128, 128 at 64), and a partial last tile
    (8, 2, 128, 1000, 90, "tiles"),
    (14, 2, 64, 1000, 90, "tiles"),
    (8, 2, 128, 1000, 48, "tileseg"),
    (14, 2, 64, 1000, 48, "tileseg"),
]


@pytest.mark.parametrize("hq,hkv,hd,t_cap,n,kind", CASES)
def test_subset_attention_vs_textbook(hq, hkv, hd, t_cap, n, kind):
    g = torch.Generator().manual_seed(hq * 1000 + n)
    q = torch.randn(n, hq, hd, generator=g).to(torch.bfloat16)
    K = torch.randn(hkv, t_cap, hd, generator=g).to(torch.bfloat16)
    V = torch.randn(hkv, t_cap, hd, generator=g).to(torch.bfloat16)
    kseg, n_shared = None, 0
    if kind == "spikes":
        kend = torch.sort(torch.randperm(t_cap, generator=g)[:n]).values
        hot = torch.randperm(t_cap // 2, generator=g)[:8] + t_cap // 2
        K[:, hot] = (K[:, hot].float() * 6).to(torch.bfloat16)
    elif kind == "subset":
        kend = torch.sort(torch.randperm(t_cap, generator=g)[:n]).values
    elif kind == "prefill":
        kend = torch.arange(n)
    elif kind == "query":  # the query rows at the end of the cache
        kend = torch.arange(t_cap - n, t_cap)
    elif kind == "tiles":  # key ends at 32 m - 1, 32 m, 32 m + 1
        ends = sorted({32 * m + d for m in range(1, 32) for d in (-1, 0, 1) if 32 * m + d < t_cap})
        kend = torch.tensor(ends[:n])
    elif kind == "tileseg":  # shared prefix ending at a tile edge - 1, segments starting at edges
        n_shared = 95
        pairs = [(s0, s0 + ln) for s0 in (96, 127, 128, 129, 191, 192, 288, 289)
                 for ln in (0, 31, 32, 95, 96, 200) if s0 + ln < t_cap]
        kseg = torch.tensor([a for a, _ in pairs][:n])
        kend = torch.tensor([b for _, b in pairs][:n])
    elif kind == "segfew":  # a few rows of packed docs: shared prefix + own segment
        n_shared = 40
        kend = torch.tensor([60, 300, 1210, 1999])[:n]
        kseg = torch.tensor([40, 250, 700, 1990])[:n]
    else:  # packed docs on a shared prefix: block-diagonal visibility
        n_shared = 40
        lens = [100, 37, n - 137]
        kend = n_shared + torch.arange(n)
        kseg = torch.cat([torch.full((Ld,), n_shared + o) for Ld, o in zip(lens, [0, 100, 137])])
    scale = hd ** -0.5
    ref = ref_attention(q, K, V, kend, scale, kseg, n_shared)
    out = _hip.subset_attn(q.to(DEV), K.to(DEV), V.to(DEV), kend.to(DEV), hq, hkv, hd, scale,
                           kseg=None if kseg is None else kseg.to(DEV), n_shared=n_shared)
    got = out.cpu().float().view(n, hq, hd)
    err = (got - ref).abs()
    if kind == "spikes":
        # The kernel's roundings (q pre-multiplied by scale * log2(e) in bf16, P in bf16 for P V,
        # fp32 sums) already move the textbook result by up to 0.04 on 6x-scaled keys; against
        # that rounding model the kernel must agree closely, whatever its running maxima did.
        emu = ref_attention_rounded(q, K, V, kend, scale)
        assert (got - emu).abs().max().item() < 2e-2, (got - emu).abs().max()
        assert err.max().item() < 6e-2 and err.mean().item() < 3e-3, (err.max(), err.mean())
        return
    assert err.max().item() < 3e-2, err.max()
    assert err.mean().item() < 3e-3, err.mean()


LONG = [
    # hq, hkv, hd, t_cap, n, kind, planted keys per (row, head)
    (28, 4, 128, 32098, 1, "query", 3),   # 7B decoding step over a 32k cache: 63 key slices
    (14, 2, 64, 8100, 1, "query", 3),     # 0.5B step: 64 slices of 4 tiles
    (12, 2, 128, 16100, 1, "query", 3),   # 1.5B step: 126 slices, two rounds of the merge's loads
    (64, 8, 128, 33000, 4, "query", 2),   # 70B, 4 tokens x 8 heads = 32 rows per KV head
    (28, 4, 128, 20000, 32, "query", 2),  # split-K work groups + the many-slice combine
    (64, 8, 128, 33000, 17, "query", 2),
    (14, 2, 64, 9000, 5, "query", 2),     # few-slice combine
    (28, 4, 128, 6000, 40, "subset", 2),  # rows scattered over the cache, split-K
]


@pytest.mark.parametrize("hq,hkv,hd,t_cap,n,kind,per_pair", LONG)
def test_long_rows_with_planted_keys(hq, hkv, hd, t_cap, n, kind, per_pair):
    """Rows over long caches, where the kernels split the keys into slices (decode), split-K
    ranges and merges (tread/blend.py:107-110; tread/engine.py:131-132). Each (row, head) gets
    `per_pair` keys of dominant score (tests/planted.py), so that dropping or double-counting the
    key range holding one of them moves the output by O(1) — at least 10x this test's error bound,
    asserted on the inputs themselves. For a one-row call every 128-key range of the cache holds a
    planted key of each KV head after the rounds run here; with several rows the rows' strata
    together cover the cache about as densely (random placement)."""
    import planted as PL
    G = hq // hkv
    g = torch.Generator().manual_seed(hq * 1000 + n + t_cap)
    gd = torch.Generator(device=DEV).manual_seed(t_cap)
    if kind == "query":
        kend = torch.arange(t_cap - n, t_cap)
    else:
        kend = torch.sort(torch.randperm(t_cap, generator=g)[:n]).values
    pairs = [(i, h) for i in range(n) for h in range(hq)]
    rounds = PL.rounds_for(G * n, per_pair, t_cap)
    scale = hd ** -0.5
    bound, margin = 0.0, float("inf")
    for rnd in range(rounds):
        q = torch.randn(n, hq, hd, generator=g).to(torch.bfloat16)
        K = torch.randn(hkv, t_cap, hd, device=DEV, generator=gd).to(torch.bfloat16)
        V = torch.randn(hkv, t_cap, hd, device=DEV, generator=gd).to(torch.bfloat16)
        keys = PL.plant(q, K, kend, pairs, g, per_pair=per_pair, rounds=rounds, rnd=rnd)
        out = _hip.subset_attn(q.to(DEV), K, V, kend.to(DEV), hq, hkv, hd, scale).view(n, hq, hd)
        ref, mag, drop = PL.reference(q, K, V, kend, pairs, scale, planted=keys)
        b, m = PL.check(torch.stack([out[i, h] for i, h in pairs]), ref, mag, drop, (rnd, kind, t_cap))
        bound, margin = max(bound, b), min(margin, m)
    print(f"\n[{hq}/{hkv}x{hd}, {n} rows over {t_cap} keys, {rounds} rounds] error bound <= {bound:.3e}; "
          f"one-key drop effect >= {margin:.1f}x the bound")


# ------------------------------------------------------------------------------------------- (d)

def test_copy_async_roundtrip_pinned():
    s = torch.cuda.Stream()
    src = torch.randn(3, 1000, 77).to(torch.bfloat16).pin_memory()
    dev = torch.empty(src.shape, dtype=src.dtype, device=DEV)
    back = torch.empty(src.shape, dtype=src.dtype).pin_memory()
    e1, e2 = torch.cuda.Event(), torch.cuda.Event()
    _hip.copy_async(dev, src, s, e1)
    s.wait_event(e1)
    _hip.copy_async(back, dev, s, e2)
    e2.synchronize()
    assert torch.equal(back, src)
