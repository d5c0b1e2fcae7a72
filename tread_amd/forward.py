"""Decoder forward over an arbitrary set of token rows against a preallocated KV cache.

Every forward on the path is the same computation with different row sets:
  - recompute of positions S (tread/blend.py:93-114): rows = positions = S, keys <= S[i];
  - the deviation pass over all candidates (tread/blend.py:117-130);
  - the query forward over the assembled cache (tread/engine.py:131-132): rows T..T+Nq-1;
  - prefix / full prefill (tread/blend.py:12-19; tread/engine.py:155-166): rows 0..N-1;
  - the packed cold prefill of missed docs (tread/engine.py:74-96): rows after the prefix,
    RoPE positions restarting at P per doc, keys = prefix + own doc (block-diagonal).
A layer is: fused residual-add + RMSNorm (HIP) -> one q|k|v GEMM (hipBLASLt via torch) ->
RoPE + splice of k/v into the cache (HIP) -> MFMA attention (HIP) -> o_proj GEMM -> fused add +
RMSNorm (HIP) -> gate|up GEMM -> SiLU-mul (HIP) -> down GEMM. The MLP output is carried as a
pending residual `delta` that the next layer's norm kernel adds.
"""
from dataclasses import dataclass
from typing import Optional

import torch
import torch.nn.functional as F

from tread_amd import _hip


@dataclass
class Rows:
    rows: torch.Tensor            # int64 [n]: cache row receiving token i's k/v
    kend: torch.Tensor            # int64 [n]: last cache row token i may attend to
    cos: torch.Tensor             # bf16 [n, hd/2]: RoPE of token i's position
    sin: torch.Tensor
    kseg: Optional[torch.Tensor] = None  # int64 [n]: first row of token i's own segment
    n_shared: int = 0             # rows [0, n_shared) are visible to every token (with kseg)
    gemm_split: int = 0           # > 0: the gate|up GEMM runs rows [0, split) and [split, n) apart

    def __len__(self):
        return self.rows.numel()

    def select(self, idx):
        """The rows at positions idx (int64 tensor) of this set."""
        pick = lambda t: None if t is None else t.index_select(0, idx)
        return Rows(rows=pick(self.rows), kend=pick(self.kend), cos=pick(self.cos), sin=pick(self.sin),
                    kseg=pick(self.kseg), n_shared=self.n_shared)


def _gate_up(x, w, split):
    """x @ w.T; with 0 < split < rows, as two GEMMs over rows [0, split) and [split, rows): when
    a few rows ride on a row count that is a multiple of the library's 256-row tiles, the
    vocabulary-wide gate|up GEMM then skips a whole extra row of tiles."""
    if not 0 < split < x.shape[0]:
        return F.linear(x, w)
    y = torch.empty(x.shape[0], w.shape[0], dtype=x.dtype, device=x.device)
    torch.mm(x[:split], w.t(), out=y[:split])
    torch.mm(x[split:], w.t(), out=y[split:])
    return y


def make_rows(P, rows, pos=None, kseg=None, n_shared=0):
    """RoPE tables for `pos` (default: rows) and causal key ends = rows."""
    rows = rows.to(torch.int64).contiguous()
    pos = rows if pos is None else pos.to(torch.int64).contiguous()
    cos, sin = _hip.rope_table(pos, P.inv_freq, P.hd)
    return Rows(rows=rows, kend=rows, cos=cos, sin=sin, kseg=kseg, n_shared=n_shared)


def layer_forward(P, l, h, delta, R: Rows, K, V, kv_only=False):
    """One decoder layer for rows R. h, delta: [n, H] (delta may be None). K, V: per-layer
    sequences of [1, hkv, t_cap, hd] cache tensors; layer l receives the rows' k/v.
    Returns (h, delta) entering layer l+1, or (h, None) when kv_only (k/v spliced, nothing else)."""
    lw = P.layers[l]
    hq, hkv, hd = P.hq, P.hkv, P.hd
    if not kv_only and _few_rows(P, lw, h.shape[0]):
        return _layer_few_rows(P, l, lw, h, delta, R, K, V)
    h, x = _hip.add_rmsnorm(h, lw.ln1, P.eps, delta=delta)
    n = h.shape[0]
    if kv_only:
        q_rows = hq * hd
        kv = F.linear(x, lw.wqkv[q_rows:], None if lw.bqkv is None else lw.bqkv[q_rows:])
        _hip.qkv_rope_splice(kv, R.cos, R.sin, R.rows, hq, hkv, hd, K[l], V[l], q_out=None, k_col=0)
        return h, None
    qkv = F.linear(x, lw.wqkv, lw.bqkv)
    q = torch.empty(n, hq, hd, dtype=h.dtype, device=h.device)
    _hip.qkv_rope_splice(qkv, R.cos, R.sin, R.rows, hq, hkv, hd, K[l], V[l], q_out=q)
    o = _hip.subset_attn(q, K[l], V[l], R.kend, hq, hkv, hd, P.scale, kseg=R.kseg, n_shared=R.n_shared)
    a = F.linear(o, lw.wo)
    h, x = _hip.add_rmsnorm(h, lw.ln2, P.eps, delta=a)
    m = _hip.silu_mul(_gate_up(x, lw.wgu, R.gemm_split))
    return h, F.linear(m, lw.wd)


# A layer of at most FEW_ROWS rows (a decoding step, a short query) runs its projections on the
# weight-streaming skinny kernels, which beat the library GEMM there on MI355X. The kernels with
# the norm (or the SiLU gating) fused in front save a launch but redo that prologue in every work
# group for every row; measured on MI355X they win up to NORM_FUSED_ROWS rows (norm) and
# SILU_FUSED_ROWS rows (SiLU) and lose beyond (at 8 rows the norm-fused lm_head takes twice the
# time of RMSNorm + skinny kernel). Fused or not, the results are the same bits. Up to the skinny
# kernels' 32 rows they lose: a 32-row query forward over a 7B-shaped model's cache of 32k rows
# took 8.5 ms on them against 6.5 ms on the library GEMMs (the whole request without recompute),
# over a 0.5B-shaped one's 1k and 8k rows 2.8 and 2.9 ms against 2.2 and 2.4 ms.
FEW_ROWS = 8
NORM_FUSED_ROWS = 2
SILU_FUSED_ROWS = 4


def _few_rows(P, lw, n):
    return n <= FEW_ROWS and all(_hip.skinny_ok(n, w.shape[0], w.shape[1]) for w in (lw.wqkv, lw.wo, lw.wgu, lw.wd))


def _norm_linear(P, h, delta, ln_w, weight, bias=None):
    """(linear(RMSNorm(h + delta)), h + delta) for a few rows, on the skinny kernels."""
    m = h.shape[0]
    if m <= NORM_FUSED_ROWS and _hip.norm_fused_ok(m, weight.shape[0], weight.shape[1]):
        return _hip.skinny_norm_linear(h, delta, ln_w, P.eps, weight, bias)
    h, x = _hip.add_rmsnorm(h, ln_w, P.eps, delta=delta)
    return _hip.skinny_linear(x, weight, bias), h


def _silu_linear(gate_up, weight):
    """linear(silu(g) * u) for a few rows, on the skinny kernels."""
    m = gate_up.shape[0]
    if m <= SILU_FUSED_ROWS and _hip.fused_ok(m, weight.shape[0], weight.shape[1]):
        return _hip.skinny_silu_linear(gate_up, weight)
    return _hip.skinny_linear(_hip.silu_mul(gate_up), weight)


def _layer_few_rows(P, l, lw, h, delta, R, K, V):
    """layer_forward for a few rows: (norm ->) q|k|v, RoPE + splice, attention, o, (norm ->)
    gate|up, (SiLU ->) down, with the same roundings as the layer for many rows."""
    hq, hkv, hd = P.hq, P.hkv, P.hd
    m = h.shape[0]
    q = torch.empty(m, hq, hd, dtype=h.dtype, device=h.device)
    if m <= NORM_FUSED_ROWS and _hip.norm_fused_ok(m, lw.wqkv.shape[0], lw.wqkv.shape[1]):
        # norm, q|k|v, RoPE and the cache splice in one launch (the same bits as the three steps)
        h = _hip.skinny_norm_qkv_rope(h, delta, lw.ln1, P.eps, lw.wqkv, lw.bqkv, hq, hkv, hd, R.cos, R.sin, R.rows,
                                      q, K[l], V[l])
    else:
        qkv, h = _norm_linear(P, h, delta, lw.ln1, lw.wqkv, lw.bqkv)
        _hip.qkv_rope_splice(qkv, R.cos, R.sin, R.rows, hq, hkv, hd, K[l], V[l], q_out=q)
    o = _hip.subset_attn(q, K[l], V[l], R.kend, hq, hkv, hd, P.scale, kseg=R.kseg, n_shared=R.n_shared)
    a = _hip.skinny_linear(o, lw.wo)
    if m <= NORM_FUSED_ROWS and _hip.norm_fused_ok(m, lw.wgu.shape[0], lw.wgu.shape[1]):
        # norm, gate|up and SiLU gating in one launch (silu_mul's bits), then a plain down projection
        act, h = _hip.skinny_norm_swiglu(h, a, lw.ln2, P.eps, lw.wgu)
        return h, _hip.skinny_linear(act, lw.wd)
    gu, h = _norm_linear(P, h, a, lw.ln2, lw.wgu)
    return h, _silu_linear(gu, lw.wd)


def run_layers(P, h, delta, R, K, V, layers, kv_only_last=False, hook=None, keep=None):
    """Run `layers` (an ordered range) for rows R; `hook(l)` runs before layer l (lazy assembly).
    With kv_only_last, the last layer only splices its k/v (its hidden output is never used),
    except for the rows at positions `keep` (int64 tensor), which then run it fully after every
    row's k/v is in place; the result is those rows' (h, delta)."""
    layers = list(layers)
    for j, l in enumerate(layers):
        if hook is not None:
            hook(l)
        last = kv_only_last and j == len(layers) - 1
        if last and keep is not None:
            hk = h.index_select(0, keep)
            dk = None if delta is None else delta.index_select(0, keep)
            layer_forward(P, l, h, delta, R, K, V, kv_only=True)
            h, delta = layer_forward(P, l, hk, dk, R.select(keep), K, V)
        else:
            h, delta = layer_forward(P, l, h, delta, R, K, V, kv_only=last)
    return h, delta


def lm_head(P, x):
    """Logits of the rows x [m, H]. A few rows stream the vocab-sized weight through the skinny
    linear kernel (measured faster than the library GEMM at m <= 8 on MI355X); more rows use the
    library GEMM."""
    if x.shape[0] <= FEW_ROWS and _hip.skinny_ok(x.shape[0], P.lm_head.shape[0], P.lm_head.shape[1]):
        return _hip.skinny_linear(x, P.lm_head)
    return F.linear(x, P.lm_head)


def norm_logits(P, h, delta):
    """Final RMSNorm + lm_head of the rows h (+ delta) [m, H]; one fused kernel for one or two rows."""
    m = h.shape[0]
    if m <= NORM_FUSED_ROWS and _hip.norm_fused_ok(m, P.lm_head.shape[0], P.lm_head.shape[1]):
        return _hip.skinny_norm_linear(h, delta, P.norm, P.eps, P.lm_head)[0]
    _, x = _hip.add_rmsnorm(h, P.norm, P.eps, delta=delta)
    return lm_head(P, x)


def final_logits(P, h, delta):
    """Final RMSNorm + lm_head on the last row only (num_logits_to_keep=1). Returns [vocab]."""
    return norm_logits(P, h[-1:].contiguous(), None if delta is None else delta[-1:].contiguous())[0]


def embed(P, ids):
    return F.embedding(ids, P.embed)


def alloc_cache(P, t_cap, device):
    shape = (P.L, 1, P.hkv, t_cap, P.hd)
    return (torch.empty(shape, dtype=P.embed.dtype, device=device),
            torch.empty(shape, dtype=P.embed.dtype, device=device))
