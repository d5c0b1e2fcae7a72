"""Qwen2 / Llama decoder math on the CPU, restated from transformers' Qwen2 modules.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py). The reference reaches this math through
transformers==4.46.3 Qwen2 modules (tread/blend.py:9,18,35-39,77,82-114); the installed
transformers restates the same formulas, cited here as site: paths under
/usr/local/lib/python3.10/dist-packages/transformers/models/qwen2/modeling_qwen2.py.

Weights come as an HF-named state dict ("model.layers.{i}.self_attn.q_proj.weight", ...), so the
same tensors can be loaded into transformers' own model to pin this restatement.
KV caches are per-layer lists of [1, kv_heads, T, head_dim] tensors, keys post-RoPE.
"""
from dataclasses import dataclass

import torch
import torch.nn.functional as F


@dataclass
class RefModel:
    cfg: object
    w: dict
    dtype: torch.dtype
    inv_freq: torch.Tensor

    @property
    def L(self):
        return self.cfg.num_hidden_layers

    @property
    def n_heads(self):
        return self.cfg.num_attention_heads

    @property
    def n_kv(self):
        return self.cfg.num_key_value_heads

    @property
    def hd(self):
        return self.cfg.head_dim

    @property
    def device(self):
        return self.inv_freq.device

    def p(self, name):
        return self.w[name]


def inv_freq_of(cfg):
    """Default RoPE inverse frequencies (site:modeling_qwen2.py:68-83): 1/theta^(2i/d) in fp32."""
    d = cfg.head_dim
    return 1.0 / (cfg.rope_theta ** (torch.arange(0, d, 2, dtype=torch.int64).float() / d))


def load(cfg, state_dict, dtype=torch.float32, device="cpu"):
    """Weights as `dtype` on `device`. The oracle normally runs on the CPU; on a GPU device the
    same torch ops run there (a second backend of the same algorithm, for comparing roundings)."""
    w = {k: v.detach().to(device, dtype).clone() for k, v in state_dict.items()}
    if "lm_head.weight" not in w:
        w["lm_head.weight"] = w["model.embed_tokens.weight"]
    return RefModel(cfg=cfg, w=w, dtype=dtype, inv_freq=inv_freq_of(cfg).to(device))


def rms_norm(x, weight, eps):
    """site:modeling_qwen2.py:238-252: fp32 variance, rsqrt, cast back, then weight * x."""
    dt = x.dtype
    h = x.to(torch.float32)
    var = h.pow(2).mean(-1, keepdim=True)
    h = h * torch.rsqrt(var + eps)
    return weight * h.to(dt)


def rope_cos_sin(m: RefModel, pos, dtype):
    """site:modeling_qwen2.py:86-102: fp32 angle pos*inv_freq, cat(freqs, freqs), cos/sin cast to dtype.

    pos: LongTensor [n]. Returns cos, sin of shape [1, n, head_dim] (the reference's rotary_emb
    output for a batch of one).
    """
    pos = pos.to(m.device)
    freqs = (m.inv_freq[:, None].float() @ pos[None, :].float()).transpose(0, 1)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype)[None], emb.sin().to(dtype)[None]


def rotate_half(x):
    """site:modeling_qwen2.py:105-109 (split-half, not interleaved)."""
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def apply_rope(x, cos, sin):
    """site:modeling_qwen2.py:113-135 with unsqueeze_dim=1: x [1, heads, n, hd], cos [1, n, hd]."""
    c, s = cos[:, None], sin[:, None]
    return x * c + rotate_half(x) * s


def repeat_kv(x, n_rep):
    """site:modeling_qwen2.py:138-147."""
    b, kv, t, d = x.shape
    if n_rep == 1:
        return x
    return x[:, :, None].expand(b, kv, n_rep, t, d).reshape(b, kv * n_rep, t, d)


def linear(x, m: RefModel, name, bias=None):
    b = m.w.get(name + ".bias") if bias is None else bias
    return F.linear(x, m.w[name + ".weight"], b)


def qkv(m: RefModel, l, x, cos, sin):
    """q/k/v projections, head split and RoPE (tread/blend.py:82-90; site:modeling_qwen2.py:196-214)."""
    pre = f"model.layers.{l}.self_attn."
    n = x.shape[1]
    q = linear(x, m, pre + "q_proj").view(1, n, m.n_heads, m.hd).transpose(1, 2)
    k = linear(x, m, pre + "k_proj").view(1, n, m.n_kv, m.hd).transpose(1, 2)
    v = linear(x, m, pre + "v_proj").view(1, n, m.n_kv, m.hd).transpose(1, 2)
    return apply_rope(q, cos, sin), apply_rope(k, cos, sin), v


def attend(m: RefModel, q, K, V, mask):
    """GQA attention of q [1, hq, n, hd] over K, V [1, kv, T, hd] with a bool or additive mask.

    The reference calls SDPA on repeat_kv'd K/V (tread/blend.py:107-110); scale = hd^-0.5
    (site:modeling_qwen2.py:186).
    """
    g = m.n_heads // m.n_kv
    args = (q, repeat_kv(K, g), repeat_kv(V, g))
    if q.is_cuda:
        # on a GPU only the memory-efficient kernel (fp32 accumulation, like the CPU kernel): the
        # math backend's batched bf16 products over transposed views are not used there
        from torch.nn.attention import SDPBackend, sdpa_kernel
        with sdpa_kernel(SDPBackend.EFFICIENT_ATTENTION):
            return F.scaled_dot_product_attention(*args, attn_mask=mask)
    return F.scaled_dot_product_attention(*args, attn_mask=mask)


def mlp(m: RefModel, l, x):
    """site:modeling_qwen2.py:35-48: down(silu(gate(x)) * up(x))."""
    pre = f"model.layers.{l}.mlp."
    return linear(F.silu(linear(x, m, pre + "gate_proj")) * linear(x, m, pre + "up_proj"), m, pre + "down_proj")


def o_proj(m: RefModel, l, o):
    n = o.shape[2]
    return linear(o.transpose(1, 2).reshape(1, n, -1), m, f"model.layers.{l}.self_attn.o_proj")


def norm(m: RefModel, name, x):
    return rms_norm(x, m.w[name + ".weight"], m.cfg.rms_norm_eps)


def embed(m: RefModel, ids):
    return F.embedding(ids, m.w["model.embed_tokens.weight"])


def forward(m: RefModel, ids, past=None, position_ids=None, mask4d=None):
    """Decoder forward over `ids` (1-D LongTensor) on top of an optional past cache.

    Mirrors `model.model(ids[None], past_key_values=..., attention_mask=..., position_ids=...)` as the
    reference uses it (tread/blend.py:18; tread/engine.py:86-88,132,148,162): positions default to
    P..P+n-1 where P is the past length; the mask defaults to causal over the concatenated cache;
    a 4D additive mask [1,1,n,P+n] is used as given. DynamicCache.update concatenates new K/V after
    the past ones (site:transformers/cache_utils.py:113-152).

    Returns (h [1, n, hidden] after the final norm, K list, V list) with K/V the full caches.
    """
    n = len(ids)
    dev = m.device
    P = 0 if past is None else past[0][0].shape[2]
    if position_ids is None:
        position_ids = torch.arange(P, P + n, device=dev)
    cos, sin = rope_cos_sin(m, position_ids, m.dtype)
    if mask4d is None:
        mask = (torch.arange(P + n, device=dev)[None, :] <= (P + torch.arange(n, device=dev))[:, None])[None, None]
    else:
        mask = mask4d
    h = embed(m, ids)[None]
    Ks, Vs = [], []
    for l in range(m.L):
        x = norm(m, f"model.layers.{l}.input_layernorm", h)
        q, k, v = qkv(m, l, x, cos, sin)
        if past is not None:
            k = torch.cat([past[0][l], k], dim=2)
            v = torch.cat([past[1][l], v], dim=2)
        Ks.append(k)
        Vs.append(v)
        h = h + o_proj(m, l, attend(m, q, k, v, mask))
        h = h + mlp(m, l, norm(m, f"model.layers.{l}.post_attention_layernorm", h))
    return norm(m, "model.norm", h), Ks, Vs


def logits_last(m: RefModel, h):
    """lm_head on the last position only (num_logits_to_keep=1): returns [vocab] in the model dtype."""
    return F.linear(h[0, -1], m.w["lm_head.weight"])
