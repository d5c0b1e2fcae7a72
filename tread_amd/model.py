"""Qwen2 / Llama-shaped decoder for the reuse engine: configs, random init, prepared weights.

`DecoderLM` mirrors the module tree of transformers' Qwen2ForCausalLM / LlamaForCausalLM
(`model.model.layers[i].self_attn.q_proj`, `.mlp.gate_proj`, `model.model.embed_tokens`,
`model.lm_head`, `model.config`, `model.dtype`), so the engine accepts either it or a transformers
model. It stores q|k|v and gate|up as single fused tensors and exposes the per-projection
weights as views of them, so one GEMM serves the three (two) projections with no extra memory.

Weights are generated directly on the target device: N(0, std) for Linear/Embedding weights,
biases N(0, bias_std) (0 by default), RMSNorm weights 1, in named_parameters() order from one
torch.Generator seeded with `seed` (CPU generation reproduces across machines; GPU generation is
used for large shapes where only timing matters).
"""
from dataclasses import dataclass, field, replace

import torch
import torch.nn as nn
import torch.nn.functional as F


@dataclass
class ModelConfig:
    vocab_size: int
    hidden_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    intermediate_size: int
    rope_theta: float = 1000000.0
    rms_norm_eps: float = 1e-6
    attention_bias: bool = True
    tie_word_embeddings: bool = False
    family: str = "qwen2"
    _name_or_path: str = ""
    rope_scaling: object = None
    max_position_embeddings: int = 131072

    @property
    def num_key_value_groups(self):
        return self.num_attention_heads // self.num_key_value_heads

    def scaled(self, **kw):
        return replace(self, **kw)


# Shapes of the public checkpoints the reference's configs name (random-init here).
PRESETS = {
    "qwen2.5-0.5b": ModelConfig(151936, 896, 24, 14, 2, 64, 4864, 1000000.0, 1e-6, True, True),
    "qwen2.5-1.5b": ModelConfig(151936, 1536, 28, 12, 2, 128, 8960, 1000000.0, 1e-6, True, True),
    "qwen2.5-7b": ModelConfig(152064, 3584, 28, 28, 4, 128, 18944, 1000000.0, 1e-6, True, False),
    "llama3-70b": ModelConfig(128256, 8192, 80, 64, 8, 128, 28672, 500000.0, 1e-5, False, False, "llama"),
}


def preset(name, **overrides):
    return replace(PRESETS[name], **overrides)


def inv_freq_of(cfg):
    """Default RoPE inverse frequencies 1/theta^(2i/d), fp32, computed on the CPU like HF."""
    d = cfg.head_dim
    return 1.0 / (cfg.rope_theta ** (torch.arange(0, d, 2, dtype=torch.int64).float() / d))


class _ViewLinear(nn.Module):
    """nn.Linear look-alike whose weight/bias are views into fused storage."""

    def __init__(self, weight, bias=None):
        super().__init__()
        self.weight = weight if isinstance(weight, nn.Parameter) else nn.Parameter(weight, requires_grad=False)
        self.bias = None if bias is None else nn.Parameter(bias, requires_grad=False)

    def forward(self, x):
        return F.linear(x, self.weight, self.bias)


class RMSNorm(nn.Module):
    def __init__(self, hidden, eps, device, dtype):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden, device=device, dtype=dtype), requires_grad=False)
        self.variance_epsilon = eps

    def forward(self, x):
        dt = x.dtype
        h = x.to(torch.float32)
        h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + self.variance_epsilon)
        return self.weight * h.to(dt)


class RotaryEmbedding(nn.Module):
    def __init__(self, cfg, device):
        super().__init__()
        self.register_buffer("inv_freq", inv_freq_of(cfg).to(device), persistent=False)
        self.attention_scaling = 1.0

    @torch.no_grad()
    def forward(self, x, position_ids):
        f = (self.inv_freq[None, :, None].float() @ position_ids[:, None, :].float()).transpose(1, 2)
        emb = torch.cat((f, f), dim=-1)
        return emb.cos().to(x.dtype), emb.sin().to(x.dtype)


class Attention(nn.Module):
    def __init__(self, cfg, device, dtype):
        super().__init__()
        hq, hkv, hd, H = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim, cfg.hidden_size
        self.num_heads, self.num_key_value_heads, self.head_dim = hq, hkv, hd
        self.num_key_value_groups = hq // hkv
        rows = (hq + 2 * hkv) * hd
        self.register_buffer("qkv_weight", torch.empty(rows, H, device=device, dtype=dtype), persistent=False)
        self.register_buffer("qkv_bias", torch.zeros(rows, device=device, dtype=dtype) if cfg.attention_bias else None,
                             persistent=False)
        w, b = self.qkv_weight, self.qkv_bias
        q, k = hq * hd, hkv * hd
        self.q_proj = _ViewLinear(w[:q], None if b is None else b[:q])
        self.k_proj = _ViewLinear(w[q:q + k], None if b is None else b[q:q + k])
        self.v_proj = _ViewLinear(w[q + k:], None if b is None else b[q + k:])
        self.o_proj = _ViewLinear(torch.empty(H, hq * hd, device=device, dtype=dtype))


class MLP(nn.Module):
    def __init__(self, cfg, device, dtype):
        super().__init__()
        H, I = cfg.hidden_size, cfg.intermediate_size
        self.register_buffer("gate_up_weight", torch.empty(2 * I, H, device=device, dtype=dtype), persistent=False)
        self.gate_proj = _ViewLinear(self.gate_up_weight[:I])
        self.up_proj = _ViewLinear(self.gate_up_weight[I:])
        self.down_proj = _ViewLinear(torch.empty(H, I, device=device, dtype=dtype))

    def forward(self, x):
        return self.down_proj(F.silu(self.gate_proj(x)) * self.up_proj(x))


class DecoderLayer(nn.Module):
    def __init__(self, cfg, device, dtype):
        super().__init__()
        self.self_attn = Attention(cfg, device, dtype)
        self.mlp = MLP(cfg, device, dtype)
        self.input_layernorm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps, device, dtype)
        self.post_attention_layernorm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps, device, dtype)


class _Body(nn.Module):
    def __init__(self, cfg, device, dtype):
        super().__init__()
        self.embed_tokens = nn.Embedding(cfg.vocab_size, cfg.hidden_size, device=device, dtype=dtype)
        self.embed_tokens.weight.requires_grad_(False)
        self.layers = nn.ModuleList(DecoderLayer(cfg, device, dtype) for _ in range(cfg.num_hidden_layers))
        self.norm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps, device, dtype)
        self.rotary_emb = RotaryEmbedding(cfg, device)


class DecoderLM(nn.Module):
    """Random-init Qwen2/Llama-shaped causal LM, built in place on `device` in `dtype`."""

    def __init__(self, cfg: ModelConfig, device="cuda", dtype=torch.bfloat16):
        super().__init__()
        self.config = cfg
        self.model = _Body(cfg, device, dtype)
        if cfg.tie_word_embeddings:
            self.lm_head = _ViewLinear(self.model.embed_tokens.weight)
        else:
            self.lm_head = _ViewLinear(torch.empty(cfg.vocab_size, cfg.hidden_size, device=device, dtype=dtype))
        self._dtype = dtype

    @property
    def dtype(self):
        return self._dtype

    @property
    def device(self):
        return self.model.embed_tokens.weight.device

    @torch.no_grad()
    def init_synthetic_(self, seed=0, std=0.02, bias_std=0.0):
        g = torch.Generator(device=self.device).manual_seed(seed)
        for name, p in self.named_parameters():
            if name.endswith("norm.weight"):
                p.fill_(1.0)
            elif name.endswith(".bias"):
                if bias_std > 0:
                    p.normal_(0.0, bias_std, generator=g)
                else:
                    p.zero_()
            else:
                p.normal_(0.0, std, generator=g)
        return self


def synthetic_model(cfg, device="cuda", dtype=torch.bfloat16, seed=0, std=0.02, bias_std=0.0):
    return DecoderLM(cfg, device, dtype).init_synthetic_(seed, std, bias_std)


# ----------------------------------------------------------------------------- prepared weights

@dataclass
class LayerW:
    ln1: torch.Tensor
    wqkv: torch.Tensor
    bqkv: object
    wo: torch.Tensor
    ln2: torch.Tensor
    wgu: torch.Tensor
    wd: torch.Tensor


@dataclass
class Prepared:
    """Flat view of a model's weights in the layout the HIP path consumes."""
    L: int
    H: int
    hq: int
    hkv: int
    hd: int
    inter: int
    eps: float
    embed: torch.Tensor
    norm: torch.Tensor
    lm_head: torch.Tensor
    inv_freq: torch.Tensor  # fp32, CPU
    layers: list = field(default_factory=list)

    @property
    def scale(self):
        return self.hd ** -0.5


def _cfg_get(cfg, *names, default=None):
    for n in names:
        v = getattr(cfg, n, None)
        if v is not None:
            return v
    return default


def rope_theta_of(cfg):
    t = getattr(cfg, "rope_theta", None)
    if t is None:
        rp = getattr(cfg, "rope_parameters", None) or {}
        t = rp.get("rope_theta")
    return t


def prepare(model) -> Prepared:
    """Build the fused weight view. DecoderLM already stores fused q|k|v and gate|up tensors;
    for a transformers model they are concatenated once (extra memory = those projections)."""
    cfg = model.config
    body = model.model
    hq = cfg.num_attention_heads
    hkv = cfg.num_key_value_heads
    H = cfg.hidden_size
    hd = _cfg_get(cfg, "head_dim", default=H // hq)
    rot = getattr(body, "rotary_emb", None)
    if rot is not None and getattr(rot, "inv_freq", None) is not None:
        inv = rot.inv_freq.detach().to("cpu", torch.float32).clone()
        if float(getattr(rot, "attention_scaling", 1.0)) != 1.0:
            raise NotImplementedError("RoPE with attention_scaling != 1 is not supported")
    else:
        inv = 1.0 / (rope_theta_of(cfg) ** (torch.arange(0, hd, 2, dtype=torch.int64).float() / hd))
    layers = []
    for lyr in body.layers:
        at, mlp = lyr.self_attn, lyr.mlp
        if hasattr(at, "qkv_weight"):
            wqkv, bqkv = at.qkv_weight, at.qkv_bias
        else:
            wqkv = torch.cat([at.q_proj.weight, at.k_proj.weight, at.v_proj.weight]).contiguous()
            bqkv = None if at.q_proj.bias is None else torch.cat(
                [at.q_proj.bias, at.k_proj.bias, at.v_proj.bias]).contiguous()
        if hasattr(mlp, "gate_up_weight"):
            wgu = mlp.gate_up_weight
        else:
            wgu = torch.cat([mlp.gate_proj.weight, mlp.up_proj.weight]).contiguous()
        layers.append(LayerW(lyr.input_layernorm.weight, wqkv, bqkv, at.o_proj.weight,
                             lyr.post_attention_layernorm.weight, wgu, mlp.down_proj.weight))
    return Prepared(L=len(layers), H=H, hq=hq, hkv=hkv, hd=hd, inter=cfg.intermediate_size,
                    eps=float(cfg.rms_norm_eps), embed=body.embed_tokens.weight, norm=body.norm.weight,
                    lm_head=model.lm_head.weight, inv_freq=inv, layers=layers)
