"""ctypes binding of libtread_hip.so (include/tread_hip.h) and torch-facing wrappers.

The wrappers validate shapes, dtypes, devices and contiguity on the host, then pass raw device
pointers and torch's current HIP stream to the C entry points. There is no fallback: if the
library is missing or a call fails, a RuntimeError says why.
"""
import ctypes
from pathlib import Path

import torch  # loads torch's HIP runtime first, so the library below binds to the same one

LIB_PATH = Path(__file__).resolve().with_name("libtread_hip.so")
ABI_VERSION = 10

c_i64, c_int, c_void, c_float, c_size = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_float, ctypes.c_size_t
P_I64 = ctypes.POINTER(ctypes.c_int64)
P_F32 = ctypes.POINTER(ctypes.c_float)


class Src(ctypes.Structure):
    """tread_src_t."""
    _fields_ = [("k", c_void), ("v", c_void), ("n_tokens", c_i64), ("dst_off", c_i64), ("delta", c_i64)]


_SIGS = {
    "tread_last_error": (ctypes.c_char_p, []),
    "tread_abi_version": (c_int, []),
    "tread_rope_assemble_bf16": (c_int, [ctypes.POINTER(Src), c_int, c_void, c_void, c_int, c_int, c_i64, c_int,
                                         P_F32, c_int, c_int, c_void]),
    "tread_rope_table_bf16": (c_int, [c_void, c_i64, P_F32, c_int, c_void, c_void, c_void]),
    "tread_qkv_rope_splice_bf16": (c_int, [c_void, c_void, c_void, c_i64, c_void, c_void, c_void, c_i64, c_int,
                                           c_int, c_int, c_void, c_void, c_void, c_i64, c_void]),
    "tread_dev_score_bf16": (c_int, [c_void, c_void, c_i64, c_void, c_void, c_void, c_i64, c_int, c_int, c_void,
                                     c_void, c_i64, c_void, c_void]),
    "tread_topk_workspace_bytes": (c_size, [c_i64]),
    "tread_topk_select_bf16": (c_int, [c_void, c_i64, c_i64, c_void, c_void, c_size, c_void]),
    "tread_subset_attn_workspace_bytes": (c_size, [c_i64, c_int, c_int, c_int, c_i64]),
    "tread_subset_attn_bf16": (c_int, [c_void, c_void, c_void, c_void, c_void, c_i64, c_i64, c_int, c_int, c_int,
                                       c_i64, c_float, c_void, c_void, c_size, c_void]),
    "tread_subset_attn_scratch_bf16": (c_int, [c_void, c_void, c_void, c_void, c_void, c_i64, c_i64, c_int, c_int,
                                               c_int, c_i64, c_float, c_void, c_void]),
    "tread_add_rmsnorm_bf16": (c_int, [c_void, c_void, c_void, c_float, c_i64, c_int, c_void, c_void, c_void]),
    "tread_silu_mul_bf16": (c_int, [c_void, c_i64, c_int, c_void, c_void]),
    "tread_skinny_workspace_bytes": (c_size, [c_i64, c_i64, c_i64]),
    "tread_skinny_linear_bf16": (c_int, [c_void, c_i64, c_void, c_void, c_i64, c_i64, c_i64, c_void, c_i64, c_void,
                                         c_size, c_void]),
    "tread_skinny_norm_linear_bf16": (c_int, [c_void, c_void, c_void, c_float, c_i64, c_i64, c_i64, c_void, c_void,
                                              c_void, c_void, c_void]),
    "tread_skinny_norm_qkv_rope_bf16": (c_int, [c_void, c_void, c_void, c_float, c_i64, c_i64, c_void, c_void, c_int,
                                                c_int, c_int, c_void, c_void, c_void, c_void, c_void, c_void, c_i64,
                                                c_void, c_void]),
    "tread_skinny_norm_swiglu_bf16": (c_int, [c_void, c_void, c_void, c_float, c_i64, c_i64, c_void, c_i64, c_void,
                                              c_void, c_void]),
    "tread_skinny_silu_workspace_bytes": (c_size, [c_i64, c_i64, c_i64]),
    "tread_skinny_silu_linear_bf16": (c_int, [c_void, c_i64, c_i64, c_void, c_i64, c_void, c_void, c_size, c_void]),
    "tread_copy_async": (c_int, [c_void, c_void, c_size, c_void, c_void]),
    "tread_copy_layers_async": (c_int, [c_void, c_void, c_void, c_int, c_int, c_void, c_void]),
}

_lib = None


def lib():
    """Load the library once; raise if it is missing (no CPU fallback exists)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built: run `python -m tread_amd.csrc.build` "
                               "(or __graft_entry__.build()) first")
        l = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            f = getattr(l, name)
            f.restype, f.argtypes = res, args
        if l.tread_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH}: ABI {l.tread_abi_version()} != {ABI_VERSION}; rebuild it")
        _lib = l
    return _lib


def exported_symbols():
    return list(_SIGS)


def _check(name, rc):
    if rc != 0:
        msg = lib().tread_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed ({rc}): {msg}")


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _need(t, name, dtype=torch.bfloat16, contig=True):
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a GPU tensor (the HIP path has no CPU fallback)")
    if dtype is not None and t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if contig and not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _freq(inv_freq):
    f = inv_freq.detach().to("cpu", torch.float32).contiguous()
    return f, ctypes.cast(f.data_ptr(), P_F32)


# ------------------------------------------------------------------------------------------- (a)

def delta_table_host(inv_freq, deltas):
    """fp32 [n, hd/2, 2] (cos, sin) of fp32(delta) * inv_freq on the host, computed with the same
    torch ops as the reference's rotary embedding (fp32 outer product, then cos / sin)."""
    pos = torch.tensor([int(d) for d in deltas], dtype=torch.int64)
    freqs = (inv_freq.detach().to("cpu", torch.float32)[:, None] @ pos[None, :].float()).transpose(0, 1)
    return torch.stack([freqs.cos(), freqs.sin()], dim=-1).contiguous()


def delta_table(inv_freq, deltas, device):
    """delta_table_host, moved to `device`."""
    return delta_table_host(inv_freq, deltas).pin_memory().to(device, non_blocking=True)


def rope_assemble(sources, dst_k, dst_v, inv_freq, layer_lo=0, layer_hi=None, table=None):
    """sources: list of (K, V, dst_off, delta) with K, V [L, 1, kv, n, hd] bf16 on the GPU.
    dst_k, dst_v: [L, 1, kv, t_cap, hd]. Rotates K by delta (fp32 cos/sin table), copies V.
    dst_v None moves K only (the sources' V may then be None).
    `table` (from delta_table over the sources' deltas) may be passed to reuse it across calls."""
    _need(dst_k, "dst_k")
    L, one, kv, t_cap, hd = dst_k.shape
    if dst_v is not None:
        _need(dst_v, "dst_v")
        if dst_v.shape != dst_k.shape:
            raise ValueError("dst_k / dst_v must both be [L, 1, kv, t_cap, hd]")
    if one != 1:
        raise ValueError("dst_k must be [L, 1, kv, t_cap, hd]")
    layer_hi = L if layer_hi is None else layer_hi
    arr = (Src * max(1, len(sources)))()
    for i, (K, V, off, delta) in enumerate(sources):
        _need(K, f"source {i} K")
        if K.shape[:3] != (L, 1, kv) or K.shape[-1] != hd:
            raise ValueError(f"source {i}: shape {tuple(K.shape)} does not match cache {tuple(dst_k.shape)}")
        if dst_v is not None:
            _need(V, f"source {i} V")
            if V.shape != K.shape:
                raise ValueError(f"source {i}: V shape {tuple(V.shape)} differs from K {tuple(K.shape)}")
        vp = V.data_ptr() if dst_v is not None else 0
        arr[i] = Src(K.data_ptr(), vp, K.shape[-2], int(off), int(delta))
    if table is None:
        table = delta_table(inv_freq, [s[3] for s in sources], dst_k.device)
    if table.shape != (len(sources), hd // 2, 2) or table.dtype != torch.float32 or not table.is_cuda:
        raise ValueError("rope_assemble: table must be fp32 [n_src, hd/2, 2] on the GPU")
    _check("tread_rope_assemble_bf16", lib().tread_rope_assemble_bf16(
        arr, len(sources), _ptr(dst_k), _ptr(dst_v), L, kv, t_cap, hd,
        ctypes.cast(table.data_ptr(), P_F32), layer_lo, layer_hi, _stream()))
    return table


# ------------------------------------------------------------------------------------ RoPE / glue

def rope_table(pos, inv_freq, head_dim):
    """bf16 cos, sin [n, head_dim/2] for int64 positions, rounded like the reference's rotary_emb."""
    _need(pos, "pos", torch.int64)
    n = pos.numel()
    cos = torch.empty(n, head_dim // 2, dtype=torch.bfloat16, device=pos.device)
    sin = torch.empty_like(cos)
    f, fp = _freq(inv_freq)
    _check("tread_rope_table_bf16", lib().tread_rope_table_bf16(_ptr(pos), n, fp, head_dim, _ptr(cos), _ptr(sin),
                                                               _stream()))
    return cos, sin


def qkv_rope_splice(qkv, cos, sin, rows, hq, hkv, hd, k_cache, v_cache, q_out=None, q_col=0, k_col=None, v_col=None):
    """qkv: [n, ld] GEMM output holding q at column q_col, k at k_col, v at v_col (defaults: q|k|v).
    k_cache / v_cache: one layer [1, hkv, t_cap, hd] (or [hkv, t_cap, hd]). q_out: [n, hq, hd] or None."""
    _need(qkv, "qkv")
    _need(rows, "rows", torch.int64)
    _need(k_cache, "k_cache")
    _need(v_cache, "v_cache")
    n, ld = qkv.shape
    k_col = hq * hd if k_col is None else k_col
    v_col = k_col + hkv * hd if v_col is None else v_col
    t_cap = k_cache.shape[-2]
    if k_cache.shape[-3] != hkv or k_cache.shape[-1] != hd or v_cache.shape != k_cache.shape:
        raise ValueError("cache shape mismatch")
    if q_out is not None:
        _need(q_out, "q_out")
        if q_out.numel() != n * hq * hd:
            raise ValueError("q_out shape mismatch")
    base = qkv.data_ptr()
    es = qkv.element_size()
    _check("tread_qkv_rope_splice_bf16", lib().tread_qkv_rope_splice_bf16(
        ctypes.c_void_p(base + q_col * es), ctypes.c_void_p(base + k_col * es), ctypes.c_void_p(base + v_col * es),
        ld, _ptr(cos), _ptr(sin), _ptr(rows), n, hq, hkv, hd, _ptr(q_out), _ptr(k_cache), _ptr(v_cache), t_cap,
        _stream()))


def add_rmsnorm(x, weight, eps, delta=None, sum_out=None, norm_out=None):
    """norm_out = weight * bf16(s * rsqrt(mean(s^2) + eps)), s = x + delta (bf16). Returns (s, norm)."""
    _need(x, "x")
    _need(weight, "weight")
    H = x.shape[-1]
    n = x.numel() // H
    if delta is not None:
        _need(delta, "delta")
        if sum_out is None:
            sum_out = torch.empty_like(x)
    if norm_out is None:
        norm_out = torch.empty_like(x)
    _check("tread_add_rmsnorm_bf16", lib().tread_add_rmsnorm_bf16(
        _ptr(x), _ptr(delta), _ptr(weight), float(eps), n, H, _ptr(sum_out), _ptr(norm_out), _stream()))
    return (sum_out if delta is not None else x), norm_out


SKINNY_MAX_ROWS = 32


def skinny_ok(m, n, k):
    """Shapes the skinny linear kernel takes (rows <= 32, n % 32 == 0, k % 128 == 0)."""
    return 0 < m <= SKINNY_MAX_ROWS and n % 32 == 0 and k % 128 == 0


def skinny_linear(x, weight, bias=None, out=None):
    """y = x @ weight.T (+ bias) for a few rows x [m, k] (m <= 32): weight-streaming MFMA kernel."""
    _need(x, "x", contig=False)
    _need(weight, "weight")
    if bias is not None:
        _need(bias, "bias")
    m, k = x.shape
    n = weight.shape[0]
    if x.stride(1) != 1 or weight.shape[1] != k or not skinny_ok(m, n, k):
        raise ValueError(f"skinny_linear: unsupported shape x {tuple(x.shape)} weight {tuple(weight.shape)}")
    if out is None:
        out = torch.empty(m, n, dtype=x.dtype, device=x.device)
    wsb = lib().tread_skinny_workspace_bytes(m, n, k)
    ws = torch.empty(wsb, dtype=torch.uint8, device=x.device) if wsb else None
    _check("tread_skinny_linear_bf16", lib().tread_skinny_linear_bf16(
        _ptr(x), x.stride(0), _ptr(weight), _ptr(bias), m, n, k, _ptr(out), out.stride(0), _ptr(ws), wsb, _stream()))
    return out


FUSED_MAX_ROWS = 8


FUSED_STAGE_BYTES = 127 * 1024  # LDS the norm-fused kernel may stage its rows in


def fused_ok(m, n, k):
    """Shapes of the fused-prologue skinny kernels (rows <= 8)."""
    return 0 < m <= FUSED_MAX_ROWS and skinny_ok(m, n, k)


def norm_fused_ok(m, n, k):
    """fused_ok, and the m normed rows of k fit in LDS."""
    return fused_ok(m, n, k) and m * k * 2 <= FUSED_STAGE_BYTES


def skinny_norm_linear(h, delta, ln_w, eps, weight, bias=None):
    """(linear(RMSNorm(h + delta)), h + delta) for a few rows h [m, k]: the layer-input norm fused in
    front of the projection. delta may be None (then the second result is h itself)."""
    _need(h, "h")
    _need(weight, "weight")
    _need(ln_w, "ln_w")
    if delta is not None:
        _need(delta, "delta")
    if bias is not None:
        _need(bias, "bias")
    m, k = h.shape
    n = weight.shape[0]
    if weight.shape[1] != k or not norm_fused_ok(m, n, k) or (delta is not None and delta.shape != h.shape):
        raise ValueError(f"skinny_norm_linear: unsupported shape h {tuple(h.shape)} weight {tuple(weight.shape)}")
    y = torch.empty(m, n, dtype=h.dtype, device=h.device)
    h_out = torch.empty_like(h) if delta is not None else None
    _check("tread_skinny_norm_linear_bf16", lib().tread_skinny_norm_linear_bf16(
        _ptr(h), _ptr(delta), _ptr(ln_w), float(eps), m, n, k, _ptr(weight), _ptr(bias), _ptr(y), _ptr(h_out),
        _stream()))
    return y, (h_out if h_out is not None else h)


def skinny_norm_qkv_rope(h, delta, ln_w, eps, wqkv, bqkv, hq, hkv, hd, cos, sin, rows, q_out, k_cache, v_cache):
    """skinny_norm_linear of the q|k|v projection and qkv_rope_splice in one launch: q (rotated)
    into q_out [m, hq, hd], k (rotated) and v into rows `rows` of one layer's k_cache / v_cache
    [(1,) hkv, t_cap, hd]. Returns h + delta (h itself when delta is None); the same bits as the two
    calls."""
    for t, name in ((h, "h"), (wqkv, "wqkv"), (ln_w, "ln_w"), (cos, "cos"), (sin, "sin"), (q_out, "q_out"),
                    (k_cache, "k_cache"), (v_cache, "v_cache")):
        _need(t, name)
    _need(rows, "rows", torch.int64)
    if delta is not None:
        _need(delta, "delta")
    if bqkv is not None:
        _need(bqkv, "bqkv")
    m, k = h.shape
    n = (hq + 2 * hkv) * hd
    t_cap = k_cache.shape[-2]
    if (wqkv.shape != (n, k) or not norm_fused_ok(m, n, k) or (delta is not None and delta.shape != h.shape)
            or rows.numel() != m or q_out.numel() != m * hq * hd or k_cache.shape[-3] != hkv
            or k_cache.shape[-1] != hd or v_cache.shape != k_cache.shape or cos.shape != (m, hd // 2)
            or sin.shape != cos.shape):
        raise ValueError(f"skinny_norm_qkv_rope: unsupported shapes h {tuple(h.shape)} wqkv {tuple(wqkv.shape)}")
    h_out = torch.empty_like(h) if delta is not None else None
    _check("tread_skinny_norm_qkv_rope_bf16", lib().tread_skinny_norm_qkv_rope_bf16(
        _ptr(h), _ptr(delta), _ptr(ln_w), float(eps), m, k, _ptr(wqkv), _ptr(bqkv), hq, hkv, hd, _ptr(cos),
        _ptr(sin), _ptr(rows), _ptr(q_out), _ptr(k_cache), _ptr(v_cache), t_cap, _ptr(h_out), _stream()))
    return h_out if h_out is not None else h


def skinny_norm_swiglu(h, delta, ln_w, eps, wgu):
    """(bf16(silu(g)) * u, h + delta) for a few rows h [m, k], [g | u] = linear(RMSNorm(h + delta),
    wgu) (wgu [2 inter, k]): the MLP's norm, gate|up and SiLU gating in one launch, the same bits
    as skinny_norm_linear followed by silu_mul. delta may be None (then h itself comes back)."""
    _need(h, "h")
    _need(wgu, "wgu")
    _need(ln_w, "ln_w")
    if delta is not None:
        _need(delta, "delta")
    m, k = h.shape
    n = wgu.shape[0]
    inter = n // 2
    if (wgu.shape[1] != k or n % 2 or inter % 16 or not norm_fused_ok(m, n, k)
            or (delta is not None and delta.shape != h.shape)):
        raise ValueError(f"skinny_norm_swiglu: unsupported shape h {tuple(h.shape)} wgu {tuple(wgu.shape)}")
    y = torch.empty(m, inter, dtype=h.dtype, device=h.device)
    h_out = torch.empty_like(h) if delta is not None else None
    _check("tread_skinny_norm_swiglu_bf16", lib().tread_skinny_norm_swiglu_bf16(
        _ptr(h), _ptr(delta), _ptr(ln_w), float(eps), m, k, _ptr(wgu), inter, _ptr(y), _ptr(h_out), _stream()))
    return y, (h_out if h_out is not None else h)


def skinny_silu_linear(gate_up, weight):
    """linear(silu(g) * u) for a few rows gate_up [m, 2 inter] = [g | u]: SiLU-gating fused into
    the down projection."""
    _need(gate_up, "gate_up")
    _need(weight, "weight")
    m, two_i = gate_up.shape
    inter, n = two_i // 2, weight.shape[0]
    if weight.shape[1] != inter or not fused_ok(m, n, inter):
        raise ValueError(f"skinny_silu_linear: unsupported shape {tuple(gate_up.shape)} x {tuple(weight.shape)}")
    y = torch.empty(m, n, dtype=gate_up.dtype, device=gate_up.device)
    wsb = lib().tread_skinny_silu_workspace_bytes(m, n, inter)
    ws = torch.empty(wsb, dtype=torch.uint8, device=gate_up.device) if wsb else None
    _check("tread_skinny_silu_linear_bf16", lib().tread_skinny_silu_linear_bf16(
        _ptr(gate_up), m, inter, _ptr(weight), n, _ptr(y), _ptr(ws), wsb, _stream()))
    return y


def silu_mul(gate_up, out=None):
    _need(gate_up, "gate_up")
    two_i = gate_up.shape[-1]
    n = gate_up.numel() // two_i
    if out is None:
        out = torch.empty(*gate_up.shape[:-1], two_i // 2, dtype=gate_up.dtype, device=gate_up.device)
    _check("tread_silu_mul_bf16", lib().tread_silu_mul_bf16(_ptr(gate_up), n, two_i // 2, _ptr(out), _stream()))
    return out


# ------------------------------------------------------------------------------------------- (b)

def dev_score(kv, cos, sin, rows, hkv, hd, k_cache, v_cache, k_col=0, v_col=None, out=None):
    """kv: [n, ld] with raw (bias added, pre-RoPE) k at k_col and v at v_col. Returns bf16 [n]."""
    _need(kv, "kv")
    _need(rows, "rows", torch.int64)
    _need(k_cache, "k_cache")
    _need(v_cache, "v_cache")
    n, ld = kv.shape
    v_col = k_col + hkv * hd if v_col is None else v_col
    if out is None:
        out = torch.empty(n, dtype=torch.bfloat16, device=kv.device)
    es = kv.element_size()
    _check("tread_dev_score_bf16", lib().tread_dev_score_bf16(
        ctypes.c_void_p(kv.data_ptr() + k_col * es), ctypes.c_void_p(kv.data_ptr() + v_col * es), ld, _ptr(cos),
        _ptr(sin), _ptr(rows), n, hkv, hd, _ptr(k_cache), _ptr(v_cache), k_cache.shape[-2], _ptr(out), _stream()))
    return out


def topk_select(score, k, out=None):
    """Indices of the k largest bf16 scores, ascending; ties at the threshold go to the lowest indices."""
    _need(score, "score")
    n = score.numel()
    if out is None:
        out = torch.empty(k, dtype=torch.int64, device=score.device)
    _check("tread_topk_select_bf16", lib().tread_topk_select_bf16(_ptr(score), n, k, _ptr(out), None, 0, _stream()))
    return out


# ------------------------------------------------------------------------------------------- (c)

def subset_attn(q, k_cache, v_cache, kend, hq, hkv, hd, scale, kseg=None, n_shared=0, out=None):
    """q: [n, hq, hd]; k_cache/v_cache: one layer [(1,) hkv, t_cap, hd]; kend/kseg: int64 [n].
    Returns out [n, hq*hd]."""
    _need(q, "q")
    _need(k_cache, "k_cache")
    _need(v_cache, "v_cache")
    _need(kend, "kend", torch.int64)
    if kseg is not None:
        _need(kseg, "kseg", torch.int64)
    n = kend.numel()
    if q.numel() != n * hq * hd:
        raise ValueError(f"q has {q.numel()} elements, expected {n}x{hq}x{hd}")
    if out is None:
        out = torch.empty(n, hq * hd, dtype=q.dtype, device=q.device)
    t_cap = k_cache.shape[-2]
    wsb = lib().tread_subset_attn_workspace_bytes(n, hq, hkv, hd, t_cap)
    ws = torch.empty(wsb, dtype=torch.uint8, device=q.device) if wsb else None
    _check("tread_subset_attn_bf16", lib().tread_subset_attn_bf16(
        _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(kend), _ptr(kseg), int(n_shared), n, hq, hkv, hd,
        t_cap, float(scale), _ptr(out), _ptr(ws), wsb, _stream()))
    return out


SUBSET_ATTN_SCRATCH_BYTES = 96 << 20  # TREAD_SUBSET_ATTN_SCRATCH_BYTES


def subset_attn_scratch(q, k_cache, v_cache, kend, hq, hkv, hd, scale, out, kseg=None, n_shared=0):
    """subset_attn through the entry point that allocates nothing: its partials live in the
    library's static per-device scratch array (shared by every call on the GPU: calls that overlap
    on one GPU race). The caller passes `out` [n, hq*hd]. Shapes whose workspace exceeds
    SUBSET_ATTN_SCRATCH_BYTES raise."""
    _need(q, "q")
    _need(k_cache, "k_cache")
    _need(v_cache, "v_cache")
    _need(kend, "kend", torch.int64)
    _need(out, "out")
    if kseg is not None:
        _need(kseg, "kseg", torch.int64)
    n = kend.numel()
    if q.numel() != n * hq * hd or out.numel() != n * hq * hd:
        raise ValueError(f"q / out must hold {n}x{hq}x{hd} elements")
    _check("tread_subset_attn_scratch_bf16", lib().tread_subset_attn_scratch_bf16(
        _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(kend), _ptr(kseg), int(n_shared), n, hq, hkv, hd,
        k_cache.shape[-2], float(scale), _ptr(out), _stream()))
    return out


# ------------------------------------------------------------------------------------------- (d)

def layer_groups(L):
    """Layer groups of a tier move, small first (the first layers are needed first): 1, 1, 2, then
    4, 4, 8, 8, 16, 16, ... layers. Layer 0 travels alone: a request's deviation pass waits for
    layer 0 (the prefix rows it attends to) before it starts, and for layer 1 only before its score
    (1.5B 16k with every block from the host tier: TTFT 21.34-21.69 ms against 21.85-21.89 ms with
    groups of 2, 2, 4, 4, 8, 8 layers and both waits up front)."""
    groups, a, n = [], 0, 0
    while a < L:
        size = (1, 1, 2)[n] if n < 3 else 4 << ((n - 3) // 2)
        groups.append((a, min(L, a + size)))
        a, n = min(L, a + size), n + 1
    return groups


def copy_layers(dsts, srcs, stream, groups, events):
    """Layer-major DMAs for blocks stacked by layer: dsts, srcs are equal-length lists of
    contiguous [L, ...] tensors (pinned host <-> device). For each layer group (a, b) in the given
    order (any order of disjoint ranges), the slices [a, b) of every pair are queued on `stream`
    (one DMA per tensor), then that group's torch.cuda.Event is recorded. One library call."""
    import numpy as np
    n, G = len(dsts), len(groups)
    if n == 0 or G == 0:
        return
    db = np.empty(n, dtype=np.uint64)
    sb = np.empty(n, dtype=np.uint64)
    lb = np.empty(n, dtype=np.uint64)
    for i, (d, s_) in enumerate(zip(dsts, srcs)):
        if d.shape != s_.shape or d.dtype != s_.dtype or d.shape[0] < max(g[1] for g in groups):
            raise ValueError(f"copy_layers: pair {i} shapes {tuple(d.shape)} / {tuple(s_.shape)}")
        if not (d.is_contiguous() and s_.is_contiguous()):
            raise ValueError(f"copy_layers: pair {i} must be contiguous")
        db[i], sb[i], lb[i] = d.data_ptr(), s_.data_ptr(), d[0].numel() * d.element_size()
    first = np.array([g[0] for g in groups], dtype=np.uint64)[:, None]
    width = np.array([g[1] - g[0] for g in groups], dtype=np.uint64)[:, None]
    dst = np.ascontiguousarray(db[None, :] + first * lb[None, :])
    src = np.ascontiguousarray(sb[None, :] + first * lb[None, :])
    size = np.ascontiguousarray(width * lb[None, :])
    for e in events:
        e.record(stream)  # creates the event; the library records it again after its group
    ev = np.array([e.cuda_event for e in events], dtype=np.uint64)
    _check("tread_copy_layers_async", lib().tread_copy_layers_async(
        dst.ctypes.data, src.ctypes.data, size.ctypes.data, n, G, ctypes.c_void_p(stream.cuda_stream), ev.ctypes.data))


def copy_async(dst, src, stream, event=None):
    """DMA src -> dst (pinned host <-> device) on `stream` (a torch.cuda.Stream); records `event`."""
    if dst.numel() * dst.element_size() != src.numel() * src.element_size():
        raise ValueError("copy_async: size mismatch")
    if not (dst.is_contiguous() and src.is_contiguous()):
        raise ValueError("copy_async: tensors must be contiguous")
    _check("tread_copy_async", lib().tread_copy_async(
        _ptr(dst), _ptr(src), src.numel() * src.element_size(), ctypes.c_void_p(stream.cuda_stream), None))
    if event is not None:
        event.record(stream)  # torch events are created lazily on first record
