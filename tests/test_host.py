"""Host-side checks that need no GPU: the C-ABI library loads and exports every entry point
include/tread_hip.h declares, the product refuses CPU tensors (no CPU fallback), and the engine's
host logic (keys, sig, budgets, bucket plans) matches the reference's."""
import re
from pathlib import Path

import pytest
import torch

from oracle import tread_ref as R

ROOT = Path(__file__).resolve().parent.parent


def header_functions():
    text = (ROOT / "include" / "tread_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tread_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from tread_amd import _hip
    lib = _hip.lib()  # raises if the library is missing or has a stale ABI
    declared = header_functions()
    assert len(declared) >= 12
    for name in declared:
        assert hasattr(lib, name), name
    assert sorted(_hip.exported_symbols()) == declared
    assert lib.tread_abi_version() == _hip.ABI_VERSION


def test_library_symbols_in_dynamic_table():
    import subprocess
    so = ROOT / "tread_amd" / "libtread_hip.so"
    out = subprocess.run(["nm", "-D", "--defined-only", str(so)], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (tread_\w+)", out))
    assert set(header_functions()) <= exported


def test_error_paths_are_reported_without_a_gpu():
    """Argument validation happens on the host before any launch: bad calls return an error code
    and a message (no device touched)."""
    import ctypes
    from tread_amd import _hip
    lib = _hip.lib()
    rc = lib.tread_subset_attn_bf16(None, None, None, None, None, 0, 5, 28, 3, 128, 100, 0.1, None, None, 0, None)
    assert rc != 0 and b"bad shape" in lib.tread_last_error()
    rc = lib.tread_topk_select_bf16(None, 10, 11, None, None, 0, None)
    assert rc != 0 and b"outside" in lib.tread_last_error()
    fake = ctypes.c_void_p(16)  # never dereferenced: the size check comes first
    rc = lib.tread_topk_select_bf16(fake, (1 << 20) + 1, 10, fake, None, 0, None)
    assert rc != 0 and b"above" in lib.tread_last_error()
    rc = lib.tread_rope_assemble_bf16(None, 1, None, None, 2, 2, 10, 128, None, 0, 2, None)
    assert rc != 0
    assert lib.tread_topk_workspace_bytes(1000) == 0
    # split-K workspace for few rows over a long cache; key-half partials for the longest quarter
    # of the row tiles otherwise: 6 400 rows x 7 heads = 175 row tiles per KV head, 44 of them
    # split: 2 halves x 4 KV heads x 44 x 256 rows x (128 fp32 + max, sum) + alignment
    assert lib.tread_subset_attn_workspace_bytes(32, 28, 4, 128, 32096) > 0
    # one decoding row of a 7B model over 32 096 keys: 63 slices of 512 keys x 4 KV heads x 32 rows
    assert lib.tread_subset_attn_workspace_bytes(1, 28, 4, 128, 32096) == 63 * 4 * 32 * (128 * 4 + 8) + 256
    # a 0.5B one over 8 100 keys: slices of 4 tiles of 32 keys (few KV heads: 64 x 2 work groups)
    assert lib.tread_subset_attn_workspace_bytes(1, 14, 2, 64, 8100) == 64 * 2 * 32 * (64 * 4 + 8) + 256
    assert lib.tread_subset_attn_workspace_bytes(2, 28, 4, 128, 300) == 3 * 4 * 32 * (128 * 4 + 8) + 256
    assert lib.tread_subset_attn_workspace_bytes(2, 28, 4, 128, 128) == 0  # one slice: no partials
    assert lib.tread_subset_attn_workspace_bytes(6400, 28, 4, 128, 32096) == 2 * 4 * 44 * 256 * (128 * 4 + 8) + 256
    assert lib.tread_subset_attn_workspace_bytes(64, 28, 4, 128, 200) == 0  # 2 row tiles: neither
    assert lib.tread_subset_attn_workspace_bytes(32000, 28, 4, 128, 32096) == 0  # 3 500 work groups: balanced


def test_product_kernels_refuse_cpu_tensors():
    from tread_amd import _hip
    x = torch.zeros(4, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU tensor"):
        _hip.add_rmsnorm(x, torch.ones(64, dtype=torch.bfloat16), 1e-6)
    with pytest.raises(RuntimeError, match="GPU tensor"):
        _hip.topk_select(torch.zeros(10, dtype=torch.bfloat16), 3)


def test_engine_sig_matches_reference_form():
    from tread_amd.engine import model_sig
    from tread_amd.model import DecoderLM, preset
    cfg = preset("qwen2.5-0.5b", num_hidden_layers=1, vocab_size=64, hidden_size=64, intermediate_size=64,
                 num_attention_heads=2, num_key_value_heads=1)

    class Shell:  # model_sig reads only config and dtype
        config = cfg
        dtype = torch.bfloat16
    assert model_sig(Shell) == ("", "torch.bfloat16", 1000000.0, None) == R.sig_of(cfg, torch.bfloat16)


def test_model_sig_reads_theta_from_rope_parameters():
    """A transformers 5.x config keeps theta in rope_parameters; the key must still carry it."""
    from transformers import Qwen2Config
    from tread_amd.engine import model_sig
    hc = Qwen2Config(hidden_size=64, num_attention_heads=2, num_key_value_heads=1, rope_theta=1000000.0)

    class Shell:
        config = hc
        dtype = torch.bfloat16
    sig = model_sig(Shell)
    assert sig[1:] == ("torch.bfloat16", 1000000.0, None)


def test_product_and_oracle_block_keys_agree():
    from tread_amd.store import block_key
    g = torch.Generator().manual_seed(0)
    for n in (0, 1, 17, 1000):
        ids = torch.randint(0, 152064, (n,), generator=g)
        parts = ("", "torch.bfloat16", 1000000.0, None, "ns", "prefix", ids)
        assert block_key(*parts) == R.block_key(*parts)
        assert block_key("abc", ids) == R.block_key("abc", ids.to(torch.int32))


def test_split_plan_and_graph_buckets():
    from tread_amd.graphs import _bucket, _q_room
    assert _bucket(6400, 32064) == (6400, 32768)  # the 7B 32k request at 20%
    assert _bucket(16000, 32064) == (16128, 32768)
    assert _bucket(1600, 8064) == (1792, 9216)
    assert _q_room(32) == 256 and _q_room(300) == 512


def test_synthetic_init_is_deterministic_and_shaped():
    from tread_amd.model import ModelConfig, prepare, synthetic_model
    cfg = ModelConfig(128, 64, 2, 4, 2, 16, 96)
    a = synthetic_model(cfg, "cpu", torch.float32, seed=3, bias_std=0.1)
    b = synthetic_model(cfg, "cpu", torch.float32, seed=3, bias_std=0.1)
    for (na, pa), (_, pb) in zip(a.state_dict().items(), b.state_dict().items()):
        assert torch.equal(pa, pb), na
    P = prepare(a)
    lw = P.layers[0]
    assert lw.wqkv.shape == ((4 + 2 * 2) * 16, 64) and lw.wgu.shape == (192, 64)
    assert lw.wqkv.data_ptr() == a.model.layers[0].self_attn.q_proj.weight.data_ptr()
    sd = a.state_dict()
    assert torch.equal(sd["model.layers.0.self_attn.k_proj.weight"], lw.wqkv[64:96])
    assert torch.allclose(sd["model.layers.0.input_layernorm.weight"], torch.ones(64))
    w = sd["model.layers.1.mlp.down_proj.weight"]
    assert abs(w.std().item() - 0.02) < 0.004


def test_prepare_fuses_a_transformers_model():
    from transformers import Qwen2Config, Qwen2ForCausalLM
    from tread_amd.model import prepare
    hf = Qwen2ForCausalLM(Qwen2Config(vocab_size=64, hidden_size=32, num_hidden_layers=1, num_attention_heads=4,
                                      num_key_value_heads=2, intermediate_size=48, rope_theta=1000000.0))
    P = prepare(hf)
    at = hf.model.layers[0].self_attn
    assert torch.equal(P.layers[0].wqkv, torch.cat([at.q_proj.weight, at.k_proj.weight, at.v_proj.weight]))
    assert torch.equal(P.inv_freq, hf.model.rotary_emb.inv_freq.float())
    assert P.hd == 8 and P.hq == 4 and P.hkv == 2


@pytest.mark.parametrize("L", [1, 2, 3, 24, 28, 80])
def test_tier_move_layer_groups_tile_the_layers(L):
    """Host-tier promotions move layers in groups that cover [0, L) in order, small ones first, layer
    0 alone (a request's deviation pass needs it before layer 1)."""
    from tread_amd import _hip as H
    g = H.layer_groups(L)
    assert g[0][0] == 0 and g[-1][1] == L
    assert all(a < b for a, b in g) and all(g[i][1] == g[i + 1][0] for i in range(len(g) - 1))
    widths = [b - a for a, b in g]
    assert all(widths[i] <= widths[i + 1] for i in range(len(widths) - 2))  # the last may be cut short
    assert widths[0] == 1 and (L < 2 or widths[1] == 1)


def test_rotation_table_equals_the_oracle_cos_sin_and_float64():
    """The fp32 (cos, sin) table kernel (a) rotates with is the oracle's fp32 cos/sin of the same
    delta bit for bit (so the kernel's rotation can be compared bit-exactly), and within one fp32
    ulp of the float64 values of the same fp32 angle."""
    import math
    from oracle import model_ref as M
    from oracle import tread_ref as R
    from tread_amd import _hip
    from tread_amd.model import preset
    for name in ("qwen2.5-7b", "qwen2.5-0.5b", "llama3-70b"):
        cfg = preset(name)
        m = M.RefModel(cfg=cfg, w={}, dtype=torch.float32, inv_freq=M.inv_freq_of(cfg))
        deltas = [0, 1, -1, 7, 999, 1000, -31000, 31000, 12345, 32064, -2**20]
        tab = _hip.delta_table_host(m.inv_freq, deltas)
        half = cfg.head_dim // 2
        for i, d in enumerate(deltas):
            c, s = R._delta_cos_sin(m, d, torch.float32)
            assert torch.equal(tab[i, :, 0], c[0, :half]) and torch.equal(tab[i, :, 1], s[0, :half]), (name, d)
            ang = (m.inv_freq * float(d)).double()  # the fp32 angle, exactly
            for j in range(half):
                for v, ref in ((tab[i, j, 0].item(), math.cos(ang[j].item())), (tab[i, j, 1].item(), math.sin(ang[j].item()))):
                    ulp = 2.0 ** (math.floor(math.log2(abs(ref))) - 23) if ref != 0 else 2 ** -149  # fp32 ulp
                    assert abs(v - ref) <= max(ulp, 2 ** -126), (name, d, j, v, ref)
