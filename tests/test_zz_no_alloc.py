"""The attention entry point that allocates nothing (tread_subset_attn_scratch_bf16), through the
C-ABI: on two calls in a row, the second with a smaller input, it gives the same bits as
tread_subset_attn_bf16 with a workspace of its own, on the shapes whose plans use the partials
(key halves of the recompute rows, key splits of the query rows, key slices of a decoding step;
head_dim 128 and 64). A shape whose partials exceed the static array is refused with a message
before anything is launched. Calls on two streams order themselves (the second waits for the
first's event), so back-to-back calls without a host synchronisation both give the right bits.
"""
import pytest
import torch

from tread_amd import _hip

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(n, hq, hkv, hd, t_cap, seed, sorted_rows=True):
    g = torch.Generator(device=DEV).manual_seed(seed)
    q = torch.randn(n, hq, hd, device=DEV, dtype=torch.bfloat16, generator=g)
    K = torch.randn(1, hkv, t_cap, hd, device=DEV, dtype=torch.bfloat16, generator=g)
    V = torch.randn_like(K)
    if sorted_rows:  # recompute rows: sorted positions over the context
        kend = torch.randperm(t_cap, device=DEV, generator=g)[:n].sort().values
    else:  # query rows: the last n positions
        kend = torch.arange(t_cap - n, t_cap, device=DEV)
    return q, K, V, kend


def _both(q, K, V, kend, hq, hkv, hd):
    n = kend.numel()
    ws_bytes = _hip.lib().tread_subset_attn_workspace_bytes(n, hq, hkv, hd, K.shape[-2])
    assert 0 < ws_bytes <= _hip.SUBSET_ATTN_SCRATCH_BYTES  # the shape's plan uses the partials
    want = _hip.subset_attn(q, K, V, kend, hq, hkv, hd, hd ** -0.5)
    out = torch.full_like(want, 7.0)
    _hip.subset_attn_scratch(q, K, V, kend, hq, hkv, hd, hd ** -0.5, out)
    torch.cuda.synchronize()
    return want, out, ws_bytes


@pytest.mark.parametrize("first,second", [
    # 7B recompute rows (key halves), then the 7B query rows (key splits) over the same context
    ((6432, 28, 4, 128, 32096, True), (32, 28, 4, 128, 32096, False)),
    # 0.5B recompute rows (head_dim 64, key splits), then fewer rows over a shorter cache
    ((1632, 14, 2, 64, 8096, True), (200, 14, 2, 64, 3000, True)),
    # a 7B decoding step (one row, keys split between waves and slices), then a 0.5B one
    ((1, 28, 4, 128, 32096, False), (1, 14, 2, 64, 8096, False)),
])
def test_scratch_entry_point_equals_workspace_entry_point(first, second):
    for i, (n, hq, hkv, hd, t_cap, srt) in enumerate((first, second)):
        q, K, V, kend = _case(n, hq, hkv, hd, t_cap, seed=17 + i, sorted_rows=srt)
        want, got, ws = _both(q, K, V, kend, hq, hkv, hd)
        print(f"\n[no-alloc attention] call {i + 1}: {n} rows x {hq} heads over {t_cap} keys, hd {hd}, "
              f"{ws} bytes of partials in the static array")
        assert torch.equal(got, want), (i, (got.float() - want.float()).abs().max().item())


def test_scratch_calls_on_two_streams_order_themselves():
    """Back-to-back calls on two streams with no host synchronisation between them: the second
    call's stream waits for the event the first recorded, so neither overwrites the other's partials
    in the shared array (both plans put theirs at its start), and both results equal the workspace
    entry point's. Repeated with the streams alternating."""
    big = _case(6432, 28, 4, 128, 32096, seed=31)  # key halves of the 7B recompute rows
    small = _case(32, 28, 4, 128, 32096, seed=32, sorted_rows=False)  # key splits of its query rows
    shapes = (28, 4, 128)
    want = [_hip.subset_attn(q, K, V, kend, *shapes, 128 ** -0.5) for q, K, V, kend in (big, small)]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for rep in range(3):
        outs = [torch.full_like(w, 7.0) for w in want]
        for s in streams:
            s.wait_stream(torch.cuda.current_stream())
        for j, (q, K, V, kend) in enumerate((big, small)):
            with torch.cuda.stream(streams[(j + rep) % 2]):
                _hip.subset_attn_scratch(q, K, V, kend, *shapes, 128 ** -0.5, outs[j])
        torch.cuda.synchronize()
        for j in range(2):
            assert torch.equal(outs[j], want[j]), (rep, j)


def test_scratch_entry_point_refuses_shapes_above_its_array():
    # 2 560 rows x 153 heads of their own over 2 560 keys: 10 row tiles per head, the longest 3 in
    # key halves, partials of ~122 MB
    n, hq, hkv, hd, t_cap = 2560, 153, 153, 128, 2560
    need = _hip.lib().tread_subset_attn_workspace_bytes(n, hq, hkv, hd, t_cap)
    assert need > _hip.SUBSET_ATTN_SCRATCH_BYTES
    q = torch.zeros(n, hq, hd, device=DEV, dtype=torch.bfloat16)
    K = torch.zeros(1, hkv, t_cap, hd, device=DEV, dtype=torch.bfloat16)
    kend = torch.arange(n, device=DEV)
    out = torch.full((n, hq * hd), 3.0, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="static maximum"):
        _hip.subset_attn_scratch(q, K, K, kend, hq, hkv, hd, hd ** -0.5, out)
    torch.cuda.synchronize()
    assert bool((out == 3.0).all())  # nothing was launched
