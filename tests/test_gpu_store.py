"""Tier moves of the block store on the GPU: batched layer-major promotions, deferred evictions on
their own stream, and the data after round trips (tread/store.py:56-125 semantics)."""
import pytest
import torch

from tread_amd import _hip
from tread_amd.store import BlockStore

pytestmark = pytest.mark.gpu
DEV = "cuda"


def blocks(n_blocks, L=3, kv=2, n=5, hd=8):
    g = torch.Generator().manual_seed(7)
    out = []
    for _ in range(n_blocks):
        K = torch.randn(L, 1, kv, n, hd, generator=g).to(torch.bfloat16)
        V = torch.randn(L, 1, kv, n, hd, generator=g).to(torch.bfloat16)
        out.append((K, V))
    return out


def test_batched_promotions_and_evictions_round_trip():
    data = blocks(4)
    nbytes = 2 * data[0][0].numel() * 2
    store = BlockStore(2 * nbytes, 1 << 30)
    keys = [f"k{i}" for i in range(4)]
    for k, (K, V) in zip(keys, data):
        store.put(k, K.to(DEV), V.to(DEV), 0)
    torch.cuda.synchronize()
    assert store.stats.offloads == 2 and len(store.blocks) == 2 and len(store.cpu_blocks) == 2
    for k in keys[:2]:
        hb = store.cpu_blocks[k]
        hb.synchronize()
        i = keys.index(k)
        assert torch.equal(hb.K, data[i][0]) and torch.equal(hb.V, data[i][1])
    # every lookup of the cycle promotes a host block and evicts the LRU GPU block (deferred)
    for rnd in range(3):
        with store.batch():
            got = [store.get(k) for k in keys]
        for i, b in enumerate(got):
            b.wait()
            assert torch.equal(b.K.cpu(), data[i][0]) and torch.equal(b.V.cpu(), data[i][1]), (rnd, i)
        torch.cuda.synchronize()
        for k, hb in store.cpu_blocks.items():
            i = keys.index(k)
            hb.synchronize()
            assert torch.equal(hb.K, data[i][0]) and torch.equal(hb.V, data[i][1]), (rnd, k)
    assert store.stats.cpu_hits == 3 * 4 and store.stats.offloads == 2 + 3 * 4
    assert store.stats.bytes_used <= store.budget


def test_promotions_in_a_batch_are_layer_major():
    """Blocks promoted in one batch share one event per layer (recorded after that layer of every
    block), and their data lands intact."""
    data = blocks(4, L=4)
    nbytes = 2 * data[0][0].numel() * 2
    store = BlockStore(nbytes, 1 << 30)  # one block: each put evicts the previous one
    for i, (K, V) in enumerate(data):
        store.put(f"h{i}", K.to(DEV), V.to(DEV), 0)
    torch.cuda.synchronize()
    assert sorted(store.cpu_blocks) == ["h0", "h1", "h2"]
    store.budget = 4 * nbytes
    with store.batch():
        got = [store.get(f"h{i}") for i in range(3)]
        assert all(b.ready == [] for b in got)  # queued at the end of the batch
    assert all(b.ready is got[0].ready for b in got) and len(got[0].ready) == 4
    for i, b in enumerate(got):
        b.wait()
        assert torch.equal(b.K.cpu(), data[i][0]) and torch.equal(b.V.cpu(), data[i][1])


def test_unqueued_batch_moves_layer0_last_on_flush():
    """batch(flush=False, layer0_last=True): nothing is queued on exit (a wait then raises instead
    of passing on an unrecorded event); the next flush() queues the schedule with layer 0 in its
    own group, last, so that its event landing means every group has; the data lands intact. A
    plain batch afterwards keeps layer 0 first."""
    L = 5
    data = blocks(4, L=L)
    nbytes = 2 * data[0][0].numel() * 2
    store = BlockStore(nbytes, 1 << 30)
    for i, (K, V) in enumerate(data):
        store.put(f"h{i}", K.to(DEV), V.to(DEV), 0)
    torch.cuda.synchronize()
    store.budget = 4 * nbytes
    with store.batch(flush=False, layer0_last=True):
        got = [store.get(f"h{i}") for i in range(2)]
    assert all(b.ready == [] for b in got)
    with pytest.raises(RuntimeError):
        got[0].wait()
    store.flush()
    ev = got[0].ready
    assert len(ev) == L and all(b.ready is ev for b in got)
    groups = _hip.layer_groups(L)
    assert groups[0] == (0, 1) and len(groups) > 2
    assert all(ev[0] is not ev[l] for l in range(1, L))  # layer 0 alone
    assert store._inflight[-1][0] is ev[0]  # the schedule's last group
    for i, b in enumerate(got):
        b.wait()
        assert torch.equal(b.K.cpu(), data[i][0]) and torch.equal(b.V.cpu(), data[i][1])
    torch.cuda.synchronize()
    store._reap()
    assert all(b.ready is None for b in got)  # landed: resident from now on
    with store.batch():
        (b2,) = [store.get("h2")]
    assert store._inflight[-1][0] is b2.ready[L - 1]  # default order: the last layers go last
    b2.wait()
    assert torch.equal(b2.K.cpu(), data[2][0]) and torch.equal(b2.V.cpu(), data[2][1])
