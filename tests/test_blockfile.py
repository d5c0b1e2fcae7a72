"""The block file / wire format and the store's disk tier, on the CPU.

Pinned by: bit-exact round trips (file and wire form), the XXH3-64 known answer of the empty input
(the checksum the format names), detection of every planted corruption (payload byte, header byte,
truncation), and the store's tier rules (LRU under a byte budget, inclusive disk tier, restart).
"""
import pytest
import torch
import xxhash

from tread_amd import blockfile as BF
from tread_amd.store import BlockStore


def _block(seed, n=37, L=3, kv=2, hd=16, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    K = torch.randn(L, 1, kv, n, hd, generator=g).to(dtype)
    V = torch.randn(L, 1, kv, n, hd, generator=g).to(dtype)
    return K, V


def _same(a, b):
    return a.dtype == b.dtype and a.shape == b.shape and torch.equal(a.view(torch.uint8), b.view(torch.uint8))


def test_xxh3_known_answer():
    # XXH3-64 of the empty input, seed 0 (the published test vector)
    assert xxhash.xxh3_64_intdigest(b"") == 0x2D06800538D394C2


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_file_round_trip_is_bit_exact(tmp_path, dtype):
    K, V = _block(1, dtype=dtype)
    key = "ab" * 32
    path = tmp_path / (key + BF.SUFFIX)
    size = BF.write_block(path, key, K, V, base=64)
    assert path.stat().st_size == size
    K2, V2, h = BF.read_block(path, pin_memory=False)
    assert _same(K, K2) and _same(V, V2)
    assert (h["key"], h["base"], h["n_tokens"], h["shape"], h["dtype"]) == (key, 64, 37, tuple(K.shape), dtype)
    assert h["k_offset"] == 4096 and h["v_offset"] % 4096 == 0 and h["v_offset"] >= 4096 + h["nbytes"]
    # the wire form is the file's bytes
    assert BF.pack(key, K, V, 64) == path.read_bytes()
    k3, K3, V3, b3 = BF.unpack(path.read_bytes())
    assert (k3, b3) == (key, 64) and _same(K, K3) and _same(V, V3)
    assert not list(tmp_path.glob("*.tmp"))


def test_corruption_is_detected(tmp_path):
    K, V = _block(2)
    key = "cd" * 32
    path = tmp_path / (key + BF.SUFFIX)
    BF.write_block(path, key, K, V, base=0)
    good = path.read_bytes()
    h = BF.parse_header(good)
    for pos in (h["k_offset"] + 5, h["v_offset"] + h["nbytes"] - 1):  # one payload byte
        bad = bytearray(good)
        bad[pos] ^= 0x40
        path.write_bytes(bytes(bad))
        with pytest.raises(BF.BlockFileError, match="payload checksum"):
            BF.read_block(path, pin_memory=False)
        with pytest.raises(BF.BlockFileError):
            BF.unpack(bytes(bad))
    bad = bytearray(good)
    bad[85] ^= 1  # a byte of `base`
    with pytest.raises(BF.BlockFileError, match="header checksum"):
        BF.parse_header(bytes(bad))
    with pytest.raises(BF.BlockFileError, match="magic"):
        BF.parse_header(b"X" + good[1:4096])
    path.write_bytes(good[:h["v_offset"] + 10])
    with pytest.raises(BF.BlockFileError, match="truncated"):
        BF.read_block(path, pin_memory=False)


def _nbytes(K, V):
    return 2 * K.numel() * K.element_size()


def test_store_spills_to_disk_and_serves_hits_exactly(tmp_path):
    blocks = {f"{i:064x}": _block(10 + i) for i in range(4)}
    nb = _nbytes(*blocks[f"{0:064x}"])
    st = BlockStore(nb, 0, disk_dir=tmp_path, disk_budget_bytes=1 << 30)
    for k, (K, V) in blocks.items():
        st.put(k, K, V, base=7)
    st.drain()
    assert st.stats.spills == 3 and st.stats.evictions == 3 and len(st.disk_blocks) == 3
    assert sorted(p.name for p in tmp_path.iterdir()) == sorted(k + BF.SUFFIX for k in list(blocks)[:3])
    k0 = f"{0:064x}"
    b = st.get(k0)  # disk hit: promoted to the GPU tier (here a CPU "device"), evicting block 3 to disk
    assert b is not None and st.stats.disk_hits == 1 and st.stats.hits == 1
    assert _same(b.K, blocks[k0][0]) and _same(b.V, blocks[k0][1]) and (b.base, b.n_tokens) == (7, 37)
    st.drain()
    assert st.stats.spills == 4 and k0 in st.disk_blocks  # inclusive: block 0's file stays
    # evicting block 0 again writes nothing (its file exists)
    st.get(f"{1:064x}")
    st.drain()
    assert st.stats.spills == 4 and st.stats.disk_hits == 2
    assert st.get("f" * 64) is None and st.stats.misses == 1


def test_store_disk_budget_is_lru_and_survives_restart(tmp_path):
    blocks = {f"{i:064x}": _block(20 + i) for i in range(5)}
    nb = _nbytes(*blocks[f"{0:064x}"])
    file_bytes = 4096 + -(-nb // 2 // 4096) * 4096 + nb // 2
    st = BlockStore(nb, 0, disk_dir=tmp_path, disk_budget_bytes=2 * file_bytes)
    for k, (K, V) in blocks.items():
        st.put(k, K, V, base=3)
    st.drain()
    keys = list(blocks)
    # blocks 0..3 left the GPU tier; the disk keeps the two most recent of them
    assert list(st.disk_blocks) == keys[2:4] and st.stats.disk_evictions == 2
    assert st.stats.disk_bytes_used == 2 * file_bytes <= st.disk_budget
    assert sorted(p.name for p in tmp_path.iterdir()) == sorted(k + BF.SUFFIX for k in keys[2:4])
    # a new store on the same directory serves them
    st2 = BlockStore(nb, 0, disk_dir=tmp_path, disk_budget_bytes=2 * file_bytes)
    assert set(st2.disk_blocks) == set(keys[2:4])
    b = st2.get(keys[3])  # a fresh store promotes to the current GPU when there is one
    assert b is not None and st2.stats.disk_hits == 1
    b.synchronize()
    assert _same(b.K.cpu(), blocks[keys[3]][0]) and _same(b.V.cpu(), blocks[keys[3]][1]) and b.base == 3
    # put() of a key drops its file (the reference's put clears the key from every tier)
    st2.put(keys[2], *blocks[keys[2]], base=3)
    assert keys[2] not in st2.disk_blocks and not (tmp_path / (keys[2] + BF.SUFFIX)).exists()


def test_scan_skips_foreign_and_partial_files(tmp_path):
    K, V = _block(30)
    key = "e" * 64
    BF.write_block(tmp_path / (key + BF.SUFFIX), key, K, V, base=1)
    (tmp_path / ("0" * 64 + BF.SUFFIX + ".tmp")).write_bytes(b"partial")
    (tmp_path / ("1" * 64 + BF.SUFFIX)).write_bytes(b"garbage")
    (tmp_path / "notes.txt").write_text("not a block")
    st = BlockStore(1 << 20, 0, disk_dir=tmp_path, disk_budget_bytes=1 << 30)
    assert list(st.disk_blocks) == [key]
    assert sorted(p.name for p in tmp_path.iterdir()) == sorted([key + BF.SUFFIX, "notes.txt"])


def _corrupt_payload(path):
    data = bytearray(path.read_bytes())
    h = BF.parse_header(bytes(data[:4096]))
    data[h["k_offset"] + 3] ^= 0x20
    path.write_bytes(bytes(data))


@pytest.mark.parametrize("batched", [False, True])
def test_corrupt_disk_block_is_a_clean_miss(tmp_path, batched):
    """A block file whose payload fails its checksum: the lookup misses (the file is dropped and
    counted), nothing half-read is served or indexed, later lookups of it miss without raising,
    and the other blocks of the same batch are served exactly."""
    blocks = {f"{i:064x}": _block(40 + i) for i in range(4)}
    keys = list(blocks)
    nb = _nbytes(*blocks[keys[0]])
    st = BlockStore(nb, 0, disk_dir=tmp_path, disk_budget_bytes=1 << 30)
    for k, (K, V) in blocks.items():
        st.put(k, K, V, base=5)
    st.drain()
    assert set(st.disk_blocks) == set(keys[:3])
    _corrupt_payload(tmp_path / (keys[1] + BF.SUFFIX))
    if batched:
        with st.batch():
            st.prefetch(keys[:3])
            got = [st.get(k) for k in keys[:3]]
    else:
        got = [st.get(k) for k in keys[:3]]
    assert got[1] is None
    assert st.stats.disk_errors == 1 and st.stats.misses == 1 and st.stats.disk_hits == st.stats.hits == 2
    assert keys[1] not in st.disk_blocks and keys[1] not in st.blocks
    assert not (tmp_path / (keys[1] + BF.SUFFIX)).exists()
    # the GPU tier holds one block: the last good lookup, served exactly
    b = got[2]
    assert b is not None and _same(b.K, blocks[keys[2]][0]) and _same(b.V, blocks[keys[2]][1])
    assert st.get(keys[1]) is None and st.stats.misses == 2 and st.stats.disk_errors == 1
    # a caller recomputing the block puts it back
    st.put(keys[1], *blocks[keys[1]], base=5)
    assert _same(st.get(keys[1]).K, blocks[keys[1]][0])


def test_prefetch_keeps_lru_order_and_stats_of_the_lookups(tmp_path):
    blocks = {f"{i:064x}": _block(50 + i) for i in range(4)}
    keys = list(blocks)
    nb = _nbytes(*blocks[keys[0]])
    st = BlockStore(nb, 0, disk_dir=tmp_path, disk_budget_bytes=1 << 30)
    for k, (K, V) in blocks.items():
        st.put(k, K, V, base=1)
    st.drain()
    order = list(st.disk_blocks)
    with st.batch():
        st.prefetch(keys)
        assert list(st.disk_blocks) == order and st.stats.disk_hits == 0 and st.stats.hits == 0
        b = st.get(keys[0])
    # the lookup moved block 0 to the LRU end; block 3, evicted by its promotion, was spilled after it
    assert st.stats.disk_hits == 1 and list(st.disk_blocks) == [keys[1], keys[2], keys[0], keys[3]]
    assert _same(b.K, blocks[keys[0]][0]) and not st._staged  # unconsumed reads are dropped at exit


def test_graph_bucket_cache_goes_stale_when_its_bucket_is_claimed():
    """A cache aliasing a graph bucket raises once a later request claims the bucket; a detached
    copy stays valid and keeps the rows."""
    from types import SimpleNamespace
    from tread_amd.cache import KVCache, StaleCacheError
    g = SimpleNamespace(generation=3)
    K = torch.arange(2 * 1 * 2 * 8 * 4, dtype=torch.float32).view(2, 1, 2, 8, 4)
    V = -K
    c = KVCache(K, V, 5, graph=g)
    kept = KVCache(K, V, 5, graph=g).detach()
    assert c.valid and torch.equal(c.K, K) and len(c.key_cache) == 2
    g.generation += 1  # the next request claims the bucket
    assert not c.valid
    for read in (lambda: c.K, lambda: c.V, lambda: c.key_cache, lambda: c.layers, lambda: c.check()):
        with pytest.raises(StaleCacheError):
            read()
    assert kept.valid and kept.graph is None and kept.K.data_ptr() != K.data_ptr()
    assert torch.equal(kept.K[..., :5, :], K[..., :5, :]) and torch.equal(kept.V[..., :5, :], V[..., :5, :])
