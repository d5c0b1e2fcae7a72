"""Content-addressed KV block store: GPU tier + pinned-host tier, byte budgets, LRU.

Same API, keys, LRU order and statistics as tread/store.py:1-125. A block is the K/V of one chunk
for all layers, stacked [layers, 1, kv_heads, tokens, head_dim], plus the position it was computed
at (`base`). What differs is how bytes move between tiers:
  - a host-tier hit (store.py:73-77) allocates the GPU tensors and queues one DMA per layer slice
    (K then V) from pinned memory on the store's copy stream, recording one event per layer in
    `Block.ready`; consumers wait on those events (`Block.wait`) on their own stream, so the
    copy overlaps whatever runs before layer l is needed;
  - an eviction (store.py:99-115) queues a D2H DMA into freshly allocated pinned memory on the
    same copy stream after the producing stream's work, instead of a synchronous copy + re-pin.
    The evicted GPU tensors are kept alive for the copy by the caching allocator's stream record.
Copies on one stream run in FIFO order, so a later H2D of a block never overtakes its D2H.
The store is single-threaded (callers serialise requests), as in the reference.
"""
import hashlib
from collections import OrderedDict
from dataclasses import dataclass, field
from typing import Optional

import torch

from tread_amd import _hip


def block_key(*parts) -> str:
    """tread/store.py:21-30: sha256 over the parts, tensors as native little-endian int64 bytes,
    everything else as str(p) in UTF-8, each part followed by one NUL byte; hex digest."""
    h = hashlib.sha256()
    for p in parts:
        if isinstance(p, torch.Tensor):
            h.update(p.detach().to("cpu", torch.int64).contiguous().numpy().tobytes())
        else:
            h.update(str(p).encode())
        h.update(b"\x00")
    return h.hexdigest()


@dataclass
class Block:
    """tread/store.py:33-41, plus the copy events of an in-flight tier move."""
    K: torch.Tensor
    V: torch.Tensor
    base: int
    n_tokens: int
    nbytes: int
    device: torch.device
    hits: int = 0
    ready: Optional[list] = field(default=None, repr=False)  # per-layer events of a pending H2D
    host_ready: Optional[object] = field(default=None, repr=False)  # event of a pending D2H

    @property
    def pending(self):
        return self.ready is not None

    def wait(self, layers=None, stream=None):
        """Make `stream` (default: current) wait until the GPU copy of `layers` has landed."""
        if self.ready is None:
            return
        s = stream or torch.cuda.current_stream()
        for l in (range(len(self.ready)) if layers is None else layers):
            s.wait_event(self.ready[l])

    def synchronize(self):
        """Block the host until every copy of this block is complete (CPU tensors readable)."""
        if self.host_ready is not None:
            self.host_ready.synchronize()
        if self.ready is not None:
            for e in self.ready:
                e.synchronize()


@dataclass
class StoreStats:
    """tread/store.py:44-53."""
    hits: int = 0  # GPU + host-tier hits
    misses: int = 0
    evictions: int = 0  # blocks leaving the GPU tier (offloaded or dropped)
    bytes_used: int = 0  # GPU tier
    cpu_hits: int = 0
    offloads: int = 0
    cpu_evictions: int = 0  # blocks dropped for good from the host tier
    cpu_bytes_used: int = 0


class BlockStore:
    def __init__(self, budget_bytes: int, cpu_budget_bytes: int = 0):
        self.budget = budget_bytes
        self.cpu_budget = cpu_budget_bytes
        self.blocks: "OrderedDict[str, Block]" = OrderedDict()  # GPU tier
        self.cpu_blocks: "OrderedDict[str, Block]" = OrderedDict()
        self.stats = StoreStats()
        self._copy_stream = None
        # (event, tensors) of DMAs in flight: pinned buffers stay referenced until their copy ends,
        # since the DMA is not visible to torch's pinned-memory allocator.
        self._inflight = []

    def _reap(self):
        if self._inflight:
            self._inflight = [(e, refs) for e, refs in self._inflight if not e.query()]

    # ---- copy engine
    def copy_stream(self, device):
        if self._copy_stream is None:
            self._copy_stream = torch.cuda.Stream(device=device)  # default priority
        return self._copy_stream

    def _to_device(self, b: Block):
        """Queue the H2D of a host-tier block, one DMA pair + event per layer."""
        dev = b.device
        if not (isinstance(dev, torch.device) and dev.type == "cuda"):
            b.K, b.V = b.K.clone(), b.V.clone()
            return
        cur = torch.cuda.current_stream(dev)
        s = self.copy_stream(dev)
        K = torch.empty(b.K.shape, dtype=b.K.dtype, device=dev)
        V = torch.empty(b.V.shape, dtype=b.V.dtype, device=dev)
        s.wait_stream(cur)  # the fresh allocation may reuse memory the current stream just released
        events = []
        for l in range(K.shape[0]):
            _hip.copy_async(K[l], b.K[l], s)
            _hip.copy_async(V[l], b.V[l], s)
            e = torch.cuda.Event()
            e.record(s)
            events.append(e)
        K.record_stream(s)
        V.record_stream(s)
        self._inflight.append((events[-1], (b.K, b.V)))
        b.K, b.V, b.ready, b.host_ready = K, V, events, None

    def _to_host(self, b: Block) -> Block:
        """Queue the D2H of an evicted GPU block into new pinned memory; returns the host Block."""
        if not b.K.is_cuda:
            return Block(K=b.K.clone(), V=b.V.clone(), base=b.base, n_tokens=b.n_tokens, nbytes=b.nbytes,
                         device=b.device, hits=b.hits)
        dev = b.K.device
        s = self.copy_stream(dev)
        s.wait_stream(torch.cuda.current_stream(dev))  # the block's producer and pending H2D land first
        K = torch.empty(b.K.shape, dtype=b.K.dtype, pin_memory=True)
        V = torch.empty(b.V.shape, dtype=b.V.dtype, pin_memory=True)
        _hip.copy_async(K, b.K, s)
        _hip.copy_async(V, b.V, s)
        e = torch.cuda.Event()
        e.record(s)
        b.K.record_stream(s)
        b.V.record_stream(s)
        self._inflight.append((e, (K, V)))
        return Block(K=K, V=V, base=b.base, n_tokens=b.n_tokens, nbytes=b.nbytes, device=b.device, hits=b.hits,
                     host_ready=e)

    # ---- tread/store.py API
    def get(self, key):
        self._reap()
        b = self.blocks.get(key)
        if b is not None:
            self.blocks.move_to_end(key)
        else:
            b = self.cpu_blocks.pop(key, None)
            if b is None:
                self.stats.misses += 1
                return None
            self.stats.cpu_bytes_used -= b.nbytes
            self.stats.cpu_hits += 1
            self._to_device(b)
            self._insert(key, b)
        b.hits += 1
        self.stats.hits += 1
        return b

    def put(self, key, K, V, base):
        self._reap()
        nbytes = sum(t.numel() * t.element_size() for t in (K, V))
        if nbytes > self.budget:
            return None  # never fits; the request is served without caching it
        for tier in (self.blocks, self.cpu_blocks):
            if key in tier:
                self._remove(tier, key)
        b = Block(K=K, V=V, base=base, n_tokens=K.shape[-2], nbytes=nbytes, device=K.device)
        self._insert(key, b)
        return b

    def _insert(self, key, b):
        while self.stats.bytes_used + b.nbytes > self.budget:
            self._evict_gpu()
        self.blocks[key] = b
        self.stats.bytes_used += b.nbytes

    def _evict_gpu(self):
        key, b = self.blocks.popitem(last=False)
        self.stats.bytes_used -= b.nbytes
        self.stats.evictions += 1
        if b.nbytes > self.cpu_budget:
            return
        while self.stats.cpu_bytes_used + b.nbytes > self.cpu_budget:
            _, old = self.cpu_blocks.popitem(last=False)
            self.stats.cpu_bytes_used -= old.nbytes
            self.stats.cpu_evictions += 1
        # A new Block, never the evicted object: a request holding the old one keeps GPU tensors.
        nb = self._to_host(b)
        self.cpu_blocks[key] = nb
        self.stats.cpu_bytes_used += nb.nbytes
        self.stats.offloads += 1

    def _remove(self, tier, key):
        b = tier.pop(key)
        if tier is self.blocks:
            self.stats.bytes_used -= b.nbytes
        else:
            self.stats.cpu_bytes_used -= b.nbytes

    def __len__(self):
        return len(self.blocks) + len(self.cpu_blocks)
