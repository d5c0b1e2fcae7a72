"""Content-addressed KV block store: GPU tier + pinned-host tier, byte budgets, LRU.

Same API, keys, LRU order and statistics as tread/store.py:1-125. A block is the K/V of one chunk
for all layers, stacked [layers, 1, kv_heads, tokens, head_dim], plus the position it was computed
at (`base`). What differs is how bytes move between tiers:
  - a host-tier hit (store.py:73-77) allocates the GPU tensors and queues DMAs from pinned memory
    on the store's H2D stream in layer groups of growing size (1, 1, 2, 4, 4, 8, 8 layers), one DMA
    per tensor and group, recording one event per group in `Block.ready` (indexed by layer);
    consumers wait on those events (`Block.wait`) on their own stream, so the copy of layer l
    overlaps whatever runs before layer l is needed. Lookups made inside `batch()` share one
    schedule: group 0 of every promoted block, then group 1, ... so that the first layers of all
    blocks land first (layer 0 last for a request that recomputes it; the schedule can also be
    left for a later flush(), so that its host-side queueing runs after the caller's first GPU
    work is launched);
  - an eviction (store.py:99-115) queues a D2H DMA into freshly allocated pinned memory on a
    second stream, after the producing stream's work (and after the block's own H2D if it was
    promoted in the same batch), instead of a synchronous copy + re-pin. The evicted GPU tensors
    are kept alive for the copy by the caching allocator's stream record. A block that came from
    the host tier keeps its pinned buffers (`shadow`; blocks never change), so evicting it again
    copies nothing: a working set cycling through a too-small GPU tier moves each block up once
    per request and never back down.
A block evicted and promoted again before its D2H was queued forces the pending copies out first,
so an H2D never reads a host buffer before its D2H filled it.

With `disk_dir`, a third tier keeps blocks as files in the format of `tread_amd.blockfile` under a
byte budget (LRU): a block leaving the host tier (or leaving the GPU tier when it does not fit the
host tier) is written there by a background thread once its D2H has landed, unless its file
already exists; blocks are immutable and content-addressed, so the disk tier is inclusive (a file
stays after its block is promoted) and a file is written once. A lookup that misses the GPU and
host tiers reads the file straight into pinned buffers, verifies its checksums and promotes the
block like a host-tier hit (`prefetch()` reads a request's files in parallel first); a file that
fails to read or verify is deleted and the lookup is a miss, so the block is computed again.
A new store on the same directory indexes the files found there, so cached blocks survive restarts.
The store is single-threaded (callers serialise requests), as in the reference; only file I/O runs
on helper threads.
"""
import hashlib
import os
from collections import OrderedDict
from concurrent.futures import ThreadPoolExecutor
from contextlib import contextmanager
from dataclasses import dataclass, field
from pathlib import Path
from typing import Optional

import torch

from tread_amd import _hip
from tread_amd import blockfile


def block_key(*parts) -> str:
    """tread/store.py:21-30: sha256 over the parts, tensors as native little-endian int64 bytes,
    everything else as str(p) in UTF-8, each part followed by one NUL byte; hex digest."""
    h = hashlib.sha256()
    for p in parts:
        if isinstance(p, torch.Tensor):
            h.update(p.detach().to("cpu", torch.int64).contiguous().numpy())  # its buffer, no copy
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
    # pinned (K, V) a promoted block came from: blocks never change, so evicting it again needs no D2H
    shadow: Optional[tuple] = field(default=None, repr=False)

    @property
    def pending(self):
        return self.ready is not None

    def wait(self, layers=None, stream=None):
        """Make `stream` (default: current) wait until the GPU copy of `layers` has landed."""
        if self.ready is None:
            return
        if not self.ready:
            raise RuntimeError("Block: its DMAs are not queued yet; flush() the store first")
        s = stream or torch.cuda.current_stream()
        seen = set()  # layers of one copy group share its event: one wait each
        for l in (range(len(self.ready)) if layers is None else layers):
            if id(self.ready[l]) not in seen:
                seen.add(id(self.ready[l]))
                s.wait_event(self.ready[l])

    def synchronize(self):
        """Block the host until every copy of this block is complete (CPU tensors readable)."""
        if self.host_ready is not None:
            self.host_ready.synchronize()
        if self.ready is not None:
            if not self.ready:
                raise RuntimeError("Block: its DMAs are not queued yet; flush() the store first")
            for e in self.ready:
                e.synchronize()


class _PendingCopy:
    """host_ready of a host block whose D2H is not queued yet (batched eviction)."""

    def synchronize(self):
        raise RuntimeError("BlockStore: flush() the batch before reading an evicted block on the host")


_Pending = _PendingCopy()


@dataclass
class StoreStats:
    """tread/store.py:44-53."""
    hits: int = 0  # GPU + host-tier hits
    misses: int = 0
    evictions: int = 0  # blocks leaving the GPU tier (offloaded or dropped)
    bytes_used: int = 0  # GPU tier
    cpu_hits: int = 0
    offloads: int = 0
    cpu_evictions: int = 0  # blocks leaving the host tier (dropped, or kept by the disk tier)
    cpu_bytes_used: int = 0
    disk_hits: int = 0  # lookups served from the disk tier (also counted in hits)
    spills: int = 0  # block files written
    disk_evictions: int = 0  # block files deleted for the disk budget
    disk_bytes_used: int = 0
    disk_errors: int = 0  # block files that failed to read or verify (dropped; the lookup missed)


class _DiskEntry:
    """A block file of the disk tier: its header, and until its write is done the host block the
    writer thread is reading (a lookup then serves that block instead of the file)."""

    def __init__(self, header, path, block=None, job=None):
        self.header, self.path, self.block, self.job = header, path, block, job

    def settle(self):
        if self.job is not None and self.job.done():
            self.job.result()  # a failed write raises here
            self.job, self.block = None, None


class BlockStore:
    def __init__(self, budget_bytes: int, cpu_budget_bytes: int = 0, disk_dir=None, disk_budget_bytes: int = 0):
        self.budget = budget_bytes
        self.cpu_budget = cpu_budget_bytes
        self.blocks: "OrderedDict[str, Block]" = OrderedDict()  # GPU tier
        self.cpu_blocks: "OrderedDict[str, Block]" = OrderedDict()
        self.stats = StoreStats()
        self.disk_dir = Path(disk_dir) if disk_dir is not None else None
        self.disk_budget = disk_budget_bytes if disk_dir is not None else 0
        self.disk_blocks: "OrderedDict[str, _DiskEntry]" = OrderedDict()
        self._writer = self._readers = None
        self._staged = {}  # key -> host Block read and verified by prefetch(), not yet looked up
        self._device = torch.device("cuda", torch.cuda.current_device()) if torch.cuda.is_available() \
            else torch.device("cpu")
        if self.disk_dir is not None:
            self.disk_dir.mkdir(parents=True, exist_ok=True)
            self._scan_disk()
        self._streams = {}  # "h2d" / "d2h" -> torch.cuda.Stream (default priority)
        # (event, tensors) of DMAs in flight: pinned buffers stay referenced until their copy ends,
        # since the DMA is not visible to torch's pinned-memory allocator.
        self._inflight = []
        self._batch = 0
        self._h2d = []  # (Block, host K, host V): promotions whose DMAs are not queued yet
        self._h2d_after = None  # (event, promotions): the current stream's state at an unqueued batch's exit
        self._h2d_layer0_last = False  # the pending schedule moves layer 0 last
        self.event_timing = False  # copy-group events with timing (for timelines; slower to record)
        self._d2h = []  # (GPU Block, host Block): evictions whose DMAs are not queued yet

    def _reap(self):
        """Drop the references of DMAs that have landed; a promoted block whose last layer group
        has landed stops being pending (consumers then take it as resident, no event wait)."""
        if self._inflight:
            keep = []
            for e, refs, blocks in self._inflight:
                if e.query():
                    for b in blocks:
                        if b.ready is not None and any(x is e for x in b.ready):
                            b.ready = None
                else:
                    keep.append((e, refs, blocks))
            self._inflight = keep

    # ---- copy engine
    def _stream(self, kind, device):
        s = self._streams.get(kind)
        if s is None:
            s = self._streams[kind] = torch.cuda.Stream(device=device)
        return s

    def copy_stream(self, device):
        """The stream host-tier promotions are copied on."""
        return self._stream("h2d", device)

    @contextmanager
    def batch(self, flush=True, layer0_last=False):
        """Lookups inside the block share one layer-major H2D schedule, queued on exit (or at an
        explicit `flush()`, which a caller must make before it reads any block obtained inside).
        flush=False leaves the schedule unqueued on exit, for the next flush(): a caller with GPU
        work to launch first hides the host time of queueing the DMAs behind that work. The
        schedule's DMAs still start after the work the current stream held at the batch's exit
        (the promoted blocks' fresh allocations may reuse memory that work released), not after
        the work launched before the flush. layer0_last: the schedule moves layer 0 last, for a
        request that recomputes layer 0 of these blocks and reads layer 1 first."""
        self._batch += 1
        if layer0_last:
            self._h2d_layer0_last = True
        try:
            yield self
        finally:
            self._batch -= 1
            if self._batch == 0:
                self._staged.clear()
                if not self._h2d:
                    self._h2d_layer0_last = False  # nothing promoted: no schedule to order
                if flush:
                    self.flush()
                elif self._h2d:
                    cur = torch.cuda.current_stream(self._h2d[0][0].K.device)
                    e = torch.cuda.Event()
                    e.record(cur)
                    self._h2d_after = (e, len(self._h2d))

    def flush(self):
        """Queue the pending DMAs: promotions layer-major on the H2D stream, then evictions on the
        D2H stream."""
        if self._h2d:
            pend, self._h2d = self._h2d, []
            after, self._h2d_after = self._h2d_after, None
            layer0_last, self._h2d_layer0_last = self._h2d_layer0_last, False
            dev = pend[0][0].K.device
            cur = torch.cuda.current_stream(dev)
            s = self.copy_stream(dev)
            # the fresh allocations may reuse memory the current stream released: wait for the work
            # it held when they were made (a batch left unqueued recorded that point on exit)
            if after is not None and after[1] == len(pend):
                s.wait_event(after[0])
            else:
                s.wait_stream(cur)
            for _, hK, hV in pend:  # host buffers filled by a queued D2H (evicted earlier)
                if getattr(hK, "_tread_ready", None) is not None:
                    s.wait_event(hK._tread_ready)
            L = pend[0][0].K.shape[0]
            groups = _hip.layer_groups(L)
            if layer0_last and len(groups) > 1:
                groups = groups[1:] + groups[:1]
            gev = [torch.cuda.Event(enable_timing=self.event_timing) for _ in groups]
            _hip.copy_layers([t for b, _, _ in pend for t in (b.K, b.V)], [t for _, hK, hV in pend for t in (hK, hV)],
                             s, groups, gev)
            group_of = {l: e for (a, b_), e in zip(groups, gev) for l in range(a, b_)}
            events = [group_of[l] for l in range(L)]  # per layer
            for b, hK, hV in pend:
                b.K.record_stream(s)
                b.V.record_stream(s)
                b.ready = events
            # the schedule's last group: once it has landed, every DMA of the schedule has
            self._inflight.append((gev[-1], tuple(t for _, hK, hV in pend for t in (hK, hV)),
                                   tuple(b for b, _, _ in pend)))
        if self._d2h:
            pend, self._d2h = self._d2h, []
            for gb, hb in pend:
                self._queue_d2h(gb, hb)

    def _queue_d2h(self, gb, hb):
        dev = gb.K.device
        s = self._stream("d2h", dev)
        s.wait_stream(torch.cuda.current_stream(dev))  # the block's producer lands first
        if gb.ready is not None:  # and its own promotion (one wait per layer group)
            for e in {id(x): x for x in gb.ready}.values():
                s.wait_event(e)
        _hip.copy_async(hb.K, gb.K, s)
        _hip.copy_async(hb.V, gb.V, s)
        e = torch.cuda.Event()
        e.record(s)
        gb.K.record_stream(s)
        gb.V.record_stream(s)
        hb.host_ready = e
        hb.K._tread_ready = e
        self._inflight.append((e, (hb.K, hb.V), ()))

    def _to_device(self, b: Block):
        """Promote a host-tier block: GPU tensors now, its DMAs with the batch's schedule."""
        dev = b.device
        if not (isinstance(dev, torch.device) and dev.type == "cuda"):
            b.K, b.V = b.K.clone(), b.V.clone()
            return
        if b.host_ready is not None and any(hb is b for _, hb in self._d2h):
            self.flush()  # its D2H is not queued yet: queue it before reading the host buffer
        hK, hV = b.K, b.V
        b.K = torch.empty(hK.shape, dtype=hK.dtype, device=dev)
        b.V = torch.empty(hV.shape, dtype=hV.dtype, device=dev)
        b.ready, b.host_ready = [], None  # pending: the layer events are set when queued
        b.shadow = (hK, hV)
        self._h2d.append((b, hK, hV))
        if self._batch == 0:
            self.flush()

    def _to_host(self, b: Block) -> Block:
        """Evict a GPU block into new pinned memory; returns the host Block (its D2H queued with
        the batch, or now)."""
        if not b.K.is_cuda:
            return Block(K=b.K.clone(), V=b.V.clone(), base=b.base, n_tokens=b.n_tokens, nbytes=b.nbytes,
                         device=b.device, hits=b.hits)
        if b.shadow is not None:  # the pinned copy it was promoted from still holds its data
            K, V = b.shadow
            return Block(K=K, V=V, base=b.base, n_tokens=b.n_tokens, nbytes=b.nbytes, device=b.device, hits=b.hits)
        K = torch.empty(b.K.shape, dtype=b.K.dtype, pin_memory=True)
        V = torch.empty(b.V.shape, dtype=b.V.dtype, pin_memory=True)
        hb = Block(K=K, V=V, base=b.base, n_tokens=b.n_tokens, nbytes=b.nbytes, device=b.device, hits=b.hits,
                   host_ready=_Pending)
        if self._batch == 0 and not any(gb is b for gb, _, _ in self._h2d):
            self._queue_d2h(b, hb)
        else:
            self._d2h.append((b, hb))
        return hb

    # ---- tread/store.py API
    def get(self, key):
        self._reap()
        b = self.blocks.get(key)
        if b is not None:
            self.blocks.move_to_end(key)
        else:
            b = self.cpu_blocks.pop(key, None)
            if b is not None:
                self.stats.cpu_bytes_used -= b.nbytes
                self.stats.cpu_hits += 1
            else:
                b = self._from_disk(key)
                if b is None:
                    self.stats.misses += 1
                    return None
                self.stats.disk_hits += 1
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
        if key in self.disk_blocks:
            self._drop_file(key)
        self._device = K.device
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
            if self._disk_wants(key, b):  # no room in the host tier: straight to disk
                self._spill(key, self._to_host(b))
            return
        while self.stats.cpu_bytes_used + b.nbytes > self.cpu_budget:
            okey, old = self.cpu_blocks.popitem(last=False)
            self.stats.cpu_bytes_used -= old.nbytes
            self.stats.cpu_evictions += 1
            if self._disk_wants(okey, old):
                self._spill(okey, old)
        # A new Block, never the evicted object: a request holding the old one keeps GPU tensors.
        nb = self._to_host(b)
        self.cpu_blocks[key] = nb
        self.stats.cpu_bytes_used += nb.nbytes
        self.stats.offloads += 1

    # ---- disk tier
    def _scan_disk(self):
        """Index the block files already in disk_dir, oldest first (partial writes are removed)."""
        for tmp in self.disk_dir.glob("*" + blockfile.SUFFIX + ".tmp"):
            tmp.unlink(missing_ok=True)
        files = sorted(self.disk_dir.glob("*" + blockfile.SUFFIX), key=lambda p: p.stat().st_mtime)
        for path in files:
            try:
                h = blockfile.read_header(path)
            except (OSError, blockfile.BlockFileError):
                path.unlink(missing_ok=True)  # not a block of this format: not ours to serve
                continue
            if path.name != h["key"] + blockfile.SUFFIX:
                continue
            self._make_room(h["file_bytes"])
            self.disk_blocks[h["key"]] = _DiskEntry(h, path)
            self.stats.disk_bytes_used += h["file_bytes"]

    def _disk_wants(self, key, b):
        if self.disk_dir is None:
            return False
        if key in self.disk_blocks:  # written before: blocks never change
            self.disk_blocks.move_to_end(key)
            return False
        return b.nbytes + blockfile.HEADER + blockfile.ALIGN <= self.disk_budget

    def _make_room(self, nbytes):
        while self.disk_blocks and self.stats.disk_bytes_used + nbytes > self.disk_budget:
            self._drop_file(next(iter(self.disk_blocks)))
            self.stats.disk_evictions += 1

    def _drop_file(self, key):
        e = self.disk_blocks.pop(key)
        if e.job is not None:
            e.job.result()
        e.path.unlink(missing_ok=True)
        self.stats.disk_bytes_used -= e.header["file_bytes"]

    def _spill(self, key, hb):
        """Write host block hb to the disk tier on the writer thread (after its D2H lands)."""
        K, V = hb.K, hb.V
        kb = K.numel() * K.element_size()
        size = blockfile.HEADER + blockfile._align(kb) + kb  # the file: header, K padded to 4 KiB, V
        self._make_room(size)
        path = self.disk_dir / (key + blockfile.SUFFIX)
        header = dict(key=key, base=hb.base, n_tokens=hb.n_tokens, shape=tuple(K.shape), dtype=K.dtype,
                      file_bytes=size)
        if self._writer is None:
            self._writer = ThreadPoolExecutor(1, thread_name_prefix="tread-spill")
        self._flush_if_pending(hb)

        def job():
            hb.synchronize()  # the D2H that fills the pinned buffers has landed
            blockfile.write_block(path, key, K, V, hb.base)

        self.disk_blocks[key] = _DiskEntry(header, path, block=hb, job=self._writer.submit(job))
        self.stats.disk_bytes_used += size
        self.stats.spills += 1

    def _flush_if_pending(self, hb):
        if hb.host_ready is _Pending:
            self.flush()  # queue its D2H so that the writer can wait for it

    def _from_disk(self, key):
        """The disk-tier block of `key` as a host Block (its bytes verified), or None: not in the
        tier, or its file failed to read or verify (then the file is dropped and counted in
        stats.disk_errors, and the lookup is a miss, so the caller recomputes the block)."""
        e = self.disk_blocks.get(key)
        if e is None:
            return None
        staged = self._staged.pop(key, None)
        if staged is not None:  # read and verified by prefetch()
            self.disk_blocks.move_to_end(key)
            return staged
        e.settle()
        if e.block is not None:  # still being written: serve the host copy the writer reads
            self.disk_blocks.move_to_end(key)
            src = e.block
            return Block(K=src.K, V=src.V, base=src.base, n_tokens=src.n_tokens, nbytes=src.nbytes,
                         device=self._device, host_ready=src.host_ready)
        b = self._read_file(e)
        if b is None:
            self._drop_corrupt(key)
            return None
        self.disk_blocks.move_to_end(key)
        return b

    def _read_file(self, e):
        """Read a block file into new (pinned) host buffers; None if it cannot be read or verified."""
        h = e.header
        nbytes = 2 * int(torch.Size(h["shape"]).numel()) * torch.empty((), dtype=h["dtype"]).element_size()
        pin = self._device.type == "cuda"
        K = torch.empty(h["shape"], dtype=h["dtype"], pin_memory=pin)
        V = torch.empty(h["shape"], dtype=h["dtype"], pin_memory=pin)
        try:
            blockfile.read_into(e.path, K, V)
        except (OSError, ValueError):  # BlockFileError is a ValueError
            return None
        return Block(K=K, V=V, base=h["base"], n_tokens=h["n_tokens"], nbytes=nbytes, device=self._device)

    def _drop_corrupt(self, key):
        e = self.disk_blocks.pop(key)
        e.path.unlink(missing_ok=True)
        self.stats.disk_bytes_used -= e.header["file_bytes"]
        self.stats.disk_errors += 1

    def prefetch(self, keys):
        """Read the disk-tier blocks among `keys` (those in neither the GPU nor the host tier) in
        parallel and verify them, before they are looked up: the lookups inside this batch() then
        take them from memory, and a file that fails to read or verify is dropped first, so its
        lookup is a clean miss. LRU order and statistics are those of the lookups alone."""
        if self.disk_dir is None or self._batch == 0:
            return
        todo = []
        for k in keys:
            if k in self.blocks or k in self.cpu_blocks or k in self._staged:
                continue
            e = self.disk_blocks.get(k)
            if e is None:
                continue
            e.settle()
            if e.block is None:
                todo.append((k, e))
        if not todo:
            return
        if len(todo) == 1:
            results = [self._read_file(todo[0][1])]
        else:
            if self._readers is None:
                self._readers = ThreadPoolExecutor(min(8, os.cpu_count() or 1), thread_name_prefix="tread-read")
            results = list(self._readers.map(lambda ke: self._read_file(ke[1]), todo))
        for (k, _), b in zip(todo, results):
            if b is None:
                self._drop_corrupt(k)
            else:
                self._staged[k] = b

    def persist(self):
        """Give every block of the GPU and host tiers that has no file yet one (within the disk
        budget), and wait for all writes: after this a store on the same directory, in this or a
        later process, finds the whole cache."""
        if self.disk_dir is None:
            return
        for key, b in list(self.cpu_blocks.items()) + list(self.blocks.items()):
            if self._disk_wants(key, b):
                self._spill(key, self._to_host(b) if b.K.is_cuda else b)
        self.flush()
        self.drain()

    def drain(self):
        """Wait for every block file write (e.g. before the process exits or the directory is read
        by another store)."""
        for e in list(self.disk_blocks.values()):
            if e.job is not None:
                e.job.result()
            e.settle()

    def _remove(self, tier, key):
        b = tier.pop(key)
        if tier is self.blocks:
            self.stats.bytes_used -= b.nbytes
        else:
            self.stats.cpu_bytes_used -= b.nbytes

    def __len__(self):
        return len(self.blocks) + len(self.cpu_blocks)  # the disk tier is inclusive, not counted
