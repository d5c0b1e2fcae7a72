"""KV cache object returned by the engine.

The reference returns a transformers DynamicCache (tread/blend.py:182-186; engine.py:131-132)
whose layers are concatenated copies. Here the cache is the assembled buffer itself,
[L, 1, kv_heads, t_cap, head_dim] for K and V with `length` valid rows, and the per-layer views
are exposed under both DynamicCache spellings: `key_cache[l]` / `value_cache[l]` (4.46) and
`layers[l].keys` / `.values` (5.x). `to_dynamic_cache()` builds a transformers DynamicCache for
decoding with a transformers model.
"""
from types import SimpleNamespace

import torch


class StaleCacheError(RuntimeError):
    """A graph-bucket cache read after a later request replayed (and overwrote) its bucket."""


class KVCache:
    """K, V: [L, 1, kv_heads, t_cap, head_dim] with `length` valid rows. A cache that is a hipGraph
    bucket's static buffer (`graph` set) is stamped with the bucket's generation when it is handed
    out; the next request that claims the bucket bumps the generation and overwrites the buffer,
    and any later read of this cache raises StaleCacheError. `detach()` (or `grow()`) moves the
    rows into buffers the cache owns, after which it stays valid."""

    def __init__(self, K, V, length, graph=None):
        self._K, self._V, self.length = K, V, int(length)
        self.graph = graph  # the hipGraph bucket whose static buffer this cache is (or None)
        self._gen = None if graph is None else graph.generation

    def check(self):
        """Raise StaleCacheError if a later request has claimed the bucket this cache aliases."""
        if self.graph is not None and self.graph.generation != self._gen:
            raise StaleCacheError("this cache aliased a hipGraph bucket that a later request has replayed and "
                                  "overwritten; detach() it before the next prefill to keep it")

    @property
    def K(self):
        self.check()
        return self._K

    @property
    def V(self):
        self.check()
        return self._V

    @property
    def valid(self):
        """False once the bucket this cache aliases has been claimed by a later request."""
        return self.graph is None or self.graph.generation == self._gen

    def detach(self):
        """Copy the valid rows into buffers this cache owns (it stops aliasing a graph bucket)."""
        if self.graph is None:
            return self
        self.grow(self.capacity, force=True)
        return self

    def grow(self, capacity, force=False):
        """Move the valid rows into a new buffer of at least `capacity` rows (decoding past the
        preallocated room). The cache stops aliasing a graph bucket."""
        K0, V0 = self.K, self.V
        if capacity <= self.capacity and not force:
            return
        capacity = max(capacity, self.capacity)
        shape = K0.shape[:-2] + (capacity, K0.shape[-1])
        K = torch.empty(shape, dtype=K0.dtype, device=K0.device)
        V = torch.empty_like(K)
        K[..., :self.length, :].copy_(K0[..., :self.length, :])
        V[..., :self.length, :].copy_(V0[..., :self.length, :])
        self._K, self._V, self.graph, self._gen = K, V, None, None

    @classmethod
    def from_layers(cls, K, V):
        """Wrap per-layer [1, kv, T, hd] lists (stacked into one buffer)."""
        Ks, Vs = torch.stack(list(K)), torch.stack(list(V))
        return cls(Ks, Vs, Ks.shape[-2])

    @property
    def key_cache(self):
        return [self.K[l][:, :, :self.length] for l in range(self.K.shape[0])]

    @property
    def value_cache(self):
        return [self.V[l][:, :, :self.length] for l in range(self.V.shape[0])]

    @property
    def layers(self):
        return [SimpleNamespace(keys=k, values=v) for k, v in zip(self.key_cache, self.value_cache)]

    @property
    def capacity(self):
        return self._K.shape[-2]

    def get_seq_length(self, layer_idx=0):
        return self.length

    def __len__(self):
        return self._K.shape[0]

    def to_dynamic_cache(self):
        from transformers import DynamicCache
        c = DynamicCache()
        for l, (k, v) in enumerate(zip(self.key_cache, self.value_cache)):
            c.update(k.clone(), v.clone(), l)
        return c
