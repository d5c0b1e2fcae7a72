"""KV cache object returned by the engine.

The reference returns a transformers DynamicCache (tread/blend.py:182-186; engine.py:256-261)
whose layers are concatenated copies. Here the cache is the assembled buffer itself,
[L, 1, kv_heads, t_cap, head_dim] for K and V with `length` valid rows, and the per-layer views
are exposed under both DynamicCache spellings: `key_cache[l]` / `value_cache[l]` (4.46) and
`layers[l].keys` / `.values` (5.x). `to_dynamic_cache()` builds a transformers DynamicCache for
decoding with a transformers model.
"""
from types import SimpleNamespace

import torch


class KVCache:
    def __init__(self, K, V, length, graph=None):
        self.K, self.V, self.length = K, V, int(length)
        self.graph = graph  # the hipGraph bucket whose static buffer this cache is (or None)

    def grow(self, capacity):
        """Move the valid rows into a new buffer of at least `capacity` rows (decoding past the
        preallocated room). The cache stops aliasing a graph bucket."""
        if capacity <= self.capacity:
            return
        shape = self.K.shape[:-2] + (capacity, self.K.shape[-1])
        K = torch.empty(shape, dtype=self.K.dtype, device=self.K.device)
        V = torch.empty_like(K)
        K[..., :self.length, :].copy_(self.K[..., :self.length, :])
        V[..., :self.length, :].copy_(self.V[..., :self.length, :])
        self.K, self.V, self.graph = K, V, None

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
        return self.K.shape[-2]

    def get_seq_length(self, layer_idx=0):
        return self.length

    def __len__(self):
        return self.K.shape[0]

    def to_dynamic_cache(self):
        from transformers import DynamicCache
        c = DynamicCache()
        for l, (k, v) in enumerate(zip(self.key_cache, self.value_cache)):
            c.update(k.clone(), v.clone(), l)
        return c
