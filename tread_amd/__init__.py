"""tread on MI355X: position-independent KV-cache reuse with hand-written CDNA4 HIP kernels.

Drop-in for tread's Engine / BlockStore API (tread/__init__.py). The HIP library
(tread_amd/libtread_hip.so, built by tread_amd.csrc.build) is loaded on first use; there is no
CPU fallback for the kernels.
"""
from tread_amd.cache import KVCache, StaleCacheError
from tread_amd.engine import Engine, RequestStats, prefill_full
from tread_amd.store import Block, BlockStore, StoreStats, block_key

__all__ = ["Engine", "BlockStore", "Block", "StoreStats", "RequestStats", "block_key", "prefill_full", "KVCache",
           "StaleCacheError"]
