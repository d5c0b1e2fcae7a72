"""On-disk / wire format of a KV block: the store's third tier (the tier SCOPE.md:34-35 of the
reference names as its stretch: "GPU, then pinned CPU RAM, then (stretch) disk").

One block = one file `<key>.trb` holding exactly what the store keeps for a block
(tread/store.py:33-41: stacked K and V [layers, 1, kv_heads, tokens, head_dim], `base`, token
count), so a new process pointed at the same directory serves the blocks an earlier one cached:
the key is the content address (model signature, chained prefix key, token ids), which is the same
across restarts. The same bytes are the wire form of a block (`pack` / `unpack`).

Layout (little-endian; offsets in bytes):
  0    8   magic b"TREADKV1"
  8    4   header length (4096)
  12   4   dtype code (1 bf16, 2 fp16, 3 fp32)
  16   64  key, ASCII hex, NUL-padded
  80   8   base (int64, position the block was computed at)
  88   8   n_tokens (int64)
  96   40  shape of K and V: 5 x int64 [layers, 1, kv_heads, tokens, head_dim]
  136  8   K offset (4096)      144  8   K bytes
  152  8   V offset             160  8   V bytes
  168  8   XXH3-64 of the K bytes followed by the V bytes
  176  8   XXH3-64 of header bytes [0, 176)
  ...      zero up to 4096
  K bytes at 4096, V bytes at the next multiple of 4096; each is the C-order element bytes.
Payload offsets are 4 KiB-aligned so that reads can go straight into page-aligned pinned buffers.
Files are written to `<key>.trb.tmp` and renamed, so a reader never sees a partial block.
"""
import os
import struct
from pathlib import Path

import torch
import xxhash

MAGIC = b"TREADKV1"
HEADER = 4096
ALIGN = 4096
SUFFIX = ".trb"
_DTYPES = {torch.bfloat16: 1, torch.float16: 2, torch.float32: 3}
_CODES = {v: k for k, v in _DTYPES.items()}
_FIXED = struct.Struct("<8sII64sqq5qQQQQQ")  # up to the payload checksum (176 bytes)
_HSUM = struct.Struct("<Q")


class BlockFileError(ValueError):
    """A block file or buffer that is not a valid block (bad magic, header, size or checksum)."""


def _align(n):
    return -(-n // ALIGN) * ALIGN


def _bytes_of(t):
    """Raw bytes of a contiguous CPU tensor (no copy)."""
    if t.device.type != "cpu" or not t.is_contiguous():
        raise ValueError("block tensors must be contiguous CPU tensors")
    return memoryview(t.view(torch.uint8).numpy()).cast("B")


def _header(key, K, V, base):
    if K.shape != V.shape or K.dtype != V.dtype or K.dim() != 5:
        raise ValueError(f"K {tuple(K.shape)} / V {tuple(V.shape)} are not one block")
    if K.dtype not in _DTYPES:
        raise ValueError(f"unsupported dtype {K.dtype}")
    kb = K.numel() * K.element_size()
    k_off, v_off = HEADER, HEADER + _align(kb)
    h = xxhash.xxh3_64()
    h.update(_bytes_of(K))
    h.update(_bytes_of(V))
    fixed = _FIXED.pack(MAGIC, HEADER, _DTYPES[K.dtype], key.encode("ascii"), int(base), K.shape[-2], *K.shape,
                        k_off, kb, v_off, kb, h.intdigest())
    return fixed + _HSUM.pack(xxhash.xxh3_64_intdigest(fixed)), k_off, v_off, kb


def parse_header(buf):
    """Fields of a block header (the first 4096 bytes of a file or packed buffer)."""
    if len(buf) < _FIXED.size + _HSUM.size:
        raise BlockFileError("truncated header")
    fixed = bytes(buf[:_FIXED.size])
    (hsum,) = _HSUM.unpack_from(buf, _FIXED.size)
    if fixed[:8] != MAGIC:
        raise BlockFileError("not a tread block (bad magic)")
    if xxhash.xxh3_64_intdigest(fixed) != hsum:
        raise BlockFileError("header checksum mismatch")
    (_, hlen, code, key, base, n_tokens, *rest) = _FIXED.unpack(fixed)
    shape, (k_off, k_bytes, v_off, v_bytes, psum) = tuple(rest[:5]), rest[5:]
    if hlen != HEADER or code not in _CODES or shape[3] != n_tokens:
        raise BlockFileError("inconsistent header")
    dtype = _CODES[code]
    nbytes = 1
    for d in shape:
        nbytes *= d
    nbytes *= torch.empty((), dtype=dtype).element_size()
    if k_bytes != nbytes or v_bytes != nbytes or k_off != HEADER or v_off != HEADER + _align(k_bytes):
        raise BlockFileError("inconsistent payload layout")
    return dict(key=key.rstrip(b"\x00").decode("ascii"), base=base, n_tokens=n_tokens, shape=shape, dtype=dtype,
                k_offset=k_off, v_offset=v_off, nbytes=nbytes, checksum=psum,
                file_bytes=v_off + v_bytes)


def _write_all(f, data):
    mv = memoryview(data).cast("B")
    while len(mv):
        n = f.write(mv)
        mv = mv[n:]


def write_block(path, key, K, V, base):
    """Write one block (contiguous CPU tensors, e.g. the pinned host-tier copy) to `path`, through
    a temporary file and a rename. Returns the file size."""
    path = Path(path)
    head, k_off, v_off, kb = _header(key, K, V, base)
    tmp = path.with_name(path.name + ".tmp")
    with open(tmp, "wb", buffering=0) as f:
        _write_all(f, head + bytes(HEADER - len(head)))
        _write_all(f, _bytes_of(K))
        if v_off - k_off - kb:
            _write_all(f, bytes(v_off - k_off - kb))
        _write_all(f, _bytes_of(V))
    os.replace(tmp, path)
    return v_off + kb


def read_header(path):
    with open(path, "rb", buffering=0) as f:
        return parse_header(f.read(HEADER))


def read_into(path, K, V, header=None, verify=True):
    """Read a block file's payload straight into the CPU tensors K and V (their shapes and dtype
    must be the header's). Returns the header."""
    with open(path, "rb", buffering=0) as f:
        h = header or parse_header(f.read(HEADER))
        if tuple(K.shape) != h["shape"] or tuple(V.shape) != h["shape"] or K.dtype != h["dtype"] or V.dtype != h["dtype"]:
            raise ValueError(f"{path}: tensors do not match the block's shape / dtype")
        for t, off in ((K, h["k_offset"]), (V, h["v_offset"])):
            f.seek(off)
            mv, got = _bytes_of(t), 0
            while got < h["nbytes"]:
                n = f.readinto(mv[got:])
                if not n:
                    raise BlockFileError(f"{path}: truncated payload")
                got += n
    if verify:
        x = xxhash.xxh3_64()
        x.update(_bytes_of(K))
        x.update(_bytes_of(V))
        if x.intdigest() != h["checksum"]:
            raise BlockFileError(f"{path}: payload checksum mismatch")
    return h


def read_block(path, pin_memory=True, verify=True, header=None):
    """Read a block file into new (pinned) CPU tensors: returns (K, V, header)."""
    h = header or read_header(path)
    K = torch.empty(h["shape"], dtype=h["dtype"], pin_memory=pin_memory)
    V = torch.empty(h["shape"], dtype=h["dtype"], pin_memory=pin_memory)
    read_into(path, K, V, header=h, verify=verify)
    return K, V, h


def pack(key, K, V, base) -> bytes:
    """The wire form of a block: the same bytes as its file."""
    head, k_off, v_off, kb = _header(key, K, V, base)
    out = bytearray(v_off + kb)
    out[:len(head)] = head
    out[k_off:k_off + kb] = _bytes_of(K)
    out[v_off:v_off + kb] = _bytes_of(V)
    return bytes(out)


def unpack(buf, verify=True):
    """Inverse of `pack`: (key, K, V, base) as CPU tensors (copies of the buffer's bytes)."""
    h = parse_header(buf)
    if len(buf) < h["file_bytes"]:
        raise BlockFileError("truncated payload")
    ts = []
    for off in (h["k_offset"], h["v_offset"]):
        t = torch.empty(h["shape"], dtype=h["dtype"])
        _bytes_of(t)[:] = memoryview(buf)[off:off + h["nbytes"]]
        ts.append(t)
    if verify:
        x = xxhash.xxh3_64()
        x.update(_bytes_of(ts[0]))
        x.update(_bytes_of(ts[1]))
        if x.intdigest() != h["checksum"]:
            raise BlockFileError("payload checksum mismatch")
    return h["key"], ts[0], ts[1], h["base"]
