"""Write the golden fixtures under tests/golden/ from constructions independent of the oracle.

- block_keys.json: SHA-256 digests of block-key part lists, built byte by byte with struct.pack
  (little-endian int64 per token id, UTF-8 str(p) otherwise, a NUL after every part) — the format
  of tread/store.py:21-30 — for the sig / namespace / prefix-chain shapes tread/engine.py:47,67 use.
- buckets.json: graph bucket sizes (tread/graphs.py:22-27) found by brute-force search over the
  allowed row counts and cache lengths.
- rotate.json: RoPE shifts of small fp32 key rows, computed in float64 with Python's math module
  from the fp32 angles fp32(delta) * inv_freq (default RoPE, split-half pairing).
- deviation.json: layer-1 deviation scores (sum over heads of L2 norms of k and v differences,
  tread/blend.py:129) of tiny fp32 inputs in float64 loops, with planted ties, and the top-k index
  sets (ties broken toward lower indices) from a full sort.

Run: python tests/golden/make_golden.py   (deterministic; uses only the standard library)
"""
import hashlib
import json
import math
import random
import struct
from pathlib import Path

HERE = Path(__file__).resolve().parent


def f32(x):
    return struct.unpack("<f", struct.pack("<f", x))[0]


def key_bytes(parts):
    out = bytearray()
    for p in parts:
        if isinstance(p, list):  # token ids
            for t in p:
                out += struct.pack("<q", t)
        elif p is None:
            out += b"None"
        else:
            out += str(p).encode("utf-8")
        out += b"\x00"
    return bytes(out)


def enc_part(p):
    if isinstance(p, list):
        return {"ids": p}
    if p is None:
        return {"none": True}
    if isinstance(p, float):
        return {"float": p}
    return {"str": p}


def block_keys():
    rnd = random.Random(7)
    cases = []
    for sig in [("", "torch.bfloat16", 1000000.0, None), ("", "torch.float32", 1000000.0, None),
                ("Qwen/Qwen2.5-0.5B-Instruct", "torch.float16", 1000000.0, None),
                ("", "torch.bfloat16", 500000.0, None)]:
        for ns in ["", "tenant-a"]:
            prefix = [rnd.randrange(0, 151936) for _ in range(rnd.choice([1, 16, 64]))]
            parts = list(sig) + [ns, "prefix", prefix]
            pkey = hashlib.sha256(key_bytes(parts)).hexdigest()
            cases.append({"parts": [enc_part(p) for p in parts], "digest": pkey})
            for n in (1, 3, 1000):
                doc = [rnd.randrange(0, 151936) for _ in range(n)]
                dparts = list(sig) + [pkey, doc]
                cases.append({"parts": [enc_part(p) for p in dparts],
                              "digest": hashlib.sha256(key_bytes(dparts)).hexdigest()})
    # edge cases: empty id list, negative ids, large ids
    for ids in ([], [-1, 0, 1], [2 ** 40, 5]):
        parts = ["", "torch.bfloat16", 1000000.0, None, "", "prefix", ids]
        cases.append({"parts": [enc_part(p) for p in parts], "digest": hashlib.sha256(key_bytes(parts)).hexdigest()})
    return cases


def buckets():
    def brute(n, T, n_min=64, n_step=256, t_step=1024):
        # smallest admissible row count >= n: a power of two >= n_min while n <= n_step, else a
        # multiple of n_step; then the smallest multiple of t_step holding T + the padded rows
        b = n
        while not ((n <= n_step and b >= n_min and b & (b - 1) == 0) or (n > n_step and b % n_step == 0)):
            b += 1
        t = t_step
        while t < T + b - n:
            t += t_step
        return b, t
    out = []
    for n in [1, 2, 63, 64, 65, 100, 128, 129, 255, 256, 257, 511, 512, 513, 1560, 6400, 16000]:
        for T in [n, n + 1, 1000, 1024, 2048, 8064, 32064]:
            if T < n:
                continue
            nb, Tb = brute(n, T)
            out.append({"n": n, "T": T, "nb": nb, "Tb": Tb})
    return out


def inv_freq(theta, d):
    return [f32(1.0 / f32(theta ** f32(f32(i) / d))) for i in range(0, d, 2)]


def rotate():
    rnd = random.Random(3)
    cases = []
    for theta, d in [(10000.0, 8), (1000000.0, 16), (500000.0, 16)]:
        # inverse frequencies as fp32 numbers: torch computes 1/(theta ** (arange(0,d,2)/d)) in fp32
        for delta in [0, 1, 37, 1000, 31000, -5]:
            rows = [[f32(rnd.gauss(0, 1)) for _ in range(d)] for _ in range(3)]
            cases.append({"theta": theta, "d": d, "delta": delta, "K": rows})
    return cases


def rotate_expected(case, inv):
    d, delta = case["d"], case["delta"]
    out = []
    for row in case["K"]:
        o = [0.0] * d
        for j in range(d // 2):
            ang = f32(f32(float(delta)) * inv[j])
            c, s = math.cos(ang), math.sin(ang)
            o[j] = row[j] * c - row[j + d // 2] * s
            o[j + d // 2] = row[j + d // 2] * c + row[j] * s
        out.append(o)
    return out


def deviation():
    rnd = random.Random(11)
    cases = []
    for hkv, hd, n in [(2, 4, 7), (1, 8, 9), (3, 2, 12)]:
        k1 = [[[f32(rnd.gauss(0, 1)) for _ in range(hd)] for _ in range(n)] for _ in range(hkv)]
        v1 = [[[f32(rnd.gauss(0, 1)) for _ in range(hd)] for _ in range(n)] for _ in range(hkv)]
        K1 = [[[f32(rnd.gauss(0, 1)) for _ in range(hd)] for _ in range(n)] for _ in range(hkv)]
        V1 = [[[f32(rnd.gauss(0, 1)) for _ in range(hd)] for _ in range(n)] for _ in range(hkv)]
        # planted ties: candidate 1 and 3 identical to candidate 0; candidate 2 exact (score 0)
        for h in range(hkv):
            for arr in (k1, v1, K1, V1):
                arr[h][1] = list(arr[h][0])
                arr[h][3] = list(arr[h][0])
            k1[h][2] = list(K1[h][2])
            v1[h][2] = list(V1[h][2])
        score = []
        for i in range(n):
            s = 0.0
            for a, b in ((k1, K1), (v1, V1)):
                for h in range(hkv):
                    s += math.sqrt(sum((a[h][i][e] - b[h][i][e]) ** 2 for e in range(hd)))
            score.append(s)
        order = sorted(range(n), key=lambda i: (-score[i], i))
        topk = {str(k): sorted(order[:k]) for k in range(0, n + 1)}
        cases.append({"k1": k1, "v1": v1, "K1": K1, "V1": V1, "score": score, "topk": topk})
    return cases


def main():
    (HERE / "block_keys.json").write_text(json.dumps(block_keys(), indent=0))
    (HERE / "buckets.json").write_text(json.dumps(buckets(), indent=0))
    rot = rotate()
    for c in rot:
        c["expected"] = rotate_expected(c, inv_freq(c["theta"], c["d"]))
    (HERE / "rotate.json").write_text(json.dumps(rot, indent=0))
    (HERE / "deviation.json").write_text(json.dumps(deviation(), indent=0))
    print("wrote", sorted(p.name for p in HERE.glob("*.json")))


if __name__ == "__main__":
    main()
