"""CPU oracle for tread's KV-reuse hot path. TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU with plain PyTorch ops, what the reference computes on the path
`Engine.prefill -> BlockStore -> rotate/assemble -> blend -> query forward`:

- `oracle.model_ref`  the Qwen2/Llama decoder math the reference reaches through transformers'
                      Qwen2 modules (RMSNorm, RoPE, GQA attention, SwiGLU MLP, causal / 4D masks).
- `oracle.tread_ref`  tread/store.py, tread/engine.py, tread/blend.py and the bucket rule of
                      tread/graphs.py, op for op, including the bf16 rounding points.

Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may import it, and
only to check results (or, for `cpu_baseline`, as the timed CPU path). The product package
`tread_amd` never imports it and has no CPU fallback. Loaded onto a GPU device
(`model_ref.load(..., device="cuda")`), the same torch code runs there as a second checker, whose
roundings differ from the CPU's only by the backends' kernels (GEMMs, attention, libm).

How each function is pinned (checks live in tests/test_oracle.py):
- model math: against transformers' own Qwen2ForCausalLM / LlamaForCausalLM on tiny configs
  (a library routine the reference calls), in fp32.
- rotate_keys: RoPE group property R(a)R(b) = R(a+b), delta 0 returns the input object,
  layer-0 keys prefilled at +d equal rotated keys (test_engine.py:46-55 re-expressed).
- block_key: an independent construction with struct.pack + hashlib, and SHA-256 known answers.
- BlockStore: random get/put scripts against an independent list-based LRU model.
- layer1_deviation score: pure-Python loops on tiny inputs, with planted ties.
- top-k selection: brute-force sort on tiny inputs.
- _bucket: brute-force search over the allowed bucket sizes.
- engine invariants: ratio=1 reproduces full prefill, reordered requests hit every block, packed
  cold prefill equals per-doc prefill after the prefix, CPU tier exactness, eviction budget
  (test_engine.py:58-178 re-expressed with random-init models).
"""
