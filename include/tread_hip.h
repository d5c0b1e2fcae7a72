/* C-ABI of libtread_hip.so: the MI355X (gfx950) kernels under tread's KV-reuse hot path.
 *
 * The reference (sykeriin/tread) has no FFI: its hot path is Python calling torch / transformers
 * ops. Each entry point below names the reference code it replaces (paths relative to the
 * reference tree). All pointers are device pointers unless marked host; tensors are contiguous,
 * row-major, bf16 unless noted. Nothing here allocates, synchronises the host or reads device
 * memory from the host, so every call is stream-ordered and can be captured into a hipGraph.
 * Return value: 0 on success, a negative errno-style code for bad arguments, or a hipError_t.
 * tread_last_error() gives a thread-local message for the last failure.
 */
#ifndef TREAD_HIP_H
#define TREAD_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* tread_stream_t; /* hipStream_t (torch.cuda.current_stream().cuda_stream) */
typedef void* tread_event_t;  /* hipEvent_t */

/* Thread-local text of the last error (empty string if none). */
const char* tread_last_error(void);
/* ABI version of this header (10); bumps on any signature change. */
int tread_abi_version(void);

/* ---------------------------------------------------------------------------------------------
 * (a) Fused RoPE re-rotation + gather/append of cached blocks into one assembled KV cache.
 * Replaces tread/blend.py:22-39 (rotate_keys: K*cos + rotate_half(K)*sin per doc block) and
 * tread/engine.py:108-120 (torch.cat of the prefix and rotated doc blocks along T, then unbind).
 * Source i holds K and V as [n_layers, n_kv, n_tokens, head_dim]; its rows land at destination
 * rows [dst_off, dst_off + n_tokens) of dst [n_layers, n_kv, t_cap, head_dim]. K is rotated by
 * `delta` positions: with c, s = cos_sin[i][j] (device fp32 [n_src][head_dim/2][2], the cos and sin
 * of fp32(delta_i) * inv_freq[j] as the reference's rotary embedding computes them), row element j
 * becomes fl(fl(x_j*c) + fl(-x_{j+hd/2}*s)) and element j+hd/2 fl(fl(x_{j+hd/2}*c) + fl(x_j*s)),
 * rounded once to bf16 (the fp32 reference rotation, op for op). delta == 0 and V are bit copies.
 * Only layers [layer_lo, layer_hi) are written. dst_v may be NULL: then only K moves (the sources'
 * v pointers are ignored), the form of a stand-alone rotate_keys.
 * srcs: HOST array (copied into the kernel arguments; at most 48 sources per internal launch).
 */
typedef struct tread_src {
  const void* k;
  const void* v;
  int64_t n_tokens;
  int64_t dst_off;
  int64_t delta;
} tread_src_t;

int tread_rope_assemble_bf16(const tread_src_t* srcs, int n_src, void* dst_k, void* dst_v, int n_layers,
                             int n_kv, int64_t t_cap, int head_dim, const float* cos_sin, int layer_lo,
                             int layer_hi, tread_stream_t stream);

/* ---------------------------------------------------------------------------------------------
 * RoPE tables with the reference's rounding: cos/sin = bf16(cos/sin(fp32(pos[i]) * inv_freq[j])),
 * shape [n, head_dim/2] each (the first half of HF's cat(freqs, freqs) table).
 * Replaces tread/blend.py:71-79 (_subset_ctx: rotary_emb for positions S, once per blend).
 * pos: int64 [n]. inv_freq: HOST array of head_dim/2 fp32 values.
 */
int tread_rope_table_bf16(const int64_t* pos, int64_t n, const float* inv_freq, int head_dim, void* cos_out,
                          void* sin_out, tread_stream_t stream);

/* ---------------------------------------------------------------------------------------------
 * q/k RoPE + splice of fresh k/v into the layer cache.
 * Replaces tread/blend.py:82-90 (_qkv: apply_rotary_pos_emb in bf16) and tread/blend.py:106
 * (K[:, :, S], V[:, :, S] = k, v). q_src/k_src/v_src point at the q, k and v columns of one GEMM
 * output with row stride `ld` elements; token i's rotated q goes to q_out [n, hq, head_dim]
 * (skipped if q_out is NULL, then q_src is ignored), its rotated k and its v to cache row rows[i]
 * of k_cache / v_cache [hkv, t_cap, head_dim]. Rounding follows the reference's bf16 torch ops:
 * bf16(bf16(x*cos) + bf16(rotate_half(x)*sin)).
 */
int tread_qkv_rope_splice_bf16(const void* q_src, const void* k_src, const void* v_src, int64_t ld,
                               const void* cos, const void* sin, const int64_t* rows, int64_t n, int hq,
                               int hkv, int head_dim, void* q_out, void* k_cache, void* v_cache, int64_t t_cap,
                               tread_stream_t stream);

/* ---------------------------------------------------------------------------------------------
 * (b) Layer-1 KV deviation score of every candidate.
 * Replaces tread/blend.py:128-129: k1 = RoPE(k_src row), then
 * score[i] = sum_h ||k1[h] - K1[h, rows[i]]||_2 + sum_h ||v_src[h] - V1[h, rows[i]]||_2 with the
 * reference's bf16 rounding points (difference, per-head norm, head sum and final add each
 * rounded to bf16; norms accumulate in fp32). Output: bf16 [n].
 */
int tread_dev_score_bf16(const void* k_src, const void* v_src, int64_t ld, const void* cos, const void* sin,
                         const int64_t* rows, int64_t n, int hkv, int head_dim, const void* k_cache,
                         const void* v_cache, int64_t t_cap, void* score_out, tread_stream_t stream);

/* Top-k selection over bf16 scores: writes the indices of the k largest scores in ASCENDING index
 * order to sel_out (int64 [k]). Among equal scores at the threshold the lowest indices win.
 * Replaces tread/blend.py:160-169 (dev.topk(budget).indices, all_c[top], S.sort()): since the
 * candidate positions are ascending, ascending indices give S already sorted.
 * n <= 2^20 candidates (TREAD_ERANGE above). Scratch: ws of at least tread_topk_workspace_bytes(n)
 * bytes (device; 0 today: the selection runs in one work group out of LDS).
 */
size_t tread_topk_workspace_bytes(int64_t n);
int tread_topk_select_bf16(const void* score, int64_t n, int64_t k, int64_t* sel_out, void* ws, size_t ws_bytes,
                           tread_stream_t stream);

/* ---------------------------------------------------------------------------------------------
 * (c) Selective-recompute attention (MFMA, GQA in-kernel, no mask tensor, no repeat_kv).
 * Replaces tread/blend.py:107-110 (repeat_kv x2 + SDPA with the bool mask arange(T) <= S) and
 * the causal / block-diagonal attention of the query forward and cold prefill
 * (tread/engine.py:81-88,132). Row i of q [n, hq, head_dim] sees cache key j of its KV head
 * iff j <= kend[i] and (j < n_shared or j >= kseg[i]); kseg may be NULL (then keys [0, kend[i]]).
 * out: [n, hq * head_dim]. scale: softmax scale (head_dim^-0.5). head_dim: 64 or 128.
 * Few rows over a long cache (the query forward) split the key axis across work groups, and a
 * launch of a few GPU rounds (the recompute rows) runs the longest quarter of its row tiles as two
 * key-half work groups; both keep fp32 partials in ws of tread_subset_attn_workspace_bytes(...)
 * bytes (device) and merge them in a second kernel. With ws NULL or too small the call still
 * succeeds, with whole row tiles and no key split.
 */
size_t tread_subset_attn_workspace_bytes(int64_t n, int hq, int hkv, int head_dim, int64_t t_cap);
int tread_subset_attn_bf16(const void* q, const void* k_cache, const void* v_cache, const int64_t* kend,
                           const int64_t* kseg, int64_t n_shared, int64_t n, int hq, int hkv, int head_dim,
                           int64_t t_cap, float scale, void* out, void* ws, size_t ws_bytes, tread_stream_t stream);

/* tread_subset_attn_bf16 without the workspace argument, for callers that cannot allocate device
 * memory (code under hipGraph capture, tight serving loops, harnesses that forbid hipMalloc). No
 * counterpart in the reference. It calls no allocator: the key-split / key-half partials live in a
 * static device array of TREAD_SUBSET_ATTN_SCRATCH_BYTES (96 MiB) that each GPU the library runs
 * on holds until the process ends; its address is looked up on the first call on each device. A
 * shape whose workspace (tread_subset_attn_workspace_bytes) exceeds that size returns TREAD_ERANGE
 * with a message and launches nothing. Every call on one GPU shares that GPU's array; calls that
 * use it are ordered on each GPU: a call on another stream than the previous call's first makes its
 * stream wait for an event that call recorded (created with the array's address lookup on the first
 * call per device). Calls on a stream under graph capture neither wait nor record, so a captured
 * call and calls on other streams that overlap it race. Same kernels and results as the workspace
 * form with a large enough workspace.
 */
#define TREAD_SUBSET_ATTN_SCRATCH_BYTES (96u << 20)
int tread_subset_attn_scratch_bf16(const void* q, const void* k_cache, const void* v_cache, const int64_t* kend,
                                   const int64_t* kseg, int64_t n_shared, int64_t n, int hq, int hkv, int head_dim,
                                   int64_t t_cap, float scale, void* out, tread_stream_t stream);

/* ---------------------------------------------------------------------------------------------
 * Decoder-layer glue for the recompute rows (transformers Qwen2RMSNorm / Qwen2MLP as called at
 * tread/blend.py:103,111-113).
 * add_rmsnorm: s = x + delta (bf16; delta may be NULL), norm_out = w * bf16(s * rsqrt(mean(s^2)+eps));
 * s is written to sum_out when it is not NULL. x, delta, sum_out, norm_out: [n, hidden].
 * silu_mul: out[n, inter] = bf16(bf16(silu(g)) * u) for gate_up [n, 2*inter] = [g | u].
 */
int tread_add_rmsnorm_bf16(const void* x, const void* delta, const void* weight, float eps, int64_t n, int hidden,
                           void* sum_out, void* norm_out, tread_stream_t stream);
int tread_silu_mul_bf16(const void* gate_up, int64_t n, int inter, void* out, tread_stream_t stream);

/* Linear layer of a few token rows (decode steps): y[m, n] = x[m, k] . weight[n, k]^T (+ bias[n]),
 * bf16, fp32 accumulation, one bf16 rounding (as F.linear). m <= 32; n a multiple of 32; k a
 * multiple of 128; x rows ldx apart (16-byte aligned), y rows ldy apart; bias may be NULL.
 * Replaces the q|k|v, o, gate|up, down and lm_head projections (transformers Qwen2Attention /
 * Qwen2MLP / lm_head) of the decoding step model(nxt.view(1, 1), past_key_values=cache) at
 * tread/server.py:207, whose GEMMs are weight-streaming. Layers with few output features split k
 * across work groups when ws holds tread_skinny_workspace_bytes(m, n, k) bytes (device, 16-byte
 * aligned); with ws NULL or too small the call still succeeds, unsplit.
 */
size_t tread_skinny_workspace_bytes(int64_t m, int64_t n, int64_t k);
int tread_skinny_linear_bf16(const void* x, int64_t ldx, const void* weight, const void* bias, int64_t m, int64_t n,
                             int64_t k, void* y, int64_t ldy, void* ws, size_t ws_bytes, tread_stream_t stream);

/* The same for m <= 8 rows with the layer's input norm fused in front: y = linear(RMSNorm(h + delta))
 * (add_rmsnorm's bits), and h_out = h + delta (may be NULL; delta may be NULL). h, delta, h_out:
 * [m, k] contiguous. Replaces input_layernorm / post_attention_layernorm + q|k|v or gate|up of a
 * decoding step (transformers Qwen2DecoderLayer under tread/server.py:207).
 */
int tread_skinny_norm_linear_bf16(const void* h, const void* delta, const void* ln_weight, float eps, int64_t m,
                                  int64_t n, int64_t k, const void* weight, const void* bias, void* y, void* h_out,
                                  tread_stream_t stream);

/* skinny_norm_linear of the q|k|v projection with tread_qkv_rope_splice_bf16 fused behind it:
 * qkv = linear(RMSNorm(h + delta), wqkv, bqkv) for m <= 8 rows (wqkv: [(hq + 2 hkv) head_dim,
 * hidden], bqkv may be NULL), then q and k rotated with cos / sin [m, head_dim / 2], q into q_out
 * [m, hq, head_dim], k and v into row rows[i] of k_cache / v_cache [hkv, t_cap, head_dim] (rows
 * outside [0, t_cap) splice nothing), h_out = h + delta (may be NULL). Bits equal to
 * tread_skinny_norm_linear_bf16 followed by tread_qkv_rope_splice_bf16, in one launch. Replaces
 * the input_layernorm + q/k/v projections + apply_rotary_pos_emb + cache update of a decoding step
 * (transformers Qwen2Attention under tread/server.py:207).
 */
int tread_skinny_norm_qkv_rope_bf16(const void* h, const void* delta, const void* ln_weight, float eps, int64_t m,
                                    int64_t hidden, const void* wqkv, const void* bqkv, int hq, int hkv, int head_dim,
                                    const void* cos, const void* sin, const int64_t* rows, void* q_out, void* k_cache,
                                    void* v_cache, int64_t t_cap, void* h_out, tread_stream_t stream);

/* skinny_norm_linear of an MLP's gate|up projection with silu_mul fused behind it: for m <= 8 rows,
 * [g | u] = linear(RMSNorm(h + delta), wgu) (wgu: [2 inter, hidden], gate rows then up rows;
 * inter a multiple of 16) and y [m, inter] = bf16(bf16(silu(g)) * u), h_out = h + delta (may be
 * NULL). Bits equal to tread_skinny_norm_linear_bf16 followed by tread_silu_mul_bf16, in one
 * launch, without the [m, 2 inter] intermediate. Replaces post_attention_layernorm + gate/up
 * projections + act_fn(gate) * up of a decoding step (transformers Qwen2MLP under
 * tread/server.py:207).
 */
int tread_skinny_norm_swiglu_bf16(const void* h, const void* delta, const void* ln_weight, float eps, int64_t m,
                                  int64_t hidden, const void* wgu, int64_t inter, void* y, void* h_out,
                                  tread_stream_t stream);

/* y[m, n] = linear(bf16(bf16(silu(g)) * u)) for gate_up [m, 2 inter] = [g | u], m <= 8 (silu_mul's
 * bits fused into the down projection of a decoding step, transformers Qwen2MLP). ws: at least
 * tread_skinny_silu_workspace_bytes(m, n, inter) bytes (device, 16-byte aligned; required when
 * that is non-zero: the k split also keeps the staged rows within LDS).
 * skinny_norm_linear requires m * k * 2 bytes to fit in LDS (about 127 KiB).
 */
size_t tread_skinny_silu_workspace_bytes(int64_t m, int64_t n, int64_t inter);
int tread_skinny_silu_linear_bf16(const void* gate_up, int64_t m, int64_t inter, const void* weight, int64_t n, void* y,
                                  void* ws, size_t ws_bytes, tread_stream_t stream);

/* ---------------------------------------------------------------------------------------------
 * (d) Block-tier copy: async DMA of `bytes` between pinned host and device memory (either
 * direction) on `stream`, then records `done` (may be NULL) on the same stream.
 * Replaces tread/store.py:75-76 (b.K.to(device, non_blocking=True)) and tread/store.py:111
 * (b.K.to("cpu").pin_memory(), a synchronous D2H).
 */
int tread_copy_async(void* dst, const void* src, size_t bytes, tread_stream_t stream, tread_event_t done);

/* Layer-major schedule of such copies: for l in [0, n_layers): the per_layer copies
 * dst[l * per_layer + i] <- src[l * per_layer + i] (bytes[...]) in order, then layer_done[l]
 * recorded (NULL array or entries skip it). One call queues the slices of every block a request
 * promotes from the host tier, layer 0 of all blocks first. Replaces the per-block
 * b.K.to(device, non_blocking=True) of tread/store.py:75-76. */
int tread_copy_layers_async(void* const* dst, const void* const* src, const size_t* bytes, int per_layer,
                            int n_layers, tread_stream_t stream, const tread_event_t* layer_done);

#ifdef __cplusplus
}
#endif

#endif /* TREAD_HIP_H */
