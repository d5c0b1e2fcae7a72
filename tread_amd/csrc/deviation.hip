// (b) Layer-1 KV deviation score and top-k selection.
//
// Score: one wave per candidate. The wave reads the candidate's fresh layer-1 k and v (one GEMM
// output row), applies RoPE to k with the reference's bf16 rounding, gathers the candidate's row
// of the assembled layer-1 cache, and reduces per-head L2 norms with wave shuffles. Bytes per
// candidate: 2 * hkv * hd * 2 (fresh k, v) + 2 * hkv * hd * 2 (cache rows) + 2 (score).
//
// Select: one work group of 1024 threads runs a two-pass radix select on the 16-bit ordered
// score keys (LDS histograms of the high then the low byte) and an order-preserving compaction,
// so the selected candidate indices come out ascending.
#include "common.h"
#include "../../include/tread_hip.h"

namespace tread {

template <int HD>
__global__ __launch_bounds__(256) void dev_score_kernel(const bf16_t* __restrict__ ksrc, const bf16_t* __restrict__ vsrc,
                                                        int64_t ld, const bf16_t* __restrict__ cosb,
                                                        const bf16_t* __restrict__ sinb, const int64_t* __restrict__ rows,
                                                        int64_t n, int hkv, const bf16_t* __restrict__ kc,
                                                        const bf16_t* __restrict__ vc, int64_t t_cap,
                                                        bf16_t* __restrict__ out) {
  constexpr int HALF = HD / 2;
  constexpr int KPL = HALF / 8;  // lanes per k head (each lane: 8 pairs)
  constexpr int VPL = HD / 8;    // lanes per v head (each lane: one 16-byte chunk)
  const int lane = threadIdx.x & 63;
  const int64_t i = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (i >= n) return;
  const int64_t row = rows[i];
  if (row < 0 || row >= t_cap) {  // out-of-range row: no cache read, NaN score
    if (lane == 0) out[i] = 0x7fc0;
    return;
  }
  const bf16_t* kr = ksrc + i * ld;
  const bf16_t* vr = vsrc + i * ld;
  const bf16_t* cs = cosb + i * HALF;
  const bf16_t* sn = sinb + i * HALF;

  float ksum = 0.f, vsum = 0.f;  // sums of per-head bf16 norms (held by group leaders)
  // k: task t -> head t / KPL, column group (t % KPL) * 8 of the first half
  for (int t0 = 0; t0 < hkv * KPL; t0 += 64) {
    int t = t0 + lane;
    float ss = 0.f;
    if (t < hkv * KPL) {
      int h = t / KPL, c = (t % KPL) * 8;
      const bf16_t* src = kr + h * HD;
      const bf16_t* cr = kc + ((int64_t)h * t_cap + row) * HD;
      u32x4_t x1 = *reinterpret_cast<const u32x4_t*>(src + c);
      u32x4_t x2 = *reinterpret_cast<const u32x4_t*>(src + c + HALF);
      u32x4_t c1 = *reinterpret_cast<const u32x4_t*>(cr + c);
      u32x4_t c2 = *reinterpret_cast<const u32x4_t*>(cr + c + HALF);
      u32x4_t cw = *reinterpret_cast<const u32x4_t*>(cs + c);
      u32x4_t sw = *reinterpret_cast<const u32x4_t*>(sn + c);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          float a = p ? hi_bf(x1[w]) : lo_bf(x1[w]);
          float b = p ? hi_bf(x2[w]) : lo_bf(x2[w]);
          float co = p ? hi_bf(cw[w]) : lo_bf(cw[w]);
          float si = p ? hi_bf(sw[w]) : lo_bf(sw[w]);
          // reference: bf16(bf16(x*cos) + bf16(rotate_half(x)*sin))
          float r1 = bf2f(f2bf(bf2f(f2bf(a * co)) + bf2f(f2bf(-b * si))));
          float r2 = bf2f(f2bf(bf2f(f2bf(b * co)) + bf2f(f2bf(a * si))));
          float k1 = p ? hi_bf(c1[w]) : lo_bf(c1[w]);
          float k2 = p ? hi_bf(c2[w]) : lo_bf(c2[w]);
          float d1 = bf2f(f2bf(r1 - k1)), d2 = bf2f(f2bf(r2 - k2));
          ss = fmaf(d1, d1, ss);
          ss = fmaf(d2, d2, ss);
        }
      }
    }
#pragma unroll
    for (int o = KPL / 2; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
    if (t < hkv * KPL && (t % KPL) == 0) ksum += bf2f(f2bf(sqrtf(ss)));
  }
  for (int t0 = 0; t0 < hkv * VPL; t0 += 64) {
    int t = t0 + lane;
    float ss = 0.f;
    if (t < hkv * VPL) {
      int h = t / VPL, c = (t % VPL) * 8;
      u32x4_t x = *reinterpret_cast<const u32x4_t*>(vr + h * HD + c);
      u32x4_t y = *reinterpret_cast<const u32x4_t*>(vc + ((int64_t)h * t_cap + row) * HD + c);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        float d1 = bf2f(f2bf(lo_bf(x[w]) - lo_bf(y[w])));
        float d2 = bf2f(f2bf(hi_bf(x[w]) - hi_bf(y[w])));
        ss = fmaf(d1, d1, ss);
        ss = fmaf(d2, d2, ss);
      }
    }
#pragma unroll
    for (int o = VPL / 2; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
    if (t < hkv * VPL && (t % VPL) == 0) vsum += bf2f(f2bf(sqrtf(ss)));
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    ksum += __shfl_xor(ksum, o);
    vsum += __shfl_xor(vsum, o);
  }
  if (lane == 0) out[i] = f2bf(bf2f(f2bf(ksum)) + bf2f(f2bf(vsum)));
}

// 16-bit key whose unsigned order is the float order of the bf16 value.
__device__ __forceinline__ uint32_t order_key(bf16_t b) {
  return (b & 0x8000u) ? (uint32_t)(~b & 0xffffu) : (uint32_t)(b | 0x8000u);
}

constexpr int SEL_THREADS = 1024;

__global__ __launch_bounds__(SEL_THREADS) void topk_select_kernel(const bf16_t* __restrict__ score, int64_t n,
                                                                  int64_t k, int64_t* __restrict__ sel) {
  __shared__ uint32_t hist[256];
  __shared__ uint32_t s_thr, s_above, s_pfx_g[SEL_THREADS], s_pfx_t[SEL_THREADS];
  const int tid = threadIdx.x;
  // pass 1: high byte
  if (tid < 256) hist[tid] = 0;
  __syncthreads();
  for (int64_t j = tid; j < n; j += SEL_THREADS) atomicAdd(&hist[order_key(score[j]) >> 8], 1u);
  __syncthreads();
  if (tid == 0) {
    uint32_t acc = 0;
    int b = 255;
    for (; b > 0; --b) {
      if (acc + hist[b] >= (uint64_t)k) break;
      acc += hist[b];
    }
    s_thr = (uint32_t)b;
    s_above = acc;
  }
  __syncthreads();
  const uint32_t hb = s_thr;
  const uint32_t above1 = s_above;
  __syncthreads();
  // pass 2: low byte among keys whose high byte is hb
  if (tid < 256) hist[tid] = 0;
  __syncthreads();
  for (int64_t j = tid; j < n; j += SEL_THREADS) {
    uint32_t key = order_key(score[j]);
    if ((key >> 8) == hb) atomicAdd(&hist[key & 0xff], 1u);
  }
  __syncthreads();
  if (tid == 0) {
    uint32_t acc = above1;
    int b = 255;
    for (; b > 0; --b) {
      if (acc + hist[b] >= (uint64_t)k) break;
      acc += hist[b];
    }
    s_thr = (hb << 8) | (uint32_t)b;
    s_above = acc;
  }
  __syncthreads();
  const uint32_t thr = s_thr;
  const int64_t need_ties = k - (int64_t)s_above;
  // pass 3: order-preserving compaction over contiguous per-thread chunks
  const int64_t chunk = (n + SEL_THREADS - 1) / SEL_THREADS;
  const int64_t lo = min<int64_t>(n, tid * chunk), hi = min<int64_t>(n, lo + chunk);
  uint32_t cg = 0, ct = 0;
  for (int64_t j = lo; j < hi; ++j) {
    uint32_t key = order_key(score[j]);
    cg += key > thr;
    ct += key == thr;
  }
  s_pfx_g[tid] = cg;
  s_pfx_t[tid] = ct;
  __syncthreads();
  // Hillis-Steele inclusive scan of both counters
  for (int off = 1; off < SEL_THREADS; off <<= 1) {
    uint32_t ag = tid >= off ? s_pfx_g[tid - off] : 0;
    uint32_t at = tid >= off ? s_pfx_t[tid - off] : 0;
    __syncthreads();
    s_pfx_g[tid] += ag;
    s_pfx_t[tid] += at;
    __syncthreads();
  }
  int64_t g_run = (int64_t)s_pfx_g[tid] - cg;
  int64_t t_run = (int64_t)s_pfx_t[tid] - ct;
  for (int64_t j = lo; j < hi; ++j) {
    uint32_t key = order_key(score[j]);
    if (key > thr) {
      sel[g_run + min(t_run, need_ties)] = j;
      ++g_run;
    } else if (key == thr) {
      if (t_run < need_ties) sel[g_run + t_run] = j;
      ++t_run;
    }
  }
}

}  // namespace tread

using namespace tread;

extern "C" int tread_dev_score_bf16(const void* k_src, const void* v_src, int64_t ld, const void* cos, const void* sin,
                                    const int64_t* rows, int64_t n, int hkv, int head_dim, const void* k_cache,
                                    const void* v_cache, int64_t t_cap, void* score_out, tread_stream_t stream) {
  if (n == 0) return 0;
  if (n < 0 || hkv <= 0 || t_cap <= 0) return fail(TREAD_EINVAL, "dev_score: bad shape");
  if (!k_src || !v_src || !cos || !sin || !rows || !k_cache || !v_cache || !score_out)
    return fail(TREAD_EINVAL, "dev_score: null pointer");
  if (head_dim != 64 && head_dim != 128) return fail(TREAD_EINVAL, "dev_score: head_dim %d not in {64,128}", head_dim);
  if (ld < (int64_t)hkv * head_dim || (ld % 8) != 0) return fail(TREAD_EINVAL, "dev_score: bad row stride %lld", (long long)ld);
  if ((((uintptr_t)k_src | (uintptr_t)v_src) & 15) != 0) return fail(TREAD_EINVAL, "dev_score: k/v source not 16-byte aligned");
  int64_t blocks = (n + 3) / 4;
  if (blocks > 0x7fffffffLL) return fail(TREAD_ERANGE, "dev_score: too many candidates");
  if (head_dim == 128)
    hipLaunchKernelGGL(dev_score_kernel<128>, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                       (const bf16_t*)k_src, (const bf16_t*)v_src, ld, (const bf16_t*)cos, (const bf16_t*)sin, rows, n,
                       hkv, (const bf16_t*)k_cache, (const bf16_t*)v_cache, t_cap, (bf16_t*)score_out);
  else
    hipLaunchKernelGGL(dev_score_kernel<64>, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                       (const bf16_t*)k_src, (const bf16_t*)v_src, ld, (const bf16_t*)cos, (const bf16_t*)sin, rows, n,
                       hkv, (const bf16_t*)k_cache, (const bf16_t*)v_cache, t_cap, (bf16_t*)score_out);
  return check_launch("dev_score");
}

extern "C" size_t tread_topk_workspace_bytes(int64_t n) {
  (void)n;
  return 0;
}

extern "C" int tread_topk_select_bf16(const void* score, int64_t n, int64_t k, int64_t* sel_out, void* ws,
                                      size_t ws_bytes, tread_stream_t stream) {
  (void)ws;
  (void)ws_bytes;
  if (n < 0 || k < 0 || k > n) return fail(TREAD_EINVAL, "topk_select: k=%lld outside [0, n=%lld]", (long long)k, (long long)n);
  if (k == 0) return 0;
  if (!score || !sel_out) return fail(TREAD_EINVAL, "topk_select: null pointer");
  if (n > 0x7fffffffLL) return fail(TREAD_ERANGE, "topk_select: n too large");
  hipLaunchKernelGGL(topk_select_kernel, dim3(1), dim3(SEL_THREADS), 0, (hipStream_t)stream, (const bf16_t*)score, n, k,
                     sel_out);
  return check_launch("topk_select");
}
