// (b) Layer-1 KV deviation score and top-k selection.
//
// Score: one half-wave (32 lanes) per candidate, two candidates per wave. The lanes read the
// candidate's fresh layer-1 k and v (one GEMM output row), apply RoPE to k with the reference's
// bf16 rounding, gather the candidate's row of the assembled layer-1 cache, and reduce per-head L2
// norms with shuffles inside the half-wave. Bytes per candidate: 2 * hkv * hd * 2 (fresh k, v) +
// 2 * hkv * hd * 2 (cache rows) + 2 (score).
//
// Select: one work group of 1024 threads stages the 16-bit ordered score keys in LDS (up to 64 Ki
// candidates), runs a two-pass radix select over them (high byte, then low byte, into a 256-bin LDS
// histogram replicated so that one wave's atomics spread over 16 words), and an order-preserving
// compaction, so the selected candidate indices come out ascending.
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
  const int lane = threadIdx.x & 31;
  const int64_t i = (int64_t)blockIdx.x * 8 + (threadIdx.x >> 5);
  if (i >= n) return;  // whole half-waves leave together: the shuffles below stay within one
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
  for (int t0 = 0; t0 < hkv * KPL; t0 += 32) {
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
  for (int t0 = 0; t0 < hkv * VPL; t0 += 32) {
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
  for (int o = 16; o >= 1; o >>= 1) {
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
constexpr int SEL_WAVES = SEL_THREADS / 64;
constexpr int64_t SEL_LDS_KEYS = 65536;  // candidates whose keys are staged in LDS (128 KiB)
constexpr int64_t SEL_MAX_N = 1 << 20;   // keeps every 16-bit histogram counter at or below 2^15
constexpr int SEL_HROWS = 16, SEL_HSTRIDE = 257;  // histogram rows; odd stride spreads rows over banks

__device__ __forceinline__ uint32_t lanes_below(uint64_t mask) {  // set bits of mask in lanes < this lane
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

__device__ __forceinline__ uint32_t wave_sum_u(uint32_t x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

// Run by one whole wave: the bin b of 256 for which the counts of the bins above b, plus `above`,
// sum to fewer than k and those of the bins from b up to at least k (the bin holding the k-th
// largest key). Lane l owns the bins 255 - 4l .. 252 - 4l; exactly one lane finds the bin, since the
// running count grows monotonically from the top bin down, and that lane stores it with the count
// above it. Requires 0 < k - above <= the count over all bins.
__device__ __forceinline__ void find_bin(const uint32_t* tot, uint32_t above, int64_t k, uint32_t* bin_out,
                                         uint32_t* above_out) {
  const int lane = threadIdx.x & 63;
  uint32_t c[4], own = 0;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    c[u] = tot[255 - 4 * lane - u];
    own += c[u];
  }
  uint32_t incl = own;  // inclusive prefix over lanes, top bins first
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t y = __shfl_up(incl, o);
    if (lane >= o) incl += y;
  }
  uint64_t before = (uint64_t)above + incl - own;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    if (before < (uint64_t)k && before + c[u] >= (uint64_t)k) {
      *bin_out = 255 - 4 * lane - u;
      *above_out = (uint32_t)before;
    }
    before += c[u];
  }
}

__global__ __launch_bounds__(SEL_THREADS) void topk_select_kernel(const bf16_t* __restrict__ score, int64_t n,
                                                                  int64_t k, int64_t* __restrict__ sel) {
  extern __shared__ uint16_t keys[];  // n ordered keys when n <= SEL_LDS_KEYS
  // One 256-bin histogram shared by all waves, replicated over 16 rows x 2 halves so that the 64
  // lanes of one atomic instruction hit 16 different words (lane l: row (l / 2) % 16, 16-bit half
  // l % 2): request scores cluster in few bins, and same-word atomics of one wave serialise.
  __shared__ uint32_t hist[SEL_HROWS * SEL_HSTRIDE];
  __shared__ uint32_t tot[256];
  __shared__ uint32_t s_thr, s_above, s_cnt_g[SEL_WAVES], s_cnt_t[SEL_WAVES];
  const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63;
  uint32_t* const hrow = hist + ((lane >> 1) & (SEL_HROWS - 1)) * SEL_HSTRIDE;
  const uint32_t hinc = (lane & 1) ? 0x10000u : 1u;
  const bool staged = n <= SEL_LDS_KEYS;
  // keys j .. j + 7 (j a multiple of 8), two per dword, low half first; keys at n and beyond are
  // unspecified and masked by the callers
  auto load8 = [&](int64_t j) -> u32x4_t {
    if (staged) return j < n ? reinterpret_cast<const u32x4_t*>(keys)[j >> 3] : u32x4_t{0u, 0u, 0u, 0u};
    u32x4_t kk;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const uint32_t a = j + 2 * w < n ? order_key(score[j + 2 * w]) : 0u;
      const uint32_t b = j + 2 * w + 1 < n ? order_key(score[j + 2 * w + 1]) : 0u;
      kk[w] = a | (b << 16);
    }
    return kk;
  };
  auto clear = [&]() {
    for (int b = tid; b < SEL_HROWS * SEL_HSTRIDE; b += SEL_THREADS) hist[b] = 0;
  };
  auto merge = [&]() {
    if (tid < 256) {
      uint32_t t = 0;
#pragma unroll
      for (int r = 0; r < SEL_HROWS; ++r) {
        const uint32_t x = hist[r * SEL_HSTRIDE + tid];
        t += (x & 0xffffu) + (x >> 16);
      }
      tot[tid] = t;
    }
  };
  // pass 1: stage the keys, histogram of the high byte. 16-byte loads, UNR of them in flight per
  // thread, when the scores are 16-byte aligned; a scalar loop for the rest.
  clear();
  __syncthreads();
  constexpr int UNR = 4;
  const int64_t nvec = (((uintptr_t)score & 15) == 0) ? n / 8 : 0;
  for (int64_t v0 = 0; v0 < nvec; v0 += (int64_t)SEL_THREADS * UNR) {
    u32x4_t x[UNR];
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int64_t v = v0 + u * SEL_THREADS + tid;
      x[u] = v < nvec ? reinterpret_cast<const u32x4_t*>(score)[v] : u32x4_t{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int64_t v = v0 + u * SEL_THREADS + tid;
      const bool ok = v < nvec;
      u32x4_t kk;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint32_t lo = order_key((bf16_t)(x[u][w] & 0xffff)), hi = order_key((bf16_t)(x[u][w] >> 16));
        kk[w] = lo | (hi << 16);
        if (ok) {
          atomicAdd(&hrow[lo >> 8], hinc);
          atomicAdd(&hrow[hi >> 8], hinc);
        }
      }
      if (ok && staged) reinterpret_cast<u32x4_t*>(keys)[v] = kk;
    }
  }
  for (int64_t j = nvec * 8 + tid; j < n; j += SEL_THREADS) {
    const uint32_t key = order_key(score[j]);
    if (staged) keys[j] = (uint16_t)key;
    atomicAdd(&hrow[key >> 8], hinc);
  }
  __syncthreads();
  merge();
  __syncthreads();
  if (wv == 0) find_bin(tot, 0, k, &s_thr, &s_above);
  clear();
  __syncthreads();
  const uint32_t hb = s_thr;
  const uint32_t above1 = s_above;
  // pass 2: low byte among keys whose high byte is hb, eight keys per thread and step
  for (int64_t j = 8 * (int64_t)tid; j < n; j += 8 * SEL_THREADS) {
    const u32x4_t kk = load8(j);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const uint32_t key = (kk[u >> 1] >> (16 * (u & 1))) & 0xffffu;
      if (j + u < n && (key >> 8) == hb) atomicAdd(&hrow[key & 0xff], hinc);
    }
  }
  __syncthreads();
  merge();
  __syncthreads();
  if (wv == 0) find_bin(tot, above1, k, &s_thr, &s_above);
  __syncthreads();
  const uint32_t thr = (hb << 8) | s_thr;
  const int64_t need_ties = k - (int64_t)s_above;
  // pass 3: order-preserving compaction. Wave w owns the contiguous range [lo, hi) and walks it 512
  // keys at a time, eight consecutive keys per lane: count first, then a scan of the 16 wave
  // totals, then write, each lane placing its keys after those of the lanes below it.
  const int64_t span = ((n + SEL_WAVES - 1) / SEL_WAVES + 511) / 512 * 512;
  const int64_t lo = min<int64_t>(n, wv * span), hi = min<int64_t>(n, lo + span);
  auto count8 = [&](int64_t j, const u32x4_t& kk, uint32_t& g, uint32_t& t) {
    g = t = 0;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const uint32_t key = (kk[u >> 1] >> (16 * (u & 1))) & 0xffffu;
      g += j + u < hi && key > thr;
      t += j + u < hi && key == thr;
    }
  };
  uint32_t cg = 0, ct = 0;
  for (int64_t j0 = lo; j0 < hi; j0 += 512) {
    const int64_t j = j0 + 8 * lane;
    uint32_t g, t;
    count8(j, load8(j), g, t);
    cg += g;
    ct += t;
  }
  cg = wave_sum_u(cg);
  ct = wave_sum_u(ct);
  if (lane == 0) {
    s_cnt_g[wv] = cg;
    s_cnt_t[wv] = ct;
  }
  __syncthreads();
  int64_t g_run = 0, t_run = 0;
  for (int w = 0; w < wv; ++w) {
    g_run += s_cnt_g[w];
    t_run += s_cnt_t[w];
  }
  for (int64_t j0 = lo; j0 < hi; j0 += 512) {
    const int64_t j = j0 + 8 * lane;
    const u32x4_t kk = load8(j);
    // keys of the lanes below this one that are greater than / equal to the threshold: one ballot
    // per key slot, counted with mbcnt
    uint32_t bg = 0, bt = 0, tg = 0, tt = 0;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const uint32_t key = (kk[u >> 1] >> (16 * (u & 1))) & 0xffffu;
      const uint64_t mg = __ballot(j + u < hi && key > thr), mt = __ballot(j + u < hi && key == thr);
      bg += lanes_below(mg);
      bt += lanes_below(mt);
      tg += __popcll(mg);
      tt += __popcll(mt);
    }
    int64_t g = g_run + bg, t = t_run + bt;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const uint32_t key = (kk[u >> 1] >> (16 * (u & 1))) & 0xffffu;
      if (j + u < hi) {
        if (key > thr) {
          sel[g + min(t, need_ties)] = j + u;
          ++g;
        } else if (key == thr) {
          if (t < need_ties) sel[g + t] = j + u;
          ++t;
        }
      }
    }
    g_run += tg;
    t_run += tt;
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
  int64_t blocks = (n + 7) / 8;
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
  if (n > SEL_MAX_N) return fail(TREAD_ERANGE, "topk_select: n=%lld above %lld candidates", (long long)n, (long long)SEL_MAX_N);
  const size_t lds = n <= SEL_LDS_KEYS ? (size_t)(n + 7) / 8 * 16 : 0;  // whole 16-byte groups of keys
  hipLaunchKernelGGL(topk_select_kernel, dim3(1), dim3(SEL_THREADS), lds, (hipStream_t)stream, (const bf16_t*)score, n,
                     k, sel_out);
  return check_launch("topk_select");
}
