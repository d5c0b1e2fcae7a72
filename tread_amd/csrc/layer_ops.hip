// Decoder-layer glue for recomputed rows: RoPE tables, q/k RoPE + cache splice, fused residual
// add + RMSNorm, and SiLU-gated product. Each follows the rounding of the torch ops it replaces
// (every bf16 torch op computes in fp32 and rounds its result to bf16 once).
#include "common.h"
#include "../../include/tread_hip.h"

namespace tread {

struct FreqArgs {
  float inv_freq[64];
};

__global__ void rope_table_kernel(const int64_t* __restrict__ pos, int64_t n, int half, const FreqArgs f,
                                  bf16_t* __restrict__ cos_out, bf16_t* __restrict__ sin_out) {
  int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n * half) return;
  int64_t i = t / half;
  int j = (int)(t % half);
  float ang = (float)pos[i] * f.inv_freq[j];
  float s, c;
  sincosf(ang, &s, &c);
  cos_out[t] = f2bf(c);
  sin_out[t] = f2bf(s);
}

// One work group per token row: rotate the hq q heads and hkv k heads, copy v, splice k/v.
template <int HD>
__global__ __launch_bounds__(256) void qkv_rope_splice_kernel(const bf16_t* __restrict__ qs, const bf16_t* __restrict__ ks,
                                                              const bf16_t* __restrict__ vs, int64_t ld,
                                                              const bf16_t* __restrict__ cosb,
                                                              const bf16_t* __restrict__ sinb,
                                                              const int64_t* __restrict__ rows, int hq, int hkv,
                                                              bf16_t* __restrict__ q_out, bf16_t* __restrict__ kc,
                                                              bf16_t* __restrict__ vc, int64_t t_cap) {
  constexpr int HALF = HD / 2;
  constexpr int PG = HALF / 8;  // pair groups per head
  const int64_t i = blockIdx.x;
  const int64_t row = rows[i];
  const bool row_ok = row >= 0 && row < t_cap;  // out-of-range rows splice nothing
  const bf16_t* cs = cosb + i * HALF;
  const bf16_t* sn = sinb + i * HALF;
  const int nq = q_out ? hq : 0;
  const int tasks = (nq + hkv) * PG;
  for (int t = threadIdx.x; t < tasks; t += blockDim.x) {
    int h = t / PG, c = (t % PG) * 8;
    const bf16_t* src;
    bf16_t* dst;
    if (h < nq) {
      src = qs + i * ld + h * HD;
      dst = q_out + (i * hq + h) * HD;
    } else {
      if (!row_ok) continue;
      int kh = h - nq;
      src = ks + i * ld + kh * HD;
      dst = kc + ((int64_t)kh * t_cap + row) * HD;
    }
    u32x4_t x1 = *reinterpret_cast<const u32x4_t*>(src + c);
    u32x4_t x2 = *reinterpret_cast<const u32x4_t*>(src + c + HALF);
    u32x4_t cw = *reinterpret_cast<const u32x4_t*>(cs + c);
    u32x4_t sw = *reinterpret_cast<const u32x4_t*>(sn + c);
    u32x4_t o1, o2;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      float r[2][2];
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        float a = p ? hi_bf(x1[w]) : lo_bf(x1[w]);
        float b = p ? hi_bf(x2[w]) : lo_bf(x2[w]);
        float co = p ? hi_bf(cw[w]) : lo_bf(cw[w]);
        float si = p ? hi_bf(sw[w]) : lo_bf(sw[w]);
        r[0][p] = bf2f(f2bf(a * co)) + bf2f(f2bf(-b * si));
        r[1][p] = bf2f(f2bf(b * co)) + bf2f(f2bf(a * si));
      }
      o1[w] = pack_bf(r[0][0], r[0][1]);
      o2[w] = pack_bf(r[1][0], r[1][1]);
    }
    *reinterpret_cast<u32x4_t*>(dst + c) = o1;
    *reinterpret_cast<u32x4_t*>(dst + c + HALF) = o2;
  }
  const int vt = row_ok ? hkv * (HD / 8) : 0;
  for (int t = threadIdx.x; t < vt; t += blockDim.x) {
    int h = t / (HD / 8), c = (t % (HD / 8)) * 8;
    *reinterpret_cast<u32x4_t*>(vc + ((int64_t)h * t_cap + row) * HD + c) =
        *reinterpret_cast<const u32x4_t*>(vs + i * ld + h * HD + c);
  }
}

// One work group per row. CPT 16-byte chunks per thread kept in registers between the two passes.
template <int CPT>
__global__ void add_rmsnorm_kernel(const bf16_t* __restrict__ x, const bf16_t* __restrict__ delta,
                                   const bf16_t* __restrict__ w, float eps, int hidden, bf16_t* __restrict__ sum_out,
                                   bf16_t* __restrict__ norm_out) {
  __shared__ float red[32];
  const int64_t i = blockIdx.x;
  add_rmsnorm_row<CPT>(x + i * hidden, delta ? delta + i * hidden : nullptr, w, eps, hidden, blockDim.x,
                       sum_out && delta ? sum_out + i * hidden : nullptr, norm_out + i * hidden, red);
}

__global__ void silu_mul_kernel(const bf16_t* __restrict__ gu, int64_t n, int inter, bf16_t* __restrict__ out) {
  const int64_t per_row = inter / 8;
  const int64_t total = n * per_row;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
    int64_t i = t / per_row, c = (t % per_row) * 8;
    u32x4_t g = *reinterpret_cast<const u32x4_t*>(gu + i * 2 * inter + c);
    u32x4_t u = *reinterpret_cast<const u32x4_t*>(gu + i * 2 * inter + inter + c);
    u32x4_t o;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float gl = lo_bf(g[q]), gh = hi_bf(g[q]);
      float sl = silu_bf16(gl);
      float sh = silu_bf16(gh);
      o[q] = pack_bf(sl * lo_bf(u[q]), sh * hi_bf(u[q]));
    }
    *reinterpret_cast<u32x4_t*>(out + i * inter + c) = o;
  }
}

}  // namespace tread

using namespace tread;

extern "C" int tread_rope_table_bf16(const int64_t* pos, int64_t n, const float* inv_freq, int head_dim, void* cos_out,
                                     void* sin_out, tread_stream_t stream) {
  if (n == 0) return 0;
  if (n < 0 || !pos || !inv_freq || !cos_out || !sin_out) return fail(TREAD_EINVAL, "rope_table: bad arguments");
  if (head_dim <= 0 || head_dim > 128 || (head_dim % 16) != 0) return fail(TREAD_EINVAL, "rope_table: bad head_dim %d", head_dim);
  FreqArgs f;
  memset(&f, 0, sizeof(f));
  for (int j = 0; j < head_dim / 2; ++j) f.inv_freq[j] = inv_freq[j];
  int64_t total = n * (head_dim / 2);
  int64_t blocks = (total + 255) / 256;
  if (blocks > 0x7fffffffLL) return fail(TREAD_ERANGE, "rope_table: n too large");
  hipLaunchKernelGGL(rope_table_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, pos, n, head_dim / 2, f,
                     (bf16_t*)cos_out, (bf16_t*)sin_out);
  return check_launch("rope_table");
}

extern "C" int tread_qkv_rope_splice_bf16(const void* q_src, const void* k_src, const void* v_src, int64_t ld,
                                          const void* cos, const void* sin, const int64_t* rows, int64_t n, int hq,
                                          int hkv, int head_dim, void* q_out, void* k_cache, void* v_cache,
                                          int64_t t_cap, tread_stream_t stream) {
  if (n == 0) return 0;
  if (n < 0 || hkv <= 0 || hq < 0 || t_cap <= 0) return fail(TREAD_EINVAL, "qkv_rope_splice: bad shape");
  if (!k_src || !v_src || !cos || !sin || !rows || !k_cache || !v_cache || (q_out && !q_src))
    return fail(TREAD_EINVAL, "qkv_rope_splice: null pointer");
  if (head_dim != 64 && head_dim != 128) return fail(TREAD_EINVAL, "qkv_rope_splice: head_dim %d not in {64,128}", head_dim);
  if ((ld % 8) != 0) return fail(TREAD_EINVAL, "qkv_rope_splice: row stride %lld not a multiple of 8", (long long)ld);
  if (((uintptr_t)k_src | (uintptr_t)v_src | (uintptr_t)(q_out ? q_src : k_src)) & 15)
    return fail(TREAD_EINVAL, "qkv_rope_splice: sources not 16-byte aligned");
  if (n > 0x7fffffffLL) return fail(TREAD_ERANGE, "qkv_rope_splice: n too large");
  if (head_dim == 128)
    hipLaunchKernelGGL(qkv_rope_splice_kernel<128>, dim3((unsigned)n), dim3(256), 0, (hipStream_t)stream,
                       (const bf16_t*)q_src, (const bf16_t*)k_src, (const bf16_t*)v_src, ld, (const bf16_t*)cos,
                       (const bf16_t*)sin, rows, hq, hkv, (bf16_t*)q_out, (bf16_t*)k_cache, (bf16_t*)v_cache, t_cap);
  else
    hipLaunchKernelGGL(qkv_rope_splice_kernel<64>, dim3((unsigned)n), dim3(256), 0, (hipStream_t)stream,
                       (const bf16_t*)q_src, (const bf16_t*)k_src, (const bf16_t*)v_src, ld, (const bf16_t*)cos,
                       (const bf16_t*)sin, rows, hq, hkv, (bf16_t*)q_out, (bf16_t*)k_cache, (bf16_t*)v_cache, t_cap);
  return check_launch("qkv_rope_splice");
}

extern "C" int tread_add_rmsnorm_bf16(const void* x, const void* delta, const void* weight, float eps, int64_t n,
                                      int hidden, void* sum_out, void* norm_out, tread_stream_t stream) {
  if (n == 0) return 0;
  if (n < 0 || !x || !weight || !norm_out) return fail(TREAD_EINVAL, "add_rmsnorm: bad arguments");
  if (hidden <= 0 || (hidden % 8) != 0 || hidden > 16384)
    return fail(TREAD_EINVAL, "add_rmsnorm: hidden %d must be a multiple of 8 and <= 16384", hidden);
  if (n > 0x7fffffffLL) return fail(TREAD_ERANGE, "add_rmsnorm: n too large");
  int nch = hidden / 8;
  int threads = rmsnorm_threads(hidden);
  int cpt = (nch + threads - 1) / threads;
  dim3 g((unsigned)n), b(threads);
  hipStream_t s = (hipStream_t)stream;
  const bf16_t *px = (const bf16_t*)x, *pd = (const bf16_t*)delta, *pw = (const bf16_t*)weight;
  bf16_t *ps = (bf16_t*)sum_out, *pn = (bf16_t*)norm_out;
  if (cpt <= 1)
    hipLaunchKernelGGL(add_rmsnorm_kernel<1>, g, b, 0, s, px, pd, pw, eps, hidden, ps, pn);
  else if (cpt <= 2)
    hipLaunchKernelGGL(add_rmsnorm_kernel<2>, g, b, 0, s, px, pd, pw, eps, hidden, ps, pn);
  else if (cpt <= 4)
    hipLaunchKernelGGL(add_rmsnorm_kernel<4>, g, b, 0, s, px, pd, pw, eps, hidden, ps, pn);
  else
    hipLaunchKernelGGL(add_rmsnorm_kernel<8>, g, b, 0, s, px, pd, pw, eps, hidden, ps, pn);
  return check_launch("add_rmsnorm");
}

extern "C" int tread_silu_mul_bf16(const void* gate_up, int64_t n, int inter, void* out, tread_stream_t stream) {
  if (n == 0) return 0;
  if (n < 0 || !gate_up || !out || inter <= 0 || (inter % 8) != 0) return fail(TREAD_EINVAL, "silu_mul: bad arguments");
  int64_t total = n * (inter / 8);
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, (const bf16_t*)gate_up, n,
                     inter, (bf16_t*)out);
  return check_launch("silu_mul");
}
