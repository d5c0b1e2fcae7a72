// Linear layers of a few token rows (decode steps): y[M, N] = x[M, K] . W[N, K]^T (+ b[N]), bf16 in
// and out, fp32 accumulation, M <= 32. Memory-bound: every weight byte is read once from HBM, so
// the kernel is built to keep enough 16-byte weight loads in flight.
//
// One work group of 8 waves per 32 output features. Each wave walks its 1/8 of K with
// v_mfma_f32_32x32x16_bf16: A = 32 weight rows x 16 K (lane l: row l % 32, 8 consecutive K at
// (l / 32) * 8 -- one 16-byte load), B = the token rows as columns (lane l: token l % 32, the same
// 8 K; tokens >= M load nothing and stay zero). The 8 partial 32 x 32 tiles meet in LDS, and one
// thread per (token, feature) sums them, adds the bias and rounds once to bf16 (as F.linear does).
#include "common.h"
#include "../../include/tread_hip.h"

namespace tread {

constexpr int SK_WAVES = 8;
constexpr int SK_ROWS = 32;  // output features per work group
constexpr int SK_U = 4;      // K steps (16 each) whose loads are issued together

__global__ __launch_bounds__(SK_WAVES * 64) void skinny_gemm_kernel(const bf16_t* __restrict__ x, int64_t ldx,
                                                                   const bf16_t* __restrict__ w,
                                                                   const bf16_t* __restrict__ bias,
                                                                   bf16_t* __restrict__ y, int64_t ldy, int M, int K) {
  __shared__ float red[SK_WAVES][16][64];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int r32 = lane & 31, half = lane >> 5;
  const int64_t n0 = (int64_t)blockIdx.x * SK_ROWS;
  const int kw = K / SK_WAVES;  // a multiple of 16
  const int kb = wv * kw + half * 8;
  const bf16_t* wp = w + (n0 + r32) * (int64_t)K + kb;
  const bool xon = r32 < M;
  const bf16_t* xp = x + (int64_t)(xon ? r32 : 0) * ldx + kb;
  const u32x4_t zero = {0u, 0u, 0u, 0u};
  f32x16_t acc = {};
  const int steps = kw / 16;
  int s = 0;
  for (; s + SK_U <= steps; s += SK_U) {
    u32x4_t a[SK_U], b[SK_U];
#pragma unroll
    for (int u = 0; u < SK_U; ++u) a[u] = *reinterpret_cast<const u32x4_t*>(wp + (s + u) * 16);
#pragma unroll
    for (int u = 0; u < SK_U; ++u) b[u] = xon ? *reinterpret_cast<const u32x4_t*>(xp + (s + u) * 16) : zero;
#pragma unroll
    for (int u = 0; u < SK_U; ++u)
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a[u]), __builtin_bit_cast(bf16x8_t, b[u]),
                                                    acc, 0, 0, 0);
  }
  for (; s < steps; ++s) {
    const u32x4_t a = *reinterpret_cast<const u32x4_t*>(wp + s * 16);
    const u32x4_t b = xon ? *reinterpret_cast<const u32x4_t*>(xp + s * 16) : zero;
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), acc,
                                                  0, 0, 0);
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) red[wv][r][lane] = acc[r];
  __syncthreads();
  // C layout: lane l holds column (token) l % 32; register r holds row (r / 4) * 8 + (l / 32) * 4 + r % 4
  for (int t = threadIdx.x; t < SK_ROWS * M; t += SK_WAVES * 64) {
    const int m = t / SK_ROWS, row = t % SK_ROWS;
    const int r = (row >> 3) * 4 + (row & 3), ln = m + 32 * ((row >> 2) & 1);
    float v = 0.f;
#pragma unroll
    for (int q = 0; q < SK_WAVES; ++q) v += red[q][r][ln];
    if (bias) v += bf2f(bias[n0 + row]);
    y[(int64_t)m * ldy + n0 + row] = f2bf(v);
  }
}

}  // namespace tread

using namespace tread;

extern "C" int tread_skinny_linear_bf16(const void* x, int64_t ldx, const void* weight, const void* bias, int64_t m,
                                        int64_t n, int64_t k, void* y, int64_t ldy, tread_stream_t stream) {
  if (m == 0 || n == 0) return 0;
  if (m < 0 || m > 32 || n < 0 || k <= 0) return fail(TREAD_EINVAL, "skinny_linear: bad shape (m=%lld n=%lld k=%lld)",
                                                      (long long)m, (long long)n, (long long)k);
  if (!x || !weight || !y) return fail(TREAD_EINVAL, "skinny_linear: null pointer");
  if ((n % SK_ROWS) != 0 || (k % (SK_WAVES * 16)) != 0)
    return fail(TREAD_EINVAL, "skinny_linear: n=%lld must be a multiple of %d and k=%lld of %d", (long long)n, SK_ROWS,
                (long long)k, SK_WAVES * 16);
  if (ldx < k || ldy < n || (ldx % 8) != 0) return fail(TREAD_EINVAL, "skinny_linear: bad leading dimensions");
  if ((((uintptr_t)x | (uintptr_t)weight) & 15) != 0) return fail(TREAD_EINVAL, "skinny_linear: x/weight not 16-byte aligned");
  if (n / SK_ROWS > 0x7fffffffLL || k > 0x7fffffffLL) return fail(TREAD_ERANGE, "skinny_linear: too large");
  hipLaunchKernelGGL(skinny_gemm_kernel, dim3((unsigned)(n / SK_ROWS)), dim3(SK_WAVES * 64), 0, (hipStream_t)stream,
                     (const bf16_t*)x, ldx, (const bf16_t*)weight, (const bf16_t*)bias, (bf16_t*)y, ldy, (int)m, (int)k);
  return check_launch("skinny_linear");
}
