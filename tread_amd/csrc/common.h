// Shared helpers for the tread HIP kernels (gfx950 / CDNA4, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

typedef uint16_t bf16_t;  // raw bfloat16 bits in memory

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4_t;
typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u32x2_t;

namespace tread {

__device__ __forceinline__ float bf2f(bf16_t b) { return __uint_as_float(((uint32_t)b) << 16); }

typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;

// Round-to-nearest-even float -> bf16 (the rounding torch uses for every bf16 result); gfx950
// does it in one instruction (v_cvt_pk_bf16_f32), two values at a time.
__device__ __forceinline__ uint32_t pack_bf(float lo, float hi) {
  bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ bf16_t f2bf(float f) { return __builtin_bit_cast(bf16_t, (__bf16)f); }

__device__ __forceinline__ float lo_bf(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_bf(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// bf16(silu(g)) with silu(g) = g / (1 + exp(-g)) in fp32 (torch's bf16 silu: fp32 math, one rounding).
__device__ __forceinline__ float silu_bf16(float g) { return bf2f(f2bf(g / (1.0f + expf(-g)))); }

// Threads used for one row of add + RMSNorm: 256, or the row's 16-byte chunks rounded up to 64.
__host__ __device__ __forceinline__ int rmsnorm_threads(int hidden) {
  const int nch = hidden / 8;
  return nch >= 256 ? 256 : ((nch + 63) / 64) * 64;
}

// add + RMSNorm of one row by the block's threads tid < nthr (a multiple of 64; every thread of the
// block must call it, for its barriers): s = bf16(x + d) (d may be null; s goes to sum_row if not
// null), out_row = bf16(w * bf16(s * r)) with r = 1 / sqrt(mean(s^2) + eps), the rounding points
// of transformers' Qwen2RMSNorm. Thread t owns the 16-byte chunks t, t + nthr, ..., sums its
// squares in that order, and the wave totals are added in wave order (by every thread, after one
// barrier), so every caller with the same nthr gets the same bits. The weight chunks are loaded
// with the row's, so the row costs one round of memory latency. red: 32 floats of shared memory.
template <int CPT>
__device__ __forceinline__ void add_rmsnorm_row(const bf16_t* __restrict__ xr, const bf16_t* __restrict__ dr,
                                                const bf16_t* __restrict__ w, float eps, int hidden, int nthr,
                                                bf16_t* __restrict__ sum_row, bf16_t* __restrict__ out_row,
                                                float* red) {
  const int tid = threadIdx.x, nch = hidden / 8;
  const bool on = tid < nthr;
  u32x4_t v[CPT], ww[CPT];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    const int c = tid + j * nthr;
    if (on && c < nch) ww[j] = *reinterpret_cast<const u32x4_t*>(w + c * 8);
  }
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    const int c = tid + j * nthr;
    if (on && c < nch) {
      u32x4_t a = *reinterpret_cast<const u32x4_t*>(xr + c * 8);
      if (dr) {
        const u32x4_t d = *reinterpret_cast<const u32x4_t*>(dr + c * 8);
#pragma unroll
        for (int q = 0; q < 4; ++q) a[q] = pack_bf(lo_bf(a[q]) + lo_bf(d[q]), hi_bf(a[q]) + hi_bf(d[q]));
        if (sum_row) *reinterpret_cast<u32x4_t*>(sum_row + c * 8) = a;
      }
      v[j] = a;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float l = lo_bf(a[q]), h = hi_bf(a[q]);
        ss = fmaf(l, l, ss);
        ss = fmaf(h, h, ss);
      }
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
  if (on && (tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  float t = 0.f;
  for (int k = 0; k < nthr / 64; ++k) t += red[k];
  const float r = 1.0f / sqrtf(t / (float)hidden + eps);
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    const int c = tid + j * nthr;
    if (on && c < nch) {
      u32x4_t o;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float l = bf2f(f2bf(lo_bf(v[j][q]) * r)) * lo_bf(ww[j][q]);
        const float h = bf2f(f2bf(hi_bf(v[j][q]) * r)) * hi_bf(ww[j][q]);
        o[q] = pack_bf(l, h);
      }
      *reinterpret_cast<u32x4_t*>(out_row + c * 8) = o;
    }
  }
  __syncthreads();  // out_row is complete for every thread, and red may be reused by the next row
}

template <typename T>
__device__ __forceinline__ T ldg_nt(const T* p) { return __builtin_nontemporal_load(p); }
template <typename T>
__device__ __forceinline__ void stg_nt(T* p, T v) { __builtin_nontemporal_store(v, p); }

}  // namespace tread

// ---- host-side error plumbing shared by every C entry point ----
namespace tread {
void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);
int check_launch(const char* what);
}  // namespace tread

#define TREAD_EINVAL (-22)
#define TREAD_ERANGE (-34)
