// Linear layers of a few token rows (decode steps): y[M, N] = x[M, K] . W[N, K]^T (+ b[N]), bf16 in
// and out, fp32 accumulation, M <= 32. Memory-bound: every weight byte is read once from HBM, so
// the kernel is built to keep enough 16-byte weight loads in flight.
//
// One work group of 8 waves per TN = 32 (or 16) output features. Each wave walks its 1/8 of K with
// v_mfma_f32_32x32x16_bf16: A = 32 weight rows x 16 K (lane l: row l % 32, 8 consecutive K at
// (l / 32) * 8 -- one 16-byte load), B = the token rows as columns (lane l: token l % 32, the same
// 8 K; tokens >= M load nothing and stay zero); with TN = 16 the same with v_mfma_f32_16x16x32_bf16
// (lane l: row / token l % 16, K at (l / 16) * 8 of a 32-K step). The 8 partial TN x TN tiles meet
// in LDS, and one thread per (token, feature) sums them, adds the bias and rounds once to bf16 (as
// F.linear does). A layer with few output features (fewer than 448 such work groups) and a long K
// also splits K across 2, 4 or 8 work groups per tile: their fp32 sums meet in a workspace, and a
// second small kernel adds them and the bias and rounds once.
#include <type_traits>

#include "common.h"
#include "../../include/tread_hip.h"

namespace tread {

constexpr int SK_WAVES = 8;
constexpr int SK_U = 4;  // MFMA K steps whose loads are issued together

enum { PRO_NONE = 0, PRO_NORM = 1, PRO_SILU = 2 };

struct SkinnyArgs {
  const bf16_t* x;  // PRO_NONE: the rows; PRO_NORM: residual rows h; PRO_SILU: gate|up rows
  int64_t ldx;
  const bf16_t* delta;  // PRO_NORM: added to h (may be null), rows ldx apart
  const bf16_t* lnw;    // PRO_NORM: RMSNorm weight
  float eps;
  bf16_t* h_out;        // PRO_NORM: h + delta, [M, K] contiguous (may be null)
  int64_t inter;        // PRO_SILU: u of column k sits at column inter + k
  const bf16_t* w;
  const bf16_t* bias;
  bf16_t* y;
  int64_t ldy;
  float* part;
  int M, K, N;
  // EPI_SWIGLU: gate|up of an MLP (N = 2 inter, the weight's rows [gate; up]): y [M, inter] =
  // bf16(bf16(silu(g)) * u) with g, u rounded to bf16 first (silu_mul's bits)
  // EPI_ROPE: q|k|v of a decoder layer (N = (hq + 2 hkv) hd): q and k rotated (cos / sin [M, hd / 2])
  // into q_out [M, hq, hd] and k_cache, v into v_cache, row rows[m] of each [hkv, t_cap, hd] cache
  const bf16_t* cosb;
  const bf16_t* sinb;
  const int64_t* rows;
  bf16_t* q_out;
  bf16_t* k_cache;
  bf16_t* v_cache;
  int64_t t_cap;
  int hq, hkv, hd;
};

enum { EPI_PLAIN = 0, EPI_ROPE = 1, EPI_SWIGLU = 2 };

// blockIdx.y = q selects the K slice [q K / ks, (q + 1) K / ks); with ks > 1 the slice's fp32 sums
// go to part[q][m][n] and skinny_reduce_kernel finishes them.
// PRO_NORM stages norm(h + delta) of the M rows in LDS first (add_rmsnorm_row: the same bits as
// the stand-alone add + RMSNorm kernel) and work group (0, 0) writes h + delta to h_out; PRO_SILU
// stages this work group's K slice of bf16(bf16(silu(g)) * u) (the same bits as silu_mul_kernel).
// EPI_ROPE (with PRO_NORM, unsplit): a q or k head's tile p holds the feature pairs (d, d + hd / 2)
// for d in [p TN / 2, (p + 1) TN / 2), so that the epilogue rotates each pair in place with the
// rounding points of qkv_rope_splice_kernel (transformers' apply_rotary_pos_emb in bf16) and writes
// q and the cache rows itself; v heads keep their features in order.
template <int PRO, int CPT, int TN, int EPI = EPI_PLAIN>
__global__ __launch_bounds__(SK_WAVES * 64) void skinny_gemm_kernel(const SkinnyArgs a) {
  static_assert(TN == 32 || TN == 16, "tile of 32 or 16 features");
  constexpr int KSTEP = 512 / TN;     // K per MFMA: 16 (32 x 32 x 16) or 32 (16 x 16 x 32)
  constexpr int NACC = TN * TN / 64;  // accumulator registers per lane
  using acc_t = std::conditional_t<TN == 32, f32x16_t, f32x4_t>;
  extern __shared__ __align__(16) bf16_t xs[];  // staged operand rows (PRO_NORM / PRO_SILU)
  __shared__ float red[SK_WAVES][NACC][64];
  __shared__ float nred[32];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int rt = lane % TN, kg = lane / TN;  // weight row and token of the tile; group of 8 K
  const int M = a.M, K = a.K;
  const int64_t n0 = (int64_t)blockIdx.x * TN;
  const int ks = gridDim.y, q = blockIdx.y;
  const int kslice = K / ks, k0 = q * kslice;
  const int kw = kslice / SK_WAVES;  // a multiple of KSTEP
  const int kb = k0 + wv * kw + kg * 8;  // this lane's first K
  // weight row of tile row rt
  int64_t wrow = n0 + rt;
  if constexpr (EPI == EPI_ROPE) {
    const int tph = a.hd / TN, hh = blockIdx.x / tph, p = blockIdx.x % tph;
    if (hh < a.hq + a.hkv)
      wrow = (int64_t)hh * a.hd + (rt < TN / 2 ? p * (TN / 2) + rt : a.hd / 2 + p * (TN / 2) + rt - TN / 2);
  } else if constexpr (EPI == EPI_SWIGLU) {  // tile p: gate rows then the matching up rows
    const int64_t j0 = (int64_t)blockIdx.x * (TN / 2);
    wrow = rt < TN / 2 ? j0 + rt : a.inter + j0 + rt - TN / 2;
  }
  const bf16_t* wp = a.w + wrow * (int64_t)K + kb;
  const bool xon = rt < M;
  const int xrow = xon ? rt : 0;
  const u32x4_t zero = {0u, 0u, 0u, 0u};
  acc_t acc = {};
  const int steps = kw / KSTEP;
  auto mma = [](u32x4_t av, u32x4_t bv, acc_t c) {
    if constexpr (TN == 32)
      return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, av), __builtin_bit_cast(bf16x8_t, bv),
                                                     c, 0, 0, 0);
    else
      return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, av), __builtin_bit_cast(bf16x8_t, bv),
                                                     c, 0, 0, 0);
  };

  auto mainloop = [&](const bf16_t* xp) {
    int s = 0;
    for (; s + SK_U <= steps; s += SK_U) {
      u32x4_t av[SK_U], bv[SK_U];
#pragma unroll
      for (int u = 0; u < SK_U; ++u) av[u] = *reinterpret_cast<const u32x4_t*>(wp + (s + u) * KSTEP);
#pragma unroll
      for (int u = 0; u < SK_U; ++u) bv[u] = xon ? *reinterpret_cast<const u32x4_t*>(xp + (s + u) * KSTEP) : zero;
#pragma unroll
      for (int u = 0; u < SK_U; ++u) acc = mma(av[u], bv[u], acc);
    }
    for (; s < steps; ++s) {
      const u32x4_t av = *reinterpret_cast<const u32x4_t*>(wp + s * KSTEP);
      const u32x4_t bv = xon ? *reinterpret_cast<const u32x4_t*>(xp + s * KSTEP) : zero;
      acc = mma(av, bv, acc);
    }
  };

  if constexpr (PRO == PRO_NONE) {
    mainloop(a.x + (int64_t)xrow * a.ldx + kb);
  } else if constexpr (PRO == PRO_NORM) {  // K is the hidden size, ks == 1
    const int nthr = rmsnorm_threads(K);
    const bool writer = a.h_out && blockIdx.x == 0 && blockIdx.y == 0;
    for (int m = 0; m < M; ++m)
      add_rmsnorm_row<CPT>(a.x + m * a.ldx, a.delta ? a.delta + m * a.ldx : nullptr, a.lnw, a.eps, K, nthr,
                           writer ? a.h_out + (int64_t)m * K : nullptr, xs + m * K, nred);
    mainloop(xs + xrow * K + (kb - k0));
  } else {
    const int cpr = kslice / 8;  // 16-byte chunks per staged row
    for (int c = threadIdx.x; c < M * cpr; c += SK_WAVES * 64) {
      const int m = c / cpr, kk = (c % cpr) * 8;
      const bf16_t* gr = a.x + m * a.ldx + k0 + kk;
      const u32x4_t g = *reinterpret_cast<const u32x4_t*>(gr);
      const u32x4_t u = *reinterpret_cast<const u32x4_t*>(gr + a.inter);
      u32x4_t o;
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = pack_bf(silu_bf16(lo_bf(g[j])) * lo_bf(u[j]), silu_bf16(hi_bf(g[j])) * hi_bf(u[j]));
      *reinterpret_cast<u32x4_t*>(xs + m * kslice + kk) = o;
    }
    __syncthreads();
    mainloop(xs + xrow * kslice + (kb - k0));
  }
#pragma unroll
  for (int r = 0; r < NACC; ++r) red[wv][r][lane] = acc[r];
  __syncthreads();
  // C layout: lane l holds column (token) l % TN; register r holds row (r / 4) * 8 + (l / 32) * 4 + r % 4
  // of the 32 x 32 tile, row (l / 16) * 4 + r of the 16 x 16 tile
  auto tile_sum = [&](int m, int row) {
    const int r = TN == 32 ? (row >> 3) * 4 + (row & 3) : (row & 3);
    const int ln = TN == 32 ? m + 32 * ((row >> 2) & 1) : m + 16 * (row >> 2);
    float v = 0.f;
#pragma unroll
    for (int p = 0; p < SK_WAVES; ++p) v += red[p][r][ln];
    return v;
  };
  if constexpr (EPI == EPI_ROPE) {
    const int tph = a.hd / TN, hh = blockIdx.x / tph, p = blockIdx.x % tph, half_hd = a.hd / 2;
    if (hh < a.hq + a.hkv) {  // q or k: rotate each (d, d + hd / 2) pair
      for (int t = threadIdx.x; t < (TN / 2) * M; t += SK_WAVES * 64) {
        const int m = t / (TN / 2), pr = t % (TN / 2), d = p * (TN / 2) + pr;
        const int64_t f = (int64_t)hh * a.hd + d;
        float lo = tile_sum(m, pr), hi = tile_sum(m, pr + TN / 2);
        if (a.bias) {
          lo += bf2f(a.bias[f]);
          hi += bf2f(a.bias[f + half_hd]);
        }
        const float x1 = bf2f(f2bf(lo)), x2 = bf2f(f2bf(hi));
        const float co = bf2f(a.cosb[(int64_t)m * half_hd + d]), si = bf2f(a.sinb[(int64_t)m * half_hd + d]);
        const bf16_t o1 = f2bf(bf2f(f2bf(x1 * co)) + bf2f(f2bf(-x2 * si)));
        const bf16_t o2 = f2bf(bf2f(f2bf(x2 * co)) + bf2f(f2bf(x1 * si)));
        bf16_t* dst;
        if (hh < a.hq) {
          dst = a.q_out + ((int64_t)m * a.hq + hh) * a.hd;
        } else {
          const int64_t row = a.rows[m];
          if (row < 0 || row >= a.t_cap) continue;  // out-of-range rows splice nothing
          dst = a.k_cache + ((int64_t)(hh - a.hq) * a.t_cap + row) * a.hd;
        }
        dst[d] = o1;
        dst[d + half_hd] = o2;
      }
    } else {  // v: into the cache unrotated
      for (int t = threadIdx.x; t < TN * M; t += SK_WAVES * 64) {
        const int m = t / TN, row = t % TN;
        const int64_t crow = a.rows[m];
        if (crow < 0 || crow >= a.t_cap) continue;
        float v = tile_sum(m, row);
        if (a.bias) v += bf2f(a.bias[n0 + row]);
        a.v_cache[((int64_t)(hh - a.hq - a.hkv) * a.t_cap + crow) * a.hd + p * TN + row] = f2bf(v);
      }
    }
    return;
  }
  if constexpr (EPI == EPI_SWIGLU) {
    for (int t = threadIdx.x; t < (TN / 2) * M; t += SK_WAVES * 64) {
      const int m = t / (TN / 2), pr = t % (TN / 2);
      const int64_t j = (int64_t)blockIdx.x * (TN / 2) + pr;
      float g = tile_sum(m, pr), u = tile_sum(m, pr + TN / 2);
      if (a.bias) {
        g += bf2f(a.bias[j]);
        u += bf2f(a.bias[a.inter + j]);
      }
      a.y[(int64_t)m * a.inter + j] = f2bf(silu_bf16(bf2f(f2bf(g))) * bf2f(f2bf(u)));
    }
    return;
  }
  for (int t = threadIdx.x; t < TN * M; t += SK_WAVES * 64) {
    const int m = t / TN, row = t % TN;
    float v = tile_sum(m, row);
    if (ks > 1) {
      a.part[((int64_t)q * M + m) * a.N + n0 + row] = v;
    } else {
      if (a.bias) v += bf2f(a.bias[n0 + row]);
      a.y[(int64_t)m * a.ldy + n0 + row] = f2bf(v);
    }
  }
}

__global__ __launch_bounds__(256) void skinny_reduce_kernel(const float* __restrict__ part, int ks, int M, int N,
                                                            const bf16_t* __restrict__ bias, bf16_t* __restrict__ y,
                                                            int64_t ldy) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= (int64_t)M * N) return;
  const int m = (int)(t / N), n = (int)(t % N);
  float v = 0.f;
  for (int q = 0; q < ks; ++q) v += part[((int64_t)q * M + m) * N + n];
  if (bias) v += bf2f(bias[n]);
  y[(int64_t)m * ldy + n] = f2bf(v);
}

// One row (a decoding step): one weight row per wave. The MFMA tiles above read 16-32 weight rows
// per wave in 64-byte pieces, which spreads HBM traffic over tens of thousands of short streams;
// at one row, streaming whole rows is faster on every decode shape (7B, weights from HBM, one
// process: gate|up 52.5 -> 43.9 us, down 29.1 -> 23.8, o 11.7 -> 7.5, q|k|v 13.1 -> 8.4). A work
// group of 8 waves stages the operand row in LDS (the same prologues as the tiles: add + RMSNorm
// or SiLU gating, the same bits), then in each of its rpw passes every wave streams one weight row
// (lane l takes the 16-byte chunks l, l + 64, ..., GV_U loads in flight), sums its fp32 products
// in chunk order, reduces across the wave and adds the bias before the one rounding. EPI_ROPE: a
// pass's 8 rows are 4 (d, d + hd/2) pairs of a q or k head, rotated together once the passes are
// done, or 8 rows of a v head, written to the cache directly.
constexpr int GV_WAVES = 8;
// 16-byte loads in flight per lane: 7, one batch for a 3 584-wide operand row (7B decoding step:
// 3.51 ms with 7, 3.54 with 4 plus the first batch queued before the prologue, 3.61 with 2; 8
// leaves the 7-chunk rows to the one-chunk tail loop, 3.81; later, 7 with the first batch queued
// before the prologue: 3.33 against 3.30)
constexpr int GV_U = 7;
constexpr int GV_MAX_RPW = 8;

// Adds to acc the fp32 products of lane's 16-byte chunks b + lane, b + lane + 64, ... (GV_U of
// them) of a weight row with the operand row xs (in LDS), in that order. The weight row is read
// through a buffer resource over it (wrs, range K * 2 bytes). FULL: every chunk lies in the row.
// Otherwise (the row's last batch) load steps wholly past the row are skipped, the same for every
// lane, and in the step that straddles its end a lane's chunk past it reads zeros instead of
// faulting and a select leaves it out: the sum has the bits of one over the row's chunks alone.
// The range check covers the whole offset, the immediate part the compiler folds the steps'
// 1 024-byte strides into included (probed on gfx950: a load at register offset 0 + immediate
// 1 024 through a 16-byte resource returns zeros), so nothing past the row is read.
// Rows whose length is no multiple of 448 chunks thereby end with one batch of loads rather than
// a loop of single loads, each waiting for the last (decoding step 0.927 -> 0.860 ms for 0.5B
// shapes, whose 896-wide rows take 2 chunks per lane, 1.55 -> 1.45 ms for 1.5B, 3.32 -> 3.31 for
// 7B). Only the FULL batches keep their loads' waits staged: in the last one the compiler waits
// for all of them at once, after the skips.
template <bool FULL>
__device__ __forceinline__ float gv_chunks(__amdgpu_buffer_rsrc_t wrs, const bf16_t* xs, int b, int lane, int nch,
                                           float acc) {
  u32x4_t av[GV_U];
#pragma unroll
  for (int u = 0; u < GV_U; ++u)
    if (FULL || b + 64 * u < nch)  // aux 2: slc, non-temporal (each weight is read once per step)
      av[u] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(wrs, (b + lane + 64 * u) * 16, 0, 2));
#pragma unroll
  for (int u = 0; u < GV_U; ++u) {
    if (!FULL && b + 64 * u >= nch) break;
    const int c = b + lane + 64 * u;
    const u32x4_t bv = *reinterpret_cast<const u32x4_t*>(xs + (FULL ? c : min(c, nch - 1)) * 8);
    float t = acc;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      t = fmaf(lo_bf(av[u][q]), lo_bf(bv[q]), t);
      t = fmaf(hi_bf(av[u][q]), hi_bf(bv[q]), t);
    }
    acc = FULL || c < nch ? t : acc;
  }
  return acc;
}

template <int PRO, int CPT, int EPI>
// Eight waves per SIMD (at most 64 VGPRs) unless the norm prologue holds more of the row per
// thread: the compiler's own choice (98-108 VGPRs, four waves) left the streams too few in flight
// (7B decoding step 3.90 -> 3.55 ms with the cap).
__global__ __launch_bounds__(GV_WAVES * 64) __attribute__((amdgpu_waves_per_eu(CPT >= 8 ? 4 : CPT >= 4 ? 6 : 8, 8)))
void gemv_kernel(const SkinnyArgs a, int rpw) {
  extern __shared__ __align__(16) bf16_t xs[];  // the operand row [K]
  __shared__ float nred[32];
  __shared__ float sums[GV_MAX_RPW][GV_WAVES];  // EPI_ROPE / EPI_SWIGLU: the passes' row sums (bias added)
  // wv in a scalar register: the weight row, and the buffer resource over it, are the wave's own
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int K = a.K, nch = K / 8;
  const int gph = EPI == EPI_ROPE ? a.hd / GV_WAVES : 1;  // passes per head (EPI_ROPE)
  // weight row of this wave in pass r (-1: past the last row)
  auto row_of = [&](int r, int& hh) -> int64_t {
    const int gi = blockIdx.x * rpw + r;
    hh = 0;
    if constexpr (EPI == EPI_ROPE) {
      hh = gi / gph;
      const int j = gi % gph;
      if (hh >= a.hq + 2 * a.hkv) return -1;
      if (hh < a.hq + a.hkv) return (int64_t)hh * a.hd + (wv < 4 ? j * 4 + wv : a.hd / 2 + j * 4 + wv - 4);
      return (int64_t)hh * a.hd + j * GV_WAVES + wv;
    } else if constexpr (EPI == EPI_SWIGLU) {  // pass gi: gate rows 4 gi .. 4 gi + 3, then their up rows
      const int64_t j = (int64_t)gi * 4;
      if (j >= a.inter) return -1;
      return wv < 4 ? j + wv : a.inter + j + wv - 4;
    } else {
      const int64_t row = (int64_t)gi * GV_WAVES + wv;
      return row < a.N ? row : -1;
    }
  };
  if constexpr (PRO == PRO_NONE) {
    for (int c = threadIdx.x; c < nch; c += GV_WAVES * 64)
      *reinterpret_cast<u32x4_t*>(xs + c * 8) = *reinterpret_cast<const u32x4_t*>(a.x + c * 8);
    __syncthreads();
  } else if constexpr (PRO == PRO_NORM) {
    // ends with a barrier; work group 0 writes h + delta
    add_rmsnorm_row<CPT>(a.x, a.delta, a.lnw, a.eps, K, rmsnorm_threads(K), blockIdx.x == 0 ? a.h_out : nullptr, xs,
                         nred);
  } else {
    for (int c = threadIdx.x; c < nch; c += GV_WAVES * 64) {
      const u32x4_t g = *reinterpret_cast<const u32x4_t*>(a.x + c * 8);
      const u32x4_t u = *reinterpret_cast<const u32x4_t*>(a.x + a.inter + c * 8);
      u32x4_t o;
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = pack_bf(silu_bf16(lo_bf(g[j])) * lo_bf(u[j]), silu_bf16(hi_bf(g[j])) * hi_bf(u[j]));
      *reinterpret_cast<u32x4_t*>(xs + c * 8) = o;
    }
    __syncthreads();
  }
  for (int r = 0; r < rpw; ++r) {
    int hh;
    const int64_t row = row_of(r, hh);
    if (row < 0) break;
    // 0x00020000: dword 3 of a gfx9 raw buffer resource (32-bit data format, untyped loads)
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc((void*)(a.w + row * K), 0, K * 2, 0x00020000);
    float acc = 0.f;
    int b = 0;  // chunks of the row before this batch (the same for every lane)
    for (; b + 64 * GV_U <= nch; b += 64 * GV_U) acc = gv_chunks<true>(wrs, xs, b, lane, nch, acc);
    if (b < nch) acc = gv_chunks<false>(wrs, xs, b, lane, nch, acc);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) acc += __shfl_xor(acc, o);
    if (a.bias) acc += bf2f(a.bias[row]);
    if constexpr (EPI == EPI_ROPE) {
      if (hh < a.hq + a.hkv) {
        if (lane == 0) sums[r][wv] = acc;
      } else if (lane == 0) {
        const int64_t crow = a.rows[0];
        if (crow >= 0 && crow < a.t_cap)
          a.v_cache[((int64_t)(hh - a.hq - a.hkv) * a.t_cap + crow) * a.hd + (row - (int64_t)hh * a.hd)] = f2bf(acc);
      }
    } else if constexpr (EPI == EPI_SWIGLU) {
      if (lane == 0) sums[r][wv] = acc;
    } else {
      if (lane == 0) a.y[row] = f2bf(acc);
    }
  }
  if constexpr (EPI == EPI_SWIGLU) {
    __syncthreads();
    for (int t = threadIdx.x; t < rpw * 4; t += GV_WAVES * 64) {
      const int r = t / 4, w = t % 4;
      const int64_t j = (int64_t)(blockIdx.x * rpw + r) * 4 + w;
      if (j >= a.inter) continue;
      a.y[j] = f2bf(silu_bf16(bf2f(f2bf(sums[r][w]))) * bf2f(f2bf(sums[r][w + 4])));
    }
  }
  if constexpr (EPI == EPI_ROPE) {
    __syncthreads();
    const int half_hd = a.hd / 2;
    for (int t = threadIdx.x; t < rpw * 4; t += GV_WAVES * 64) {
      const int r = t / 4, w = t % 4, gi = blockIdx.x * rpw + r, hh = gi / gph;
      if (hh >= a.hq + a.hkv) continue;  // v heads (or past the last head): written already
      const int d = (gi % gph) * 4 + w;
      const float x1 = bf2f(f2bf(sums[r][w])), x2 = bf2f(f2bf(sums[r][w + 4]));
      const float co = bf2f(a.cosb[d]), si = bf2f(a.sinb[d]);
      const bf16_t o1 = f2bf(bf2f(f2bf(x1 * co)) + bf2f(f2bf(-x2 * si)));
      const bf16_t o2 = f2bf(bf2f(f2bf(x2 * co)) + bf2f(f2bf(x1 * si)));
      bf16_t* dst;
      if (hh < a.hq) {
        dst = a.q_out + (int64_t)hh * a.hd;
      } else {
        const int64_t crow = a.rows[0];
        if (crow < 0 || crow >= a.t_cap) continue;
        dst = a.k_cache + ((int64_t)(hh - a.hq) * a.t_cap + crow) * a.hd;
      }
      dst[d] = o1;
      dst[d + half_hd] = o2;
    }
  }
}

// Passes per work group of gemv_kernel (8 rows per pass): one, up to 4 096 work groups, then as
// few more as keep the launch under that (the prologue is repeated by every work group; 2 048 or
// 768 work groups measured 3-16 % slower per step, 8 192 the same). Rows shorter than 2 048 take
// at most 1 024 work groups: a pass over them is a batch of 2-3 loads per lane, short against the
// prologue (gate|up of a 0.5B step, 1 216 work groups -> 608 x 2 passes, of a 1.5B step 2 240 ->
// 560 x 4: decoding step 0.831 -> 0.803 and 1.409 -> 1.375 ms; at most 512: 0.837 and 1.425).
static int gemv_rpw(int64_t groups, int K) {
  const int64_t most = K < 2048 ? 1024 : 4096;
  int rpw = 1;
  while (rpw < GV_MAX_RPW && (groups + rpw - 1) / rpw > most) rpw *= 2;
  return rpw;
}

template <int PRO, int EPI>
static int launch_gemv(int cpt, const SkinnyArgs& a, int64_t groups, hipStream_t s) {
  const int rpw = gemv_rpw(groups, a.K);
  const dim3 grid((unsigned)((groups + rpw - 1) / rpw));
  const size_t lds = (size_t)a.K * sizeof(bf16_t);
  if constexpr (PRO == PRO_NORM) {
    if (cpt <= 1) hipLaunchKernelGGL((gemv_kernel<PRO, 1, EPI>), grid, dim3(GV_WAVES * 64), lds, s, a, rpw);
    else if (cpt <= 2) hipLaunchKernelGGL((gemv_kernel<PRO, 2, EPI>), grid, dim3(GV_WAVES * 64), lds, s, a, rpw);
    else if (cpt <= 4) hipLaunchKernelGGL((gemv_kernel<PRO, 4, EPI>), grid, dim3(GV_WAVES * 64), lds, s, a, rpw);
    else hipLaunchKernelGGL((gemv_kernel<PRO, 8, EPI>), grid, dim3(GV_WAVES * 64), lds, s, a, rpw);
  } else {
    hipLaunchKernelGGL((gemv_kernel<PRO, 1, EPI>), grid, dim3(GV_WAVES * 64), lds, s, a, rpw);
  }
  return check_launch("skinny gemv");
}

// Tile width: 16 features (twice the work groups, 64 contiguous weight bytes per row per step) for
// one or two rows and fewer than 128 tiles of 32, measured faster there at one row: 11-17 % on a 7B
// model's down projection (3 584 x 18 944, with and without the SiLU prologue) and 8 % on o
// (3 584 x 3 584); 32 elsewhere (at 144 tiles the norm prologue, repeated by twice the work groups,
// made 16 slower; so did the SiLU prologue at 4 and 8 rows). The choice depends on the shape alone,
// so the fused prologues give the plain kernel's bits.
static int skinny_tn(int64_t m, int64_t n, int64_t k) {
  return (m <= 2 && n / 32 < 128 && (k % (SK_WAVES * 32)) == 0) ? 16 : 32;
}

// K slices per tile: enough work groups to cover the GPU when the feature count is small (448 of
// the 32-feature tiles, 224 of the 16-feature ones: at one row the 224 unsplit 16-feature groups of
// a 7B down projection measured 9-20 % faster than 448 split ones plus their reduction), as long as
// every wave keeps at least 512 K (shorter slices measured slower than one work group per tile) and
// K splits into whole MFMA steps.
static int skinny_ksplit(int tn, int64_t n, int64_t k) {
  const int64_t tiles = n / tn, kstep = 512 / tn, want = tn == 16 ? 224 : 448;
  int ks = 1;
  while (ks < 8 && tiles * ks < want && (k % ((int64_t)SK_WAVES * kstep * ks * 2)) == 0 &&
         k / ((int64_t)SK_WAVES * ks * 2) >= 512)
    ks *= 2;
  return ks;
}

}  // namespace tread

using namespace tread;

template <int PRO, int CPT, int EPI = EPI_PLAIN>
static void launch_tile(int tn, dim3 grid, size_t lds, hipStream_t s, const SkinnyArgs& a) {
  if (tn == 16) hipLaunchKernelGGL((skinny_gemm_kernel<PRO, CPT, 16, EPI>), grid, dim3(SK_WAVES * 64), lds, s, a);
  else hipLaunchKernelGGL((skinny_gemm_kernel<PRO, CPT, 32, EPI>), grid, dim3(SK_WAVES * 64), lds, s, a);
}

template <int EPI>
static void launch_norm(int cpt, int tn, dim3 grid, size_t lds, hipStream_t s, const SkinnyArgs& a) {
  if (cpt <= 1) launch_tile<PRO_NORM, 1, EPI>(tn, grid, lds, s, a);
  else if (cpt <= 2) launch_tile<PRO_NORM, 2, EPI>(tn, grid, lds, s, a);
  else if (cpt <= 4) launch_tile<PRO_NORM, 4, EPI>(tn, grid, lds, s, a);
  else launch_tile<PRO_NORM, 8, EPI>(tn, grid, lds, s, a);
}

static int launch_skinny(int pro, int cpt, int tn, const SkinnyArgs& a, int ks, size_t lds, hipStream_t s) {
  const dim3 grid((unsigned)(a.N / tn), (unsigned)ks);
  if (pro == PRO_NONE) launch_tile<PRO_NONE, 1>(tn, grid, lds, s, a);
  else if (pro == PRO_SILU) launch_tile<PRO_SILU, 1>(tn, grid, lds, s, a);
  else launch_norm<EPI_PLAIN>(cpt, tn, grid, lds, s, a);
  int rc = check_launch("skinny_linear");
  if (rc || ks <= 1) return rc;
  const int64_t total = (int64_t)a.M * a.N;
  hipLaunchKernelGGL(skinny_reduce_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, (const float*)a.part,
                     ks, a.M, a.N, a.bias, a.y, a.ldy);
  return check_launch("skinny_linear");
}

// Dynamic LDS the staged operand rows may take: gfx950's 160 KiB per work group less the kernel's
// static arrays (partial tiles of the 32-feature tile, 32 KiB; norm scratch) and some headroom.
constexpr size_t SK_STAGE_MAX = 160 * 1024 - sizeof(float) * (SK_WAVES * 16 * 64 + 32) - 256;

// Dynamic LDS of gemv_kernel's operand row: 160 KiB less its static arrays and some headroom.
constexpr size_t GV_STAGE_MAX = 160 * 1024 - sizeof(float) * (GV_MAX_RPW * GV_WAVES + 32) - 256;

// K slices of the SiLU-gated projection: the plain rule, then more slices until this work group's
// staged rows fit in LDS (0: no split fits).
static int silu_ksplit(int tn, int64_t m, int64_t n, int64_t k) {
  int ks = skinny_ksplit(tn, n, k);
  while ((size_t)m * (k / ks) * sizeof(bf16_t) > SK_STAGE_MAX) {
    if (ks >= 64 || (k % ((int64_t)SK_WAVES * (512 / tn) * ks * 2)) != 0) return 0;
    ks *= 2;
  }
  return ks;
}

static int check_shape(const char* what, int64_t m, int64_t mmax, int64_t n, int64_t k) {
  if (m < 0 || m > mmax || n < 0 || k <= 0)
    return fail(TREAD_EINVAL, "%s: bad shape (m=%lld n=%lld k=%lld)", what, (long long)m, (long long)n, (long long)k);
  if ((n % 32) != 0 || (k % (SK_WAVES * 16)) != 0)
    return fail(TREAD_EINVAL, "%s: n=%lld must be a multiple of 32 and k=%lld of %d", what, (long long)n,
                (long long)k, SK_WAVES * 16);
  if (n / 16 > 0x7fffffffLL || k > 0x7fffffffLL) return fail(TREAD_ERANGE, "%s: too large", what);
  return 0;
}

extern "C" size_t tread_skinny_workspace_bytes(int64_t m, int64_t n, int64_t k) {
  if (m <= 1 || m > 32 || n <= 0 || (n % 32) != 0 || k <= 0 || (k % (SK_WAVES * 16)) != 0) return 0;
  const int ks = skinny_ksplit(skinny_tn(m, n, k), n, k);
  return ks > 1 ? (size_t)ks * m * n * sizeof(float) : 0;
}

extern "C" size_t tread_skinny_silu_workspace_bytes(int64_t m, int64_t n, int64_t inter) {
  if (m <= 1 || m > 8 || n <= 0 || (n % 32) != 0 || inter <= 0 || (inter % (SK_WAVES * 16)) != 0) return 0;
  const int ks = silu_ksplit(skinny_tn(m, n, inter), m, n, inter);
  return ks > 1 ? (size_t)ks * m * n * sizeof(float) : 0;
}

extern "C" int tread_skinny_linear_bf16(const void* x, int64_t ldx, const void* weight, const void* bias, int64_t m,
                                        int64_t n, int64_t k, void* y, int64_t ldy, void* ws, size_t ws_bytes,
                                        tread_stream_t stream) {
  if (m == 0 || n == 0) return 0;
  if (int rc = check_shape("skinny_linear", m, 32, n, k)) return rc;
  if (!x || !weight || !y) return fail(TREAD_EINVAL, "skinny_linear: null pointer");
  if (ldx < k || ldy < n || (ldx % 8) != 0) return fail(TREAD_EINVAL, "skinny_linear: bad leading dimensions");
  if ((((uintptr_t)x | (uintptr_t)weight) & 15) != 0) return fail(TREAD_EINVAL, "skinny_linear: x/weight not 16-byte aligned");
  if (m == 1 && (size_t)k * sizeof(bf16_t) > GV_STAGE_MAX)
    return fail(TREAD_EINVAL, "skinny_linear: a row of %lld does not fit in LDS", (long long)k);
  const int tn = skinny_tn(m, n, k);
  int ks = m == 1 ? 1 : skinny_ksplit(tn, n, k);
  if (ks > 1 && (!ws || ws_bytes < (size_t)ks * m * n * sizeof(float) || (((uintptr_t)ws) & 15) != 0)) ks = 1;
  SkinnyArgs a;
  memset(&a, 0, sizeof(a));
  a.x = (const bf16_t*)x;
  a.ldx = ldx;
  a.w = (const bf16_t*)weight;
  a.bias = (const bf16_t*)bias;
  a.y = (bf16_t*)y;
  a.ldy = ldy;
  a.part = (float*)ws;
  a.M = (int)m;
  a.K = (int)k;
  a.N = (int)n;
  if (m == 1) return launch_gemv<PRO_NONE, EPI_PLAIN>(1, a, n / GV_WAVES, (hipStream_t)stream);
  return launch_skinny(PRO_NONE, 1, tn, a, ks, 0, (hipStream_t)stream);
}

extern "C" int tread_skinny_norm_linear_bf16(const void* h, const void* delta, const void* ln_weight, float eps,
                                             int64_t m, int64_t n, int64_t k, const void* weight, const void* bias,
                                             void* y, void* h_out, tread_stream_t stream) {
  if (m == 0 || n == 0) return 0;
  if (int rc = check_shape("skinny_norm_linear", m, 8, n, k)) return rc;
  if (k > 16384) return fail(TREAD_EINVAL, "skinny_norm_linear: hidden %lld above 16384", (long long)k);
  if ((size_t)m * k * sizeof(bf16_t) > SK_STAGE_MAX)
    return fail(TREAD_EINVAL, "skinny_norm_linear: %lld rows of %lld do not fit in LDS", (long long)m, (long long)k);
  if (!h || !ln_weight || !weight || !y) return fail(TREAD_EINVAL, "skinny_norm_linear: null pointer");
  if ((((uintptr_t)h | (uintptr_t)delta | (uintptr_t)ln_weight | (uintptr_t)weight | (uintptr_t)h_out) & 15) != 0)
    return fail(TREAD_EINVAL, "skinny_norm_linear: operands not 16-byte aligned");
  SkinnyArgs a;
  memset(&a, 0, sizeof(a));
  a.x = (const bf16_t*)h;
  a.ldx = k;
  a.delta = (const bf16_t*)delta;
  a.lnw = (const bf16_t*)ln_weight;
  a.eps = eps;
  a.h_out = (bf16_t*)h_out;
  a.w = (const bf16_t*)weight;
  a.bias = (const bf16_t*)bias;
  a.y = (bf16_t*)y;
  a.ldy = n;
  a.M = (int)m;
  a.K = (int)k;
  a.N = (int)n;
  const int nthr = rmsnorm_threads((int)k), cpt = (int)((k / 8 + nthr - 1) / nthr);
  if (m == 1) return launch_gemv<PRO_NORM, EPI_PLAIN>(cpt, a, n / GV_WAVES, (hipStream_t)stream);
  return launch_skinny(PRO_NORM, cpt, skinny_tn(m, n, k), a, 1, (size_t)m * k * sizeof(bf16_t), (hipStream_t)stream);
}

extern "C" int tread_skinny_norm_qkv_rope_bf16(const void* h, const void* delta, const void* ln_weight, float eps,
                                               int64_t m, int64_t hidden, const void* wqkv, const void* bqkv, int hq,
                                               int hkv, int head_dim, const void* cos, const void* sin,
                                               const int64_t* rows, void* q_out, void* k_cache, void* v_cache,
                                               int64_t t_cap, void* h_out, tread_stream_t stream) {
  if (m == 0) return 0;
  if (hq <= 0 || hkv <= 0 || (head_dim != 64 && head_dim != 128) || t_cap <= 0)
    return fail(TREAD_EINVAL, "skinny_norm_qkv_rope: bad heads (hq=%d hkv=%d head_dim=%d t_cap=%lld)", hq, hkv,
                head_dim, (long long)t_cap);
  const int64_t n = (int64_t)(hq + 2 * hkv) * head_dim;
  if (int rc = check_shape("skinny_norm_qkv_rope", m, 8, n, hidden)) return rc;
  if (hidden > 16384) return fail(TREAD_EINVAL, "skinny_norm_qkv_rope: hidden %lld above 16384", (long long)hidden);
  if ((size_t)m * hidden * sizeof(bf16_t) > SK_STAGE_MAX)
    return fail(TREAD_EINVAL, "skinny_norm_qkv_rope: %lld rows of %lld do not fit in LDS", (long long)m,
                (long long)hidden);
  if (!h || !ln_weight || !wqkv || !cos || !sin || !rows || !q_out || !k_cache || !v_cache)
    return fail(TREAD_EINVAL, "skinny_norm_qkv_rope: null pointer");
  if ((((uintptr_t)h | (uintptr_t)delta | (uintptr_t)ln_weight | (uintptr_t)wqkv | (uintptr_t)h_out) & 15) != 0)
    return fail(TREAD_EINVAL, "skinny_norm_qkv_rope: operands not 16-byte aligned");
  SkinnyArgs a;
  memset(&a, 0, sizeof(a));
  a.x = (const bf16_t*)h;
  a.ldx = hidden;
  a.delta = (const bf16_t*)delta;
  a.lnw = (const bf16_t*)ln_weight;
  a.eps = eps;
  a.h_out = (bf16_t*)h_out;
  a.w = (const bf16_t*)wqkv;
  a.bias = (const bf16_t*)bqkv;
  a.M = (int)m;
  a.K = (int)hidden;
  a.N = (int)n;
  a.cosb = (const bf16_t*)cos;
  a.sinb = (const bf16_t*)sin;
  a.rows = rows;
  a.q_out = (bf16_t*)q_out;
  a.k_cache = (bf16_t*)k_cache;
  a.v_cache = (bf16_t*)v_cache;
  a.t_cap = t_cap;
  a.hq = hq;
  a.hkv = hkv;
  a.hd = head_dim;
  const int tn = skinny_tn(m, n, hidden);  // the tile skinny_norm_linear picks: the same sums
  const int nthr = rmsnorm_threads((int)hidden), cpt = (int)((hidden / 8 + nthr - 1) / nthr);
  if (m == 1) return launch_gemv<PRO_NORM, EPI_ROPE>(cpt, a, n / GV_WAVES, (hipStream_t)stream);
  launch_norm<EPI_ROPE>(cpt, tn, dim3((unsigned)(n / tn), 1), (size_t)m * hidden * sizeof(bf16_t), (hipStream_t)stream, a);
  return check_launch("skinny_norm_qkv_rope");
}

extern "C" int tread_skinny_norm_swiglu_bf16(const void* h, const void* delta, const void* ln_weight, float eps,
                                             int64_t m, int64_t hidden, const void* wgu, int64_t inter, void* y,
                                             void* h_out, tread_stream_t stream) {
  if (m == 0) return 0;
  if (inter <= 0 || (inter % 16) != 0)
    return fail(TREAD_EINVAL, "skinny_norm_swiglu: inter %lld must be a positive multiple of 16", (long long)inter);
  const int64_t n = 2 * inter;
  if (int rc = check_shape("skinny_norm_swiglu", m, 8, n, hidden)) return rc;
  if (hidden > 16384) return fail(TREAD_EINVAL, "skinny_norm_swiglu: hidden %lld above 16384", (long long)hidden);
  if ((size_t)m * hidden * sizeof(bf16_t) > SK_STAGE_MAX)
    return fail(TREAD_EINVAL, "skinny_norm_swiglu: %lld rows of %lld do not fit in LDS", (long long)m,
                (long long)hidden);
  if (!h || !ln_weight || !wgu || !y) return fail(TREAD_EINVAL, "skinny_norm_swiglu: null pointer");
  if ((((uintptr_t)h | (uintptr_t)delta | (uintptr_t)ln_weight | (uintptr_t)wgu | (uintptr_t)h_out) & 15) != 0)
    return fail(TREAD_EINVAL, "skinny_norm_swiglu: operands not 16-byte aligned");
  SkinnyArgs a;
  memset(&a, 0, sizeof(a));
  a.x = (const bf16_t*)h;
  a.ldx = hidden;
  a.delta = (const bf16_t*)delta;
  a.lnw = (const bf16_t*)ln_weight;
  a.eps = eps;
  a.h_out = (bf16_t*)h_out;
  a.w = (const bf16_t*)wgu;
  a.inter = inter;
  a.y = (bf16_t*)y;
  a.M = (int)m;
  a.K = (int)hidden;
  a.N = (int)n;
  const int tn = skinny_tn(m, n, hidden);  // the tile skinny_norm_linear picks: the same sums
  const int nthr = rmsnorm_threads((int)hidden), cpt = (int)((hidden / 8 + nthr - 1) / nthr);
  if (m == 1) return launch_gemv<PRO_NORM, EPI_SWIGLU>(cpt, a, n / GV_WAVES, (hipStream_t)stream);
  launch_norm<EPI_SWIGLU>(cpt, tn, dim3((unsigned)(n / tn), 1), (size_t)m * hidden * sizeof(bf16_t), (hipStream_t)stream, a);
  return check_launch("skinny_norm_swiglu");
}

extern "C" int tread_skinny_silu_linear_bf16(const void* gate_up, int64_t m, int64_t inter, const void* weight,
                                             int64_t n, void* y, void* ws, size_t ws_bytes, tread_stream_t stream) {
  if (m == 0 || n == 0) return 0;
  if (int rc = check_shape("skinny_silu_linear", m, 8, n, inter)) return rc;
  if (!gate_up || !weight || !y) return fail(TREAD_EINVAL, "skinny_silu_linear: null pointer");
  if ((((uintptr_t)gate_up | (uintptr_t)weight) & 15) != 0)
    return fail(TREAD_EINVAL, "skinny_silu_linear: operands not 16-byte aligned");
  if (m == 1) {
    if ((size_t)inter * sizeof(bf16_t) > GV_STAGE_MAX)
      return fail(TREAD_EINVAL, "skinny_silu_linear: a row of %lld does not fit in LDS", (long long)inter);
    SkinnyArgs a;
    memset(&a, 0, sizeof(a));
    a.x = (const bf16_t*)gate_up;
    a.inter = inter;
    a.w = (const bf16_t*)weight;
    a.y = (bf16_t*)y;
    a.M = 1;
    a.K = (int)inter;
    a.N = (int)n;
    return launch_gemv<PRO_SILU, EPI_PLAIN>(1, a, n / GV_WAVES, (hipStream_t)stream);
  }
  const int tn = skinny_tn(m, n, inter);
  const int ks = silu_ksplit(tn, m, n, inter);
  if (ks == 0) return fail(TREAD_EINVAL, "skinny_silu_linear: %lld rows of %lld do not fit in LDS", (long long)m,
                           (long long)inter);
  if (ks > 1 && (!ws || ws_bytes < (size_t)ks * m * n * sizeof(float) || (((uintptr_t)ws) & 15) != 0))
    return fail(TREAD_EINVAL, "skinny_silu_linear: needs a workspace of tread_skinny_silu_workspace_bytes() bytes");
  SkinnyArgs a;
  memset(&a, 0, sizeof(a));
  a.x = (const bf16_t*)gate_up;
  a.ldx = 2 * inter;
  a.inter = inter;
  a.w = (const bf16_t*)weight;
  a.y = (bf16_t*)y;
  a.ldy = n;
  a.part = (float*)ws;
  a.M = (int)m;
  a.K = (int)inter;
  a.N = (int)n;
  return launch_skinny(PRO_SILU, 1, tn, a, ks, (size_t)m * (inter / ks) * sizeof(bf16_t), (hipStream_t)stream);
}
