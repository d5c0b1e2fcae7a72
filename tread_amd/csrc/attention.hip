// (c) Selective-recompute attention on CDNA4 MFMA (v_mfma_f32_32x32x16_bf16).
//
// Rows are (query token, query head) pairs of one KV head group: row r of KV head h is token
// r / G, query head h*G + r % G (G = hq / hkv), so the G heads that share a KV head share every
// K/V tile staged in LDS (GQA in-kernel, no repeat_kv). A work group of 8 waves owns 256 rows
// (ATT_QB 32-row query blocks per wave; one fits the register file best, 198 VGPRs and two waves
// per SIMD) and each wave computes the transposed score blocks S^T = K Q^T, so that after the
// softmax its probabilities already sit in the B-operand layout of O^T = V^T P^T: every lane
// holds one query column for both products, and the online-softmax rescale is a per-lane scalar.
// K and V tiles go from global memory straight into LDS (no register staging), row-major
// [key][d] with XOR-swizzled chunks; the A operand of the PV product (V^T) is read with gfx950's
// transposing LDS read, two 8-byte reads per lane and fragment. Tiles are
// double-buffered in LDS with one barrier per 64-key tile. The online softmax keeps a stale row
// max until it is 2^8 too small, so the O rescale runs a handful of times per row, not per tile. The key range of a work group is the union of [0, n_shared) and
// [min kseg, max kend]; the visibility predicate (key <= kend[row] and key outside the row's
// masked gap) is evaluated in registers only on tiles that cross a row's boundary.
//
// Work groups are mapped XCD-aware: the hardware deals work group ids round-robin over the 8
// XCDs, so ids are remapped such that every XCD works on one KV head at a time, longest row tiles
// first, and the K/V tiles that its CUs stream are shared through that XCD's L2.
//
// Few rows (the query forward: tens of rows over a long cache) would leave most CUs idle, so the
// key range is then split across work groups (split-K): each writes its unnormalised fp32 O and
// its running (max, sum) to a workspace, and a combine kernel merges the splits per row.
#include "common.h"
#include "../../include/tread_hip.h"

namespace tread {

constexpr int ATT_WAVES = 8;
constexpr int ATT_THREADS = ATT_WAVES * 64;
constexpr int ATT_QB = 1;                      // 32-row query blocks per wave
constexpr int ATT_BM = ATT_WAVES * 32 * ATT_QB;  // rows per work group
constexpr int ATT_BK = 64;                     // keys per tile
constexpr int N_XCD = 8;
constexpr int ATT_TARGET_WGS = 512;     // split-K when fewer (head, row tile) work groups than this
constexpr int ATT_MIN_SPLIT_KEYS = 1024;

struct AttnArgs {
  const bf16_t* q;
  const bf16_t* k;
  const bf16_t* v;
  const int64_t* kend;
  const int64_t* kseg;
  bf16_t* out;
  float* ws_o;   // split-K partial O [nsplit][hkv][tiles][BM][HD] (nsplit > 1)
  float* ws_ml;  // split-K partial (max, sum) [nsplit][hkv][tiles][BM][2]
  int64_t n_shared;
  int64_t n;
  int64_t t_cap;
  int32_t hq, hkv, G;
  int32_t tiles;  // row tiles per KV head
  int32_t xpg;    // XCDs per KV head (0: plain mapping)
  int32_t nsplit;
  int32_t split_len;  // keys per split (multiple of ATT_BK)
  float scale_log2;
};

// K and V tiles live in LDS as unpadded [key][hd] rows of 16-byte chunks, filled straight from
// global memory (global_load_lds_dwordx4: a wave's 64 x 16 B land contiguously). Bank conflicts
// are avoided by XOR-swizzling the chunk index within a row instead of padding:
//  - K: chunk j of row r sits at j ^ (r % NCH). A wave's A-operand reads take the same chunk of 32
//    consecutive rows, which then spread over every bank;
//  - V: chunk j of row r sits at j ^ fV(r), fV moving the chunk's upper bits with the low row
//    bits, so a transposing read (8 rows x 64 contiguous bytes per wave) hits each bank twice.
template <int HD>
struct AttnSmem {
  static constexpr int NCH = HD / 8;  // 16-byte chunks per row
  static constexpr int K_ELEMS = ATT_BK * HD;
  static constexpr int V_ELEMS = ATT_BK * HD;
  static constexpr int BUF = K_ELEMS + V_ELEMS;
  static __device__ __forceinline__ int k_swz(int r) { return r & (NCH - 1); }
  static __device__ __forceinline__ int v_swz(int r) {
    return HD == 128 ? ((r & 3) << 2) : (((r >> 1) & 1) << 2);
  }
};

// Transposing LDS read (ds_read_b64_tr_b16): in each group of 16 lanes, lane i receives element
// (i % 4) of the 8-byte chunks addressed by lanes 4k + i / 4, k = 0..3.
typedef __attribute__((__vector_size__(4 * sizeof(short)))) short s16x4_t;
__device__ __forceinline__ s16x4_t lds_read_tr16(const bf16_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4_t*)((__attribute__((address_space(3))) char*)(uintptr_t)p));
}

// 16 bytes per lane from global memory straight into LDS: lane l's bytes land at lds + 16 l
// (lds is wave-uniform).
__device__ __forceinline__ void lds_load16(const bf16_t* g, bf16_t* lds) {
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)(uintptr_t)lds, 16, 0, 0);
}

constexpr float ATT_RESCALE_LOG2 = 8.0f;  // keep a stale row max until it is 2^8 too small

__device__ __forceinline__ int wave_max(int v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = max(v, __shfl_xor(v, o));
  return v;
}
__device__ __forceinline__ int wave_min(int v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = min(v, __shfl_xor(v, o));
  return v;
}

template <int HD>
__global__ __launch_bounds__(ATT_THREADS) void subset_attn_kernel(const AttnArgs a) {
  using SM = AttnSmem<HD>;
  constexpr int KS = HD / 16;   // k-steps of the QK product
  constexpr int DB = HD / 32;   // 32-row d blocks of O^T
  constexpr int KCH = HD / 8;   // 16-byte chunks per K/V row
  constexpr int K_LD = ATT_BK * KCH / ATT_THREADS;  // K (and V) 16-byte chunks per thread per tile
  extern __shared__ __align__(16) bf16_t smem[];
  __shared__ int red[4][ATT_WAVES];

  // ---- work group -> (split, kv head, row tile)
  int bid = blockIdx.x, split = 0, head, td;
  if (a.nsplit > 1) {
    split = bid % a.nsplit;
    bid /= a.nsplit;
    head = bid % a.hkv;
    td = bid / a.hkv;
  } else if (a.xpg > 0) {  // XCD-aware, longest tiles first
    const int xcd = bid % N_XCD, k = bid / N_XCD;
    head = xcd / a.xpg;
    td = k * a.xpg + xcd % a.xpg;
  } else {
    head = bid % a.hkv;
    td = bid / a.hkv;
  }
  if (td >= a.tiles) return;
  const int tile = a.tiles - 1 - td;

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int c = lane & 31, half = lane >> 5;
  const int64_t R = a.n * a.G;
  const int n_shared = a.kseg ? (int)min<int64_t>(a.n_shared, a.t_cap) : 0;
  // this lane's query column in each of the wave's query blocks
  bool valid[ATT_QB];
  int64_t qi[ATT_QB];
  int qh[ATT_QB], my_end[ATT_QB], my_seg[ATT_QB];
  int vmax = -1, vmin = 0x7fffffff, smax = 0, smin = 0x7fffffff;
#pragma unroll
  for (int b = 0; b < ATT_QB; ++b) {
    const int64_t r = (int64_t)tile * ATT_BM + (wv * ATT_QB + b) * 32 + c;
    valid[b] = r < R;
    qi[b] = valid[b] ? r / a.G : 0;
    qh[b] = head * a.G + (int)(valid[b] ? r % a.G : 0);
    my_end[b] = -1;
    my_seg[b] = 0;
    if (valid[b]) {
      my_end[b] = (int)min<int64_t>(max<int64_t>(a.kend[qi[b]], -1), a.t_cap - 1);
      if (a.kseg) my_seg[b] = (int)min<int64_t>(max<int64_t>(a.kseg[qi[b]], 0), a.t_cap);
      vmax = max(vmax, my_end[b]);
      vmin = min(vmin, my_end[b]);
      smax = max(smax, my_seg[b]);
      smin = min(smin, my_seg[b]);
    }
  }

  // ---- work-group key range
  {
    vmax = wave_max(vmax);
    vmin = wave_min(vmin);
    smax = wave_max(smax);
    smin = wave_min(smin);
    if (lane == 0) {
      red[0][wv] = vmax;
      red[1][wv] = vmin;
      red[2][wv] = smax;
      red[3][wv] = smin;
    }
  }
  __syncthreads();
  int kmax = red[0][0], kmin = red[1][0], segmax = red[2][0], segmin = red[3][0];
#pragma unroll
  for (int w = 1; w < ATT_WAVES; ++w) {
    kmax = max(kmax, red[0][w]);
    kmin = min(kmin, red[1][w]);
    segmax = max(segmax, red[2][w]);
    segmin = min(segmin, red[3][w]);
  }
  int startA = 0, endA = min(n_shared, kmax + 1);
  int startB = max(n_shared, segmin), endB = kmax + 1;
  if (a.nsplit > 1) {  // this work group's slice of the key axis
    const int lo = split * a.split_len, hi = lo + a.split_len;
    startA = max(startA, lo);
    endA = min(endA, hi);
    startB = max(startB, lo);
    endB = min(endB, hi);
  }
  const int nA = endA > startA ? (endA - startA + ATT_BK - 1) / ATT_BK : 0;
  const int nB = endB > startB ? (endB - startB + ATT_BK - 1) / ATT_BK : 0;
  const int ntiles = nA + nB;

  // ---- Q^T fragments (B operand), resident for the whole kernel
  bf16x8_t qf[ATT_QB][KS];
#pragma unroll
  for (int b = 0; b < ATT_QB; ++b) {
    const bf16_t* qp = a.q + (qi[b] * a.hq + qh[b]) * HD + half * 8;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      u32x4_t t = {0, 0, 0, 0};
      if (valid[b]) t = *reinterpret_cast<const u32x4_t*>(qp + s * 16);
      qf[b][s] = __builtin_bit_cast(bf16x8_t, t);
    }
  }

  const bf16_t* kbase = a.k + (int64_t)head * a.t_cap * HD;
  const bf16_t* vbase = a.v + (int64_t)head * a.t_cap * HD;
  // this lane's part of a V^T fragment read (see lds_read_tr16): tile row (key) offset, and the
  // column (d) offset within a 32-wide d block
  const int tr_g = lane >> 4, tr_j = lane & 15;
  const int tr_row = half * 4 + (tr_j >> 2);
  const int tr_col = (tr_g & 1) * 16 + (tr_j & 3) * 4;
  const int tr_swz = SM::v_swz(tr_row);  // equal for every row this lane reads (rows differ by multiples of 8)

  auto tile_bounds = [&](int j, int& s0, int& s1) {
    if (j < nA) {
      s0 = startA + j * ATT_BK;
      s1 = min(s0 + ATT_BK, endA);
    } else {
      s0 = startB + (j - nA) * ATT_BK;
      s1 = min(s0 + ATT_BK, endB);
    }
  };
  // Queue the tile's K and V rows straight into LDS buffer `buf`. Load x of this wave fills LDS
  // chunk positions [(x * ATT_WAVES + wv) * 64, +64), lane l position +l; the lane fetches the
  // global chunk that the swizzle places there. Rows past the tile's end re-read its last row
  // (finite data; those keys are masked), so nothing outside the cache is touched.
  auto issue_tile = [&](int j, int buf) {
    int s0, s1;
    tile_bounds(j, s0, s1);
    bf16_t* Ks = smem + buf * SM::BUF;
    bf16_t* Vs = Ks + SM::K_ELEMS;
#pragma unroll
    for (int x = 0; x < K_LD; ++x) {
      const int base = (x * ATT_WAVES + wv) * 64;  // first chunk position of this wave-wide load
      const int pos = base + lane;
      const int r = pos / KCH, p = pos % KCH;
      const int64_t grow = min(s0 + r, s1 - 1);
      lds_load16(kbase + grow * HD + (p ^ SM::k_swz(r)) * 8, Ks + base * 8);
      lds_load16(vbase + grow * HD + (p ^ SM::v_swz(r)) * 8, Vs + base * 8);
    }
  };

  f32x16_t oacc[ATT_QB][DB];
#pragma unroll
  for (int b = 0; b < ATT_QB; ++b)
#pragma unroll
    for (int d = 0; d < DB; ++d)
#pragma unroll
      for (int x = 0; x < 16; ++x) oacc[b][d][x] = 0.f;
  // running max (log2-scaled units) and sum of this lane's query rows
  float m_run[ATT_QB], l_run[ATT_QB];
#pragma unroll
  for (int b = 0; b < ATT_QB; ++b) {
    m_run[b] = -1e30f;
    l_run[b] = 0.f;
  }
  const float cs = a.scale_log2;

  if (ntiles > 0) issue_tile(0, 0);
  for (int j = 0; j < ntiles; ++j) {
    const int buf = j & 1;
    // tile j's LDS loads (this wave's) have landed; the barrier makes every wave's visible and
    // guarantees nobody still reads buffer buf ^ 1 (tile j - 1), which the next loads overwrite
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (j + 1 < ntiles) issue_tile(j + 1, buf ^ 1);
    const bf16_t* Ks = smem + buf * SM::BUF;
    const bf16_t* Vs = Ks + SM::K_ELEMS;
    int s0, s1;
    tile_bounds(j, s0, s1);

    const bool full = (s1 - s0 == ATT_BK) && (s1 - 1 <= kmin) && (j < nA || s0 >= segmax);
    // each 32-key half of the tile: S^T = K Q^T for every query block (a K fragment read from
    // LDS feeds them all), online softmax, then O^T += V^T P^T for those 32 keys
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      f32x16_t sacc[ATT_QB];
#pragma unroll
      for (int b = 0; b < ATT_QB; ++b)
#pragma unroll
        for (int x = 0; x < 16; ++x) sacc[b][x] = 0.f;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const int kr = kb * 32 + c;
        const bf16x8_t af = *reinterpret_cast<const bf16x8_t*>(Ks + kr * HD + ((2 * s + half) ^ SM::k_swz(kr)) * 8);
#pragma unroll
        for (int b = 0; b < ATT_QB; ++b)
          sacc[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, qf[b][s], sacc[b], 0, 0, 0);
      }
#pragma unroll
      for (int b = 0; b < ATT_QB; ++b) {
        if (!full) {
#pragma unroll
          for (int x = 0; x < 16; ++x) {
            int key = s0 + kb * 32 + (x >> 2) * 8 + half * 4 + (x & 3);
            bool vis = key < s1 && key <= my_end[b] && (key < n_shared || key >= my_seg[b]);
            sacc[b][x] = vis ? sacc[b][x] : -INFINITY;
          }
        }
        float tmax = -INFINITY;
#pragma unroll
        for (int x = 0; x < 16; ++x) tmax = fmaxf(tmax, sacc[b][x]);
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
        // Lazy rescale: exponentiate against a stale row max m_run and move it (rescaling the
        // running sum and O) only when some row's max outgrew it by more than 2^8; p then stays
        // <= 256, and the final division by the sum is exact either way.
        const float m_cand = fmaxf(m_run[b], tmax * cs);
        if (__ballot(m_cand > m_run[b] + ATT_RESCALE_LOG2)) {
          const float corr = __builtin_amdgcn_exp2f(m_run[b] - m_cand);
          l_run[b] *= corr;
#pragma unroll
          for (int d = 0; d < DB; ++d)
#pragma unroll
            for (int x = 0; x < 16; ++x) oacc[b][d][x] *= corr;
          m_run[b] = m_cand;
        }
        const float m_use = m_run[b];
        float rs = 0.f;
#pragma unroll
        for (int x = 0; x < 16; ++x) {
          float p = __builtin_amdgcn_exp2f(fmaf(sacc[b][x], cs, -m_use));
          sacc[b][x] = p;
          rs += p;
        }
        rs += __shfl_xor(rs, 32);
        l_run[b] += rs;
      }
      // O^T += V^T P^T over the 2 k-steps (16 keys each) of this half; each V fragment feeds
      // every query block
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        const int s = kb * 2 + h2, base = h2 * 8;
        bf16x8_t pb[ATT_QB];
#pragma unroll
        for (int b = 0; b < ATT_QB; ++b) {
          u32x4_t pw;
#pragma unroll
          for (int q = 0; q < 4; ++q) pw[q] = pack_bf(sacc[b][base + 2 * q], sacc[b][base + 2 * q + 1]);
          pb[b] = __builtin_bit_cast(bf16x8_t, pw);
        }
#pragma unroll
        for (int d = 0; d < DB; ++d) {
          // V^T fragment: keys s*16 + half*4 + (0..3) and s*16 + 8 + half*4 + (0..3) of column
          // d*32 + lane%32, transposed on the fly out of the row-major V tile
          const int col = d * 32 + tr_col;
          const bf16_t* vr = Vs + (s * 16 + tr_row) * HD + (((col >> 3) ^ tr_swz) << 3) + (col & 7);
          const s16x4_t lo = lds_read_tr16(vr);
          const s16x4_t hi = lds_read_tr16(vr + 8 * HD);
          const bf16x8_t va = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
          for (int b = 0; b < ATT_QB; ++b)
            oacc[b][d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pb[b], oacc[b][d], 0, 0, 0);
        }
      }
    }
  }

#pragma unroll
  for (int b = 0; b < ATT_QB; ++b) {
    if (!valid[b]) continue;
    if (a.nsplit > 1) {
      // partial for the combine kernel: unnormalised O, running max and sum
      const int64_t p = (((int64_t)split * a.hkv + head) * a.tiles + tile) * ATT_BM + (wv * ATT_QB + b) * 32 + c;
      float* po = a.ws_o + p * HD;
#pragma unroll
      for (int d = 0; d < DB; ++d)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          f32x4_t o = {oacc[b][d][g4 * 4 + 0], oacc[b][d][g4 * 4 + 1], oacc[b][d][g4 * 4 + 2], oacc[b][d][g4 * 4 + 3]};
          *reinterpret_cast<f32x4_t*>(po + d * 32 + g4 * 8 + half * 4) = o;
        }
      if (half == 0) {
        a.ws_ml[p * 2] = m_run[b];
        a.ws_ml[p * 2 + 1] = l_run[b];
      }
      continue;
    }
    const float inv = l_run[b] > 0.f ? 1.0f / l_run[b] : 0.f;
    bf16_t* op = a.out + (qi[b] * a.hq + qh[b]) * HD;
#pragma unroll
    for (int d = 0; d < DB; ++d)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        u32x2_t o = {pack_bf(oacc[b][d][g4 * 4 + 0] * inv, oacc[b][d][g4 * 4 + 1] * inv),
                     pack_bf(oacc[b][d][g4 * 4 + 2] * inv, oacc[b][d][g4 * 4 + 3] * inv)};
        *reinterpret_cast<u32x2_t*>(op + d * 32 + g4 * 8 + half * 4) = o;
      }
  }
}

// Merge split-K partials: one wave per (kv head, row); each lane owns HD/64 output elements.
template <int HD>
__global__ __launch_bounds__(256) void attn_combine_kernel(const AttnArgs a) {
  constexpr int EPL = HD / 64;
  const int64_t w = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int64_t R = a.n * a.G;
  if (w >= (int64_t)a.hkv * R) return;
  const int head = (int)(w / R);
  const int64_t r = w % R;
  const int tile = (int)(r / ATT_BM), in_tile = (int)(r % ATT_BM);
  const int64_t qi = r / a.G;
  const int qh = head * a.G + (int)(r % a.G);
  const int64_t stride = (int64_t)a.hkv * a.tiles * ATT_BM;
  const int64_t p0 = ((int64_t)head * a.tiles + tile) * ATT_BM + in_tile;
  float M = -INFINITY;
  for (int s = 0; s < a.nsplit; ++s) M = fmaxf(M, a.ws_ml[(p0 + s * stride) * 2]);
  float L = 0.f, acc[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) acc[e] = 0.f;
  for (int s = 0; s < a.nsplit; ++s) {
    const int64_t p = p0 + s * stride;
    const float l = a.ws_ml[p * 2 + 1];
    if (l == 0.f) continue;  // empty split
    const float wgt = __builtin_amdgcn_exp2f(a.ws_ml[p * 2] - M);
    L += wgt * l;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[e] += wgt * a.ws_o[p * HD + lane * EPL + e];
  }
  const float inv = L > 0.f ? 1.0f / L : 0.f;
  bf16_t* op = a.out + (qi * a.hq + qh) * HD + lane * EPL;
  if constexpr (EPL == 2) {
    *reinterpret_cast<uint32_t*>(op) = pack_bf(acc[0] * inv, acc[1] * inv);
  } else {
    op[0] = f2bf(acc[0] * inv);
  }
}

struct SplitPlan {
  int nsplit, split_len;
  int64_t tiles;
};

static SplitPlan plan_split(int64_t n, int hq, int hkv, int64_t t_cap) {
  SplitPlan sp;
  sp.tiles = (n * (hq / hkv) + ATT_BM - 1) / ATT_BM;
  const int64_t base = (int64_t)hkv * sp.tiles;
  sp.nsplit = 1;
  sp.split_len = 0;
  if (base < ATT_TARGET_WGS && t_cap >= 2 * ATT_MIN_SPLIT_KEYS) {
    int64_t want = (ATT_TARGET_WGS + base - 1) / base;
    int64_t most = t_cap / ATT_MIN_SPLIT_KEYS;
    int64_t ns = want < most ? want : most;
    if (ns > 1) {
      int64_t len = (t_cap + ns - 1) / ns;
      len = (len + ATT_BK - 1) / ATT_BK * ATT_BK;
      sp.nsplit = (int)((t_cap + len - 1) / len);
      sp.split_len = (int)len;
    }
  }
  return sp;
}

static size_t split_ws_bytes(const SplitPlan& sp, int hkv, int head_dim) {
  if (sp.nsplit <= 1) return 0;
  size_t rows = (size_t)sp.nsplit * hkv * sp.tiles * ATT_BM;
  return rows * (size_t)head_dim * 4 + rows * 8 + 256;
}

}  // namespace tread

using namespace tread;

extern "C" size_t tread_subset_attn_workspace_bytes(int64_t n, int hq, int hkv, int head_dim, int64_t t_cap) {
  if (n <= 0 || hq <= 0 || hkv <= 0 || (hq % hkv) != 0 || t_cap <= 0) return 0;
  return split_ws_bytes(plan_split(n, hq, hkv, t_cap), hkv, head_dim);
}

extern "C" int tread_subset_attn_bf16(const void* q, const void* k_cache, const void* v_cache, const int64_t* kend,
                                      const int64_t* kseg, int64_t n_shared, int64_t n, int hq, int hkv, int head_dim,
                                      int64_t t_cap, float scale, void* out, void* ws, size_t ws_bytes,
                                      tread_stream_t stream) {
  if (n == 0) return 0;
  if (n < 0 || hq <= 0 || hkv <= 0 || (hq % hkv) != 0 || t_cap <= 0)
    return fail(TREAD_EINVAL, "subset_attn: bad shape (n=%lld hq=%d hkv=%d)", (long long)n, hq, hkv);
  if (!q || !k_cache || !v_cache || !kend || !out) return fail(TREAD_EINVAL, "subset_attn: null pointer");
  if (head_dim != 64 && head_dim != 128) return fail(TREAD_EINVAL, "subset_attn: head_dim %d not in {64,128}", head_dim);
  if (t_cap > 0x7fffffffLL - 128) return fail(TREAD_ERANGE, "subset_attn: t_cap too large");
  if (n_shared < 0) return fail(TREAD_EINVAL, "subset_attn: negative n_shared");
  if ((((uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache | (uintptr_t)out) & 15) != 0)
    return fail(TREAD_EINVAL, "subset_attn: operands must be 16-byte aligned");
  AttnArgs a;
  memset(&a, 0, sizeof(a));
  a.q = (const bf16_t*)q;
  a.k = (const bf16_t*)k_cache;
  a.v = (const bf16_t*)v_cache;
  a.kend = kend;
  a.kseg = kseg;
  a.out = (bf16_t*)out;
  a.n_shared = n_shared;
  a.n = n;
  a.t_cap = t_cap;
  a.hq = hq;
  a.hkv = hkv;
  a.G = hq / hkv;
  SplitPlan sp = plan_split(n, hq, hkv, t_cap);
  const size_t need = split_ws_bytes(sp, hkv, head_dim);
  if (sp.nsplit > 1 && (!ws || ws_bytes < need)) sp.nsplit = 1;  // no workspace: one pass per row tile
  if (sp.tiles > 0x7fffffffLL / N_XCD) return fail(TREAD_ERANGE, "subset_attn: too many rows");
  a.tiles = (int32_t)sp.tiles;
  a.nsplit = sp.nsplit;
  a.split_len = sp.split_len;
  if (sp.nsplit > 1) {
    uintptr_t base = ((uintptr_t)ws + 255) & ~(uintptr_t)255;
    a.ws_ml = (float*)base;
    a.ws_o = a.ws_ml + (size_t)sp.nsplit * hkv * sp.tiles * ATT_BM * 2;
  }
  a.scale_log2 = scale * 1.4426950408889634f;
  int64_t grid;
  if (sp.nsplit > 1) {
    a.xpg = 0;
    grid = (int64_t)sp.nsplit * hkv * sp.tiles;
  } else if (hkv <= N_XCD && (N_XCD % hkv) == 0) {
    a.xpg = N_XCD / hkv;
    grid = (int64_t)N_XCD * ((sp.tiles + a.xpg - 1) / a.xpg);
  } else {
    a.xpg = 0;
    grid = (int64_t)hkv * sp.tiles;
  }
  if (grid > 0x7fffffffLL) return fail(TREAD_ERANGE, "subset_attn: grid too large");
  size_t smem = (head_dim == 128 ? AttnSmem<128>::BUF : AttnSmem<64>::BUF) * 2 * sizeof(bf16_t);
  hipStream_t s = (hipStream_t)stream;
  if (head_dim == 128)
    hipLaunchKernelGGL(subset_attn_kernel<128>, dim3((unsigned)grid), dim3(ATT_THREADS), smem, s, a);
  else
    hipLaunchKernelGGL(subset_attn_kernel<64>, dim3((unsigned)grid), dim3(ATT_THREADS), smem, s, a);
  int rc = check_launch("subset_attn");
  if (rc || sp.nsplit <= 1) return rc;
  const int64_t waves = (int64_t)hkv * n * a.G;
  const int64_t blocks = (waves + 3) / 4;
  if (head_dim == 128)
    hipLaunchKernelGGL(attn_combine_kernel<128>, dim3((unsigned)blocks), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(attn_combine_kernel<64>, dim3((unsigned)blocks), dim3(256), 0, s, a);
  return check_launch("subset_attn combine");
}
