// (c) Selective-recompute attention on CDNA4 MFMA (v_mfma_f32_32x32x16_bf16).
//
// Rows are (query token, query head) pairs of one KV head group: row r of KV head h is token
// r / G, query head h*G + r % G (G = hq / hkv), so the G heads that share a KV head share every
// K/V tile staged in LDS (GQA in-kernel, no repeat_kv). A work group of 8 waves owns 256 rows (32
// per wave, two waves per SIMD) and each wave computes the transposed score blocks S^T = K Q^T, so
// that after the softmax its probabilities already sit in the B-operand layout of O^T = V^T P^T:
// every lane holds one query column for both products, and the online-softmax rescale is a
// per-lane scalar. Q is pre-multiplied by scale * log2(e) and the score MFMAs start from -m (the
// running max), so they produce the exponent of exp2 directly. The online softmax keeps a stale
// row max until it is 2^8 too small, so the O rescale runs a handful of times per row, not per
// tile.
//
// K and V tiles go from global memory straight into LDS (no register staging), row-major
// [key][d] with XOR-swizzled chunks, three tile buffers deep; the A operand of the PV product
// (V^T) is read with gfx950's transposing LDS read. Fragment reads are inline asm with explicit
// waits, streaming ahead of the MFMAs. One step per key tile: an MFMA phase (scores of the next
// tile, then the PV product of this one) and a softmax phase (mask, row max, rescale,
// exponentials), which the two waves sharing a SIMD run in opposite order (ping-pong). The key
// range of a work group is the union of [0, n_shared) and [min kseg, max kend]; the visibility
// predicate (key <= kend[row] and key outside the row's masked gap) is evaluated in registers only
// on tiles that cross a row's boundary.
//
// Work groups are mapped XCD-aware: the hardware deals work group ids round-robin over the 8
// XCDs, so ids are remapped such that every XCD works on one KV head at a time, longest row tiles
// first, and the K/V tiles that its CUs stream are shared through that XCD's L2.
//
// Few rows (the query forward: tens of rows over a long cache) would leave most CUs idle, so the
// key range is then split across work groups (split-K): each writes its unnormalised fp32 O and
// its running (max, sum) to a workspace, and a combine kernel merges the splits per row.
#include <utility>

#include <mutex>

#include "common.h"
#include "../../include/tread_hip.h"

namespace tread {

constexpr int ATT_WAVES = 8;
constexpr int ATT_THREADS = ATT_WAVES * 64;
constexpr int ATT_BM = ATT_WAVES * 32;         // rows per work group (32 per wave)
// keys per pipeline step: as many as three LDS tile buffers of K and V hold in 160 KB, so that a
// step's fixed costs (barrier, first fragment latencies, tile bookkeeping) are spread over as much
// MFMA work as fits: 96 at head_dim 128 (3 x 48 KB; 1.6-2.8 % faster than 64-key steps on the
// recompute and causal shapes), 128 at head_dim 64 (3 x 32 KB)
constexpr int att_bk(int head_dim) { return head_dim == 64 ? 128 : 96; }
constexpr int ATT_NBUF = 3;                    // LDS tile buffers (software pipeline depth)
constexpr int N_XCD = 8;
constexpr int ATT_TARGET_WGS = 512;     // split-K when fewer (head, row tile) work groups than this
constexpr int ATT_MIN_SPLIT_KEYS = 512;
constexpr int ATT_MANY_TILE_WGS = 64;   // (head, row tile) work groups from which the split aims higher

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
  int32_t split_len;  // keys per split (multiple of att_bk(HD))
  int32_t nlong;      // (nsplit 1) the nlong longest row tiles per KV head run as two work groups
  int32_t prow;       // rows per row tile in the split-K partials (ATT_BM; DEC_ROWS for decode_attn)
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
  static constexpr int BK = att_bk(HD);
  static constexpr int K_ELEMS = BK * HD;
  static constexpr int V_ELEMS = BK * HD;
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
__device__ __forceinline__ float wave_max_f(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}
__device__ __forceinline__ float wave_sum_f(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
__device__ __forceinline__ int wave_min(int v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = min(v, __shfl_xor(v, o));
  return v;
}

// LDS byte address of a pointer into the work group's shared memory (the low 32 bits of its
// generic address; the LDS aperture is 4 GiB-aligned).
__device__ __forceinline__ uint32_t lds_addr(const void* p) { return (uint32_t)(uintptr_t)p; }

// V^T fragment halves by inline asm rather than the intrinsic: the compiler would otherwise wait
// for every outstanding global->LDS load (the next tiles' prefetch) before the first transposing
// read of a tile. The caller orders the results with lgkm_wait before use.
template <int OFF>
__device__ __forceinline__ s16x4_t tr_read(uint32_t addr) {
  s16x4_t r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "n"(OFF));
  return r;
}

// Wait until at most N LDS operations of this wave are outstanding (they complete in order), and
// tie the fragments read by tr_read to that point.
template <int N, int M>
__device__ __forceinline__ void lgkm_wait(s16x4_t (&v)[M]) {
  static_assert(M == 4 || M == 8, "fragment count");
  if constexpr (M == 8)
    asm volatile("s_waitcnt lgkmcnt(%8)"
                 : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]), "+v"(v[6]), "+v"(v[7])
                 : "n"(N));
  else
    asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]) : "n"(N));
}

template <int OFF>
__device__ __forceinline__ bf16x8_t lds_read128(uint32_t addr) {
  u32x4_t r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "n"(OFF));
  return __builtin_bit_cast(bf16x8_t, r);
}
template <int N>
__device__ __forceinline__ void lgkm_wait(bf16x8_t& v) {
  asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(v) : "n"(N));
}

template <int... I, typename F>
__device__ __forceinline__ void static_for_impl(std::integer_sequence<int, I...>, F&& f) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(std::make_integer_sequence<int, N>{}, f);
}

template <int N>
__device__ __forceinline__ void vm_wait() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Work-group barrier of the tile pipelines, after each wave has waited (vm_wait) for its own
// global->LDS loads of the tiles the barrier publishes. __syncthreads() would also wait for every
// outstanding vector memory operation (vmcnt(0)), i.e. for the tiles still being prefetched,
// taking the pipeline's load lead away at every barrier.
__device__ __forceinline__ void tile_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// max over lanes l and l ^ 32 (the two key halves of one query column)
__device__ __forceinline__ float xhalf_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xhalf_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

template <int HD>
__global__ __launch_bounds__(ATT_THREADS) void subset_attn_kernel(const AttnArgs a) {
  using SM = AttnSmem<HD>;
  constexpr int BK = SM::BK;    // keys per tile
  constexpr int NKB = BK / 32;  // 32-key blocks of a tile (score MFMA blocks)
  constexpr int NST = BK / 16;  // k-steps of the PV product
  constexpr int KS = HD / 16;   // k-steps of the QK product
  constexpr int DB = HD / 32;   // 32-row d blocks of O^T
  constexpr int KCH = HD / 8;   // 16-byte chunks per K/V row
  constexpr int K_LD = BK * KCH / ATT_THREADS;  // K (and V) 16-byte chunks per thread per tile
  static_assert(BK * KCH % ATT_THREADS == 0, "a tile's chunks split evenly over the threads");
  static_assert(BK % 32 == 0 && SM::BUF * ATT_NBUF * 2 <= 160 * 1024, "key tile size");
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
  // Balance: the row tiles are ordered longest first (td 0 is the last row tile, whose rows see
  // the most keys when rows are sorted by position), and the nlong longest run as two work groups
  // over the two halves of their key tiles, dispatched first; the rest follow longest first.
  int kpart = -1;
  if (a.nsplit <= 1 && a.nlong > 0) {
    if (td < 2 * a.nlong) {
      kpart = td & 1;
      td >>= 1;
    } else {
      td -= a.nlong;
    }
  }
  if (td >= a.tiles) return;
  const int tile = a.tiles - 1 - td;

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int c = lane & 31, half = lane >> 5;
  const int64_t R = a.n * a.G;
  const int n_shared = a.kseg ? (int)min<int64_t>(a.n_shared, a.t_cap) : 0;
  // this lane's query column: row r of the head group
  const int64_t r = (int64_t)tile * ATT_BM + wv * 32 + c;
  const bool valid = r < R;
  const int64_t qi = valid ? r / a.G : 0;
  const int qh = head * a.G + (int)(valid ? r % a.G : 0);
  int my_end = -1, my_seg = 0;
  int vmax = -1, vmin = 0x7fffffff, smax = 0, smin = 0x7fffffff;
  if (valid) {
    my_end = (int)min<int64_t>(max<int64_t>(a.kend[qi], -1), a.t_cap - 1);
    if (a.kseg) my_seg = (int)min<int64_t>(max<int64_t>(a.kseg[qi], 0), a.t_cap);
    vmax = vmin = my_end;
    smax = smin = my_seg;
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
  const int nA = endA > startA ? (endA - startA + BK - 1) / BK : 0;
  const int nB = endB > startB ? (endB - startB + BK - 1) / BK : 0;
  // this work group's key tiles [jbase, jbase + ntiles) of the nA + nB (a half for kpart 0 / 1)
  int jbase = 0, ntiles = nA + nB;
  if (kpart >= 0) {
    const int h = ntiles / 2;
    jbase = kpart ? h : 0;
    ntiles = kpart ? ntiles - h : h;
  }

  // ---- Q^T fragments (B operand), resident for the whole kernel, pre-multiplied by
  // scale * log2(e) (rounded to bf16, as the reference's math path rounds its scaled q), so that
  // the MFMA, started from -m_run, yields the exponent of exp2 directly
  bf16x8_t qf[KS];
  {
    const bf16_t* qp = a.q + (qi * a.hq + qh) * HD + half * 8;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      u32x4_t t = {0, 0, 0, 0};
      if (valid) t = *reinterpret_cast<const u32x4_t*>(qp + s * 16);
#pragma unroll
      for (int w = 0; w < 4; ++w) t[w] = pack_bf(lo_bf(t[w]) * a.scale_log2, hi_bf(t[w]) * a.scale_log2);
      qf[s] = __builtin_bit_cast(bf16x8_t, t);
    }
  }

  const bf16_t* kbase = a.k + (int64_t)head * a.t_cap * HD;
  const bf16_t* vbase = a.v + (int64_t)head * a.t_cap * HD;
  // this lane's V^T fragment read addresses (see lds_read_tr16) in buffer 0, one per d block:
  // tile row (key) half * 4 + (lane % 16) / 4, column d * 32 + (lane / 16 % 2) * 16 + lane % 4 * 4
  uint32_t vaddr[DB];
  {
    const int tr_g = lane >> 4, tr_j = lane & 15;
    const int tr_row = half * 4 + (tr_j >> 2);
    const int tr_col = (tr_g & 1) * 16 + (tr_j & 3) * 4;
    const int tr_swz = SM::v_swz(tr_row);  // equal for every row this lane reads (rows differ by multiples of 8)
#pragma unroll
    for (int d = 0; d < DB; ++d) {
      const int col = d * 32 + tr_col;
      vaddr[d] = lds_addr(smem + SM::K_ELEMS + tr_row * HD + (((col >> 3) ^ tr_swz) << 3) + (col & 7));
    }
  }

  auto tile_bounds = [&](int jl, int& s0, int& s1) {
    const int j = jbase + jl;
    if (j < nA) {
      s0 = startA + j * BK;
      s1 = min(s0 + BK, endA);
    } else {
      s0 = startB + (j - nA) * BK;
      s1 = min(s0 + BK, endB);
    }
  };
  // Queue tile j's K and V rows straight into LDS buffer `buf`, one wave-wide 16-byte load at a
  // time (LPT loads per wave and tile). Load x of this wave fills LDS chunk positions
  // [(x * ATT_WAVES + wv) * 64, +64), lane l position +l; the lane fetches the global chunk that
  // the swizzle places there. Rows past the tile's end re-read its last row (finite data; those
  // keys are masked), so nothing outside the cache is touched.
  constexpr int LPT = 2 * K_LD;
  int ld_row[K_LD], ld_kch[K_LD], ld_vch[K_LD];
#pragma unroll
  for (int x = 0; x < K_LD; ++x) {
    const int pos = (x * ATT_WAVES + wv) * 64 + lane;
    ld_row[x] = pos / KCH;
    ld_kch[x] = ((pos % KCH) ^ SM::k_swz(ld_row[x])) * 8;
    ld_vch[x] = ((pos % KCH) ^ SM::v_swz(ld_row[x])) * 8;
  }
  auto issue_load = [&](int q, int s0, int s1, int buf) {
    const int x = q >> 1;
    const int64_t grow = min(s0 + ld_row[x], s1 - 1);
    bf16_t* dst = smem + buf * SM::BUF + ((q & 1) ? SM::K_ELEMS : 0) + (x * ATT_WAVES + wv) * 64 * 8;
    if (q & 1)
      lds_load16(vbase + grow * HD + ld_vch[x], dst);
    else
      lds_load16(kbase + grow * HD + ld_kch[x], dst);
  };
  auto issue_tile = [&](int j, int buf) {
    int s0, s1;
    tile_bounds(j, s0, s1);
#pragma unroll
    for (int q = 0; q < LPT; ++q) issue_load(q, s0, s1, buf);
  };

  f32x16_t oacc[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d)
#pragma unroll
    for (int x = 0; x < 16; ++x) oacc[d][x] = 0.f;
  // running max (log2-scaled units, shared by lanes l and l ^ 32) and this lane's partial sums
  float m_run = 0.f;     // scores arrive as s * scale_log2 - m_run (the MFMA starts from -m_run)
  bool m_set = false;     // m_run holds a real row max (else 0, and nothing is accumulated yet)
  f32x16_t mneg;
#pragma unroll
  for (int x = 0; x < 16; ++x) mneg[x] = 0.f;
  float lsum[4] = {0.f, 0.f, 0.f, 0.f};

  // this lane's A-operand (K) fragment addresses for the 32-key half 0 of buffer 0, one per
  // k-step: row c, chunk (2 st + half) swizzled; half 1 and the buffers are fixed offsets
  uint32_t kaddr[KS];
#pragma unroll
  for (int st = 0; st < KS; ++st) kaddr[st] = lds_addr(smem + c * HD + ((2 * st + half) ^ SM::k_swz(c)) * 8);
  constexpr int NK = NKB * KS;  // K fragments per tile
  constexpr int RING = 4;     // K fragment reads in flight ahead of the MFMAs
  constexpr int NV = 2 * DB;  // transposing reads per PV k-step

  // V^T fragments of PV k-step ST from the buffer at byte offset `off`
  auto v_read = [&](auto st_c, uint32_t off, s16x4_t (&f)[NV]) {
    constexpr int ST = decltype(st_c)::value;
#pragma unroll
    for (int d = 0; d < DB; ++d) {
      f[2 * d] = tr_read<ST * 16 * HD * 2>(vaddr[d] + off);
      f[2 * d + 1] = tr_read<(ST * 16 + 8) * HD * 2>(vaddr[d] + off);
    }
  };
  // S^T = K Q^T for the tile in buffer `buf`: s[kb] holds keys kb * 32 + (x / 4) * 8 + half * 4 + x % 4
  // (register x) of this lane's query column. K fragments stream RING reads ahead of the MFMAs.
  auto qk = [&](int buf, f32x16_t (&s)[NKB]) {
    const uint32_t ko = (uint32_t)(buf * SM::BUF * 2);
    bf16x8_t kf[NK];
    static_for<RING>([&](auto I) {
      constexpr int i = decltype(I)::value;
      kf[i] = lds_read128<(i % NKB) * 32 * HD * 2>(kaddr[i / NKB] + ko);
    });
    static_for<NK>([&](auto I) {
      constexpr int i = decltype(I)::value;
      constexpr int k_after = (i + RING - 1 < NK - 1 ? i + RING - 1 : NK - 1) - i;
      lgkm_wait<k_after>(kf[i]);
      constexpr int kb = i % NKB, st = i / NKB;
      if constexpr (st == 0) {
        s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[i], qf[st], mneg, 0, 0, 0);
      } else {
        s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[i], qf[st], s[kb], 0, 0, 0);
      }
      if constexpr (i + RING < NK) {
        constexpr int m = i + RING;
        kf[m] = lds_read128<(m % NKB) * 32 * HD * 2>(kaddr[m / NKB] + ko);
      }
    });
  };
  // visibility mask (tiles crossing a row boundary), row max, lazy rescale of O and the sums:
  // the scores arrive relative to a stale max m_run and move (with O and the sums) only when some
  // row's max outgrew it by more than 2^8, or on a row's first visible keys; p then stays <= 256
  // and the final division by the sum is exact either way
  auto settle = [&](int j, f32x16_t (&s)[NKB]) {
    int s0, s1;
    tile_bounds(j, s0, s1);
    const bool full = (s1 - s0 == BK) && (s1 - 1 <= kmin) && (jbase + j < nA || s0 >= segmax);
    if (!full) {
      asm volatile("");  // keeps this rare path a branch: no speculated predicates on full tiles
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int x = 0; x < 16; ++x) {
          const int key = s0 + kb * 32 + (x >> 2) * 8 + half * 4 + (x & 3);
          const bool vis = key < s1 && key <= my_end && (key < n_shared || key >= my_seg);
          s[kb][x] = vis ? s[kb][x] : -INFINITY;
        }
    }
    float mx[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      mx[q] = fmaxf(fmaxf(s[0][q], s[0][q + 4]), s[0][q + 8]);
      mx[q] = fmaxf(mx[q], s[0][q + 12]);
#pragma unroll
      for (int kb = 1; kb < NKB; ++kb) {
        mx[q] = fmaxf(fmaxf(mx[q], s[kb][q]), s[kb][q + 4]);
        mx[q] = fmaxf(fmaxf(mx[q], s[kb][q + 8]), s[kb][q + 12]);
      }
    }
    const float tmax = xhalf_max(fmaxf(fmaxf(mx[0], mx[1]), fmaxf(mx[2], mx[3])));
    const bool need = m_set ? tmax > ATT_RESCALE_LOG2 : tmax > -INFINITY;
    if (__ballot(need)) {
      const float sh = need ? tmax : 0.f;
      const float corr = __builtin_amdgcn_exp2f(-sh);
#pragma unroll
      for (int q = 0; q < 4; ++q) lsum[q] *= corr;
#pragma unroll
      for (int d = 0; d < DB; ++d)
#pragma unroll
        for (int x = 0; x < 16; ++x) oacc[d][x] *= corr;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int x = 0; x < 16; ++x) s[kb][x] -= sh;
      m_run += sh;
      m_set = m_set || need;
#pragma unroll
      for (int x = 0; x < 16; ++x) mneg[x] = -m_run;
    }
  };
  // P = exp2(S') (S' = s * scale * log2(e) - m) as the B operand of the NST PV k-steps (16 keys
  // each); register x of s[kb] feeds k-step kb * 2 + x / 8
  auto to_p = [&](f32x16_t (&s)[NKB], bf16x8_t (&pb)[NST]) {
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int x = 0; x < 16; ++x) {
        const float p = __builtin_amdgcn_exp2f(s[kb][x]);
        s[kb][x] = p;
        lsum[x & 3] += p;
      }
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        u32x4_t pw;
#pragma unroll
        for (int q = 0; q < 4; ++q) pw[q] = pack_bf(s[kb][h2 * 8 + 2 * q], s[kb][h2 * 8 + 2 * q + 1]);
        pb[kb * 2 + h2] = __builtin_bit_cast(bf16x8_t, pw);
      }
  };
  // O^T += V^T P^T over the tile in buffer `buf`: k-step st covers tile keys st * 16 + half * 4 +
  // (0..3) and st * 16 + 8 + half * 4 + (0..3); fragment reads run one k-step ahead of the MFMAs.
  // v0 holds k-step 0's fragments, already queued.
  auto pv = [&](int buf, const bf16x8_t (&pb)[NST], s16x4_t (&v0)[NV]) {
    const uint32_t off = (uint32_t)(buf * SM::BUF * 2);
    s16x4_t v1[NV];
    auto mm = [&](const s16x4_t (&f)[NV], const bf16x8_t& p) {
#pragma unroll
      for (int d = 0; d < DB; ++d) {
        const bf16x8_t va = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(f[2 * d], f[2 * d + 1], 0, 1, 2, 3, 4, 5, 6, 7));
        oacc[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, p, oacc[d], 0, 0, 0);
      }
    };
    // k-steps alternate between the fragment sets v0 and v1: the next step's reads are queued
    // (NV LDS reads) before this step's fragments are waited for
    static_for<NST>([&](auto I) {
      constexpr int st = decltype(I)::value;
      s16x4_t(&cur)[NV] = (st & 1) ? v1 : v0;
      s16x4_t(&nxt)[NV] = (st & 1) ? v0 : v1;
      if constexpr (st + 1 < NST) {
        v_read(std::integral_constant<int, st + 1>{}, off, nxt);
        lgkm_wait<NV>(cur);
      } else {
        lgkm_wait<0>(cur);
      }
      mm(cur, pb[st]);
    });
  };

  // Software pipeline over tiles with ATT_NBUF LDS buffers (tile t in buffer t % ATT_NBUF): the
  // MFMA phase of a step computes the scores of tile t + 1 and accumulates tile t, whose
  // probabilities the softmax phase produced; tile t + ATT_NBUF - 1 is loaded meanwhile. The two
  // waves sharing a SIMD (wave w and w + 4) run the softmax and the MFMA phase in opposite order,
  // so that after each barrier one of them issues MFMAs while the other exponentiates: the early
  // group settles and exponentiates tile t + 1 after its MFMA phase, the late group tile t before.
  // Each wave's outstanding global loads are whole tiles of LPT instructions.
  // A wave none of whose 32 rows exists (the last row tile of a group; few query rows) only loads
  // its share of every tile and meets every barrier of the pipeline below, leaving its SIMD to the
  // waves with rows.
  const bool idle = __builtin_amdgcn_readfirstlane(__ballot(valid) == 0ull ? 1 : 0) != 0;
  if (idle) {
    if (ntiles > 0) {
#pragma unroll
      for (int t = 0; t < ATT_NBUF - 1; ++t)
        if (t < ntiles) issue_tile(t, t);
      if constexpr (ATT_NBUF >= 4) {
        if (ntiles > 2) vm_wait<2 * LPT>();
        else if (ntiles > 1) vm_wait<LPT>();
        else vm_wait<0>();
      } else {
        if (ntiles > 1) vm_wait<LPT>();
        else vm_wait<0>();
      }
      tile_barrier();
      int bj = 0;
      for (int j = 0; j + 1 < ntiles; ++j) {
        if constexpr (ATT_NBUF >= 4) {
          if (j + 2 < ntiles) vm_wait<LPT>();
          else vm_wait<0>();
        } else {
          vm_wait<0>();
        }
        tile_barrier();
        const int bn = bj == ATT_NBUF - 1 ? 0 : bj + 1, bprev = bj == 0 ? ATT_NBUF - 1 : bj - 1;
        const int tl = j + ATT_NBUF - 1;
        if (tl < ntiles) issue_tile(tl, bprev);
        bj = bn;
      }
    }
    return;  // no rows: nothing to write
  }
  if (ntiles > 0) {
#pragma unroll
    for (int t = 0; t < ATT_NBUF - 1; ++t)
      if (t < ntiles) issue_tile(t, t);
    // tile 0 landed: the tiles queued after it may still fly
    if constexpr (ATT_NBUF >= 4) {
      if (ntiles > 2) vm_wait<2 * LPT>();
      else if (ntiles > 1) vm_wait<LPT>();
      else vm_wait<0>();
    } else {
      if (ntiles > 1) vm_wait<LPT>();
      else vm_wait<0>();
    }
    tile_barrier();
    const bool late = wv >= ATT_WAVES / 2;
    f32x16_t sc[NKB];
    bf16x8_t pb[NST];
    qk(0, sc);
    int j = 0, bj = 0;  // bj = j % ATT_NBUF
    if (!late) {
      settle(0, sc);
      to_p(sc, pb);
    }
    while (j + 1 < ntiles) {
      // every wave's loads of tile j + 1 landed, and every wave is done with tile j - 1, whose
      // buffer receives tile j + ATT_NBUF - 1
      if constexpr (ATT_NBUF >= 4) {
        if (j + 2 < ntiles) vm_wait<LPT>();
        else vm_wait<0>();
      } else {
        vm_wait<0>();
      }
      tile_barrier();
      const int bn = bj == ATT_NBUF - 1 ? 0 : bj + 1, bprev = bj == 0 ? ATT_NBUF - 1 : bj - 1;
      const int tl = j + ATT_NBUF - 1;
      if (tl < ntiles) issue_tile(tl, bprev);
      if (late) {
        settle(j, sc);
        to_p(sc, pb);
      }
      // the scores of tile j are in pb now, so sc takes tile j + 1's. The MFMA phase runs at raised
      // wave priority, so its MFMAs and fragment reads issue ahead of the partner wave's softmax
      // VALU work on the same SIMD (measured 0.7-1 % faster on the recompute and causal shapes).
      __builtin_amdgcn_s_setprio(1);
      qk(bn, sc);
      s16x4_t v0[NV];
      v_read(std::integral_constant<int, 0>{}, (uint32_t)(bj * SM::BUF * 2), v0);
      pv(bj, pb, v0);
      __builtin_amdgcn_s_setprio(0);
      ++j;
      bj = bn;
      if (!late) {
        settle(j, sc);
        to_p(sc, pb);
      }
    }
    if (late) {
      settle(j, sc);
      to_p(sc, pb);
    }
    s16x4_t v0[NV];
    v_read(std::integral_constant<int, 0>{}, (uint32_t)(bj * SM::BUF * 2), v0);
    pv(bj, pb, v0);
  }

  if (!valid) return;
  // row sum over both key halves
  const float l_run = xhalf_sum((lsum[0] + lsum[1]) + (lsum[2] + lsum[3]));
  if (a.nsplit > 1 || kpart >= 0) {
    // partial for the combine kernel: unnormalised O, running max and sum
    const int64_t p = a.nsplit > 1 ? (((int64_t)split * a.hkv + head) * a.tiles + tile) * ATT_BM + wv * 32 + c
                                   : (((int64_t)kpart * a.hkv + head) * a.nlong + td) * ATT_BM + wv * 32 + c;
    float* po = a.ws_o + p * HD;
#pragma unroll
    for (int d = 0; d < DB; ++d)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        f32x4_t o = {oacc[d][g4 * 4 + 0], oacc[d][g4 * 4 + 1], oacc[d][g4 * 4 + 2], oacc[d][g4 * 4 + 3]};
        *reinterpret_cast<f32x4_t*>(po + d * 32 + g4 * 8 + half * 4) = o;
      }
    if (half == 0) {
      a.ws_ml[p * 2] = m_run;
      a.ws_ml[p * 2 + 1] = l_run;
    }
    return;
  }
  const float inv = l_run > 0.f ? 1.0f / l_run : 0.f;
  bf16_t* op = a.out + (qi * a.hq + qh) * HD;
#pragma unroll
  for (int d = 0; d < DB; ++d)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      u32x2_t o = {pack_bf(oacc[d][g4 * 4 + 0] * inv, oacc[d][g4 * 4 + 1] * inv),
                   pack_bf(oacc[d][g4 * 4 + 2] * inv, oacc[d][g4 * 4 + 3] * inv)};
      *reinterpret_cast<u32x2_t*>(op + d * 32 + g4 * 8 + half * 4) = o;
    }
}

// (d) A few query rows against a long cache (decoding steps). One work group per (key slice, KV
// head) holds every row of the launch (query tokens x the G query heads of the KV head, at most
// DEC_ROWS: one MFMA column block) and splits the slice's keys between its waves instead of its
// rows: wave w takes the slice's 32-key tiles w, w + 8, ..., each into its own 16 KB of LDS (K rows
// then V rows, swizzled as in subset_attn_kernel), computes S^T = K Q^T and O^T += V^T P^T with the
// same MFMA layouts on one 32-key block, and keeps its own running max and sums. No wave waits for
// another inside the loop: a wave queues its next K tile as soon as its score MFMAs have read this
// one, and its next V tile after its PV MFMAs, so its loads overlap its own arithmetic and the
// other wave of its SIMD; its first K and V tiles go out together once the rows' key ends are in.
// At the end the 8 waves' (max, sum, O) meet in LDS; one partial per row
// goes to the split-K workspace for the combine kernels, or, with a single slice, the normalised
// output is written directly.
constexpr int DEC_WAVES = 8;
constexpr int DEC_THREADS = DEC_WAVES * 64;
constexpr int DEC_BK = 32;    // keys per wave tile
constexpr int DEC_ROWS = 32;  // rows per launch and KV head

template <int HD>
__global__ __launch_bounds__(DEC_THREADS) void decode_attn_kernel(const AttnArgs a) {
  using SM = AttnSmem<HD>;
  constexpr int KS = HD / 16;            // k-steps of the score product
  constexpr int DB = HD / 32;            // 32-row d blocks of O^T
  constexpr int KCH = HD / 8;            // 16-byte chunks per K/V row
  constexpr int TE = DEC_BK * HD;        // elements of one K (or V) tile
  constexpr int LPK = TE / 8 / 64;       // 16-byte loads per lane for one K (or V) tile
  constexpr int NV = 2 * DB;             // transposing reads per PV k-step
  constexpr int RING = KS < 4 ? KS : 4;  // K fragment reads in flight ahead of the MFMAs
  // per wave [K tile | V tile] while the tiles stream; the 8 waves' fp32 O rows for the merge after
  extern __shared__ __align__(16) bf16_t smem[];
  __shared__ float mrg_m[DEC_WAVES][DEC_ROWS], mrg_l[DEC_WAVES][DEC_ROWS];

  const int split = blockIdx.x, head = blockIdx.y;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int c = lane & 31, half = lane >> 5;
  const int k_lo = split * a.split_len;
  bf16_t* const kbuf = smem + wv * 2 * TE;
  bf16_t* const vbuf = kbuf + TE;
  const bf16_t* kbase = a.k + (int64_t)head * a.t_cap * HD;
  const bf16_t* vbase = a.v + (int64_t)head * a.t_cap * HD;
  // Load x of a tile fills LDS chunk positions [x * 64, x * 64 + 64) of the wave's tile, lane l
  // position x * 64 + l, with the global chunk the swizzle places there; rows from k1 on re-read
  // row k1 - 1.
  auto issue = [&](int k0, int k1, const bf16_t* base, bf16_t* buf, bool is_v) {
#pragma unroll
    for (int x = 0; x < LPK; ++x) {
      const int pos = x * 64 + lane, row = pos / KCH, ch = pos % KCH;
      const int sw = is_v ? SM::v_swz(row) : SM::k_swz(row);
      const int64_t grow = min(k0 + row, k1 - 1);
      lds_load16(base + grow * HD + (ch ^ sw) * 8, buf + x * 64 * 8);
    }
  };
  // The rows' key ends and Q are loaded before any tile: the compiler waits for all outstanding
  // vector memory (vmcnt(0)) before using a plain load's value while global -> LDS loads are in
  // flight, so these go first, and the wave's first K and V tiles follow together. A lane past the
  // launch's rows reads row 0 (unconditional loads: one under a branch is waited for at its end);
  // its column's scores and output are never used.
  const int64_t R = a.n * a.G;
  const bool valid = c < R;  // this lane's query column: row c = (token c / G, head head * G + c % G)
  const int64_t qi = valid ? c / a.G : 0;
  const int qh = head * a.G + (int)(valid ? c % a.G : 0);
  const int n_shared = a.kseg ? (int)min<int64_t>(a.n_shared, a.t_cap) : 0;
  const int64_t end_raw = a.kend[qi];
  const int64_t seg_raw = (a.kseg ? a.kseg : a.kend)[qi];
  u32x4_t qraw[KS];
  {
    const bf16_t* qp = a.q + (qi * a.hq + qh) * HD + half * 8;
#pragma unroll
    for (int s = 0; s < KS; ++s) qraw[s] = *reinterpret_cast<const u32x4_t*>(qp + s * 16);
  }
  const int64_t tcap1 = a.t_cap - 1;
  const int my_end = !valid ? -1 : (int)(end_raw < -1 ? -1 : end_raw > tcap1 ? tcap1 : end_raw);
  const int my_seg = !(valid && a.kseg) ? 0 : (int)(seg_raw < 0 ? 0 : seg_raw > a.t_cap ? a.t_cap : seg_raw);
  // every wave holds the same rows, so wave reductions give the work group's key bounds
  const int kmax = wave_max(my_end);
  const int kmin = wave_min(valid ? my_end : 0x7fffffff);
  const int segmax = wave_max(valid && a.kseg ? my_seg : 0);
  const int k_hi = min(k_lo + a.split_len, kmax + 1);
  const int ntiles = k_hi > k_lo ? (k_hi - k_lo + DEC_BK - 1) / DEC_BK : 0;
  // Q^T fragments (B operand), pre-multiplied by scale * log2(e) and rounded to bf16, as in
  // subset_attn_kernel (before the tile loads go out, for the reason above)
  bf16x8_t qf[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    u32x4_t t = qraw[s];
#pragma unroll
    for (int w = 0; w < 4; ++w) t[w] = pack_bf(lo_bf(t[w]) * a.scale_log2, hi_bf(t[w]) * a.scale_log2);
    qf[s] = __builtin_bit_cast(bf16x8_t, t);
    asm volatile("" : "+v"(qf[s]));  // computed here, not next to its first use
  }
  // K rows only up to the last visible key as well: keys past a row's end are masked from the
  // scores, and V rows past the work group's last visible key are never read
  if (wv < ntiles) {
    const int k0 = k_lo + wv * DEC_BK, k1 = min(k0 + DEC_BK, k_hi);
    issue(k0, k1, kbase, kbuf, false);
    issue(k0, k1, vbase, vbuf, true);
  }

  auto tile_keys = [&](int j, int& k0, int& k1) {
    k0 = k_lo + j * DEC_BK;
    k1 = min(k0 + DEC_BK, k_hi);
  };

  // K fragment addresses (A operand of the score product): row c, chunk 2 s + half, swizzled
  uint32_t kaddr[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) kaddr[s] = lds_addr(kbuf + c * HD + ((2 * s + half) ^ SM::k_swz(c)) * 8);
  // V^T fragment addresses (transposing reads), as in subset_attn_kernel
  uint32_t vaddr[DB];
  {
    const int tr_g = lane >> 4, tr_j = lane & 15;
    const int tr_row = half * 4 + (tr_j >> 2);
    const int tr_col = (tr_g & 1) * 16 + (tr_j & 3) * 4;
    const int tr_swz = SM::v_swz(tr_row);
#pragma unroll
    for (int d = 0; d < DB; ++d) {
      const int col = d * 32 + tr_col;
      vaddr[d] = lds_addr(vbuf + tr_row * HD + (((col >> 3) ^ tr_swz) << 3) + (col & 7));
    }
  }
  auto v_read = [&](auto st_c, s16x4_t (&f)[NV]) {
    constexpr int ST = decltype(st_c)::value;
#pragma unroll
    for (int d = 0; d < DB; ++d) {
      f[2 * d] = tr_read<ST * 16 * HD * 2>(vaddr[d]);
      f[2 * d + 1] = tr_read<(ST * 16 + 8) * HD * 2>(vaddr[d]);
    }
  };

  f32x16_t oacc[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d)
#pragma unroll
    for (int x = 0; x < 16; ++x) oacc[d][x] = 0.f;
  float m_run = -INFINITY;  // log2-scaled running max of this lane's row (-inf: nothing visible yet)
  float lsum[4] = {0.f, 0.f, 0.f, 0.f};

  for (int j = wv; j < ntiles; j += DEC_WAVES) {
    const int jn = j + DEC_WAVES;
    const bool more = jn < ntiles;
    vm_wait<LPK>();  // this tile's K landed (its V may still fly)
    // S^T = K Q^T: register x of sc holds key (x / 4) * 8 + half * 4 + x % 4 of the tile
    f32x16_t sc;
#pragma unroll
    for (int x = 0; x < 16; ++x) sc[x] = 0.f;
    {
      bf16x8_t kf[KS];
      static_for<RING>([&](auto I) {
        constexpr int i = decltype(I)::value;
        kf[i] = lds_read128<0>(kaddr[i]);
      });
      static_for<KS>([&](auto I) {
        constexpr int i = decltype(I)::value;
        constexpr int k_after = (i + RING - 1 < KS - 1 ? i + RING - 1 : KS - 1) - i;
        lgkm_wait<k_after>(kf[i]);
        sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[i], qf[i], sc, 0, 0, 0);
        if constexpr (i + RING < KS) kf[i + RING] = lds_read128<0>(kaddr[i + RING]);
      });
    }
    if (more) {  // every K fragment read has completed
      int n0, n1;
      tile_keys(jn, n0, n1);
      issue(n0, n1, kbase, kbuf, false);
    }
    int k0, k1;
    tile_keys(j, k0, k1);
    const bool full = (k1 - k0 == DEC_BK) && (k1 - 1 <= kmin) && (k0 >= segmax || k1 <= n_shared || !a.kseg);
    if (!full) {
#pragma unroll
      for (int x = 0; x < 16; ++x) {
        const int key = k0 + (x >> 2) * 8 + half * 4 + (x & 3);
        const bool vis = key < k1 && key <= my_end && (!a.kseg || key < n_shared || key >= my_seg);
        sc[x] = vis ? sc[x] : -INFINITY;
      }
    }
    float mx = sc[0];
#pragma unroll
    for (int x = 1; x < 16; ++x) mx = fmaxf(mx, sc[x]);
    const float m_new = fmaxf(m_run, xhalf_max(mx));
    const bool any = m_new > -INFINITY;
    const float corr = any ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.f;
    const float msub = any ? m_new : 0.f;
    m_run = m_new;
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) lsum[q4] *= corr;
#pragma unroll
    for (int d = 0; d < DB; ++d)
#pragma unroll
      for (int x = 0; x < 16; ++x) oacc[d][x] *= corr;
    bf16x8_t pb[2];
#pragma unroll
    for (int x = 0; x < 16; ++x) {
      const float p = __builtin_amdgcn_exp2f(sc[x] - msub);
      sc[x] = p;
      lsum[x & 3] += p;
    }
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      u32x4_t pw;
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) pw[q4] = pack_bf(sc[h2 * 8 + 2 * q4], sc[h2 * 8 + 2 * q4 + 1]);
      pb[h2] = __builtin_bit_cast(bf16x8_t, pw);
    }
    // this tile's V landed (the next K tile may still fly)
    if (more) vm_wait<LPK>();
    else vm_wait<0>();
    // O^T += V^T P^T: k-step st covers tile keys st * 16 + half * 4 + (0..3) and st * 16 + 8 + half * 4 + (0..3)
    {
      s16x4_t v0[NV], v1[NV];
      v_read(std::integral_constant<int, 0>{}, v0);
      v_read(std::integral_constant<int, 1>{}, v1);
      auto mm = [&](const s16x4_t (&f)[NV], const bf16x8_t& p) {
#pragma unroll
        for (int d = 0; d < DB; ++d) {
          const bf16x8_t va = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(f[2 * d], f[2 * d + 1], 0, 1, 2, 3, 4, 5, 6, 7));
          oacc[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, p, oacc[d], 0, 0, 0);
        }
      };
      lgkm_wait<NV>(v0);
      mm(v0, pb[0]);
      lgkm_wait<0>(v1);
      mm(v1, pb[1]);
    }
    if (more) {  // every V fragment read has completed
      int n0, n1;
      tile_keys(jn, n0, n1);
      issue(n0, n1, vbase, vbuf, true);
    }
  }

  // ---- merge the 8 waves' partials of each row
  const float l_row = xhalf_sum((lsum[0] + lsum[1]) + (lsum[2] + lsum[3]));
  __syncthreads();  // every wave is done with its tile buffers
  // [wave][row][HD + 4]: the 16-byte pad per row puts the 32 rows a store instruction writes in
  // different banks (with a stride of HD floats every lane of a store hit the same banks, and the
  // 8 waves' writes took 3.5 us)
  constexpr int MO_LD = HD + 4;
  float* const mo = reinterpret_cast<float*>(smem);
  if (valid) {  // only the launch's rows are merged
#pragma unroll
    for (int d = 0; d < DB; ++d)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const f32x4_t o = {oacc[d][g4 * 4 + 0], oacc[d][g4 * 4 + 1], oacc[d][g4 * 4 + 2], oacc[d][g4 * 4 + 3]};
        *reinterpret_cast<f32x4_t*>(mo + (wv * DEC_ROWS + c) * MO_LD + d * 32 + g4 * 8 + half * 4) = o;
      }
  }
  if (half == 0) {
    mrg_m[wv][c] = m_run;
    mrg_l[wv][c] = l_row;
  }
  __syncthreads();
  constexpr int DQ = HD / 4;
  for (int it = threadIdx.x; it < (int)R * DQ; it += DEC_THREADS) {
    const int rr = it / DQ, dq = it % DQ;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < DEC_WAVES; ++w)
      if (mrg_l[w][rr] > 0.f) M = fmaxf(M, mrg_m[w][rr]);
    float L = 0.f;
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < DEC_WAVES; ++w) {
      const float l = mrg_l[w][rr];
      if (l > 0.f) {
        const float wgt = __builtin_amdgcn_exp2f(mrg_m[w][rr] - M);
        L += wgt * l;
        acc += wgt * *reinterpret_cast<const f32x4_t*>(mo + (w * DEC_ROWS + rr) * MO_LD + dq * 4);
      }
    }
    if (a.nsplit > 1) {
      const int64_t p = ((int64_t)split * a.hkv + head) * DEC_ROWS + rr;
      *reinterpret_cast<f32x4_t*>(a.ws_o + p * HD + dq * 4) = acc;
      if (dq == 0) {
        a.ws_ml[p * 2] = L > 0.f ? M : 0.f;
        a.ws_ml[p * 2 + 1] = L;
      }
    } else {
      const float inv = L > 0.f ? 1.0f / L : 0.f;
      const int64_t qr = rr / a.G;
      const int qhr = head * a.G + rr % a.G;
      const u32x2_t o2 = {pack_bf(acc[0] * inv, acc[1] * inv), pack_bf(acc[2] * inv, acc[3] * inv)};
      *reinterpret_cast<u32x2_t*>(a.out + (qr * a.hq + qhr) * HD + dq * 4) = o2;
    }
  }
}

// Merge split-K partials: one work group per (kv head, row). The split maxima and sums go through
// LDS; each thread then owns 4 output elements of one split group (every SG-th split), and the
// groups' weighted partial sums are reduced in LDS.
constexpr int CMB_THREADS = 256;
constexpr int CMB_MAX_SPLITS = 1024;
template <int HD>
__global__ __launch_bounds__(CMB_THREADS) void attn_combine_kernel(const AttnArgs a) {
  constexpr int DQ = HD / 4;              // float4 groups of a row
  constexpr int SG = CMB_THREADS / DQ;    // split groups
  __shared__ float sm_w[CMB_MAX_SPLITS];  // split weight exp2(m_s - M) (0 for empty splits)
  __shared__ float red[CMB_THREADS / 64];
  __shared__ f32x4_t part[SG][DQ];
  const int64_t R = a.n * a.G;
  const int64_t w = blockIdx.x;
  const int head = (int)(w / R);
  const int64_t r = w % R;
  const int tile = (int)(r / a.prow), in_tile = (int)(r % a.prow);
  const int64_t stride = (int64_t)a.hkv * a.tiles * a.prow;
  const int64_t p0 = ((int64_t)head * a.tiles + tile) * a.prow + in_tile;
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int dq = t % DQ, sg = t / DQ;  // this thread's 4 output elements and split group
  // The (max, sum) of slice t and the split group's first UNR partial rows are all issued before any
  // of them is used: one round of memory latency when nsplit <= UNR * SG (a decoding step's 64
  // slices), where the maxima, then the weights, then the rows took three.
  constexpr int UNR = 8;
  f32x4_t o[UNR];
  auto load_rows = [&](int s0) {
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int s = s0 + u * SG;
      if (s < a.nsplit) o[u] = *reinterpret_cast<const f32x4_t*>(a.ws_o + (p0 + s * stride) * HD + dq * 4);
    }
  };
  float2 ml0 = {0.f, 0.f};
  if (t < a.nsplit) ml0 = *reinterpret_cast<const float2*>(a.ws_ml + (p0 + t * stride) * 2);
  load_rows(sg);
  // global max of the split maxima
  float m = ml0.y > 0.f ? ml0.x : -INFINITY;
  for (int s = t + CMB_THREADS; s < a.nsplit; s += CMB_THREADS)
    if (a.ws_ml[(p0 + s * stride) * 2 + 1] > 0.f) m = fmaxf(m, a.ws_ml[(p0 + s * stride) * 2]);
  m = wave_max_f(m);
  if (lane == 0) red[wv] = m;
  __syncthreads();
  float M = red[0];
#pragma unroll
  for (int q = 1; q < CMB_THREADS / 64; ++q) M = fmaxf(M, red[q]);
  __syncthreads();
  // weights and the weighted sum of the split sums
  float lw = 0.f;
  if (t < a.nsplit) {
    const float wgt = ml0.y > 0.f ? __builtin_amdgcn_exp2f(ml0.x - M) : 0.f;
    sm_w[t] = wgt;
    lw += wgt * ml0.y;
  }
  for (int s = t + CMB_THREADS; s < a.nsplit; s += CMB_THREADS) {
    const int64_t p = p0 + s * stride;
    const float l = a.ws_ml[p * 2 + 1];
    const float wgt = l > 0.f ? __builtin_amdgcn_exp2f(a.ws_ml[p * 2] - M) : 0.f;
    sm_w[s] = wgt;
    lw += wgt * l;
  }
  lw = wave_sum_f(lw);
  if (lane == 0) red[wv] = lw;
  __syncthreads();
  float L = 0.f;
#pragma unroll
  for (int q = 0; q < CMB_THREADS / 64; ++q) L += red[q];
  // the group's slices in order, UNR at a time (empty slices have weight 0 and are skipped)
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = sg;;) {
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int s = s0 + u * SG;
      const float wg = s < a.nsplit ? sm_w[s] : 0.f;
      if (wg != 0.f) acc += wg * o[u];
    }
    s0 += UNR * SG;
    if (s0 >= a.nsplit) break;
    load_rows(s0);
  }
  part[sg][dq] = acc;
  __syncthreads();
  if (sg != 0) return;
#pragma unroll
  for (int g = 1; g < SG; ++g) acc += part[g][dq];
  const float inv = L > 0.f ? 1.0f / L : 0.f;
  const int64_t qi = r / a.G;
  const int qh = head * a.G + (int)(r % a.G);
  bf16_t* op = a.out + (qi * a.hq + qh) * HD + dq * 4;
  const u32x2_t o2 = {pack_bf(acc[0] * inv, acc[1] * inv), pack_bf(acc[2] * inv, acc[3] * inv)};
  *reinterpret_cast<u32x2_t*>(op) = o2;
}

// Merge the two key halves of the long row tiles (nlong > 0): one wave per (KV head, row), the
// same weighting as attn_combine_kernel for two partials.
constexpr int HALF_ROWS = 4;  // rows (waves) per work group
template <int HD>
__global__ __launch_bounds__(HALF_ROWS * 64) void attn_halves_kernel(const AttnArgs a) {
  constexpr int EPL = HD / 64;  // elements per lane
  const int lane = threadIdx.x & 63;
  const int64_t per_head = (int64_t)a.nlong * ATT_BM;
  const int64_t w = (int64_t)blockIdx.x * HALF_ROWS + (threadIdx.x >> 6);
  if (w >= a.hkv * per_head) return;
  const int head = (int)(w / per_head);
  const int64_t rem = w % per_head;
  const int td = (int)(rem / ATT_BM), rt = (int)(rem % ATT_BM);
  const int64_t r = (int64_t)(a.tiles - 1 - td) * ATT_BM + rt;
  if (r >= a.n * a.G) return;
  const int64_t p0 = ((int64_t)head * a.nlong + td) * ATT_BM + rt;
  const int64_t p1 = ((int64_t)(a.hkv + head) * a.nlong + td) * ATT_BM + rt;
  const float m0 = a.ws_ml[p0 * 2], l0 = a.ws_ml[p0 * 2 + 1];
  const float m1 = a.ws_ml[p1 * 2], l1 = a.ws_ml[p1 * 2 + 1];
  const float M = fmaxf(l0 > 0.f ? m0 : -INFINITY, l1 > 0.f ? m1 : -INFINITY);
  const float w0 = l0 > 0.f ? __builtin_amdgcn_exp2f(m0 - M) : 0.f;
  const float w1 = l1 > 0.f ? __builtin_amdgcn_exp2f(m1 - M) : 0.f;
  const float L = w0 * l0 + w1 * l1;
  const float inv = L > 0.f ? 1.0f / L : 0.f;
  const float* o0 = a.ws_o + p0 * HD + lane * EPL;
  const float* o1 = a.ws_o + p1 * HD + lane * EPL;
  const int64_t qi = r / a.G;
  const int qh = head * a.G + (int)(r % a.G);
  bf16_t* op = a.out + (qi * a.hq + qh) * HD + lane * EPL;
  if constexpr (EPL == 2) {
    const float2 x0 = *reinterpret_cast<const float2*>(o0), x1 = *reinterpret_cast<const float2*>(o1);
    *reinterpret_cast<uint32_t*>(op) = pack_bf((w0 * x0.x + w1 * x1.x) * inv, (w0 * x0.y + w1 * x1.y) * inv);
  } else {
    op[0] = f2bf((w0 * o0[0] + w1 * o1[0]) * inv);
  }
}

// Merge split-K partials of launches with few key slices (nsplit <= CMB_FEW_SPLITS): HD / 4 lanes
// per (KV head, row), each owning 4 output elements (one 16-byte load per slice), so a wave merges
// 64 / (HD / 4) rows; the slices are walked in order. Same weights as attn_combine_kernel
// (exp2(m_s - M), empty slices skipped). Against one wave per row with HD / 64 elements per lane
// (4- or 8-byte loads), same bits: a 0.5B-shaped recompute's merge (1 632 rows x 14 heads, 7
// slices) took 18.0 us, a 1.5B-shaped one (3 232 x 12, 7 slices) 34 us; one wave per row
// instead of a 256-thread work group had taken a 1.5B-shaped call 321 -> 292 us.
constexpr int CMB_FEW_SPLITS = 16;
template <int HD>
__global__ __launch_bounds__(HALF_ROWS * 64) void attn_combine_few_kernel(const AttnArgs a) {
  constexpr int LPR = HD / 4;    // lanes per row, 4 elements each
  constexpr int RPW = 64 / LPR;  // rows per wave
  const int lane = threadIdx.x & 63;
  const int q4 = lane % LPR;
  const int64_t R = a.n * a.G;
  const int64_t w = ((int64_t)blockIdx.x * HALF_ROWS + (threadIdx.x >> 6)) * RPW + lane / LPR;
  if (w >= (int64_t)a.hkv * R) return;  // lanes work alone: no cross-lane operation below
  const int head = (int)(w / R);
  const int64_t r = w % R;
  const int tile = (int)(r / a.prow), in_tile = (int)(r % a.prow);
  const int64_t stride = (int64_t)a.hkv * a.tiles * a.prow;
  const int64_t p0 = ((int64_t)head * a.tiles + tile) * a.prow + in_tile;
  // every slice's (max, sum) and partial O are loaded up front (one round of memory latency, not
  // one per slice); the merge then walks the slices in order
  float mv[CMB_FEW_SPLITS], lv[CMB_FEW_SPLITS];
  f32x4_t ov[CMB_FEW_SPLITS];
#pragma unroll
  for (int sp = 0; sp < CMB_FEW_SPLITS; ++sp) {
    if (sp < a.nsplit) {
      const int64_t p = p0 + sp * stride;
      const float2 ml = *reinterpret_cast<const float2*>(a.ws_ml + p * 2);
      mv[sp] = ml.x;
      lv[sp] = ml.y;
      ov[sp] = *reinterpret_cast<const f32x4_t*>(a.ws_o + p * HD + q4 * 4);
    }
  }
  float M = -INFINITY;
#pragma unroll
  for (int sp = 0; sp < CMB_FEW_SPLITS; ++sp)
    if (sp < a.nsplit && lv[sp] > 0.f) M = fmaxf(M, mv[sp]);
  float L = 0.f;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int sp = 0; sp < CMB_FEW_SPLITS; ++sp) {
    if (sp < a.nsplit && lv[sp] > 0.f) {
      const float wgt = __builtin_amdgcn_exp2f(mv[sp] - M);
      L += wgt * lv[sp];
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] += wgt * ov[sp][e];
    }
  }
  const float inv = L > 0.f ? 1.0f / L : 0.f;
  const int64_t qi = r / a.G;
  const int qh = head * a.G + (int)(r % a.G);
  bf16_t* op = a.out + (qi * a.hq + qh) * HD + q4 * 4;
  const u32x2_t o2 = {pack_bf(acc[0] * inv, acc[1] * inv), pack_bf(acc[2] * inv, acc[3] * inv)};
  *reinterpret_cast<u32x2_t*>(op) = o2;
}

struct SplitPlan {
  int nsplit, split_len;
  int64_t tiles;
  int nlong;    // one work group per key half for the nlong longest row tiles of each KV head
  bool decode;  // decode_attn_kernel: at most DEC_ROWS rows per KV head, keys split between waves
};

// Keys per decode_attn work group: at most about DEC_TARGET_WGS work groups over the cache (one
// per CU: each holds 134 KiB of LDS, so a few more would run as a second round), in whole 32-key
// tiles, at least four tiles (half the waves one each), and at most CMB_MAX_SPLITS slices. The
// floor matters for few KV heads over a short cache: at two tiles per wave a 0.5B-shaped step
// (2 KV heads, 8k keys) ran 38 work groups and a 1.5B-shaped one (16k keys) 66, each bound by one
// CU's share of HBM; with four tiles per work group, 130 and 254 (decoding step 0.867 -> 0.834 and
// 1.454 -> 1.409 ms; one tile per wave: 0.842 and 1.414).
constexpr int DEC_TARGET_WGS = 256;
constexpr int DEC_MIN_SPLIT = 4 * DEC_BK;

// Row tiles per KV head run as two half-range work groups when there is no key split and the
// launch is a few rounds of the GPU: a quarter of them (the longest). Simulated dispatch of the
// recompute shape (rows sorted by position, so row tile t sees about t / tiles of the context) on
// the 32 CUs of an XCD: 90 % of the ideal makespan with whole tiles longest first, 97-98 % with
// the longest quarter halved and dispatched first; measured 5 % faster (any quarter to two
// fifths alike). Launches of more rounds are balanced already and measured slower with halves:
// 1 % at 1 600 work groups (a 70B-shaped recompute, 8 KV heads), 1-2 % at 3 500 (a 32 000-row
// causal pass).
constexpr int ATT_LONG_MIN_TILES = 8;
constexpr int64_t ATT_LONG_MAX_WGS = 1536;

// Compute units of the current device, looked up once per device.
static int cu_count() {
  static std::mutex mu;
  static int cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  std::lock_guard<std::mutex> lock(mu);
  if (!cache[dev]) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
    cache[dev] = v;
  }
  return cache[dev];
}

static SplitPlan plan_split(int64_t n, int hq, int hkv, int head_dim, int64_t t_cap) {
  SplitPlan sp;
  sp.decode = false;
  if (n * (hq / hkv) <= DEC_ROWS) {
    sp.decode = true;
    sp.tiles = 1;
    sp.nlong = 0;
    const int64_t unit = DEC_BK;  // whole tiles; the waves take them round-robin
    int64_t len = (t_cap * hkv + DEC_TARGET_WGS - 1) / DEC_TARGET_WGS;
    if (len < DEC_MIN_SPLIT) len = DEC_MIN_SPLIT;
    if (len < (t_cap + CMB_MAX_SPLITS - 1) / CMB_MAX_SPLITS) len = (t_cap + CMB_MAX_SPLITS - 1) / CMB_MAX_SPLITS;
    len = (len + unit - 1) / unit * unit;
    sp.nsplit = (int)((t_cap + len - 1) / len);
    sp.split_len = (int)len;
    return sp;
  }
  sp.tiles = (n * (hq / hkv) + ATT_BM - 1) / ATT_BM;
  const int64_t base = (int64_t)hkv * sp.tiles;
  sp.nsplit = 1;
  sp.split_len = 0;
  sp.nlong = 0;
  if (base < ATT_TARGET_WGS && t_cap >= 2 * ATT_MIN_SPLIT_KEYS) {
    const bool many = base >= ATT_MANY_TILE_WGS;
    int64_t want = (ATT_TARGET_WGS + base - 1) / base;
    if (many) {
      // Many row tiles with ragged key ranges (recompute rows sorted by position): about three
      // work groups per CU over the launch, rounded, skipping multiples of 4; none when the row
      // tiles alone fill the CUs (then whole tiles, the longest in key halves). Swept in whole
      // requests on MI355X (deviation-selected rows, graph buckets, TTFT in one process): 0.5B 8k
      // (100 row-tile groups) 8.10 / 7.01 / 6.46 / 6.36 / 6.28 / 6.45 / 6.43 ms with 2 / 3 / 5 /
      // 6 / 7 / 9 / 11 slices, 1.5B 16k (158 groups) 21.76 / 19.63 / 19.42 / 19.94 / 19.74 /
      // 19.95 ms with 2 / 3 / 5 / 6 / 7 / 9; slice counts that are multiples of 4 were slow on
      // every shape swept. The 0.5B deviation pass (438 groups) ran 245 us in 3 slices and 201 us
      // in whole tiles with key halves.
      const int64_t cus = cu_count();
      want = base >= cus ? 1 : (6 * cus / base + 1) / 2;
      if (want >= 4 && want % 4 == 0) --want;
    }
    int64_t most = t_cap / (many ? 2 * ATT_MIN_SPLIT_KEYS : ATT_MIN_SPLIT_KEYS);
    int64_t ns = want < most ? want : most;
    if (ns > CMB_MAX_SPLITS) ns = CMB_MAX_SPLITS;
    if (ns > 1) {
      int64_t len = (t_cap + ns - 1) / ns;
      const int64_t bk = att_bk(head_dim);
      len = (len + bk - 1) / bk * bk;
      sp.nsplit = (int)((t_cap + len - 1) / len);
      sp.split_len = (int)len;
    }
  }
  if (sp.nsplit == 1 && sp.tiles >= ATT_LONG_MIN_TILES && base <= ATT_LONG_MAX_WGS) sp.nlong = (int)((sp.tiles + 2) / 4);
  return sp;
}

static size_t split_rows(const SplitPlan& sp, int hkv) {
  if (sp.decode) return sp.nsplit > 1 ? (size_t)sp.nsplit * hkv * DEC_ROWS : 0;
  if (sp.nsplit > 1) return (size_t)sp.nsplit * hkv * sp.tiles * ATT_BM;
  return (size_t)2 * hkv * sp.nlong * ATT_BM;
}

static size_t split_ws_bytes(const SplitPlan& sp, int hkv, int head_dim) {
  const size_t rows = split_rows(sp, hkv);
  return rows ? rows * (size_t)head_dim * 4 + rows * 8 + 256 : 0;
}

}  // namespace tread

using namespace tread;

static int subset_attn_impl(const void* q, const void* k_cache, const void* v_cache, const int64_t* kend,
                            const int64_t* kseg, int64_t n_shared, int64_t n, int hq, int hkv, int head_dim,
                            int64_t t_cap, float scale, void* out, void* ws, size_t ws_bytes, tread_stream_t stream);

// Merge the a.nsplit key-slice partials of every row (one work group, or with few slices one wave,
// per (KV head, row)).
static int launch_combine(const AttnArgs& a, int head_dim, hipStream_t s) {
  const int64_t blocks = (int64_t)a.hkv * a.n * a.G;
  if (a.nsplit <= CMB_FEW_SPLITS) {
    const int64_t rows_per_wg = (int64_t)HALF_ROWS * (64 / (head_dim / 4));
    const dim3 fgrid((unsigned)((blocks + rows_per_wg - 1) / rows_per_wg));
    if (head_dim == 128)
      hipLaunchKernelGGL(attn_combine_few_kernel<128>, fgrid, dim3(HALF_ROWS * 64), 0, s, a);
    else
      hipLaunchKernelGGL(attn_combine_few_kernel<64>, fgrid, dim3(HALF_ROWS * 64), 0, s, a);
    return check_launch("subset_attn combine");
  }
  if (head_dim == 128)
    hipLaunchKernelGGL(attn_combine_kernel<128>, dim3((unsigned)blocks), dim3(CMB_THREADS), 0, s, a);
  else
    hipLaunchKernelGGL(attn_combine_kernel<64>, dim3((unsigned)blocks), dim3(CMB_THREADS), 0, s, a);
  return check_launch("subset_attn combine");
}

// decode_attn_kernel over (key slice, KV head) work groups, then the slice merge (nsplit > 1).
static int decode_attn_launch(AttnArgs& a, const SplitPlan& sp, int head_dim, hipStream_t s) {
  a.prow = DEC_ROWS;
  const dim3 grid((unsigned)sp.nsplit, (unsigned)a.hkv);
  // the 8 waves' padded fp32 O rows of the merge (slightly more than their K and V tiles)
  const size_t smem = (size_t)DEC_WAVES * DEC_ROWS * (head_dim + 4) * sizeof(float);
  if (head_dim == 128)
    hipLaunchKernelGGL(decode_attn_kernel<128>, grid, dim3(DEC_THREADS), smem, s, a);
  else
    hipLaunchKernelGGL(decode_attn_kernel<64>, grid, dim3(DEC_THREADS), smem, s, a);
  int rc = check_launch("subset_attn decode");
  if (rc || sp.nsplit <= 1) return rc;
  return launch_combine(a, head_dim, s);
}

extern "C" size_t tread_subset_attn_workspace_bytes(int64_t n, int hq, int hkv, int head_dim, int64_t t_cap) {
  if (n <= 0 || hq <= 0 || hkv <= 0 || (hq % hkv) != 0 || t_cap <= 0) return 0;
  return split_ws_bytes(plan_split(n, hq, hkv, head_dim, t_cap), hkv, head_dim);
}

extern "C" int tread_subset_attn_bf16(const void* q, const void* k_cache, const void* v_cache, const int64_t* kend,
                                      const int64_t* kseg, int64_t n_shared, int64_t n, int hq, int hkv, int head_dim,
                                      int64_t t_cap, float scale, void* out, void* ws, size_t ws_bytes,
                                      tread_stream_t stream) {
  return subset_attn_impl(q, k_cache, v_cache, kend, kseg, n_shared, n, hq, hkv, head_dim, t_cap, scale, out, ws,
                          ws_bytes, stream);
}

// ---- the same attention with its fp32 partials in a static per-device scratch array -------------
// For callers that cannot allocate (graph capture, serving loops): the key-split and key-half
// partials live in `scratch`, a file-scope device array of TREAD_SUBSET_ATTN_SCRATCH_BYTES that each
// GPU the library runs on holds until the process ends. Host code never passes the array's name to
// a kernel (on the host it is only a stand-in): its device address is looked up once per device
// with hipGetSymbolAddress and kept in g_scratch_ptr. Every call on one GPU shares that GPU's
// array; nothing in it has to start at zero (every partial the merge kernels read is written by the
// attention kernel of the same call). Calls that use the array are ordered among themselves on
// each GPU: a call on another stream than the previous one first makes its stream wait for the
// event the previous call recorded after its launches (a host mutex orders the bookkeeping of calls
// from several threads). Calls on a stream under graph capture neither wait nor record (an event
// recorded outside the capture cannot be waited on inside it): ordering a captured graph against
// calls on other streams is the caller's, and such calls that overlap race.
static __device__ __align__(256) unsigned char scratch[TREAD_SUBSET_ATTN_SCRATCH_BYTES];

namespace {
constexpr int SCRATCH_MAX_DEVICES = 64;
std::mutex g_scratch_mu;
struct ScratchState {
  void* ptr = nullptr;          // device address of `scratch` on this device
  hipEvent_t done = nullptr;    // recorded after the last call's launches that used the array
  hipStream_t stream = nullptr; // that call's stream
  bool recorded = false;
};
ScratchState g_scratch[SCRATCH_MAX_DEVICES];
}  // namespace

// Set-up on the first call on a device (that device current): the address of `scratch` and the
// ordering event. Called with g_scratch_mu held.
static int scratch_state_for_current_device(ScratchState** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail((int)e, "subset_attn_scratch: hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= SCRATCH_MAX_DEVICES)
    return fail(TREAD_ERANGE, "subset_attn_scratch: device %d outside the %d supported", dev, SCRATCH_MAX_DEVICES);
  ScratchState& st = g_scratch[dev];
  if (!st.ptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(e != hipSuccess ? (int)e : TREAD_EINVAL, "subset_attn_scratch: hipGetSymbolAddress: %s",
                  hipGetErrorString(e));
    e = hipEventCreateWithFlags(&st.done, hipEventDisableTiming);
    if (e != hipSuccess) return fail((int)e, "subset_attn_scratch: hipEventCreate: %s", hipGetErrorString(e));
    st.ptr = p;
  }
  *out = &st;
  return 0;
}

extern "C" int tread_subset_attn_scratch_bf16(const void* q, const void* k_cache, const void* v_cache,
                                              const int64_t* kend, const int64_t* kseg, int64_t n_shared, int64_t n,
                                              int hq, int hkv, int head_dim, int64_t t_cap, float scale, void* out,
                                              tread_stream_t stream) {
  if (n == 0) return 0;
  if (n < 0 || hq <= 0 || hkv <= 0 || (hq % hkv) != 0 || t_cap <= 0)
    return fail(TREAD_EINVAL, "subset_attn_scratch: bad shape (n=%lld hq=%d hkv=%d)", (long long)n, hq, hkv);
  const size_t need = split_ws_bytes(plan_split(n, hq, hkv, head_dim, t_cap), hkv, head_dim);
  if (need > (size_t)TREAD_SUBSET_ATTN_SCRATCH_BYTES)
    return fail(TREAD_ERANGE,
                "subset_attn_scratch: this shape (n=%lld hq=%d hkv=%d head_dim=%d t_cap=%lld) needs %zu bytes of "
                "scratch, above the static maximum of %zu; call tread_subset_attn_bf16 with a workspace instead",
                (long long)n, hq, hkv, head_dim, (long long)t_cap, need, (size_t)TREAD_SUBSET_ATTN_SCRATCH_BYTES);
  if (!need)  // this plan keeps no partials: the array is not touched
    return subset_attn_impl(q, k_cache, v_cache, kend, kseg, n_shared, n, hq, hkv, head_dim, t_cap, scale, out,
                            nullptr, 0, stream);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  ScratchState* st = nullptr;
  int rc = scratch_state_for_current_device(&st);
  if (rc) return rc;
  hipStream_t s = (hipStream_t)stream;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(s, &cap);
  if (e != hipSuccess) return fail((int)e, "subset_attn_scratch: hipStreamIsCapturing: %s", hipGetErrorString(e));
  const bool capturing = cap != hipStreamCaptureStatusNone;
  if (!capturing && st->recorded && st->stream != s) {
    e = hipStreamWaitEvent(s, st->done, 0);
    if (e != hipSuccess) return fail((int)e, "subset_attn_scratch: hipStreamWaitEvent: %s", hipGetErrorString(e));
  }
  rc = subset_attn_impl(q, k_cache, v_cache, kend, kseg, n_shared, n, hq, hkv, head_dim, t_cap, scale, out, st->ptr,
                        (size_t)TREAD_SUBSET_ATTN_SCRATCH_BYTES, stream);
  if (rc || capturing) return rc;
  e = hipEventRecord(st->done, s);
  if (e != hipSuccess) return fail((int)e, "subset_attn_scratch: hipEventRecord: %s", hipGetErrorString(e));
  st->stream = s;
  st->recorded = true;
  return 0;
}

static int subset_attn_impl(const void* q, const void* k_cache, const void* v_cache, const int64_t* kend,
                            const int64_t* kseg, int64_t n_shared, int64_t n, int hq, int hkv, int head_dim,
                            int64_t t_cap, float scale, void* out, void* ws, size_t ws_bytes, tread_stream_t stream) {
  if (n == 0) return 0;
  if (n < 0 || hq <= 0 || hkv <= 0 || (hq % hkv) != 0 || t_cap <= 0)
    return fail(TREAD_EINVAL, "subset_attn: bad shape (n=%lld hq=%d hkv=%d)", (long long)n, hq, hkv);
  if (!q || !k_cache || !v_cache || !kend || !out) return fail(TREAD_EINVAL, "subset_attn: null pointer");
  if (head_dim != 64 && head_dim != 128) return fail(TREAD_EINVAL, "subset_attn: head_dim %d not in {64,128}", head_dim);
  // the one-slice decode plan rounds t_cap up to whole 256-key rounds of its waves in an int
  if (t_cap > 0x7fffffffLL - DEC_WAVES * DEC_BK) return fail(TREAD_ERANGE, "subset_attn: t_cap too large");
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
  SplitPlan sp = plan_split(n, hq, hkv, head_dim, t_cap);
  const size_t need = split_ws_bytes(sp, hkv, head_dim);
  if (need && (!ws || ws_bytes < need)) {  // no workspace: one pass per row tile (decode: one slice)
    sp.nsplit = 1;
    sp.nlong = 0;
    if (sp.decode) sp.split_len = (int)((t_cap + DEC_WAVES * DEC_BK - 1) / (DEC_WAVES * DEC_BK) * (DEC_WAVES * DEC_BK));
  }
  const int64_t vtiles = sp.tiles + sp.nlong;  // work groups per KV head without a key split
  if (vtiles > 0x7fffffffLL / N_XCD) return fail(TREAD_ERANGE, "subset_attn: too many rows");
  a.tiles = (int32_t)sp.tiles;
  a.nsplit = sp.nsplit;
  a.split_len = sp.split_len;
  a.nlong = sp.nlong;
  if (sp.nsplit > 1 || sp.nlong > 0) {
    uintptr_t base = ((uintptr_t)ws + 255) & ~(uintptr_t)255;
    a.ws_ml = (float*)base;
    a.ws_o = a.ws_ml + split_rows(sp, hkv) * 2;
  }
  a.scale_log2 = scale * 1.4426950408889634f;
  if (sp.decode) return decode_attn_launch(a, sp, head_dim, (hipStream_t)stream);
  a.prow = ATT_BM;
  int64_t grid;
  if (sp.nsplit > 1) {
    a.xpg = 0;
    grid = (int64_t)sp.nsplit * hkv * sp.tiles;
  } else if (hkv <= N_XCD && (N_XCD % hkv) == 0) {
    a.xpg = N_XCD / hkv;
    grid = (int64_t)N_XCD * ((vtiles + a.xpg - 1) / a.xpg);
  } else {
    a.xpg = 0;
    grid = (int64_t)hkv * vtiles;
  }
  if (grid > 0x7fffffffLL) return fail(TREAD_ERANGE, "subset_attn: grid too large");
  size_t smem = (head_dim == 128 ? AttnSmem<128>::BUF : AttnSmem<64>::BUF) * ATT_NBUF * sizeof(bf16_t);
  hipStream_t s = (hipStream_t)stream;
  if (head_dim == 128)
    hipLaunchKernelGGL(subset_attn_kernel<128>, dim3((unsigned)grid), dim3(ATT_THREADS), smem, s, a);
  else
    hipLaunchKernelGGL(subset_attn_kernel<64>, dim3((unsigned)grid), dim3(ATT_THREADS), smem, s, a);
  int rc = check_launch("subset_attn");
  if (rc) return rc;
  if (sp.nlong > 0) {
    const int64_t rows = (int64_t)hkv * sp.nlong * ATT_BM;
    const dim3 hgrid((unsigned)((rows + HALF_ROWS - 1) / HALF_ROWS));
    if (head_dim == 128)
      hipLaunchKernelGGL(attn_halves_kernel<128>, hgrid, dim3(HALF_ROWS * 64), 0, s, a);
    else
      hipLaunchKernelGGL(attn_halves_kernel<64>, hgrid, dim3(HALF_ROWS * 64), 0, s, a);
    return check_launch("subset_attn halves");
  }
  if (sp.nsplit <= 1) return rc;
  return launch_combine(a, head_dim, s);
}
