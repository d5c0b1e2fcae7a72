// (c) Selective-recompute attention on CDNA4 MFMA (v_mfma_f32_32x32x16_bf16).
//
// Rows are (query token, query head) pairs of one KV head group: row r of KV head h is token
// r / G, query head h*G + r % G (G = hq / hkv), so the G heads that share a KV head share every
// K/V tile staged in LDS (GQA in-kernel, no repeat_kv). A work group of 4 waves owns 128 rows;
// each wave owns 32 rows and computes the transposed score block S^T = K Q^T, so that after the
// softmax its probabilities already sit in the B-operand layout of O^T = V^T P^T: every lane
// holds one query column for both products, and the online-softmax rescale is a per-lane scalar.
// K tiles are staged row-major [key][d]; V tiles are staged transposed [d][key] so the A operand
// of the PV product is two 8-byte LDS reads per lane. Tiles are double-buffered in LDS with one
// barrier per 64-key tile. The key range of a work group is the union of [0, n_shared) and
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

constexpr int ATT_WAVES = 4;
constexpr int ATT_THREADS = ATT_WAVES * 64;
constexpr int ATT_BM = ATT_WAVES * 32;  // rows per work group
constexpr int ATT_BK = 64;              // keys per tile
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

template <int HD>
struct AttnSmem {
  static constexpr int KSTR = HD + 8;      // Ks row stride (elements)
  static constexpr int VSTR = ATT_BK + 4;  // VT row stride (elements)
  static constexpr int K_ELEMS = ATT_BK * KSTR;
  static constexpr int V_ELEMS = HD * VSTR;
  static constexpr int BUF = K_ELEMS + V_ELEMS;
};

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
  constexpr int K_LD = ATT_BK * KCH / ATT_THREADS;  // K chunks per thread per tile
  constexpr int KPT = HD / 32;  // keys per thread in the V transpose (4 or 2)
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
  const int64_t r = (int64_t)tile * ATT_BM + wv * 32 + c;
  const bool valid = r < R;
  const int64_t qi = valid ? r / a.G : 0;
  const int qh = head * a.G + (int)(valid ? r % a.G : 0);
  int my_end = -1, my_seg = 0;
  if (valid) {
    int64_t e = a.kend[qi];
    my_end = (int)min<int64_t>(max<int64_t>(e, -1), a.t_cap - 1);
    if (a.kseg) my_seg = (int)min<int64_t>(max<int64_t>(a.kseg[qi], 0), a.t_cap);
  }
  const int n_shared = a.kseg ? (int)min<int64_t>(a.n_shared, a.t_cap) : 0;

  // ---- work-group key range
  {
    int vmax = wave_max(my_end);
    int vmin = wave_min(valid ? my_end : 0x7fffffff);
    int smax = wave_max(valid ? my_seg : 0);
    int smin = wave_min(valid ? my_seg : 0x7fffffff);
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
  bf16x8_t qf[KS];
  {
    const bf16_t* qp = a.q + (qi * a.hq + qh) * HD + half * 8;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      u32x4_t t = {0, 0, 0, 0};
      if (valid) t = *reinterpret_cast<const u32x4_t*>(qp + s * 16);
      qf[s] = __builtin_bit_cast(bf16x8_t, t);
    }
  }

  const bf16_t* kbase = a.k + (int64_t)head * a.t_cap * HD;
  const bf16_t* vbase = a.v + (int64_t)head * a.t_cap * HD;
  const int vdg = tid % KCH, vkg = tid / KCH;  // V transpose: d group, key group

  u32x4_t kreg[K_LD], vreg[KPT];
  auto tile_bounds = [&](int j, int& s0, int& s1) {
    if (j < nA) {
      s0 = startA + j * ATT_BK;
      s1 = min(s0 + ATT_BK, endA);
    } else {
      s0 = startB + (j - nA) * ATT_BK;
      s1 = min(s0 + ATT_BK, endB);
    }
  };
  auto gload = [&](int j) {
    int s0, s1;
    tile_bounds(j, s0, s1);
#pragma unroll
    for (int x = 0; x < K_LD; ++x) {
      int ch = tid + x * ATT_THREADS;
      int key = ch / KCH, cc = ch % KCH;
      u32x4_t t = {0, 0, 0, 0};
      if (s0 + key < s1) t = *reinterpret_cast<const u32x4_t*>(kbase + (int64_t)(s0 + key) * HD + cc * 8);
      kreg[x] = t;
    }
#pragma unroll
    for (int x = 0; x < KPT; ++x) {
      int key = vkg * KPT + x;
      u32x4_t t = {0, 0, 0, 0};
      if (s0 + key < s1) t = *reinterpret_cast<const u32x4_t*>(vbase + (int64_t)(s0 + key) * HD + vdg * 8);
      vreg[x] = t;
    }
  };
  auto lstore = [&](int buf) {
    bf16_t* Ks = smem + buf * SM::BUF;
    bf16_t* VT = Ks + SM::K_ELEMS;
#pragma unroll
    for (int x = 0; x < K_LD; ++x) {
      int ch = tid + x * ATT_THREADS;
      int key = ch / KCH, cc = ch % KCH;
      *reinterpret_cast<u32x4_t*>(Ks + key * SM::KSTR + cc * 8) = kreg[x];
    }
    // transpose: element e of key (vkg*KPT + x) goes to VT[vdg*8 + e][vkg*KPT + x]
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      uint32_t w[KPT];
#pragma unroll
      for (int x = 0; x < KPT; ++x) w[x] = (e & 1) ? (vreg[x][e >> 1] >> 16) : (vreg[x][e >> 1] & 0xffffu);
      bf16_t* dst = VT + (vdg * 8 + e) * SM::VSTR + vkg * KPT;
      if constexpr (KPT == 4) {
        u32x2_t pk = {w[0] | (w[1] << 16), w[2] | (w[3] << 16)};
        *reinterpret_cast<u32x2_t*>(dst) = pk;
      } else {
        *reinterpret_cast<uint32_t*>(dst) = w[0] | (w[1] << 16);
      }
    }
  };

  f32x16_t oacc[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d)
#pragma unroll
    for (int x = 0; x < 16; ++x) oacc[d][x] = 0.f;
  // running max (log2-scaled units) and sum of this lane's query row
  float m_run = -1e30f, l_run = 0.f;
  const float cs = a.scale_log2;

  if (ntiles > 0) {
    gload(0);
    lstore(0);
  }
  for (int j = 0; j < ntiles; ++j) {
    const int buf = j & 1;
    __syncthreads();
    if (j + 1 < ntiles) gload(j + 1);
    const bf16_t* Ks = smem + buf * SM::BUF;
    const bf16_t* VT = Ks + SM::K_ELEMS;
    int s0, s1;
    tile_bounds(j, s0, s1);

    // S^T = K Q^T for two 32-key blocks (raw, unscaled scores)
    f32x16_t sacc[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int x = 0; x < 16; ++x) sacc[kb][x] = 0.f;
      const bf16_t* kr = Ks + (kb * 32 + c) * SM::KSTR + half * 8;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        bf16x8_t af = *reinterpret_cast<const bf16x8_t*>(kr + s * 16);
        sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, qf[s], sacc[kb], 0, 0, 0);
      }
    }
    // mask, row max (raw scores; the scale is positive so it commutes with max)
    const bool full = (s1 - s0 == ATT_BK) && (s1 - 1 <= kmin) && (j < nA || s0 >= segmax);
    if (!full) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int x = 0; x < 16; ++x) {
          int key = s0 + kb * 32 + (x >> 2) * 8 + half * 4 + (x & 3);
          bool vis = key < s1 && key <= my_end && (key < n_shared || key >= my_seg);
          sacc[kb][x] = vis ? sacc[kb][x] : -INFINITY;
        }
    }
    float tmax = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int x = 0; x < 16; ++x) tmax = fmaxf(tmax, sacc[kb][x]);
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
    const float m_new = fmaxf(m_run, tmax * cs);
    // rescale the running sum and O only if some row's max moved (rare after the first tiles)
    if (__ballot(m_new > m_run)) {
      const float corr = __builtin_amdgcn_exp2f(m_run - m_new);
      l_run *= corr;
#pragma unroll
      for (int d = 0; d < DB; ++d)
#pragma unroll
        for (int x = 0; x < 16; ++x) oacc[d][x] *= corr;
    }
    m_run = m_new;
    float rs = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int x = 0; x < 16; ++x) {
        float p = __builtin_amdgcn_exp2f(fmaf(sacc[kb][x], cs, -m_new));
        sacc[kb][x] = p;
        rs += p;
      }
    rs += __shfl_xor(rs, 32);
    l_run += rs;

    // O^T += V^T P^T over 4 k-steps of 16 keys
#pragma unroll
    for (int s = 0; s < ATT_BK / 16; ++s) {
      const int kb = s >> 1, base = (s & 1) * 8;
      u32x4_t pw;
#pragma unroll
      for (int q = 0; q < 4; ++q) pw[q] = pack_bf(sacc[kb][base + 2 * q], sacc[kb][base + 2 * q + 1]);
      const bf16x8_t pb = __builtin_bit_cast(bf16x8_t, pw);
#pragma unroll
      for (int d = 0; d < DB; ++d) {
        const bf16_t* vr = VT + (d * 32 + c) * SM::VSTR + s * 16 + half * 4;
        u32x2_t lo = *reinterpret_cast<const u32x2_t*>(vr);
        u32x2_t hi = *reinterpret_cast<const u32x2_t*>(vr + 8);
        u32x4_t av = {lo[0], lo[1], hi[0], hi[1]};
        oacc[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, av), pb, oacc[d], 0, 0, 0);
      }
    }
    if (j + 1 < ntiles) lstore(buf ^ 1);
  }

  if (!valid) return;
  if (a.nsplit > 1) {
    // partial for the combine kernel: unnormalised O, running max and sum
    const int64_t p = (((int64_t)split * a.hkv + head) * a.tiles + tile) * ATT_BM + wv * 32 + c;
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
