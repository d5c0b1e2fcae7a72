// (a) Fused RoPE re-rotation + gather/append of cached KV blocks into the assembled cache.
//
// One streaming pass over HBM: every source row is read once and written once. Within a work unit
// (source, layer, kv head, a span of token rows) the source rows and the destination rows are each
// one contiguous span, so K and V move as 16-byte vectors with non-temporal loads and stores. A
// unit is 4 KiB of ONE tensor, K or V (16 token rows at head_dim 128, 32 at 64), and thread t
// moves one 16-byte chunk of that span: the one-chunk-per-thread, one-stream-per-group shape of the
// fastest plain copy on this part (the 7B request's bytes without rotation: 6.1 TB/s, against
// 5.4-5.8 with K and V in one group). rotate_half's partner of a K chunk comes from another lane of
// the same 16-lane DPP row (row_ror:8). The source's cos/sin table (HD * 4 bytes) is staged in LDS
// once per group: read from the cache by every thread it would be 4x the unit's own bytes
// (measured 730 vs 627 us per 7B request).
// cos/sin come from a per-source fp32 table that the caller builds exactly as the reference's
// rotary embedding does. The rotation keeps the reference's fp32 op order with no contraction,
// fl(fl(x1*c) + fl(-x2*s)) and fl(fl(x2*c) + fl(x1*s)), then one RNE to bf16.
#include "common.h"
#include "../../include/tread_hip.h"

namespace tread {

constexpr int ASM_MAX_SRC = 48;
constexpr int ASM_THREADS = 256;

struct AsmSrc {
  const bf16_t* k;
  const bf16_t* v;
  int64_t n;
  int64_t dst_off;
  int32_t delta;
  int32_t unit_begin;
  int32_t chunks;
  int32_t pad;
};

constexpr int ASM_BUCKETS = 512;
static_assert(ASM_MAX_SRC < 128, "a bucket entry holds the source index in 7 bits");

struct AsmArgs {
  AsmSrc src[ASM_MAX_SRC];
  // byte b % 4 of word b / 4: the source of the first unit of work-group bucket b, bit 7 set when
  // the bucket's units reach into a later source
  uint32_t bucket_src[ASM_BUCKETS / 4];
  const float* cos_sin;  // [n_src][HD/2][2]: cos, sin of this launch's sources
  bf16_t* dk;
  bf16_t* dv;
  int64_t t_cap;
  int32_t n_src;
  int32_t n_kv;
  int32_t layer_lo;
  int32_t n_lr;  // layers in this launch
};

// Rows per work unit: one 16-byte chunk per thread of one row span of K or V.
template <int HD>
constexpr int asm_rows() { return ASM_THREADS / (HD / 8); }

// The unit's source (binary search over the sources' first units) and its row spans.
struct AsmUnit {
  int s;          // source index
  int rows;       // valid rows of the unit
  int64_t soff;   // element offset of the unit's first row in the source's K (and V)
  int64_t doff;   // element offset of its first destination row in the cache
};
// Work group b finds its source through bucket b >> GS of the launch's bucket table: GS is the
// smallest of ASM_SHIFTS that keeps the grid within ASM_BUCKETS buckets, a template argument of the
// kernels, so that the bucket word's address depends on the group index alone and its load is the
// group's first. A binary search over the sources instead took ~6 dependent scalar loads before
// the group's one 16-byte load per thread could go out (7B request: 646-652 -> 607-609 us).
constexpr int ASM_SHIFTS[] = {0, 4, 6, 8, 10, 12, 14, 16, 18, 20, 22};
static int asm_bucket_shift(int64_t groups) {
  for (int s : ASM_SHIFTS)
    if (((groups - 1) >> s) < ASM_BUCKETS) return s;
  return -1;
}

// The unit's source (the last one whose first unit is <= u: the bucket entry e's source, then, if
// the bucket reaches into later sources, forward past those that begin at or before u) and its
// row spans.
template <int HD>
__device__ __forceinline__ AsmUnit asm_unit_from(const AsmArgs& a, int u, uint32_t e) {
  constexpr int ROWS = asm_rows<HD>();
  int lo = e & 0x7f;
  if (e & 0x80)
    while (lo + 1 < a.n_src && a.src[lo + 1].unit_begin <= u) ++lo;
  const AsmSrc& src = a.src[lo];
  const int local = u - src.unit_begin;
  const int chunk = local % src.chunks;
  const int lh = local / src.chunks;
  const int head = lh % a.n_kv;
  const int layer = a.layer_lo + lh / a.n_kv;
  const int64_t row0 = (int64_t)chunk * ROWS;
  AsmUnit r;
  r.s = lo;
  r.rows = (int)min<int64_t>(ROWS, src.n - row0);
  r.soff = (((int64_t)layer * a.n_kv + head) * src.n + row0) * HD;
  r.doff = (((int64_t)layer * a.n_kv + head) * a.t_cap + src.dst_off + row0) * HD;
  return r;
}

// lane l ^ 8 of the same 16-lane row (DPP row_ror:8)
__device__ __forceinline__ uint32_t lane_xor8(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xf, 0xf, false);
}

// Work group b is unit b / 2, its K span for even b and its V span for odd b (K only, one group
// per unit, when the launch moves no V); thread t moves one 16-byte chunk of the span's 4 KiB.
// rotate_half's partner of K chunk j is chunk j ^ (CH / 2) of the same row; the chunks are dealt
// so that it sits at lane l ^ 8 of the same 16-lane DPP row (row_ror:8): at head_dim 128 thread t
// takes chunk t (16 chunks a row); at head_dim 64 (8 chunks a row) each 16-lane row takes two rows,
// lanes 0-3 / 4-7 the first / second row's chunks 0-3 and lanes 8-11 / 12-15 their chunks 4-7 (a
// wave still covers 1 KiB of contiguous rows).
template <int HD, int GS>
__global__ __launch_bounds__(ASM_THREADS) void rope_assemble_kernel(const AsmArgs a) {
  constexpr int HALF = HD / 2, CH = HD / 8;
  const int b = blockIdx.x;
  const int bk = b >> GS;  // this group's bucket word: the first load
  const uint32_t e = (a.bucket_src[bk >> 2] >> ((bk & 3) * 8)) & 0xffu;
  const bool has_v = a.dv != nullptr;  // uniform: a K-only launch (rotate_keys) moves no V
  const int u = has_v ? b >> 1 : b;  // the grid holds exactly the launch's (unit, tensor) spans
  const bool is_v = has_v && (b & 1);
  const AsmUnit w = asm_unit_from<HD>(a, u, e);
  const AsmSrc& src = a.src[w.s];
  const int c = threadIdx.x;
  if (is_v) {
    if (c / CH < w.rows)
      stg_nt(reinterpret_cast<u32x4_t*>(a.dv + w.doff) + c, ldg_nt(reinterpret_cast<const u32x4_t*>(src.v + w.soff) + c));
    return;
  }
  int sc = c;  // this thread's chunk of the K span
  if constexpr (HD == 64) {
    const int i = c & 15;
    sc = ((c >> 4) * 2 + ((i >> 2) & 1)) * CH + ((i & 3) | ((i >> 3) << 2));
  }
  const int r = sc / CH, j = sc % CH;
  const bool ok = r < w.rows;
  u32x4_t x = {0, 0, 0, 0};
  if (ok) x = ldg_nt(reinterpret_cast<const u32x4_t*>(src.k + w.soff) + sc);
  if (src.delta == 0) {  // a bit copy
    if (ok) stg_nt(reinterpret_cast<u32x4_t*>(a.dk + w.doff) + sc, x);
    return;
  }
  __shared__ f32x4_t tab_s[HALF * 2 / 4];  // (cos, sin) of the source's HALF columns
  if (c < HALF * 2 / 4) tab_s[c] = reinterpret_cast<const f32x4_t*>(a.cos_sin + (int64_t)w.s * HALF * 2)[c];
  __syncthreads();
  const int g = (j % (CH / 2)) * 4;  // columns (j % (CH / 2)) * 8 .. + 7
  const f32x4_t t0 = tab_s[g], t1 = tab_s[g + 1], t2 = tab_s[g + 2], t3 = tab_s[g + 3];
  u32x4_t p;  // partner chunk j ^ (CH / 2) (every lane of the row takes part, valid or not)
#pragma unroll
  for (int q = 0; q < 4; ++q) p[q] = lane_xor8(x[q]);
  if (!ok) return;
  const float cv[8] = {t0[0], t0[2], t1[0], t1[2], t2[0], t2[2], t3[0], t3[2]};
  const float sv[8] = {t0[1], t0[3], t1[1], t1[3], t2[1], t2[3], t3[1], t3[3]};
  // own chunk y, partner chunk p: first half y c + (-p) s, second half y c + p s
  const float sg = j < CH / 2 ? -1.f : 1.f;
  u32x4_t o;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float cl = cv[2 * q], ch = cv[2 * q + 1], sl = sv[2 * q], sh = sv[2 * q + 1];
    const float yl = lo_bf(x[q]), yh = hi_bf(x[q]);
    const float pl = sg * lo_bf(p[q]), ph = sg * hi_bf(p[q]);
    {
#pragma clang fp contract(off)
      o[q] = pack_bf(yl * cl + pl * sl, yh * ch + ph * sh);
    }
  }
  stg_nt(reinterpret_cast<u32x4_t*>(a.dk + w.doff) + sc, o);
}

}  // namespace tread

using namespace tread;

template <int GS>
static void launch_gs(int head_dim, dim3 grid, dim3 block, hipStream_t s, const AsmArgs& a) {
  if (head_dim == 128)
    hipLaunchKernelGGL((rope_assemble_kernel<128, GS>), grid, block, 0, s, a);
  else
    hipLaunchKernelGGL((rope_assemble_kernel<64, GS>), grid, block, 0, s, a);
}

static void launch_assemble(int head_dim, int gs, dim3 grid, dim3 block, hipStream_t s, const AsmArgs& a) {
  switch (gs) {
    case 0: launch_gs<0>(head_dim, grid, block, s, a); break;
    case 4: launch_gs<4>(head_dim, grid, block, s, a); break;
    case 6: launch_gs<6>(head_dim, grid, block, s, a); break;
    case 8: launch_gs<8>(head_dim, grid, block, s, a); break;
    case 10: launch_gs<10>(head_dim, grid, block, s, a); break;
    case 12: launch_gs<12>(head_dim, grid, block, s, a); break;
    case 14: launch_gs<14>(head_dim, grid, block, s, a); break;
    case 16: launch_gs<16>(head_dim, grid, block, s, a); break;
    case 18: launch_gs<18>(head_dim, grid, block, s, a); break;
    case 20: launch_gs<20>(head_dim, grid, block, s, a); break;
    default: launch_gs<22>(head_dim, grid, block, s, a); break;
  }
}

extern "C" int tread_rope_assemble_bf16(const tread_src_t* srcs, int n_src, void* dst_k, void* dst_v,
                                        int n_layers, int n_kv, int64_t t_cap, int head_dim,
                                        const float* cos_sin, int layer_lo, int layer_hi,
                                        tread_stream_t stream) {
  if (n_src < 0 || (n_src > 0 && !srcs)) return fail(TREAD_EINVAL, "rope_assemble: bad source list");
  if (n_src == 0) return 0;
  if (!dst_k || !cos_sin) return fail(TREAD_EINVAL, "rope_assemble: null pointer");
  if (head_dim != 64 && head_dim != 128) return fail(TREAD_EINVAL, "rope_assemble: head_dim %d not in {64,128}", head_dim);
  if (n_kv <= 0 || n_layers <= 0 || t_cap <= 0) return fail(TREAD_EINVAL, "rope_assemble: bad shape");
  if (layer_lo < 0 || layer_hi > n_layers || layer_lo >= layer_hi)
    return fail(TREAD_EINVAL, "rope_assemble: layer range [%d,%d) outside [0,%d)", layer_lo, layer_hi, n_layers);
  for (int i = 0; i < n_src; ++i) {
    const tread_src_t& s = srcs[i];
    if (s.n_tokens > 0 && (!s.k || (dst_v && !s.v)))  // an empty source moves nothing
      return fail(TREAD_EINVAL, "rope_assemble: source %d has a null pointer", i);
    if (s.n_tokens < 0 || s.dst_off < 0 || s.dst_off + s.n_tokens > t_cap)
      return fail(TREAD_ERANGE, "rope_assemble: source %d rows [%lld,%lld) outside the cache (t_cap %lld)", i,
                  (long long)s.dst_off, (long long)(s.dst_off + s.n_tokens), (long long)t_cap);
    if (s.delta > 0x7fffffffLL || s.delta < -0x7fffffffLL)
      return fail(TREAD_ERANGE, "rope_assemble: source %d delta out of range", i);
  }
  const int n_lr = layer_hi - layer_lo;
  for (int base = 0; base < n_src; base += ASM_MAX_SRC) {
    AsmArgs a;
    memset(&a, 0, sizeof(a));
    int cnt = 0;
    int64_t units = 0;
    const int end = n_src < base + ASM_MAX_SRC ? n_src : base + ASM_MAX_SRC;
    for (int i = base; i < end; ++i) {  // empty sources keep their slot: table row == source index
      const tread_src_t& s = srcs[i];
      AsmSrc& d = a.src[cnt++];
      d.k = (const bf16_t*)s.k;
      d.v = (const bf16_t*)s.v;
      d.n = s.n_tokens;
      d.dst_off = s.dst_off;
      d.delta = (int32_t)s.delta;
      const int rows_per_unit = head_dim == 128 ? asm_rows<128>() : asm_rows<64>();
      d.chunks = (int32_t)((s.n_tokens + rows_per_unit - 1) / rows_per_unit);
      d.unit_begin = (int32_t)units;
      units += (int64_t)n_lr * n_kv * d.chunks;
    }
    if (units == 0) continue;
    if (units > 0x7fffffffLL) return fail(TREAD_ERANGE, "rope_assemble: too many work units");
    // one work group per unit and tensor (K, V)
    const int64_t groups = dst_v ? 2 * units : units;
    const int gshift = asm_bucket_shift(groups), ushift = groups == units ? 0 : 1;
    if (groups > 0x7fffffffLL || gshift < 0) return fail(TREAD_ERANGE, "rope_assemble: too many work units");
    for (int b = 0, si = 0; b < ASM_BUCKETS; ++b) {  // the units of bucket b's groups
      const int64_t first = ((int64_t)b << gshift) >> ushift;
      const int64_t last = ((((int64_t)b + 1) << gshift) - 1) >> ushift;
      while (si + 1 < cnt && a.src[si + 1].unit_begin <= first) ++si;
      const bool mixed = si + 1 < cnt && a.src[si + 1].unit_begin <= last;
      a.bucket_src[b >> 2] |= (uint32_t)(si | (mixed ? 0x80 : 0)) << ((b & 3) * 8);
    }
    a.n_src = cnt;
    a.cos_sin = cos_sin + (int64_t)base * (head_dim / 2) * 2;
    a.dk = (bf16_t*)dst_k;
    a.dv = (bf16_t*)dst_v;
    a.t_cap = t_cap;
    a.n_kv = n_kv;
    a.layer_lo = layer_lo;
    a.n_lr = n_lr;
    dim3 grid((unsigned)groups), block(ASM_THREADS);
    launch_assemble(head_dim, gshift, grid, block, (hipStream_t)stream, a);
    int rc = check_launch("rope_assemble");
    if (rc) return rc;
  }
  return 0;
}
