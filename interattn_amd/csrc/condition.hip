// Condition-block (eps-threshold) routing for gfx950: the reference's own
// selection rule, next to the top-k rule of select_topk.hip.
//
//   ia_condition_block_selection_stats  (CBT/core.py:747-814)
//     grid = (n_chunks, Hkv, batch), 256 threads: workgroup c owns chunk c of 16
//     blocks (the reference's _SELECT_CHUNK), wave w its step of 4 blocks, so each
//     wave runs a short dependency chain and a SIMD holds several.  Per block and
//     query row: s = q.k_bar/sqrt(D), the range bound upper/lower
//     from the sign of q against k_max/k_min, delta = max(|upper-s|, |lower-s|),
//     z = s + log(max(count,1)), zc = z + log cosh(delta) (or z + delta for the
//     term1-mass-exp variant); one k_bar/k_max/k_min row per 16 lanes, DPP row
//     sums.  Writes s, delta and the chunk's (max, sum-exp) partials of z and zc.
//   ia_condition_block_selection_reduce  (CBT/core.py:821-847)
//     log-sum-exp merge of the chunk partials into per-row globals.
//   ia_condition_block_selection_select  (CBT/core.py:854-905)
//     term1 = 2 B_all e^(z-c_m)/c_l (cosh delta - 1), term2 = 2 b_c e^(z-z_m)/z_l
//     tanh(delta/2); selected = mean_g(term1 + term2) > eps (and the block exists).
//   ia_condition_block_route  (CBT/page_attention.py:104-204)
//     one workgroup per 256 blocks of a (sequence, kv head): reduces the chunk
//     partials inline, thresholds, writes the selected flags, compacts the
//     selected block ids (wave ballots) for the finalize, and computes the
//     representative softmax partial of the unselected blocks: logit z, value
//     v_bar, weight beta, fp32 sums.  For bfloat16 caches value and weight are
//     rounded to bfloat16 (the reference's cast points, CBT/page_attention.py:
//     194-201); float32 caches stay float32 throughout.  In fixed-mask mode the
//     selection comes from a caller mask and the logit is recomputed as
//     q.k_bar/sqrt(D) + log(count), with q and k_bar rounded to bfloat16 for
//     bfloat16 caches (CBG/real_attention_benchmark/fixed_mask.py:86-107).
//   The selected blocks and the exact suffix are then streamed by the paged
//   finalize (kSrcLists) and merged with the representative partials.
#include <algorithm>
#include <string>

#include "paged_decode_kernel.hpp"

namespace ia {
namespace {

constexpr int kChunk16 = 16;  // blocks per selection-stats partial

struct CondParams {
  const void* q;
  int64_t q_batch_stride, q_row_stride;
  int32_t q_f32;
  const void* k_bar;
  const void* k_max;
  const void* k_min;
  int32_t bounds_packed;  // k_max is the packed k_bounds (pairs per dimension), k_min unused
  const void* v_bar;
  const float* v_norm_max;  // [batch, Hkv, nb]
  const float* v_norm_all;  // [batch, Hkv]
  const int32_t* counts;    // [batch, nb]
  int32_t nb, n_kv_heads, n_chunks;
  float scale;  // 1/sqrt(D)
  int32_t mass_exp;
  float eps;
  float* s;        // [batch, rows, nb]
  float* delta;    // [batch, rows, nb]
  float* partial;  // [batch, 4, rows, n_chunks]
  float* globals;  // [batch, 4, rows]
  uint8_t* selected;  // [batch, rows, nb] (optional)
  float* z_out;       // [batch, rows, nb] (optional)
  int32_t* rc_counts;  // [batch*Hkv, n_rc]
  int32_t* rc_lists;   // [batch*Hkv, n_rc, kRouteChunk]
  int32_t n_rc;
  float* rep_ml;   // [batch*Hkv, n_rc, G, 2]
  float* rep_acc;  // [batch*Hkv, n_rc, G, D]
  const uint8_t* mask;  // fixed-mask mode: [batch, Hkv, nb]
  int32_t rep_bf16;     // bfloat16 caches: representative operands rounded to bfloat16
};

// Raw words of one row slice of DPL elements (bf16 pairs or floats): loads are
// issued before any use so a wave keeps all of its rows in flight at once.
template <bool BF16, int DPL>
struct RawRow {
  static constexpr int kWords = BF16 ? DPL / 2 : DPL;
  u32 w[kWords];
  __device__ __forceinline__ void load(const void* base, int64_t off) {
    if constexpr (BF16) {
      const unsigned short* p = reinterpret_cast<const unsigned short*>(base) + off;
      if constexpr (DPL == 8) {
        const u32x4_t v = ld_stream16(p);
        w[0] = v[0]; w[1] = v[1]; w[2] = v[2]; w[3] = v[3];
      } else {
        const u32x2_t v = ld_stream8(p);
        w[0] = v[0]; w[1] = v[1];
      }
    } else {
      const float* p = reinterpret_cast<const float*>(base) + off;
#pragma unroll
      for (int e = 0; e < DPL; e += 4) {
        const u32x4_t v = ld_stream16(p + e);
        w[e] = v[0]; w[e + 1] = v[1];
        w[e + 2] = v[2]; w[e + 3] = v[3];
      }
    }
  }
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int i = 0; i < kWords; ++i) w[i] = 0u;
  }
  __device__ __forceinline__ float operator[](int e) const {
    if constexpr (BF16) return (e & 1) ? bf16_hi(w[e >> 1]) : bf16_lo(w[e >> 1]);
    else return __uint_as_float(w[e]);
  }
};

// k_max / k_min of one row slice: the separate rows, or the packed k_bounds row whose
// pair (k_max, k_min) of dimension e sits at [2e, 2e + 1] (CBT/core.py:490-499).  The
// same two loads of DPL elements either way, chosen without a branch.
template <bool BF16, int DPL>
struct RawBounds {
  RawRow<BF16, DPL> a, b;
  bool packed;
  __device__ __forceinline__ void load(const void* kmax, const void* kmin, int64_t off, bool pk) {
    packed = pk;
    a.load(kmax, pk ? 2 * off : off);
    b.load(pk ? kmax : kmin, pk ? 2 * off + DPL : off);
  }
  __device__ __forceinline__ void zero() {
    a.zero();
    b.zero();
    packed = false;
  }
  // (both candidates are read first and passed through an empty asm, so the choice
  // is between two values: a choice between two elements of one row would be turned
  // into a row index chosen at run time, which puts the rows in scratch memory)
  __device__ __forceinline__ static float pick(bool pk, float x, float y) {
    asm("" : "+v"(x), "+v"(y));
    return pk ? x : y;
  }
  __device__ __forceinline__ float mx(int e) const {
    return e < DPL / 2 ? pick(packed, a[2 * e], a[e]) : pick(packed, b[2 * e - DPL], a[e]);
  }
  __device__ __forceinline__ float mn(int e) const {
    return e < DPL / 2 ? pick(packed, a[2 * e + 1], b[e]) : pick(packed, b[2 * e + 1 - DPL], b[e]);
  }
};

__device__ __forceinline__ float q_elem(const CondParams& p, int64_t off) {
  return p.q_f32 ? reinterpret_cast<const float*>(p.q)[off]
                 : __uint_as_float((u32)reinterpret_cast<const unsigned short*>(p.q)[off] << 16);
}

// (m, l) <- log-sum-exp merge of (m, l) and (m2, l2); m = -inf marks an empty partial
__device__ __forceinline__ void lse_merge(float& m, float& l, float m2, float l2) {
  const float mn = fmaxf(m, m2);
  if (mn == kNegInf) return;
  l = (m == kNegInf ? 0.f : l * __expf(m - mn)) + (m2 == kNegInf ? 0.f : l2 * __expf(m2 - mn));
  m = mn;
}

// Per-row globals (z_m, z_l, c_m, c_l) of the G query rows of kv head h from the
// 16-block chunk partials, by a whole 256-thread workgroup: every chunk's partials
// are loaded at once (one round trip), merged per thread, then the maxima and the
// rescaled sums are reduced over lanes and waves.  glob[v][g] in LDS on return
// (v = 0..3 as above).
template <int G>
__device__ __forceinline__ void reduce_globals(const CondParams& p, int b, int h, float (*glob)[G],
                                               float (*red)[2 * G]) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int rows = p.n_kv_heads * G;
  const int64_t plane = (int64_t)rows * p.n_chunks;
  const float* base = p.partial + (int64_t)b * 4 * plane + (int64_t)h * G * p.n_chunks;
  float m[2 * G], l[2 * G];  // pair i = (value v = i / G, row g = i % G)
#pragma unroll
  for (int i = 0; i < 2 * G; ++i) {
    m[i] = kNegInf;
    l[i] = 0.f;
  }
  for (int c = threadIdx.x; c < p.n_chunks; c += 256) {
    float mc[2 * G], lc[2 * G];
#pragma unroll
    for (int i = 0; i < 2 * G; ++i) {
      const float* row = base + (int64_t)(i % G) * p.n_chunks + c;
      mc[i] = row[(2 * (i / G)) * plane];
      lc[i] = row[(2 * (i / G) + 1) * plane];
    }
#pragma unroll
    for (int i = 0; i < 2 * G; ++i) lse_merge(m[i], l[i], mc[i], lc[i]);
  }
  float M[2 * G];
#pragma unroll
  for (int i = 0; i < 2 * G; ++i) {
    const float mw = wave_max(m[i]);
    if (lane == 0) red[wave][i] = mw;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 2 * G; ++i) M[i] = fmaxf(fmaxf(red[0][i], red[1][i]), fmaxf(red[2][i], red[3][i]));
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 2 * G; ++i) {
    const float t = wave_sum(m[i] == kNegInf ? 0.f : l[i] * __expf(m[i] - M[i]));
    if (lane == 0) red[wave][i] = t;
  }
  __syncthreads();
  if (threadIdx.x < 2 * G) {
    const int i = threadIdx.x;
    glob[2 * (i / G)][i % G] = M[i];
    glob[2 * (i / G) + 1][i % G] = red[0][i] + red[1][i] + red[2][i] + red[3][i];
  }
  __syncthreads();
}

// ---------------------------------------------------------------- selection stats

template <int D, int G, bool KBH, bool BDH>
__global__ __launch_bounds__(256) void ia_condition_block_selection_stats(CondParams p) {
  constexpr int DPL = D / 16;
  __shared__ float z_lds[2][4][64];  // (z, zc) of step w at lane (r, c16) of wave w
  const int lane = threadIdx.x & 63;
  const int step = threadIdx.x >> 6;  // wave w scores step w: blocks chunk*16 + 4w + (0..3)
  const int c16 = lane & 15;
  const int r = lane >> 4;
  const int chunk = blockIdx.x;
  const int h = blockIdx.y;
  const int b = blockIdx.z;

  // this wave's four key rows (k_bar, k_max, k_min), its counts and the group's
  // query slices, all issued before any use
  const int64_t vbase = ((int64_t)b * p.n_kv_heads + h) * p.nb;
  const int j = chunk * kChunk16 + 4 * step + r;
  const bool inb = j < p.nb;
  const int cnt = inb ? p.counts[(int64_t)b * p.nb + j] : 0;
  RawRow<KBH, DPL> rb;
  RawBounds<BDH, DPL> rx;
  if (inb) {
    const int64_t off = (vbase + j) * D + c16 * DPL;
    rb.load(p.k_bar, off);
    rx.load(p.k_max, p.k_min, off, p.bounds_packed);
  } else {
    rb.zero();
    rx.zero();
  }
  // q rows h*G + g at dims c16*DPL ..: one 16-byte (bf16) or DPL/4 16-byte (f32) loads
  u32 qw[G][DPL];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int64_t qo = (int64_t)b * p.q_batch_stride + (int64_t)(h * G + g) * p.q_row_stride + c16 * DPL;
    if (p.q_f32) {
      const u32* qp = reinterpret_cast<const u32*>(p.q) + qo;
#pragma unroll
      for (int e = 0; e < DPL; ++e) qw[g][e] = qp[e];
    } else {
      const unsigned short* qp = reinterpret_cast<const unsigned short*>(p.q) + qo;
#pragma unroll
      for (int e = 0; e < DPL; ++e) qw[g][e] = (u32)qp[e] << 16;
    }
  }

  const bool active = cnt > 0;
  // upper/lower = sum q+ k_max + q- k_min / sum q+ k_min + q- k_max, i.e. with
  // A = sum q (k_max + k_min) and B = sum |q| (k_max - k_min) >= 0:
  // upper = (A + B)/2, lower = (A - B)/2 and delta = |A/2 - s| + B/2
  float ksum[DPL], kdif[DPL];
#pragma unroll
  for (int e = 0; e < DPL; ++e) {
    ksum[e] = rx.mx(e) + rx.mn(e);
    kdif[e] = rx.mx(e) - rx.mn(e);
  }
  float ps[G], pa[G], pb[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float a = 0.f, sa = 0.f, sb = 0.f;
#pragma unroll
    for (int e = 0; e < DPL; ++e) {
      const float qv = __uint_as_float(qw[g][e]);
      a = fmaf(qv, rb[e], a);
      sa = fmaf(qv, ksum[e], sa);
      sb = fmaf(fabsf(qv), kdif[e], sb);
    }
    ps[g] = row16_sum(a);
    pa[g] = row16_sum(sa);
    pb[g] = row16_sum(sb);
  }
  // lane c16 < G finishes row g = c16
  float sv = 0.f, av = 0.f, bv = 0.f;
#pragma unroll
  for (int g = 0; g < G; ++g)
    if (g == c16) {
      sv = ps[g];
      av = pa[g];
      bv = pb[g];
    }
  sv *= p.scale;
  const float dl = fabsf(0.5f * av * p.scale - sv) + 0.5f * bv * p.scale;
  const float z = active ? sv + __logf((float)max(cnt, 1)) : kNegInf;
  const float zc = active ? (p.mass_exp ? z + dl : z + log_cosh(dl)) : kNegInf;
  if (c16 < G && inb) {
    const int64_t o = ((int64_t)b * (p.n_kv_heads * G) + h * G + c16) * p.nb + j;
    p.s[o] = active ? sv : 0.f;
    p.delta[o] = active ? dl : 0.f;
  }
  z_lds[0][step][lane] = z;
  z_lds[1][step][lane] = zc;
  __syncthreads();
  if (step != 0) return;
  // chunk partials over the 16 blocks: 4 steps in-lane, 4 rows across lanes (wave 0
  // reads every step's values at its own lane, so the sums run in step order)
  float zs[4], zcs[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    zs[t] = z_lds[0][t][lane];
    zcs[t] = z_lds[1][t][lane];
  }
  float mz = fmaxf(fmaxf(zs[0], zs[1]), fmaxf(zs[2], zs[3]));
  float mc = fmaxf(fmaxf(zcs[0], zcs[1]), fmaxf(zcs[2], zcs[3]));
  mz = rows_max(mz);
  mc = rows_max(mc);
  float lz = 0.f, lc = 0.f;
  if (mz != kNegInf) {
#pragma unroll
    for (int t = 0; t < 4; ++t) lz += (zs[t] == kNegInf) ? 0.f : __expf(zs[t] - mz);
  }
  if (mc != kNegInf) {
#pragma unroll
    for (int t = 0; t < 4; ++t) lc += (zcs[t] == kNegInf) ? 0.f : __expf(zcs[t] - mc);
  }
  lz = rows_sum(lz);
  lc = rows_sum(lc);
  if (r == 0 && c16 < G) {
    const int rows = p.n_kv_heads * G;
    const int64_t base = (int64_t)b * 4 * rows * p.n_chunks + (int64_t)(h * G + c16) * p.n_chunks + chunk;
    const int64_t plane = (int64_t)rows * p.n_chunks;
    p.partial[base] = mz;
    p.partial[base + plane] = lz;
    p.partial[base + 2 * plane] = mc;
    p.partial[base + 3 * plane] = lc;
  }
}

// grid (Hkv, batch): the chunk partials of one kv head's rows -> globals [batch, 4, rows]
template <int G>
__global__ __launch_bounds__(256) void ia_condition_block_selection_reduce(CondParams p) {
  __shared__ float glob[4][G];
  __shared__ float red[4][2 * G];
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  reduce_globals<G>(p, b, h, glob, red);
  if (threadIdx.x < 4 * G) {
    const int v = threadIdx.x / G, g = threadIdx.x % G;
    const int rows = p.n_kv_heads * G;
    p.globals[(int64_t)b * 4 * rows + (int64_t)v * rows + h * G + g] = glob[v][g];
  }
}

template <int G>
__global__ __launch_bounds__(256) void ia_condition_block_selection_select(CondParams p) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  const int h = blockIdx.y;
  const int b = blockIdx.z;
  if (j >= p.nb) return;
  const int rows = p.n_kv_heads * G;
  const int cnt = p.counts[(int64_t)b * p.nb + j];
  const bool active = cnt > 0;
  const float lc = __logf((float)max(cnt, 1));
  const float b_c = active ? p.v_norm_max[((int64_t)b * p.n_kv_heads + h) * p.nb + j] : 0.f;
  const float b_all = p.v_norm_all[(int64_t)b * p.n_kv_heads + h];
  float z[G], mean = 0.f;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int row = h * G + g;
    const int64_t o = ((int64_t)b * rows + row) * p.nb + j;
    const float s = active ? p.s[o] : 0.f;
    const float dl = active ? p.delta[o] : 0.f;
    z[g] = active ? s + lc : kNegInf;
    const float* gl = p.globals + (int64_t)b * 4 * rows;
    if (active)
      mean += condition_value(dl, z[g], gl[row], 1.f / gl[rows + row], gl[2 * rows + row], 1.f / gl[3 * rows + row],
                              b_c, b_all, p.mass_exp);
  }
  mean /= (float)G;
  const uint8_t sel = (active && mean > p.eps) ? 1 : 0;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int64_t o = ((int64_t)b * rows + h * G + g) * p.nb + j;
    if (p.selected) p.selected[o] = sel;
    if (p.z_out) p.z_out[o] = z[g];
  }
}

// ---------------------------------------------------------------- route + representatives

template <int D, int G, bool VBH, bool KBH, bool MASK>
__global__ __launch_bounds__(256) void ia_condition_block_route(CondParams p) {
  constexpr int DPL = D / 16;
  __shared__ float z_lds[G][kRouteChunk];
  __shared__ float red[8][G];
  __shared__ float glob[4][G];
  __shared__ float gred[4][2 * G];
  __shared__ int wcnt[4];
  __shared__ float wacc[4][G * D];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c16 = lane & 15;
  const int r = lane >> 4;
  const int rc = blockIdx.x;
  const int h = blockIdx.y;
  const int b = blockIdx.z;
  const int bh = b * p.n_kv_heads + h;
  const int rows = p.n_kv_heads * G;
  const int j = rc * kRouteChunk + threadIdx.x;
  const bool inb = j < p.nb;

  // ---- v_bar rows of the chunk (16 per 16-lane row), issued first: at low selection
  // fractions almost every block is a representative, so they are all needed
  constexpr int kRows = kRouteChunk / 16;
  RawRow<VBH, DPL> vr[kRows];
#pragma unroll
  for (int t = 0; t < kRows; ++t) {
    const int jj = rc * kRouteChunk + 16 * t + 4 * wave + r;
    if (jj < p.nb) vr[t].load(p.v_bar, ((int64_t)bh * p.nb + jj) * D + c16 * DPL);
    else vr[t].zero();
  }
  // fixed-mask mode with bfloat16 k_bar: the k_bar rows of the same rows, issued with
  // them (every row: the few selected ones are read and not used); float32 k_bar rows
  // are read later, a batch at a time (registers)
  constexpr bool kPreK = MASK && KBH;
  RawRow<KBH, DPL> kr[kPreK ? kRows : 1];
  if constexpr (kPreK) {
#pragma unroll
    for (int t = 0; t < kRows; ++t) {
      const int jj = rc * kRouteChunk + 16 * t + 4 * wave + r;
      if (jj < p.nb) kr[t].load(p.k_bar, ((int64_t)bh * p.nb + jj) * D + c16 * DPL);
      else kr[t].zero();
    }
  }

  // ---- this thread's block: count and statistics, loaded before the globals reduce
  const int cnt = inb ? p.counts[(int64_t)b * p.nb + j] : 0;
  float s_g[G], d_g[G];
  float b_c = 0.f, b_all = 0.f;
  bool msel = false;
  if constexpr (MASK) {
    msel = inb && p.mask[(int64_t)bh * p.nb + j] != 0;
  } else {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int64_t o = ((int64_t)b * rows + h * G + g) * p.nb + j;
      s_g[g] = inb ? p.s[o] : 0.f;
      d_g[g] = inb ? p.delta[o] : 0.f;
    }
    b_c = inb ? p.v_norm_max[(int64_t)bh * p.nb + j] : 0.f;
    b_all = p.v_norm_all[bh];
    reduce_globals<G>(p, b, h, glob, gred);
  }
  const bool active = cnt > 0;
  const float logc = __logf((float)max(cnt, 1));

  // ---- routing of this thread's block
  bool sel = false;
  if constexpr (MASK) {
    sel = active && msel;  // (the logits are computed below)
  } else {
    float z[G], mean = 0.f;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      z[g] = active ? s_g[g] + logc : kNegInf;
      if (active)
        mean += condition_value(d_g[g], z[g], glob[0][g], 1.f / glob[1][g], glob[2][g], 1.f / glob[3][g], b_c, b_all,
                                p.mass_exp);
    }
    mean /= (float)G;
    sel = active && mean > p.eps;
#pragma unroll
    for (int g = 0; g < G; ++g) z_lds[g][threadIdx.x] = (active && !sel) ? z[g] : kNegInf;
  }
  if (p.selected && inb) {
#pragma unroll
    for (int g = 0; g < G; ++g) p.selected[((int64_t)b * rows + h * G + g) * p.nb + j] = sel ? 1 : 0;
  }

  // ---- compaction of the selected blocks, ascending
  const unsigned long long ballot = __ballot(sel);
  if (lane == 0) wcnt[wave] = __popcll(ballot);
  __syncthreads();
  int off = 0;
  for (int w = 0; w < wave; ++w) off += wcnt[w];
  if (sel)
    p.rc_lists[((int64_t)bh * p.n_rc + rc) * kRouteChunk + off + __popcll(ballot & ((1ull << lane) - 1ull))] =
        list_entry(j, cnt);
  if (threadIdx.x == 0) p.rc_counts[(int64_t)bh * p.n_rc + rc] = wcnt[0] + wcnt[1] + wcnt[2] + wcnt[3];

  // ---- fixed-mask mode: representative logits q.k_bar/sqrt(D) + log(count)
  if constexpr (MASK) {
    float qb[G][DPL];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < DPL; ++e) {
        const float qv = q_elem(p, (int64_t)b * p.q_batch_stride + (int64_t)(h * G + g) * p.q_row_stride + c16 * DPL + e);
        qb[g][e] = round_if(qv, p.rep_bf16);
      }
    // q_g . k_bar of the lane-row's blocks: the lane's partial sums of RPG rows x G
    // query rows are reduce-scattered over the 16 lanes of the row (four DPP steps for
    // all of them) and each complete sum goes to z_lds; the block's owner then applies
    // the scale and log(count), or -inf for a selected or empty block
    // (bfloat16 rows: all kRows preloaded; float32 rows: 8 at a time, so at most 8 rows
    // per reduce-scatter)
    constexpr int kRowsIn = KBH ? kRows : 8;                    // k_bar rows in flight
    constexpr int NVR = G * kRowsIn >= 32 ? 32 : G * kRowsIn;  // values per reduce-scatter
    constexpr int RPG = NVR / G;                                // rows per reduce-scatter
    auto dots = [&](int tbase, auto&& kval) {
      float v[NVR];
#pragma unroll
      for (int tt = 0; tt < RPG; ++tt)
#pragma unroll
        for (int g = 0; g < G; ++g) {
          float a = 0.f;
#pragma unroll
          for (int e = 0; e < DPL; ++e) a = fmaf(qb[g][e], kval(tt, e), a);
          v[tt * G + g] = a;
        }
      reduce_scatter16<NVR>(v, lane);
      const int b16 = lane & 15;
#pragma unroll
      for (int k = 0; k < NVR / 16; ++k) {
        const int x = NVR == 32 ? 2 * b16 + k : b16 / (16 / NVR);  // value index held in v[k]
        const int tt = x / G;
        z_lds[x - tt * G][16 * (tbase + tt) + 4 * wave + r] = v[k];
      }
    };
    if constexpr (kPreK) {
#pragma unroll
      for (int t0 = 0; t0 < kRows; t0 += RPG) dots(t0, [&](int tt, int e) { return kr[t0 + tt][e]; });
    } else {
      for (int t0 = 0; t0 < kRows; t0 += kRowsIn) {
        RawRow<KBH, DPL> kq[kRowsIn];
#pragma unroll
        for (int u = 0; u < kRowsIn; ++u) {
          const int jj = rc * kRouteChunk + 16 * (t0 + u) + 4 * wave + r;
          if (jj < p.nb) kq[u].load(p.k_bar, ((int64_t)bh * p.nb + jj) * D + c16 * DPL);
          else kq[u].zero();
        }
#pragma unroll
        for (int u0 = 0; u0 < kRowsIn; u0 += RPG)
          dots(t0 + u0, [&](int tt, int e) { return round_if(kq[u0 + tt][e], p.rep_bf16); });
      }
    }
    __syncthreads();  // every block's dots in z_lds
    {  // thread t owns block t of the chunk
      const bool rep = active && !msel;
#pragma unroll
      for (int g = 0; g < G; ++g) z_lds[g][threadIdx.x] = rep ? z_lds[g][threadIdx.x] * p.scale + logc : kNegInf;
    }
  }
  __syncthreads();

  // ---- representative softmax partial: max, weights, weighted v_bar
  float mg[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float m = wave_max(z_lds[g][threadIdx.x]);
    if (lane == 0) red[wave][g] = m;
  }
  __syncthreads();
#pragma unroll
  for (int g = 0; g < G; ++g) mg[g] = fmaxf(fmaxf(red[0][g], red[1][g]), fmaxf(red[2][g], red[3][g]));
  __syncthreads();
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float zv = z_lds[g][threadIdx.x];
    const float beta = (zv == kNegInf) ? 0.f : __expf(zv - mg[g]);
    z_lds[g][threadIdx.x] = beta;  // reuse as the fp32 weight
    const float l = wave_sum(beta);
    if (lane == 0) red[4 + wave][g] = l;
  }
  __syncthreads();

  float acc[G][DPL];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < DPL; ++e) acc[g][e] = 0.f;
#pragma unroll
  for (int t = 0; t < kRows; ++t) {
    const int jl = 16 * t + 4 * wave + r;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float bw = round_if(z_lds[g][jl], p.rep_bf16);
#pragma unroll
      for (int e = 0; e < DPL; ++e) acc[g][e] = fmaf(bw, round_if(vr[t][e], !VBH && p.rep_bf16), acc[g][e]);
    }
  }
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < DPL; ++e) {
      float v = acc[g][e];
      v = rows_sum(v);
      if (r == 0) wacc[wave][g * D + c16 * DPL + e] = v;
    }
  __syncthreads();
  const int64_t slot = (int64_t)bh * p.n_rc + rc;
  for (int o = threadIdx.x; o < G * D; o += 256) {
    const int g = o / D;
    p.rep_acc[slot * (G * D) + o] = wacc[0][o] + wacc[1][o] + wacc[2][o] + wacc[3][o];
    if (o % D == 0) {
      // partials use the finalize's log2 domain
      p.rep_ml[(slot * G + g) * 2 + 0] = mg[g] == kNegInf ? kNegInf : mg[g] * kLog2e;
      p.rep_ml[(slot * G + g) * 2 + 1] = red[4][g] + red[5][g] + red[6][g] + red[7][g];
    }
  }
}

// ---------------------------------------------------------------- host

int check_summaries(const ia_block_summaries* sm, bool need_bounds, bool need_v) {
  if (!sm || !sm->k_bar || !sm->counts) return fail(IA_ERR_INVALID, "summaries need k_bar and counts");
  if (sm->bounds_packed != 0 && sm->bounds_packed != 1) return fail(IA_ERR_INVALID, "bounds_packed must be 0 or 1");
  if (need_bounds && (!sm->k_max || (!sm->bounds_packed && !sm->k_min)))
    return fail(IA_ERR_INVALID, "summaries need k_max and k_min (or packed bounds at k_max)");
  if (need_v && (!sm->v_bar || !sm->v_norm_max || !sm->v_norm_all))
    return fail(IA_ERR_INVALID, "summaries need v_bar, v_norm_max and v_norm_all");
  const int32_t dts[3] = {sm->k_bar_dtype, sm->bounds_dtype, sm->v_bar_dtype};
  for (int32_t dt : dts)
    if (dt != IA_F32 && dt != IA_BF16) return fail(IA_ERR_INVALID, "summary dtypes must be IA_F32 or IA_BF16");
  if (sm->nb < 0 || sm->block_size <= 0 || sm->block_size % 16 || sm->block_size > 32768)
    return fail(IA_ERR_INVALID, "nb must be >= 0 and block_size a positive multiple of 16, at most 32768");
  const void* ptrs[4] = {sm->k_bar, sm->k_max, sm->bounds_packed ? nullptr : sm->k_min, sm->v_bar};
  for (const void* q : ptrs)
    if (reinterpret_cast<uintptr_t>(q) % 16) return fail(IA_ERR_INVALID, "summary arrays must be 16-byte aligned");
  return IA_OK;
}

CondParams cond_params(const ia_decode_shape* shape, const void* q, const ia_block_summaries* sm) {
  CondParams p{};
  p.q = q;
  p.q_batch_stride = shape->q_batch_stride;
  p.q_row_stride = shape->q_row_stride;
  p.q_f32 = shape->q_dtype == IA_F32;
  p.k_bar = sm->k_bar;
  p.k_max = sm->k_max;
  p.k_min = sm->bounds_packed ? sm->k_max : sm->k_min;
  p.bounds_packed = sm->bounds_packed;
  p.v_bar = sm->v_bar;
  p.v_norm_max = sm->v_norm_max;
  p.v_norm_all = sm->v_norm_all;
  p.counts = sm->counts;
  p.nb = sm->nb;
  p.n_kv_heads = shape->n_kv_heads;
  p.n_chunks = std::max(1, (sm->nb + kChunk16 - 1) / kChunk16);
  p.scale = 1.0f / std::sqrt((float)shape->head_dim);
  return p;
}

template <int D, int G>
void launch_stats(const CondParams& p, bool kbh, bool bdh, int batch, hipStream_t st) {
  dim3 grid(p.n_chunks, p.n_kv_heads, batch);
  if (kbh) {
    if (bdh) hipLaunchKernelGGL((ia_condition_block_selection_stats<D, G, true, true>), grid, dim3(256), 0, st, p);
    else hipLaunchKernelGGL((ia_condition_block_selection_stats<D, G, true, false>), grid, dim3(256), 0, st, p);
  } else {
    if (bdh) hipLaunchKernelGGL((ia_condition_block_selection_stats<D, G, false, true>), grid, dim3(256), 0, st, p);
    else hipLaunchKernelGGL((ia_condition_block_selection_stats<D, G, false, false>), grid, dim3(256), 0, st, p);
  }
}

template <int D, int G, bool MASK>
void launch_route(const CondParams& p, bool vbh, bool kbh, int batch, hipStream_t st) {
  dim3 grid(p.n_rc, p.n_kv_heads, batch);
  if (vbh) {
    if (kbh) hipLaunchKernelGGL((ia_condition_block_route<D, G, true, true, MASK>), grid, dim3(256), 0, st, p);
    else hipLaunchKernelGGL((ia_condition_block_route<D, G, true, false, MASK>), grid, dim3(256), 0, st, p);
  } else {
    if (kbh) hipLaunchKernelGGL((ia_condition_block_route<D, G, false, true, MASK>), grid, dim3(256), 0, st, p);
    else hipLaunchKernelGGL((ia_condition_block_route<D, G, false, false, MASK>), grid, dim3(256), 0, st, p);
  }
}

#define IA_DG_SWITCH(D, G, CALL)                                 \
  do {                                                           \
    if (D == 128 && G == 4) { constexpr int DD = 128, GG = 4; CALL; } \
    else if (D == 128 && G == 8) { constexpr int DD = 128, GG = 8; CALL; } \
    else if (D == 128 && G == 2) { constexpr int DD = 128, GG = 2; CALL; } \
    else if (D == 128 && G == 1) { constexpr int DD = 128, GG = 1; CALL; } \
    else if (D == 64 && G == 4) { constexpr int DD = 64, GG = 4; CALL; } \
    else if (D == 64 && G == 8) { constexpr int DD = 64, GG = 8; CALL; } \
    else if (D == 64 && G == 2) { constexpr int DD = 64, GG = 2; CALL; } \
    else if (D == 64 && G == 1) { constexpr int DD = 64, GG = 1; CALL; } \
    else return fail(IA_ERR_UNSUPPORTED, "head_dim / group combination"); \
  } while (0)

struct CondWs {
  float* s;
  float* delta;
  float* partial;
  int32_t* rc_counts;
  int32_t* rc_lists;
  float* rep_ml;
  float* rep_acc;
  char* decode;
  size_t decode_bytes;
  size_t total;
};

CondWs cond_ws_layout(int batch, int hkv, int g, int d, int nb, int max_items, char* base) {
  CondWs w{};
  const size_t rows = (size_t)hkv * g;
  const size_t bh = (size_t)batch * hkv;
  const size_t n16 = std::max(1, (nb + kChunk16 - 1) / kChunk16);
  const size_t nrc = std::max(1, (nb + kRouteChunk - 1) / kRouteChunk);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off = align_up(off + bytes, 256);
    return base ? base + o : nullptr;
  };
  w.s = reinterpret_cast<float*>(take((size_t)batch * rows * std::max(nb, 1) * 4));
  w.delta = reinterpret_cast<float*>(take((size_t)batch * rows * std::max(nb, 1) * 4));
  w.partial = reinterpret_cast<float*>(take((size_t)batch * 4 * rows * n16 * 4));
  w.rc_counts = reinterpret_cast<int32_t*>(take(bh * nrc * 4));
  w.rc_lists = reinterpret_cast<int32_t*>(take(bh * nrc * kRouteChunk * 4));
  w.rep_ml = reinterpret_cast<float*>(take(bh * nrc * g * 2 * 4));
  w.rep_acc = reinterpret_cast<float*>(take(bh * nrc * g * d * 4));
  w.decode_bytes = decode_ws_size(batch, hkv, g, d, max_items);
  w.decode = take(w.decode_bytes);
  w.total = off;
  return w;
}

int64_t cond_units_max(int nb, int32_t sfx_cap) {
  return (int64_t)nb + (std::max(sfx_cap, 0) + kDenseTile - 1) / kDenseTile;
}

int run_condition(bool mask_mode, const ia_decode_shape* shape, const void* q, const ia_block_summaries* sm,
                  const uint8_t* mask, const ia_paged_kv* prompt, const ia_suffix_kv* sfx, float eps,
                  int32_t mass_exp, uint8_t* selected, float scale, void* out, int32_t out_dtype, void* workspace,
                  size_t workspace_bytes, void* stream) {
  int rc = check_shape(shape);
  if (rc) return rc;
  rc = check_summaries(sm, !mask_mode, true);
  if (rc) return rc;
  rc = check_kv(prompt, shape->head_dim);
  if (rc) return rc;
  if (prompt->dtype == IA_FP8_E4M3) return fail(IA_ERR_UNSUPPORTED, "condition-mode decode takes f32 or bf16 K/V");
  if (mask_mode && !mask) return fail(IA_ERR_INVALID, "fixed-mask decode needs a mask");
  if (!q || !out) return fail(IA_ERR_INVALID, "q and out must be non-null");
  if (out_dtype != IA_F32 && out_dtype != IA_BF16) return fail(IA_ERR_INVALID, "out dtype must be IA_F32 or IA_BF16");
  if (!(scale > 0.f) || !std::isfinite(scale)) return fail(IA_ERR_INVALID, "scale must be positive and finite");
  if (sfx && sfx->cap > 0) {
    if (!sfx->k || !sfx->v || !sfx->len) return fail(IA_ERR_INVALID, "suffix needs k, v and a device length");
    const int eb = prompt->dtype == IA_F32 ? 4 : 2;
    const int64_t st6[6] = {sfx->k_batch_stride, sfx->k_head_stride, sfx->k_token_stride,
                            sfx->v_batch_stride, sfx->v_head_stride, sfx->v_token_stride};
    for (int64_t s6 : st6)
      if (s6 < 0 || (s6 * eb) % 16) return fail(IA_ERR_INVALID, "suffix strides must be 16-byte multiples");
    if ((reinterpret_cast<uintptr_t>(sfx->k) | reinterpret_cast<uintptr_t>(sfx->v)) % 16)
      return fail(IA_ERR_INVALID, "suffix pointers must be 16-byte aligned");
  }
  const int G = shape->n_q_heads / shape->n_kv_heads;
  const int D = shape->head_dim;
  const int nb = sm->nb;
  const int n_rc = std::max(1, (nb + kRouteChunk - 1) / kRouteChunk);
  if (n_rc > kMaxRouteChunks) return fail(IA_ERR_UNSUPPORTED, "too many blocks per sequence for condition mode");
  const int32_t sfx_cap = (sfx && sfx->cap > 0) ? sfx->cap : 0;
  const int64_t units_max = cond_units_max(nb, sfx_cap);
  const int cap_items = units_cap_items(units_max);
  const CondWs need = cond_ws_layout(shape->batch, shape->n_kv_heads, G, D, nb, cap_items, nullptr);
  if (!workspace || workspace_bytes < need.total)
    return fail(IA_ERR_WORKSPACE, "workspace too small: need " + std::to_string(need.total) + " bytes");
  if (reinterpret_cast<uintptr_t>(workspace) % 256)
    return fail(IA_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  if (shape->batch == 0) return IA_OK;
  const CondWs ws = cond_ws_layout(shape->batch, shape->n_kv_heads, G, D, nb, cap_items,
                                   reinterpret_cast<char*>(workspace));
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);

  CondParams cp = cond_params(shape, q, sm);
  cp.mass_exp = mass_exp;
  cp.eps = eps;
  cp.s = ws.s;
  cp.delta = ws.delta;
  cp.partial = ws.partial;
  cp.selected = selected;
  cp.rc_counts = ws.rc_counts;
  cp.rc_lists = ws.rc_lists;
  cp.n_rc = n_rc;
  cp.rep_ml = ws.rep_ml;
  cp.rep_acc = ws.rep_acc;
  cp.mask = mask;
  cp.rep_bf16 = prompt->dtype == IA_BF16;
  const bool kbh = sm->k_bar_dtype == IA_BF16, bdh = sm->bounds_dtype == IA_BF16, vbh = sm->v_bar_dtype == IA_BF16;
  if (nb > 0) {
    if (!mask_mode) {
      IA_DG_SWITCH(D, G, (launch_stats<DD, GG>(cp, kbh, bdh, shape->batch, st)));
      rc = check_launch("condition stats");
      if (rc) return rc;
      IA_DG_SWITCH(D, G, (launch_route<DD, GG, false>(cp, vbh, kbh, shape->batch, st)));
    } else {
      IA_DG_SWITCH(D, G, (launch_route<DD, GG, true>(cp, vbh, kbh, shape->batch, st)));
    }
    rc = check_launch("condition route");
    if (rc) return rc;
  }

  DecodeParams p{};
  p.q = q;
  p.q_batch_stride = shape->q_batch_stride;
  p.q_row_stride = shape->q_row_stride;
  p.kv = *prompt;
  p.n_kv_heads = shape->n_kv_heads;
  p.unit_tokens = sm->block_size;
  p.scale_log2 = scale * kLog2e;
  p.q_f32 = shape->q_dtype == IA_F32;
  p.out_f32 = out_dtype == IA_F32;
  p.out = out;
  p.rc_counts = ws.rc_counts;
  p.rc_lists = ws.rc_lists;
  p.n_rc = nb > 0 ? n_rc : 0;
  p.nb_max = nb;
  if (sfx_cap > 0) {
    p.sfx_k = sfx->k;
    p.sfx_v = sfx->v;
    p.sfx_k_batch_stride = sfx->k_batch_stride;
    p.sfx_k_head_stride = sfx->k_head_stride;
    p.sfx_k_token_stride = sfx->k_token_stride;
    p.sfx_v_batch_stride = sfx->v_batch_stride;
    p.sfx_v_head_stride = sfx->v_head_stride;
    p.sfx_v_token_stride = sfx->v_token_stride;
    p.sfx_len = sfx->len;
    p.sfx_len_stride = sfx->len_stride;
    p.sfx_cap = sfx_cap;
  }
  p.rep_ml = nb > 0 ? ws.rep_ml : nullptr;
  p.rep_acc = ws.rep_acc;
  p.max_items = cap_items;
  p.part_ml = reinterpret_cast<float*>(ws.decode);
  p.part_acc = reinterpret_cast<float*>(ws.decode + align_up((size_t)shape->batch * shape->n_kv_heads * cap_items * G * 2 * 4, 256));
  const int nsub_u = (std::max(sm->block_size, kDenseTile) + 15) / 16;
  int items = 1;
  rc = decode_items(p, prompt->dtype, D, G, kSrcLists, (int64_t)shape->batch * shape->n_kv_heads, units_max, nsub_u,
                    cap_items, st, &items);
  if (rc) return rc;
  return dispatch_decode(p, prompt->dtype, D, G, kSrcLists, dim3(items, shape->n_kv_heads, shape->batch), st,
                         nullptr);
}

// ---------------------------------------------------------------- one-launch call

// Workspace of the one-launch condition call, sized by (batch, Hkv, G, D) only so one
// zero-filled buffer serves every prompt length and eps: the rows' lines (finished
// items, epoch), the items' statistics partials [rows, kMaxItemsPerBh, 4 G] as tagged
// words, and split-K partials for rows x kMaxItemsPerBh workgroup slots (untagged
// (m, l) and accumulators, and tagged words for rows of at most 8 items).
struct CondFusedWs {
  size_t sbuf, part_ml, part_acc, tpart, total;
};

CondFusedWs cond_fused_ws_layout(int batch, int hkv, int g, int d) {
  const size_t rows = (size_t)batch * hkv;
  const size_t slots = rows * kMaxItemsPerBh;
  CondFusedWs w{};
  w.sbuf = align_up(rows * kFlagStride * 4, 256);
  w.part_ml = align_up(w.sbuf + rows * kMaxItemsPerBh * 4 * g * 8, 256);
  w.part_acc = align_up(w.part_ml + slots * g * 2 * 4, 256);
  w.tpart = align_up(w.part_acc + slots * g * d * 4, 256);
  w.total = align_up(w.tpart + slots * (g * d + 2 * g) * 8, 256);
  return w;
}

// Items per (sequence, kv head) row of the one-launch call on the current device, or
// 0 when the call does not fit one launch: every row's items must be resident at
// once (they exchange their statistics), an item owns at most kCondItemBlocks
// blocks and its selected blocks plus the suffix must fit the finalize's LDS lists.
int cond_fused_items(int batch, int hkv, int g, int d, int nb, int block_size, int sfx_cap, int kv_dtype,
                     bool q_f32, hipStream_t st) {
  if (g > 4 || (d != 64 && d != 128) || nb <= 0 || nb > 65535 || batch <= 0) return 0;
  if (kv_dtype != IA_BF16 && kv_dtype != IA_F32) return 0;
  if ((kv_dtype == IA_F32) != q_f32) return 0;
  DecodeParams probe{};
  probe.q_f32 = q_f32;
  int resident = 0;
  if (dispatch_decode(probe, kv_dtype, d, g, kSrcCondFused, dim3(1), st, &resident) != IA_OK || resident <= 0)
    return 0;
  const int64_t rows = (int64_t)batch * hkv;
  const int nsub_b = (block_size + 15) / 16;
  const int sfx_sub = (std::max(sfx_cap, 0) + 15) / 16;
  const int sfx_units = (std::max(sfx_cap, 0) + kDenseTile - 1) / kDenseTile;
  const int m_cap = std::min({kCondItemBlocks, (kMaxSubsPerItem - sfx_sub) / std::max(nsub_b, 1),
                              kMaxUnitsPerItem - sfx_units});
  if (m_cap < 1) return 0;
  const int64_t n_min = (nb + m_cap - 1) / m_cap;
  // about one resident round, items of at least 32 blocks where the row allows.
  // Measured at batch 1 x 8 kv heads (graph replays, one box): 32K (512 blocks) 16
  // items 19.4 us against 20.3 with 32 and 21.1 with 12; 64K 16 items 21.5, 32 items
  // 21.7; 128K 32 items 22.9 against 24.7-26.4 with 20-28.
  int64_t n = std::min<int64_t>({resident / rows, (int64_t)kMaxItemsPerBh, std::max<int64_t>(n_min, (nb + 31) / 32),
                                 (int64_t)nb});
  if (n < n_min || n < 1 || rows * n > resident) return 0;
  return (int)n;
}

int run_condition_fused(const uint8_t* mask, const ia_decode_shape* shape, const void* q,
                        const ia_block_summaries* sm, const ia_paged_kv* prompt, const ia_suffix_kv* sfx, float eps,
                        int32_t mass_exp, uint8_t* selected, float scale, void* out, int32_t out_dtype,
                        void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_shape(shape);
  if (rc) return rc;
  rc = check_summaries(sm, !mask, true);
  if (rc) return rc;
  rc = check_kv(prompt, shape->head_dim);
  if (rc) return rc;
  if (!q || !out) return fail(IA_ERR_INVALID, "q and out must be non-null");
  if (out_dtype != IA_F32 && out_dtype != IA_BF16) return fail(IA_ERR_INVALID, "out dtype must be IA_F32 or IA_BF16");
  if (!(scale > 0.f) || !std::isfinite(scale)) return fail(IA_ERR_INVALID, "scale must be positive and finite");
  if (sfx && sfx->cap > 0) {
    if (!sfx->k || !sfx->v || !sfx->len) return fail(IA_ERR_INVALID, "suffix needs k, v and a device length");
    const int eb = prompt->dtype == IA_F32 ? 4 : 2;
    const int64_t st6[6] = {sfx->k_batch_stride, sfx->k_head_stride, sfx->k_token_stride,
                            sfx->v_batch_stride, sfx->v_head_stride, sfx->v_token_stride};
    for (int64_t s6 : st6)
      if (s6 < 0 || (s6 * eb) % 16) return fail(IA_ERR_INVALID, "suffix strides must be 16-byte multiples");
    if ((reinterpret_cast<uintptr_t>(sfx->k) | reinterpret_cast<uintptr_t>(sfx->v)) % 16)
      return fail(IA_ERR_INVALID, "suffix pointers must be 16-byte aligned");
  }
  const int G = shape->n_q_heads / shape->n_kv_heads;
  const int D = shape->head_dim;
  const int32_t sfx_cap = (sfx && sfx->cap > 0) ? sfx->cap : 0;
  const CondFusedWs L = cond_fused_ws_layout(shape->batch, shape->n_kv_heads, G, D);
  if (!workspace || workspace_bytes < L.total)
    return fail(IA_ERR_WORKSPACE, "workspace too small: need " + std::to_string(L.total) + " bytes");
  if (reinterpret_cast<uintptr_t>(workspace) % 256)
    return fail(IA_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  if (shape->batch == 0) return IA_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int n_it = cond_fused_items(shape->batch, shape->n_kv_heads, G, D, sm->nb, sm->block_size, sfx_cap,
                                    prompt->dtype, shape->q_dtype == IA_F32, st);
  if (n_it <= 0)
    return fail(IA_ERR_UNSUPPORTED, "this condition call does not fit one launch; use ia_condition_decode");
  char* ws = reinterpret_cast<char*>(workspace);

  DecodeParams p{};
  p.q = q;
  p.q_batch_stride = shape->q_batch_stride;
  p.q_row_stride = shape->q_row_stride;
  p.kv = *prompt;
  p.n_kv_heads = shape->n_kv_heads;
  p.unit_tokens = sm->block_size;
  p.scale_log2 = scale * kLog2e;
  p.q_f32 = shape->q_dtype == IA_F32;
  p.out_f32 = out_dtype == IA_F32;
  p.out = out;
  p.nb_max = sm->nb;
  if (sfx_cap > 0) {
    p.sfx_k = sfx->k;
    p.sfx_v = sfx->v;
    p.sfx_k_batch_stride = sfx->k_batch_stride;
    p.sfx_k_head_stride = sfx->k_head_stride;
    p.sfx_k_token_stride = sfx->k_token_stride;
    p.sfx_v_batch_stride = sfx->v_batch_stride;
    p.sfx_v_head_stride = sfx->v_head_stride;
    p.sfx_v_token_stride = sfx->v_token_stride;
    p.sfx_len = sfx->len;
    p.sfx_len_stride = sfx->len_stride;
    p.sfx_cap = sfx_cap;
  }
  p.n_rows = shape->batch * shape->n_kv_heads;
  p.max_items = n_it;
  p.rowctr = reinterpret_cast<u32*>(ws);
  p.sbuf = reinterpret_cast<unsigned long long*>(ws + L.sbuf);
  p.part_ml = reinterpret_cast<float*>(ws + L.part_ml);
  p.part_acc = reinterpret_cast<float*>(ws + L.part_acc);
  p.tpart = reinterpret_cast<unsigned long long*>(ws + L.tpart);
  p.wait_ticks = wait_limit_ticks();
  p.c_kbar = sm->k_bar;
  p.c_kmax = sm->k_max;
  p.c_kmin = sm->bounds_packed ? sm->k_max : sm->k_min;
  p.c_bounds_packed = sm->bounds_packed;
  p.c_vbar = sm->v_bar;
  p.c_kbar_bf16 = sm->k_bar_dtype == IA_BF16;
  p.c_bounds_bf16 = sm->bounds_dtype == IA_BF16;
  p.c_vbar_bf16 = sm->v_bar_dtype == IA_BF16;
  p.c_vnorm_max = sm->v_norm_max;
  p.c_vnorm_all = sm->v_norm_all;
  p.c_counts = sm->counts;
  p.c_items = n_it;
  p.c_eps = eps;
  p.c_mass_exp = mass_exp;
  p.c_scale = 1.0f / std::sqrt((float)D);
  p.c_rep_bf16 = prompt->dtype == IA_BF16;
  p.c_selected = mask ? nullptr : selected;
  p.c_mask = mask;
  return dispatch_decode(p, prompt->dtype, D, G, kSrcCondFused, dim3(p.n_rows * n_it), st, nullptr);
}

}  // namespace
}  // namespace ia

extern "C" {

size_t ia_condition_decode_fused_workspace_size(int32_t batch, int32_t n_kv_heads, int32_t group,
                                                int32_t head_dim) {
  return ia::cond_fused_ws_layout(std::max(batch, 0), std::max(n_kv_heads, 0), std::max(group, 1),
                                  std::max(head_dim, 1))
      .total;
}

int32_t ia_condition_decode_fused_items(const ia_decode_shape* shape, const ia_block_summaries* sm,
                                        int32_t kv_dtype, int32_t suffix_cap) {
  if (ia::check_shape(shape) || !sm) return 0;
  return ia::cond_fused_items(shape->batch, shape->n_kv_heads, shape->n_q_heads / shape->n_kv_heads,
                              shape->head_dim, sm->nb, sm->block_size, suffix_cap, kv_dtype,
                              shape->q_dtype == IA_F32, nullptr);
}

int ia_condition_decode_fused(const ia_decode_shape* shape, const void* q, const ia_block_summaries* sm,
                              const ia_paged_kv* prompt, const ia_suffix_kv* suffix, float eps,
                              int32_t term1_mass_exp, uint8_t* selected, float scale, void* out, int32_t out_dtype,
                              void* workspace, size_t workspace_bytes, void* stream) {
  return ia::run_condition_fused(nullptr, shape, q, sm, prompt, suffix, eps, term1_mass_exp, selected, scale, out,
                                 out_dtype, workspace, workspace_bytes, stream);
}

int ia_fixed_mask_decode_fused(const ia_decode_shape* shape, const void* q, const ia_block_summaries* sm,
                               const uint8_t* mask, const ia_paged_kv* prompt, const ia_suffix_kv* suffix,
                               float scale, void* out, int32_t out_dtype, void* workspace, size_t workspace_bytes,
                               void* stream) {
  if (!mask) return ia::fail(IA_ERR_INVALID, "fixed-mask decode needs a mask");
  return ia::run_condition_fused(mask, shape, q, sm, prompt, suffix, 0.f, 0, nullptr, scale, out, out_dtype,
                                 workspace, workspace_bytes, stream);
}

size_t ia_condition_workspace_size(int32_t batch, int32_t n_kv_heads, int32_t group, int32_t head_dim, int32_t nb,
                                   int32_t suffix_cap) {
  const int cap_items = ia::units_cap_items(ia::cond_units_max(nb, suffix_cap));
  return ia::cond_ws_layout(batch, n_kv_heads, group, head_dim, nb, cap_items, nullptr).total;
}

int ia_condition_selection_stats(const ia_decode_shape* shape, const void* q, const ia_block_summaries* sm,
                                 int32_t term1_mass_exp, float* s, float* delta, float* partial, float* globals,
                                 void* stream) {
  using namespace ia;
  int rc = check_shape(shape);
  if (rc) return rc;
  rc = check_summaries(sm, true, false);
  if (rc) return rc;
  if (!q || !s || !delta || !partial) return fail(IA_ERR_INVALID, "null pointer argument");
  if (shape->batch == 0 || sm->nb == 0) return IA_OK;
  CondParams cp = cond_params(shape, q, sm);
  cp.mass_exp = term1_mass_exp;
  cp.s = s;
  cp.delta = delta;
  cp.partial = partial;
  cp.globals = globals;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int G = shape->n_q_heads / shape->n_kv_heads;
  const int D = shape->head_dim;
  const bool kbh = sm->k_bar_dtype == IA_BF16, bdh = sm->bounds_dtype == IA_BF16;
  IA_DG_SWITCH(D, G, (launch_stats<DD, GG>(cp, kbh, bdh, shape->batch, st)));
  rc = check_launch("condition stats");
  if (rc || !globals) return rc;
  const dim3 grid(shape->n_kv_heads, shape->batch);
  switch (G) {
    case 1: hipLaunchKernelGGL(ia_condition_block_selection_reduce<1>, grid, dim3(256), 0, st, cp); break;
    case 2: hipLaunchKernelGGL(ia_condition_block_selection_reduce<2>, grid, dim3(256), 0, st, cp); break;
    case 4: hipLaunchKernelGGL(ia_condition_block_selection_reduce<4>, grid, dim3(256), 0, st, cp); break;
    default: hipLaunchKernelGGL(ia_condition_block_selection_reduce<8>, grid, dim3(256), 0, st, cp); break;
  }
  return check_launch("condition reduce");
}

int ia_condition_select(const ia_decode_shape* shape, const ia_block_summaries* sm, const float* s,
                        const float* delta, const float* globals, float eps, int32_t term1_mass_exp,
                        uint8_t* selected, float* z, void* stream) {
  using namespace ia;
  int rc = check_shape(shape);
  if (rc) return rc;
  rc = check_summaries(sm, false, true);
  if (rc) return rc;
  if (!s || !delta || !globals || !selected) return fail(IA_ERR_INVALID, "null pointer argument");
  if (shape->batch == 0 || sm->nb == 0) return IA_OK;
  CondParams cp = cond_params(shape, nullptr, sm);
  cp.mass_exp = term1_mass_exp;
  cp.eps = eps;
  cp.s = const_cast<float*>(s);
  cp.delta = const_cast<float*>(delta);
  cp.globals = const_cast<float*>(globals);
  cp.selected = selected;
  cp.z_out = z;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  dim3 grid((sm->nb + 255) / 256, shape->n_kv_heads, shape->batch);
  const int G = shape->n_q_heads / shape->n_kv_heads;
  switch (G) {
    case 1: hipLaunchKernelGGL(ia_condition_block_selection_select<1>, grid, dim3(256), 0, st, cp); break;
    case 2: hipLaunchKernelGGL(ia_condition_block_selection_select<2>, grid, dim3(256), 0, st, cp); break;
    case 4: hipLaunchKernelGGL(ia_condition_block_selection_select<4>, grid, dim3(256), 0, st, cp); break;
    case 8: hipLaunchKernelGGL(ia_condition_block_selection_select<8>, grid, dim3(256), 0, st, cp); break;
    default: return fail(IA_ERR_UNSUPPORTED, "GQA group size");
  }
  return check_launch("condition select");
}

int ia_condition_decode(const ia_decode_shape* shape, const void* q, const ia_block_summaries* sm,
                        const ia_paged_kv* prompt, const ia_suffix_kv* suffix, float eps, int32_t term1_mass_exp,
                        uint8_t* selected, float scale, void* out, int32_t out_dtype, void* workspace,
                        size_t workspace_bytes, void* stream) {
  return ia::run_condition(false, shape, q, sm, nullptr, prompt, suffix, eps, term1_mass_exp, selected, scale, out,
                           out_dtype, workspace, workspace_bytes, stream);
}

int ia_fixed_mask_decode(const ia_decode_shape* shape, const void* q, const ia_block_summaries* sm,
                         const uint8_t* mask, const ia_paged_kv* prompt, const ia_suffix_kv* suffix, float scale,
                         void* out, int32_t out_dtype, void* workspace, size_t workspace_bytes, void* stream) {
  return ia::run_condition(true, shape, q, sm, mask, prompt, suffix, 0.f, 0, nullptr, scale, out, out_dtype,
                           workspace, workspace_bytes, stream);
}

}  // extern "C"
