// Paged decode attention for gfx950: the selected-block finalize (sparse) and
// the dense fallback share one kernel template.
//
// Work decomposition
//   grid = (items, Hkv, batch); one 512-thread workgroup (8 waves) per split-K
//   item of one (sequence, kv head).  An item is a run of "units": selected
//   blocks (sparse) or 128-token tiles (dense).  A prologue stages the item's
//   unit token ranges and one page id per 16-token subtile in LDS (so the
//   streaming loop never waits on a dependent scalar load).  Waves take units
//   round-robin and stream them one page-resident subtile at a time, keeping
//   their own online-softmax state; the workgroup folds its eight waves in LDS
//   and writes one (m, l, acc) partial (an empty partial when the (sequence,
//   kv head) needs fewer items than the grid row), or the output rows directly
//   when the grid has a single item per row.  A second small kernel merges the
//   partials.
//   There is no cross-workgroup synchronisation inside a launch.
//
// Lane layout (head_dim D, DPL = D/16 dims per lane; lane = 16*r + c)
//   K and V of the next subtiles are in flight in a ring of register buffers
//   while the current one is consumed (two subtiles, 16 KiB per wave, for bf16).
//   bf16 and fp8 caches (MFMA): V is read as four steps i = 0..3, row r holding
//   token 4i + r and lane c dims [c*DPL, (c+1)*DPL); K is read as 16-byte pieces,
//   lane c taking token c/4 + 4 (c%4).  Q.K runs as v_mfma_f32_16x16x32_bf16 with
//   the G query rows replicated over the 16 columns, which leaves each lane the
//   scores of tokens r, r+4, r+8, r+12 for query row c % G: exactly the k-slice
//   of the P operand of the P.V product (v_mfma_f32_16x16x16_bf16, one per dim
//   group), whose V operand is the lane's own four row loads interleaved by
//   v_perm.  fp8 codes are widened to bf16 in registers (exact).
//   fp32 caches (VALU): the same V layout for K; Q.K partial sums for the 4 steps
//   x G query rows are reduce-scattered over the 16-lane row with DPP, leaving
//   each lane the complete score of one (token, query row) pair; the softmax
//   weights reach the V lanes of the same row through DPP row broadcasts.
//
// Numerics follow the reference's fused kernel (CBT/page_attention.py):
//   bf16 K/V: scores = bf16(q) . K accumulated in fp32, fp32 online softmax,
//   weights rounded to bf16 for the P.V product (:248-252), fp32 normaliser
//   (:253).  fp32 K/V: everything in fp32.  fp8 K/V: as bf16 on the widened
//   codes; the per-(page, head) scale multiplies the score and is folded into
//   the weight before its bf16 rounding.
#pragma once

#include <algorithm>
#include <atomic>
#include <type_traits>

#include "cond_rule.hpp"
#include "plan.hpp"
#include "topk_select.hpp"

namespace ia {

// Waits of one workgroup on another that reached their bound: the waiting workgroup
// then computed the missing data itself (score and statistics hand-offs: same
// results, later) or, for a merge read of a finished item's partial, wrote NaN.
// One counter per device in each translation unit that instantiates the kernels
// (device variables are not shared between translation units), summed by
// ia_wait_fallbacks.  A vector atomic, taken only on that rare path.
static __device__ u32 g_wait_fallbacks[1];
__device__ __forceinline__ void note_wait_fallback() {
  __hip_atomic_fetch_add(g_wait_fallbacks, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Host: this translation unit's counter on the current device (a synchronous read;
// reset to zero when `reset`).
static inline uint64_t tu_wait_fallbacks(bool reset) {
  u32 v = 0u;
  if (hipMemcpyFromSymbol(&v, HIP_SYMBOL(g_wait_fallbacks), sizeof(v), 0, hipMemcpyDeviceToHost) != hipSuccess) return 0;
  if (reset) {
    const u32 zero = 0u;
    (void)hipMemcpyToSymbol(HIP_SYMBOL(g_wait_fallbacks), &zero, sizeof(zero), 0, hipMemcpyHostToDevice);
  }
  return v;
}

// kRing: register buffers in the load pipeline (subtiles in flight = kRing - 1),
// sized so a wave stays within 256 registers (two waves per SIMD).
struct KvBf16 {
  static constexpr int kBytes = 2;
  static constexpr int kRing = 3;
};
struct KvF32 {
  static constexpr int kBytes = 4;
  static constexpr int kRing = 2;
};
struct KvFp8 {
  static constexpr int kBytes = 1;
  static constexpr int kRing = 3;
};

// NW words (2 or 4) at p with one plain, cached load
template <int NW>
__device__ __forceinline__ void load_cached_words(const char* p, u32* w) {
  static_assert(NW == 2 || NW == 4, "8- or 16-byte pieces");
  if constexpr (NW == 4) {
    const u32x4_t a = *reinterpret_cast<const u32x4_t*>(p);
    w[0] = a[0]; w[1] = a[1]; w[2] = a[2]; w[3] = a[3];
  } else {
    const u32x2_t a = *reinterpret_cast<const u32x2_t*>(p);
    w[0] = a[0]; w[1] = a[1];
  }
}

// NWD words of one K/V row slice, as streaming loads
template <int NWD>
__device__ __forceinline__ void load_words(const char* p, u32* w) {
  if constexpr (NWD == 8) {
    const u32x4_t a = ld_stream16(p);
    const u32x4_t b = ld_stream16(p + 16);
    w[0] = a[0]; w[1] = a[1]; w[2] = a[2]; w[3] = a[3];
    w[4] = b[0]; w[5] = b[1]; w[6] = b[2]; w[7] = b[3];
  } else if constexpr (NWD == 4) {
    const u32x4_t a = ld_stream16(p);
    w[0] = a[0]; w[1] = a[1]; w[2] = a[2]; w[3] = a[3];
  } else if constexpr (NWD == 2) {
    const u32x2_t a = ld_stream8(p);
    w[0] = a[0]; w[1] = a[1];
  } else {
    w[0] = ld_stream4(p);
  }
}

// Where a finalize launch takes its units from.
constexpr int kSrcTopk = 0;   // idx[b, h, 0:n_sel[b, h]] blocks of unit_tokens tokens
constexpr int kSrcDense = 1;  // every 128-token tile of [0, seq_len)
constexpr int kSrcLists = 2;  // route-chunk lists of selected blocks, then the exact suffix
constexpr int kSrcTopkFused = 3;  // top-k of a score row selected in the prologue, then as kSrcTopk
constexpr int kSrcCondFused = 4;  // condition rule over the item's own blocks in the prologue, then as kSrcLists
constexpr int kFusedMaxBlocks = 4096;  // score row staged in LDS by the fused top-k source
constexpr int kCondItemBlocks = 512;   // blocks one item of the one-launch condition call owns at most
// sources that merge their split-K partials inside the launch (the row's last item)
constexpr bool src_fused(int src) { return src == kSrcTopkFused || src == kSrcCondFused; }

constexpr int kRouteChunk = 256;      // blocks per route workgroup (condition mode)
constexpr int kMaxRouteChunks = 256;  // route chunks per (sequence, kv head)
constexpr int kMaxItemsPerBh = 64;  // upper bound of split-K items per (sequence, kv head)
// Sources whose launch is planned by work (one flat grid, items per (sequence, kv
// head) in proportion to its subtiles); kSrcLists keeps a fixed item count per row.
constexpr bool src_balanced(int src) { return src != kSrcLists; }
constexpr int kSpecEntries = 2048;  // list entries a finalize item stages without waiting for the counts
constexpr int kNoPage = -1;
constexpr int kSfxPage = -2;          // subtile of the contiguous suffix source

struct DecodeParams {
  const void* q;
  int64_t q_batch_stride, q_row_stride;
  ia_paged_kv kv;
  const int32_t* seq_lens;
  const int32_t* idx;  // kSrcTopk
  const int32_t* n_sel;
  int32_t k_cap;
  // kSrcTopkFused: block scores [batch*Hkv, nb_max] and the selection rule; item 0
  // of each (b, h) also writes the chosen ids / counts when idx_out is set
  float* scores;
  const int32_t* k_per_seq;
  int32_t topk_k, forced_first, forced_last, forced_in_k;
  int32_t* idx_out;
  int32_t* n_sel_out;
  int32_t unit_tokens;  // tokens per unit: block_size (blocks) or the dense tile
  int32_t max_items;    // stride of the item partials per (b, h)
  // kSrcLists: selected blocks per route chunk, valid tokens per block, suffix
  const int32_t* rc_counts;   // [batch*Hkv, n_rc]
  const int32_t* rc_lists;    // [batch*Hkv, n_rc, kRouteChunk]
  int32_t n_rc;
  int32_t nb_max;
  const void* sfx_k;
  const void* sfx_v;
  int64_t sfx_k_batch_stride, sfx_k_head_stride, sfx_k_token_stride;
  int64_t sfx_v_batch_stride, sfx_v_head_stride, sfx_v_token_stride;
  const int32_t* sfx_len;     // device: suffix length (entry b, or entry 0 when sfx_len_stride == 0)
  int32_t sfx_len_stride;
  int32_t sfx_cap;            // host bound on the suffix length
  // representative partials folded by the merge (condition mode)
  const float* rep_ml;        // [batch*Hkv, n_rc, G, 2]
  const float* rep_acc;       // [batch*Hkv, n_rc, G, D]
  int32_t n_kv_heads;
  float scale_log2;  // softmax scale * log2(e)
  int32_t q_f32;     // q is fp32 (else bf16)
  int32_t out_f32;   // out is fp32 (else bf16)
  void* out;
  float* part_ml;  // [batch*Hkv, max_items, G, 2] (fused top-k call: [workgroup, G, 2])
  float* part_acc; // [batch*Hkv, max_items, G, D] (fused top-k call: [workgroup, G, D])
  // balanced sources: items of each (b, h) row, written by the row's item 0 and
  // read by the merge; the plan's workgroup budget and the row count; the fused
  // top-k source reads its plan entries (one per workgroup) from the scorer launch
  int32_t* part_n;  // [batch*Hkv]
  int32_t plan_budget;
  int32_t n_rows;
  // fused top-k call: block keys scored in the prologue (k_bar for the mean-key
  // score, or k_max / k_min for the Quest score), rows of D contiguous elements at
  // b * kb_batch_stride + h * kb_head_stride + j * D; hand-off flags between the
  // items of a row (zero between calls) and the bound of every wait on them
  const void* kb;
  const void* kb2;
  int64_t kb_batch_stride, kb_head_stride;
  int32_t kb_bf16;
  int32_t score_quest;
  float score_scale;
  int32_t key_rows;          // one-launch top-k call: run the instance that loads keys as whole rows
  unsigned long long* sbuf;  // [rows, nb_max] published scores: tag << 32 | score bits
  unsigned long long* tpart; // [workgroups, G D + 2 G] tagged partials (acc, then (m, l)) of rows of <= 8 items
  u32* rowctr;               // [rows, kFlagStride]: finished partials (word 0), row epoch (word 1)
  int64_t wait_ticks;
  // one-launch condition call (kSrcCondFused): the prompt blocks' summaries, rows of
  // D elements at ((b * Hkv + h) * nb_max + j) * D (bf16 or fp32 each), their norm
  // bounds [batch, Hkv, nb_max] and [batch, Hkv] and valid counts [batch, nb_max];
  // the items per row; the rule's eps, variant (term1 mass exp) and 1/sqrt(D); the
  // representatives' bf16 rounding (bf16 caches); the optional selected flags
  // [batch, Hkv * G, nb_max].  The items' statistics partials travel through sbuf
  // ([rows, kMaxItemsPerBh * 4 G] tagged words).
  const void* c_kbar;
  const void* c_kmax;
  const void* c_kmin;
  const void* c_vbar;
  int32_t c_kbar_bf16, c_bounds_bf16, c_vbar_bf16;
  int32_t c_bounds_packed;  // k_max is the packed k_bounds (pairs per dimension), k_min unused
  const float* c_vnorm_max;
  const float* c_vnorm_all;
  const int32_t* c_counts;
  int32_t c_items;
  float c_eps;
  int32_t c_mass_exp;
  float c_scale;
  int32_t c_rep_bf16;
  uint8_t* c_selected;
  const uint8_t* c_mask;  // external-mask mode: the selection [batch, Hkv, nb_max] (no statistics)
};

constexpr int kWaves = 8;  // split-K merge: up to kWaves x kMergeFastSlots slots in one round trip
constexpr int kThreads = kWaves * 64;
// finalize: one 8-wave workgroup per CU (two waves per SIMD), so the waves that
// share a CU share one work list
constexpr int kFinWaves = 8;
constexpr int kFinThreads = kFinWaves * 64;
constexpr int kDenseTile = 128;
constexpr int kMaxUnitsPerItem = kPlanMaxUnits;  // LDS unit ranges per item
constexpr int kMaxSubsPerItem = kPlanMaxSubs;  // LDS page ids per item (16 tokens each)

// Lane (within the 16-lane row) and slot holding the reduce-scattered value of
// index x = i*G + g (see reduce_scatter16).
template <int G>
struct ScoreMap {
  static constexpr int NV = 4 * G;
  static constexpr int KG = NV >= 16 ? NV / 16 : 1;
  static constexpr int lane_of(int x) { return NV >= 16 ? x / (NV / 16) : x * (16 / NV); }
  static constexpr int slot_of(int x) { return NV >= 16 ? x % (NV / 16) : 0; }
};

template <int CTRL>
__device__ __forceinline__ float bcast_row(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}

// max / sum over the lanes that hold the same query row g
template <int G, bool MAX>
__device__ __forceinline__ float fold_g(float v) {
  auto op = [](float a, float b) { return MAX ? fmaxf(a, b) : a + b; };
  v = op(v, dpp<kDppRowRor4>(v));
  v = op(v, dpp<kDppRowRor8>(v));
  if constexpr (G <= 2) v = op(v, dpp<kDppXor1>(v));
  if constexpr (G == 1) v = op(v, dpp<kDppXor2>(v));
  return MAX ? rows_max(v) : rows_sum(v);
}

template <int G, int D>
__device__ __forceinline__ void store_decode_out(const DecodeParams& p, int b, int h, int o, float v) {
  const int g = o / D, d = o % D;
  const int64_t off = ((int64_t)b * (p.n_kv_heads * G) + h * G + g) * D + d;
  if (p.out_f32) {
    reinterpret_cast<float*>(p.out)[off] = v;
  } else {
    reinterpret_cast<unsigned short*>(p.out)[off] = f32_to_bf16_bits(v);
  }
}

// Softmax-weight rescale factor of query row g, taken from the lane of the
// same quad that owns g (quad_perm broadcast [q,q,q,q] = q * 0x55).
template <int G>
__device__ __forceinline__ float alpha_of_row(const float* alpha, int g) {
  if constexpr (G == 4) {
    switch (g) {
      case 0: return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(alpha[0]), 0x00, 0xf, 0xf, false));
      case 1: return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(alpha[0]), 0x55, 0xf, 0xf, false));
      case 2: return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(alpha[0]), 0xAA, 0xf, 0xf, false));
      default: return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(alpha[0]), 0xFF, 0xf, 0xf, false));
    }
  } else if constexpr (G == 8) {  // g = 2*(c16 & 3) + k
    const float v = (g & 1) ? alpha[1] : alpha[0];
    switch (g >> 1) {
      case 0: return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x00, 0xf, 0xf, false));
      case 1: return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x55, 0xf, 0xf, false));
      case 2: return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xAA, 0xf, 0xf, false));
      default: return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xFF, 0xf, 0xf, false));
    }
  } else if constexpr (G == 2) {  // g = (c16 >> 1) & 1: quad lanes 2g, 2g+1
    return g ? __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(alpha[0]), 0xAA, 0xf, 0xf, false))
             : __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(alpha[0]), 0x00, 0xf, 0xf, false));
  } else {
    return alpha[0];
  }
}

// pb[i][g] = weight of (token 4i + r, row g), read from the row lane that owns
// index x = i*G + g after the reduce-scatter (compile-time lane and slot).
template <int G, int X>
struct WeightBcast {
  __device__ __forceinline__ static void run(const float* pw, float (*pb)[G]) {
    WeightBcast<G, X - 1>::run(pw, pb);
    constexpr int x = X - 1;
    constexpr int L = ScoreMap<G>::lane_of(x);
    constexpr int S = ScoreMap<G>::slot_of(x);
    pb[x / G][x % G] = bcast_row<0x150 + L>(pw[S]);
  }
};
template <int G>
struct WeightBcast<G, 0> {
  __device__ __forceinline__ static void run(const float*, float (*)[G]) {}
};

// First of the 8 dims that lane row r (lane / 16) feeds into k-slice kk of the Q.K
// MFMA.  K is read in 16-byte pieces at byte 64*pc + 16*r of the token row: 8 bf16
// dims per piece (one k-slice) or 16 e4m3 dims (two k-slices).  Q is loaded at the
// same dims, so the order of dims inside the dot product is the only change.
template <int KBYTES>
__device__ __forceinline__ int mfma_kslice(int kk, int r) {
  return KBYTES == 2 ? 32 * kk + 8 * r : 64 * (kk >> 1) + 16 * r + 8 * (kk & 1);
}

// Softmax rescale factor of accumulator row i of lane row r (query row (4r + i) % G)
// from a lane that owns that query row: quad lane i of the same quad for G | 4
// (quad_perm [i,i,i,i]), lane 4 (r & 1) + i of the same lane row for G = 8.
template <int G>
__device__ __forceinline__ float mfma_row_alpha(float alpha, int i, int lane) {
  if constexpr (G == 8) {
    return __shfl(alpha, (lane & 48) + 4 * ((lane >> 4) & 1) + i, 64);
  } else {
    const int a = __float_as_int(alpha);
    switch (i) {
      case 0: return __int_as_float(__builtin_amdgcn_mov_dpp(a, 0x00, 0xf, 0xf, false));
      case 1: return __int_as_float(__builtin_amdgcn_mov_dpp(a, 0x55, 0xf, 0xf, false));
      case 2: return __int_as_float(__builtin_amdgcn_mov_dpp(a, 0xAA, 0xf, 0xf, false));
      default: return __int_as_float(__builtin_amdgcn_mov_dpp(a, 0xFF, 0xf, 0xf, false));
    }
  }
}

// ------------------------------------------------------------ balanced launch plan
// (plan.hpp).  Units of row r for the finalize's own plan: top-k, the row's selected
// blocks; dense, its 128-token tiles.
// Dense units are capped at k_cap = ceil(max_seq_len / tile): tokens past the host's
// bound are never read, and no row needs more than max_items items.
template <int SRC>
__device__ __forceinline__ int plan_row_units(const DecodeParams& p, int r) {
  if constexpr (SRC == kSrcTopk) {
    return min(max(p.n_sel[r], 0), p.k_cap);
  } else {
    return min(cdiv_pos(max(p.seq_lens[r / p.n_kv_heads], 0), p.unit_tokens), p.k_cap);
  }
}


// ------------------------------------------------------------ fused top-k call helpers

// Block scores of one (sequence, kv head), blocks [lo, hi), by the whole workgroup:
// in step t wave w scores block base + 32 t + 4 w + r (lane row r; 16 lanes per key
// row), NB steps in flight.  Mean key: s = sum_g q_g . k_bar / (G sqrt(D)); Quest:
// s = sum_g sum_d max(q_gd k_max_d, q_gd k_min_d) / G = (q+ . k_max + q- . k_min) / G
// with q+ = sum_g max(q_g, 0), q- = sum_g min(q_g, 0) (qa, qb).  The arithmetic is
// the standalone selector's (block_score / block_score_quest), so both give the same
// bits.  Scores land in s_lds[j].  qw holds the raw query words of the group's rows
// at this lane's dims (f32 q: floats; bf16 q: pairs in the first D/32 words); they
// are summed after the first step batch's loads are issued, so the caller's query
// loads share that round trip.  SHARED: the rows are read by other workgroups of the
// same XCD too (plain loads, so their lines stay in L2 for them); else streaming loads.
// key words per lane in flight in one step batch of the scorer (a value: registers,
// never memory)
template <int D>
using ScoreWords = u32 __attribute__((ext_vector_type(D >= 128 ? 64 : 32)));

template <int D, int G, bool KBF16, bool QUEST, bool SHARED>
struct BlockScorer {
  static constexpr int DPL = D / 16;
  static constexpr int EB = KBF16 ? 2 : 4;
  static constexpr int NWR = DPL * EB / 4;                        // words per lane per key row
  static constexpr int NW = D >= 128 ? 64 : 32;                   // key words per lane in flight
  static constexpr int NS = NW / NWR / (QUEST ? 2 : 1);           // steps in flight (Quest reads two rows per block)
  // whole-row scorers sum a batch's steps with one reduce-scatter; range scorers (a
  // step or two per item) keep a row sum per step, which costs less there
  static constexpr bool kScatter = SHARED && NS >= 4 && NS <= 32;
  using words_t = ScoreWords<D>;

  // the loads of every step of the batch at base that holds a block of [.., hi), without
  // a per-lane condition (rows past hi re-read row hi - 1); steps past it are skipped
  __device__ __forceinline__ static void issue(const DecodeParams& p, int64_t kb_off, int base, int hi, words_t& w) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int c16 = lane & 15;
    const int r = lane >> 4;
    const char* k1 = reinterpret_cast<const char*>(p.kb) + kb_off * EB;
    const char* k2 = reinterpret_cast<const char*>(p.kb2) + kb_off * EB;
#pragma unroll
    for (int t = 0; t < NS; ++t) {
      if (base + 32 * t >= hi) break;  // uniform
      const int j = min(base + 32 * t + 4 * wave + r, hi - 1);
#pragma unroll
      for (int q = 0; q < (QUEST ? 2 : 1); ++q) {
        const char* rowp = (q ? k2 : k1) + ((int64_t)j * D + c16 * DPL) * EB;
        const int o = (QUEST ? 2 * t + q : t) * NWR;
        if constexpr (NWR >= 4) {
#pragma unroll
          for (int v4 = 0; v4 < NWR; v4 += 4) {
            const u32x4_t x = SHARED ? *reinterpret_cast<const u32x4_t*>(rowp + 4 * v4) : ld_stream16(rowp + 4 * v4);
            w[o + v4] = x[0];
            w[o + v4 + 1] = x[1];
            w[o + v4 + 2] = x[2];
            w[o + v4 + 3] = x[3];
          }
        } else {
          const u32x2_t x = SHARED ? *reinterpret_cast<const u32x2_t*>(rowp) : ld_stream8(rowp);
          w[o] = x[0];
          w[o + 1] = x[1];
        }
      }
    }
  }

  // Scores of blocks [lo, hi) into s_lds
  __device__ __forceinline__ static void run(const DecodeParams& p, int64_t kb_off, int lo, int hi,
                                             const u32 (&qw)[G][D / 16], float* s_lds, words_t& w) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int c16 = lane & 15;
    const int r = lane >> 4;
    auto compute = [&](int base, const words_t& wv, const float* qa, const float* qb) {
      if constexpr (kScatter) {
        // whole-row scoring runs full batches: the NS steps' lane shares are summed by
        // one reduce-scatter over the 16-lane row (4 DPP rounds for all of them)
        // instead of a row sum per step; each lane then holds whole scores
        float v[NS];
#pragma unroll
        for (int t = 0; t < NS; ++t) {
          v[t] = 0.f;
          if (base + 32 * t >= hi) continue;  // uniform
          u32 w1[NWR], w2[NWR];
#pragma unroll
          for (int e = 0; e < NWR; ++e) {
            w1[e] = wv[(QUEST ? 2 * t : t) * NWR + e];
            w2[e] = QUEST ? wv[(2 * t + 1) * NWR + e] : 0u;
          }
          v[t] = QUEST ? block_dot_quest<DPL, KBF16>(w1, w2, qa, qb) : block_dot<DPL, KBF16>(w1, qa);
        }
        reduce_scatter16<NS>(v, lane);
        constexpr int kHeld = NS >= 16 ? NS / 16 : 1;  // steps a lane holds
        constexpr int kCopies = NS >= 16 ? 1 : 16 / NS;  // lanes holding each step
#pragma unroll
        for (int k = 0; k < kHeld; ++k) {
          const int t = NS == 32 ? 2 * c16 + k : c16 / kCopies;
          const int j = base + 32 * t + 4 * wave + r;
          if (c16 % kCopies == 0 && base + 32 * t < hi && j < hi) s_lds[j] = v[k] * p.score_scale;
        }
      } else {
#pragma unroll
        for (int t = 0; t < NS; ++t) {
          if (base + 32 * t >= hi) break;  // uniform
          const int j = base + 32 * t + 4 * wave + r;
          u32 w1[NWR], w2[NWR];
#pragma unroll
          for (int e = 0; e < NWR; ++e) {
            w1[e] = wv[(QUEST ? 2 * t : t) * NWR + e];
            w2[e] = QUEST ? wv[(2 * t + 1) * NWR + e] : 0u;
          }
          const float a = QUEST ? block_score_quest<DPL, KBF16>(w1, w2, qa, qb, p.score_scale)
                                : block_score<DPL, KBF16>(w1, qa, p.score_scale);
          if (c16 == 0 && j < hi) s_lds[j] = a;
        }
      }
    };
    if (lo >= hi) return;
    issue(p, kb_off, lo, hi, w);
    // qa = sum_g q_g (mean key); Quest: qa = sum_g q_g+, qb = sum_g q_g- (the standalone
    // selector's order), while the first batch is in flight
    float qa[DPL], qb[DPL];
#pragma unroll
    for (int e = 0; e < DPL; ++e) {
      qa[e] = 0.f;
      qb[e] = 0.f;
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int e = 0; e < DPL; ++e) {
        const float v = p.q_f32 ? __uint_as_float(qw[g][e]) : ((e & 1) ? bf16_hi(qw[g][e >> 1]) : bf16_lo(qw[g][e >> 1]));
        if constexpr (QUEST) {
          qa[e] += fmaxf(v, 0.f);
          qb[e] += fminf(v, 0.f);
        } else {
          qa[e] += v;
        }
      }
    }
    compute(lo, w, qa, qb);
    for (int base = lo + 32 * NS; base < hi; base += 32 * NS) {
      issue(p, kb_off, base, hi, w);
      compute(base, w, qa, qb);
    }
  }
};

template <int D, int G, bool KBF16, bool QUEST, bool SHARED>
__device__ __forceinline__ void score_blocks(const DecodeParams& p, int64_t kb_off, int lo, int hi,
                                             const u32 (&qw)[G][D / 16], float* s_lds) {
  ScoreWords<D> w;
  BlockScorer<D, G, KBF16, QUEST, SHARED>::run(p, kb_off, lo, hi, qw, s_lds, w);
}

constexpr int kMaxMergeSlots = kMaxItemsPerBh + kMaxRouteChunks;  // split-K items + representative partials
constexpr int kMergeFastSlots = 8;  // slots per wave read in the merge's one-round-trip path
constexpr int kMergeGroup = kMergeFastSlots;            // slots per merge group
constexpr int kMergeGroups = kMaxItemsPerBh / kMergeGroup;  // groups of a row's split-K items
constexpr int kFlagStride = 64;  // u32 words between hand-off flags (one 256-byte line each)
constexpr int kSoloItems = 3;    // fused top-k call: rows of at most this many items score the whole row per item

// The split-K merge of a row's items (balanced launches: the merge kernel and the
// fused top-k call's in-kernel merge share it, so both give the same bits).  Slots
// are taken in groups of kMergeGroup: a group's partial is M = max_j m_j,
// L = sum_j f_j l_j, a = sum_j f_j acc_j with f_j = 2^(m_j - M), slots in order
// (absent slots hold m = -inf); the groups are combined the same way, in order, and
// out = a / max(L, 1e-30) (CBT/legacy.py:765-794).  One lane holds PER consecutive
// outputs of the row's [G, D] block, all of one query row.
template <int PER>
__device__ __forceinline__ void merge_group(const float* mv, const float* lv, const float (*av)[PER], float& M,
                                            float& L, float* a) {
  M = kNegInf;
#pragma unroll
  for (int j = 0; j < kMergeGroup; ++j) M = fmaxf(M, mv[j]);
  L = 0.f;
#pragma unroll
  for (int e = 0; e < PER; ++e) a[e] = 0.f;
  if (M != kNegInf) {
#pragma unroll
    for (int j = 0; j < kMergeGroup; ++j) {
      const float f = (mv[j] == kNegInf) ? 0.f : exp2f(mv[j] - M);
      L += f * lv[j];
#pragma unroll
      for (int e = 0; e < PER; ++e) a[e] = fmaf(f, av[j][e], a[e]);
    }
  }
}

// Combine ng <= kMergeGroups group partials in order (gm/gl/ga give group g's M, L
// and outputs; the loop bound is a constant so that register arrays stay in
// registers); writes the PER outputs of the lane through store(e, value).
template <int PER, typename GM, typename GL, typename GA, typename Store>
__device__ __forceinline__ void merge_combine(int ng, GM gm, GL gl, GA ga, Store store) {
  float M = kNegInf;
#pragma unroll
  for (int g = 0; g < kMergeGroups; ++g)
    if (g < ng) M = fmaxf(M, gm(g));
  float L = 0.f, a[PER];
#pragma unroll
  for (int e = 0; e < PER; ++e) a[e] = 0.f;
  if (M != kNegInf) {
#pragma unroll
    for (int g = 0; g < kMergeGroups; ++g) {
      if (g < ng) {
        const float mg = gm(g);
        const float f = (mg == kNegInf) ? 0.f : exp2f(mg - M);
        L += f * gl(g);
#pragma unroll
        for (int e = 0; e < PER; ++e) a[e] = fmaf(f, ga(g, e), a[e]);
      }
    }
  }
#pragma unroll
  for (int e = 0; e < PER; ++e) store(e, a[e] / fmaxf(L, 1e-30f));
}

// The fused call's in-kernel split-K merge, run by the row's last item to finish
// (every thread of its workgroup calls it): the row's n partials are read at the
// coherence point and merged with the merge kernel's merge_group / merge_combine
// arithmetic, so the output equals the two-step path's bit for bit (which lane
// computes an output does not change its arithmetic).  The row's partials sit in
// the slots of its workgroups, slot0 .. slot0 + n - 1.  Each thread merges outputs
// o = threadIdx.x + kFinThreads k.  NGL = the merge groups loaded (a power of two
// >= ceil(n / 8), chosen by the caller): every load is unconditional (slot indices
// clamped; slots past n are weighed by 0), the (m, l) words first and the first
// pass's accumulators after them, so the wait for the (m, l) words leaves the
// accumulators in flight and the merge of up to 32 slots costs one round trip
// (more slots: a second batch of four groups after the first).  (Loads under
// per-group branches made the compiler wait for half of them at a branch join
// before the (m, l) loads went out: two round trips.)
template <int D, int G, int NGL>
__device__ __forceinline__ void fused_merge(const DecodeParams& p, int b, int h, int64_t slot0, int n) {
  static_assert(NGL >= 1 && NGL <= kMergeGroups, "merge groups");
  constexpr int NO = (G * D + kFinThreads - 1) / kFinThreads;  // outputs per thread
  constexpr int NB = NGL < 4 ? NGL : 4;                        // groups per load batch
  constexpr int NBATCH = NGL / NB;
  __shared__ float ml_lds[kMaxItemsPerBh][G][2];
  constexpr int kMlPer = (kMaxItemsPerBh * G + kFinThreads - 1) / kFinThreads;
  float mlv[kMlPer][2];
#pragma unroll
  for (int i = 0; i < kMlPer; ++i) {
    const int t = min(threadIdx.x + kFinThreads * i, n * G - 1);
    mlv[i][0] = ld_agent(p.part_ml + (slot0 * G + t) * 2);
    mlv[i][1] = ld_agent(p.part_ml + (slot0 * G + t) * 2 + 1);
  }
  float acc[NB][kMergeGroup];
  auto load_acc = [&](int o, int gb) {  // groups gb .. gb + NB - 1
#pragma unroll
    for (int g = 0; g < NB; ++g)
#pragma unroll
      for (int j = 0; j < kMergeGroup; ++j)
        acc[g][j] = ld_agent(p.part_acc + (slot0 + min(kMergeGroup * (gb + g) + j, n - 1)) * (G * D) + o);
  };
  load_acc(threadIdx.x < G * D ? threadIdx.x : 0, 0);
#pragma unroll
  for (int i = 0; i < kMlPer; ++i) {
    const int t = threadIdx.x + kFinThreads * i;
    if (t < n * G) {
      ml_lds[t / G][t % G][0] = mlv[i][0];
      ml_lds[t / G][t % G][1] = mlv[i][1];
    }
  }
  const int ng = (n + kMergeGroup - 1) / kMergeGroup;
  __syncthreads();
  // one output per pass (G * D > kFinThreads takes several passes)
#pragma unroll 1
  for (int k = 0; k < NO; ++k) {
    const int o = threadIdx.x + kFinThreads * k;
    if (o >= G * D) break;
    const int g0 = o / D;
    float gM[kMergeGroups], gL[kMergeGroups], ga[kMergeGroups][1];
#pragma unroll
    for (int g = 0; g < kMergeGroups; ++g) {
      gM[g] = kNegInf;
      gL[g] = 0.f;
      ga[g][0] = 0.f;
    }
#pragma unroll
    for (int bt = 0; bt < NBATCH; ++bt) {
      if (k > 0 || bt > 0) load_acc(o, NB * bt);
#pragma unroll
      for (int gi = 0; gi < NB; ++gi) {
        const int g = NB * bt + gi;
        if (g < ng) {
          float mv[kMergeGroup], lv[kMergeGroup], av[kMergeGroup][1];
#pragma unroll
          for (int j = 0; j < kMergeGroup; ++j) {
            const int s = kMergeGroup * g + j;
            mv[j] = s < n ? ml_lds[s][g0][0] : kNegInf;
            lv[j] = s < n ? ml_lds[s][g0][1] : 0.f;
            av[j][0] = acc[gi][j];
          }
          merge_group<1>(mv, lv, av, gM[g], gL[g], ga[g]);
        }
      }
    }
    merge_combine<1>(
        ng, [&](int g) { return gM[g]; }, [&](int g) { return gL[g]; }, [&](int g, int) { return ga[g][0]; },
        [&](int, float v) { store_decode_out<G, D>(p, b, h, o, v); });
  }
}

// Tag of a row's published words (score entries and tagged partials): a slot or an
// entry serves whichever row the launch plan (and the call shape) gives it, so the
// tag names the row too: row << 19 | (epoch mod (2^19 - 1)) + 1 (rows < 2^13).  The
// low part is never 0, so a zero-filled word never matches, and the row's epoch only
// grows (it is never reset between calls of any shape), so a word left by an earlier
// call of any row never matches unless it is 2^19 - 1 split calls of the same row old.
__device__ __forceinline__ u32 partial_tag(int bh, u32 row_epoch) {
  return ((u32)bh << 19) | ((row_epoch % 0x7ffffu) + 1u);
}

// The merge of a row of at most kMergeGroup items whose partials were published as
// tagged 8-byte words (value bits | tag << 32, tag = partial_tag): every
// slot's words are loaded at once and a word whose tag has not arrived yet is read
// again (its publisher has passed the row's counter, so its stores are in flight).
// One merge group: the merge kernel's arithmetic, the same bits.  These reads wait
// for stores already issued, so their bound is at least kMergeWaitTicks whatever the
// caller's wait limit (which governs the score hand-off, where a fallback exists); a
// word still missing then turns the output into NaN (never silent).
constexpr long long kMergeWaitTicks = 2000000;  // 20 ms of the 100 MHz clock
template <int D, int G>
__device__ __forceinline__ void fused_merge_tagged(const DecodeParams& p, int b, int h, int64_t slot0, int n, u32 tag) {
  constexpr int NO = (G * D + kFinThreads - 1) / kFinThreads;  // outputs per thread
  constexpr int W = G * D + 2 * G;                             // words per slot
  __shared__ float mlt_lds[kMergeGroup][G][2];
  const unsigned long long t0 = clock_100mhz();
  const long long bound = max((long long)p.wait_ticks, kMergeWaitTicks);
  auto value = [&](const unsigned long long* ptr, unsigned long long v) -> float {
    while ((u32)(v >> 32) != tag && (long long)(clock_100mhz() - t0) <= bound) {
      __builtin_amdgcn_s_sleep(1);
      v = ld_agent_u64(ptr);
    }
    if ((u32)(v >> 32) == tag) return __uint_as_float((u32)v);
    note_wait_fallback();
    return __builtin_nanf("");
  };
  // (m, l) of every slot, staged in LDS
  if (threadIdx.x < kMergeGroup * G * 2) {
    const int s = threadIdx.x / (G * 2), e = threadIdx.x % (G * 2);
    const unsigned long long* ptr = p.tpart + (slot0 + min(s, n - 1)) * W + G * D + e;
    const float v = value(ptr, ld_agent_u64(ptr));
    if (s < n) mlt_lds[s][e / 2][e % 2] = v;
  }
#pragma unroll 1
  for (int k = 0; k < NO; ++k) {
    const int o = threadIdx.x + kFinThreads * k;
    unsigned long long raw[kMergeGroup];
    const bool active = o < G * D;
    const int oc = active ? o : 0;
#pragma unroll
    for (int j = 0; j < kMergeGroup; ++j) raw[j] = ld_agent_u64(p.tpart + (slot0 + min(j, n - 1)) * W + oc);
    float av[kMergeGroup][1];
#pragma unroll
    for (int j = 0; j < kMergeGroup; ++j)
      av[j][0] = j < n ? value(p.tpart + (slot0 + j) * W + oc, raw[j]) : 0.f;
    if (k == 0) __syncthreads();  // the (m, l) staging
    if (!active) continue;
    const int g0 = o / D;
    float mv[kMergeGroup], lv[kMergeGroup];
#pragma unroll
    for (int j = 0; j < kMergeGroup; ++j) {
      mv[j] = j < n ? mlt_lds[j][g0][0] : kNegInf;
      lv[j] = j < n ? mlt_lds[j][g0][1] : 0.f;
    }
    float gM, gL, ga[1];
    merge_group<1>(mv, lv, av, gM, gL, ga);
    merge_combine<1>(
        1, [&](int) { return gM; }, [&](int) { return gL; }, [&](int, int) { return ga[0]; },
        [&](int, float v) { store_decode_out<G, D>(p, b, h, o, v); });
  }
}

}  // namespace ia

#include "cond_fused.hpp"

namespace ia {

template <int D, int G, typename KV, int SRC, bool KROWS = false>
__global__ __launch_bounds__(kFinThreads, 2) void ia_condition_block_paged_finalize(DecodeParams p) {
  constexpr int DPL = D / 16;
  constexpr int NWD = DPL * KV::kBytes / 4;
  using SM = ScoreMap<G>;
  constexpr int NV = SM::NV;
  constexpr int KG = SM::KG;
  constexpr bool kBf16 = KV::kBytes == 2;
  constexpr bool kFp8 = KV::kBytes == 1;
  // bf16 caches, and fp8 caches whose e4m3 codes widen exactly to bf16, run Q.K and
  // P.V as bf16 pairs through v_dot2_f32_bf16; fp32 caches stay fp32
  constexpr bool kDot2 = kBf16 || kFp8;
  constexpr int NWB = DPL / 2;  // bf16 words per lane per token row
  // bf16 / fp8 caches: Q.K and P.V on MFMA (query rows padded to the 16-row tile)
  constexpr bool kMfma = kDot2;
  constexpr int kMfmaK = D / 32;  // 32-dim k-slices of Q.K
  // fp32 caches with G x D / 16 >= 32 query words per lane (G >= 4 at D = 128): the
  // query rows are read from LDS inside the subtile loop instead of being held in
  // registers, which keeps the instance within 256 registers (no spill)
  constexpr bool kQLds = !kDot2 && G * DPL >= 32;

  __shared__ int unit_lo[kMaxUnitsPerItem];
  __shared__ int unit_hi[kMaxUnitsPerItem];
  __shared__ int sub_pg[kMaxSubsPerItem];    // page id of each valid subtile (kSfxPage: suffix)
  __shared__ int sub_info[kMaxSubsPerItem];  // first row in the page (or suffix token) << 5 | valid rows
  __shared__ int sub_sc[kFp8 ? kMaxSubsPerItem : 1];  // fp8 with sequence scales: 2 x logical page
  __shared__ int wcnt_p[kFinWaves];
  __shared__ int wprog[kFinWaves];  // subtiles consumed per wave
  __shared__ int rc_prefix[SRC == kSrcLists ? kMaxRouteChunks + 1 : 1];
  __shared__ int rc_entries[SRC == kSrcLists ? kSpecEntries : 1];
  __shared__ float fsc[SRC == kSrcTopkFused ? kFusedMaxBlocks : 1];
  __shared__ int fsel[SRC == kSrcTopkFused ? kMaxUnitsPerItem : 1];
  __shared__ TopkLds<kFinThreads> ftk;
  __shared__ float wacc_lds[kFinWaves][G * D];
  // bf16 caches at D = 128: each wave's key subtile (16 token rows of 16 16-byte
  // pieces) on its way from whole-row loads to the MFMA operand layout (slots
  // XOR-swizzled per row).  Whole-row loads use full cache lines per instruction (the
  // operand layout's loads read 64 bytes of sixteen rows), which raises one CU's
  // stream rate where HBM is not saturated: items of uneven length (ragged rows, the
  // condition calls' few-subtile items).  Where every workgroup streams equal shares
  // at the HBM rate the transpose costs more than it gains (C4 +0.66 us), so the
  // one-launch top-k call takes it in its KROWS instance only (the host picks that
  // one for launches with per-sequence k, its variable-length batches), and the dense
  // and top-k-list sources never.
  constexpr bool kKeyLdsAny =
      kMfma && kBf16 && D == 128 && ((SRC == kSrcTopkFused && KROWS) || SRC == kSrcLists || SRC == kSrcCondFused);
  __shared__ u32x4_t key_lds[kKeyLdsAny ? kFinWaves : 1][kKeyLdsAny ? 256 : 1];
  __shared__ float q_lds[kQLds ? G * D : 1];
  __shared__ float wm_lds[kFinWaves][G];
  __shared__ float wl_lds[kFinWaves][G];

  __shared__ PlanEntry plan_lds;
  __shared__ u32 merge_todo[1];  // fused calls: this workgroup merges its row
  __shared__ std::conditional_t<SRC == kSrcCondFused, CondLds<D, G>, char> cond_lds;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c16 = lane & 15;
  const int r = lane >> 4;
  constexpr bool kBalanced = src_balanced(SRC);
  constexpr bool kListUnits = SRC == kSrcLists || SRC == kSrcCondFused;  // blocks then suffix tiles
  const int nsub_u = ((kListUnits ? max(p.unit_tokens, kDenseTile) : p.unit_tokens) + 15) / 16;
  if (threadIdx.x < kFinWaves) wprog[threadIdx.x] = 0;  // read after the prologue's barriers

  // ---- this workgroup's (b, h) row and its item: from the launch plan (balanced
  // sources; the fused top-k plan comes from the scorer launch), else from the grid
  int b, h, item, n_items_row = 1, slot_lo = 0, slot_hi = 0, seq_len = 0, n_units = 0, n_blk_units = 0, sfx_len = 0;
  int k_b = p.topk_k;

  // query rows of kv head hq of sequence bq: raw loads, converted after the
  // prologue.  Vector path: every row at the lane's dim slice c16*DPL ..; MFMA path:
  // row c16 % G at the dims of the lane's k-slices.
  constexpr int QR0 = kMfma ? kMfmaK : G;
  constexpr int QR1 = kMfma ? 8 : DPL;
  u32 qraw[QR0][QR1];  // f32 q: floats; bf16 q: pairs in the lower half (upper half unused)
  // One-launch top-k call: the same two plain loads on both q dtypes, straight into
  // qraw, with no load under a branch and no arithmetic on the loaded words until they
  // are used (f32 rows read their two halves, bf16 rows their one half twice, the copy
  // landing in the unused upper half): loads under the dtype branch made the compiler
  // wait for every load in flight before each of them, in the middle of the selection
  // (C3 -0.5, C5 -0.4, C2 -0.2 us).  The other sources load q at the start, where the
  // branch-free form's extra loads sit ahead of the first summary rows and measured
  // slower (one-launch eps-rule call +0.4-0.7 us), so they keep the dtype branch.
  auto load_q = [&](int bq, int hq) {
    const bool qf = p.q_f32 != 0;
#pragma unroll
    for (int x = 0; x < QR0; ++x) {
      const int g = kMfma ? c16 % G : x;
      const int d0 = kMfma ? mfma_kslice<KV::kBytes>(x, r) : c16 * DPL;
      constexpr int NE = kMfma ? 8 : DPL;
      static_assert(NE == QR1, "one query slice per row of qraw");
      const int64_t row = (int64_t)bq * p.q_batch_stride + (int64_t)(hq * G + g) * p.q_row_stride;
      if constexpr (SRC == kSrcTopkFused) {
        const char* q0 = reinterpret_cast<const char*>(p.q) + (row + d0) * (qf ? 4 : 2);
        load_cached_words<NE / 2>(q0, qraw[x]);
        load_cached_words<NE / 2>(qf ? q0 + NE * 2 : q0, qraw[x] + NE / 2);
      } else if (qf) {
        const u32* qp = reinterpret_cast<const u32*>(p.q) + row + d0;
#pragma unroll
        for (int e = 0; e < NE; ++e) qraw[x][e] = qp[e];
      } else {
        const unsigned short* qp = reinterpret_cast<const unsigned short*>(p.q) + row + d0;
#pragma unroll
        for (int e = 0; e < NE / 2; ++e) qraw[x][e] = (u32)qp[2 * e] | ((u32)qp[2 * e + 1] << 16);
#pragma unroll
        for (int e = NE / 2; e < QR1; ++e) qraw[x][e] = 0u;
      }
    }
  };
  u32 row_epoch = 0u;  // fused top-k call: calls so far that split this row
  // fused top-k call: the plan slot of this workgroup.  Workgroup w runs on XCD w % 8
  // (the dispatcher deals workgroups to the XCDs in turn), so slot
  // (w % 8) * (grid / 8) + w / 8 puts consecutive slots -- the items of one row -- on
  // one XCD, where they share the row's block-key lines through its L2.  (Placement
  // only: any mapping gives the same results.)
  constexpr int SDPL = D / 16;  // key dims per lane in the scorer (16 lanes per key row)
  const int fused_slot = (gridDim.x % 8 == 0)
                             ? (int)((blockIdx.x % 8) * (gridDim.x / 8) + blockIdx.x / 8)
                             : (int)blockIdx.x;
  if constexpr (kBalanced) {
    PlanEntry e;
    if constexpr (SRC == kSrcTopkFused) {
      // every wave evaluates the launch plan itself (no barrier, no round trip to a
      // plan written elsewhere): a row's units are the blocks the top-k rule takes.
      // The lengths and k of the rows a lane holds in registers are loaded first, all
      // in one round trip (clamped indices, no per-lane branch).
      int pre_len[kPlanRegRows], pre_k[kPlanRegRows];
      const int last_row = max(p.n_rows - 1, 0);
#pragma unroll
      for (int k = 0; k < kPlanRegRows; ++k) pre_len[k] = p.seq_lens[min(lane + 64 * k, last_row) / p.n_kv_heads];
      if (p.k_per_seq) {
#pragma unroll
        for (int k = 0; k < kPlanRegRows; ++k) pre_k[k] = p.k_per_seq[min(lane + 64 * k, last_row) / p.n_kv_heads];
      } else {
#pragma unroll
        for (int k = 0; k < kPlanRegRows; ++k) pre_k[k] = p.topk_k;
      }
      auto row_slots = [&](int len, int kr) -> int {
        const int nbs_r = min(cdiv_pos(max(len, 0), p.unit_tokens), p.nb_max);
        return topk_count(nbs_r, TopkRule{p.forced_first, p.forced_last, max(kr, 0), p.forced_in_k, p.k_cap}) *
               nsub_u;
      };
      auto slots_of = [&](int rr) -> int {
        if ((rr & 63) == lane && (rr >> 6) < kPlanRegRows) {
          int len = pre_len[0], kr = pre_k[0];
#pragma unroll
          for (int k = 1; k < kPlanRegRows; ++k)
            if ((rr >> 6) == k) {
              len = pre_len[k];
              kr = pre_k[k];
            }
          return row_slots(len, kr);
        }
        const int bb = rr / p.n_kv_heads;
        return row_slots(p.seq_lens[bb], p.k_per_seq ? p.k_per_seq[bb] : p.topk_k);
      };
      PlanRows rows;
      const PlanRule rule = plan_rule_wave(slots_of, p.n_rows, p.plan_budget, p.max_items, nsub_u, rows);
      e = plan_entry_wave(slots_of, rows, p.n_rows, rule, fused_slot, nsub_u);
      // the row's length and k from the lane that holds it
      const int row_e = __builtin_amdgcn_readfirstlane(e.row);
      if (row_e >= 0 && row_e < 64 * kPlanRegRows) {
        int len = pre_len[0], kr = pre_k[0];
#pragma unroll
        for (int k = 1; k < kPlanRegRows; ++k)
          if ((row_e >> 6) == k) {
            len = pre_len[k];
            kr = pre_k[k];
          }
        e.seq_len = __builtin_amdgcn_readlane(len, row_e & 63);
        e.k_row = __builtin_amdgcn_readlane(kr, row_e & 63);
      } else if (row_e >= 0) {
        e.seq_len = p.seq_lens[row_e / p.n_kv_heads];
        e.k_row = p.k_per_seq ? p.k_per_seq[row_e / p.n_kv_heads] : p.topk_k;
      }
    } else if constexpr (SRC == kSrcCondFused) {
      // every row alike: n items per row, consecutive plan slots (the items' units
      // are known only after their routing)
      const int n_it = p.c_items;
      const int row = fused_slot / n_it;
      e.row = row < p.n_rows ? row : -1;
      e.item = fused_slot - row * n_it;
      e.n_items = n_it;
      e.slot_lo = e.slot_hi = e.n_units = e.seq_len = e.k_row = 0;
    } else {
      if (wave == 0) {
        PlanRows rows;
        auto slots_of = [&](int rr) -> int { return plan_row_units<SRC>(p, rr) * nsub_u; };
        const PlanRule rule = plan_rule_wave(slots_of, p.n_rows, p.plan_budget, p.max_items, nsub_u, rows);
        const PlanEntry pe = plan_entry_wave(slots_of, rows, p.n_rows, rule, (int)blockIdx.x, nsub_u);
        if (lane == 0) plan_lds = pe;
      }
      __syncthreads();
      e = plan_lds;
    }
    const int row = __builtin_amdgcn_readfirstlane(e.row);
    if (row < 0) return;  // idle workgroup (the whole workgroup)
    b = row / p.n_kv_heads;
    h = row - b * p.n_kv_heads;
    item = __builtin_amdgcn_readfirstlane(e.item);
    n_items_row = __builtin_amdgcn_readfirstlane(e.n_items);
    slot_lo = __builtin_amdgcn_readfirstlane(e.slot_lo);
    slot_hi = __builtin_amdgcn_readfirstlane(e.slot_hi);
    n_units = __builtin_amdgcn_readfirstlane(e.n_units);
    if constexpr (SRC == kSrcTopkFused) {
      seq_len = max(__builtin_amdgcn_readfirstlane(e.seq_len), 0);
      k_b = max(__builtin_amdgcn_readfirstlane(e.k_row), 0);
    } else if constexpr (SRC != kSrcCondFused) {
      seq_len = max(p.seq_lens[b], 0);
    }
  } else {
    b = blockIdx.z;
    h = blockIdx.y;
    item = blockIdx.x;
  }
  const int bh = b * p.n_kv_heads + h;
  // (the epoch stays in a vector register until the publish, so its load is not
  // waited for here)
  u32 row_epoch_v = 0u;
  if constexpr (src_fused(SRC)) row_epoch_v = ld_agent_u32(p.rowctr + (int64_t)bh * kFlagStride + 1);
  if constexpr (SRC != kSrcTopkFused) load_q(b, h);

  if constexpr (SRC == kSrcTopkFused) {
    // ---- block scores: item i of the row's n scores blocks [i nbs / n, (i+1) nbs / n)
    // into LDS and publishes them as tagged 8-byte entries, score bits | tag << 32 with
    // tag = partial_tag(row, epoch) (the epoch counts the calls that split the row, so
    // an entry left by an earlier call, of this row or another, never matches).  Each item takes the other items'
    // blocks from the entries whose tag has arrived; when one is still missing at the
    // wait bound, it scores the other items' blocks itself (same arithmetic, same
    // bits).  Every item then holds the whole row and applies the shared top-k rule
    // (item 0 publishes the chosen blocks).
    const int nbs = min(cdiv_pos(seq_len, p.unit_tokens), p.nb_max);
    const int n_it = n_items_row;
    // (G > 4 keeps the hand-off: its query words leave no room for a second scorer form)
    constexpr bool kSoloG = G <= 4;
    // rows of up to kSoloItems items: every item scores the whole row itself (the
    // row's items sit on one XCD and read the key lines in the same order, so the
    // second read of a line is an L2 hit) and no scores are handed over; rows of more
    // items split the scoring and hand the scores to each other.  Measured
    // (alternating builds on one box): C5 66.4 against 67.8 us, C4 unchanged; ragged
    // C3 rows of 1-3 items -0.4 to -0.5 us; 32-item rows (C2) +0.4 us whole-row.
    const bool solo = kSoloG && n_it <= kSoloItems;
    auto range_lo = [&](int i) { return (i * nbs) / n_it; };  // (< 2^19: 32-bit arithmetic)
    unsigned long long* row_entries = p.sbuf + (int64_t)bh * p.nb_max;
    const int own_lo = solo ? 0 : range_lo(item), own_hi = solo ? nbs : range_lo(item + 1);
    const TopkRule rule{p.forced_first, p.forced_last, k_b, p.forced_in_k, p.k_cap};
    const TopkForced forced(rule, nbs);
    // the candidates' largest key and largest ~key, taken while the scores pass by
    u32 kmx = 0u, kmn_inv = 0u;
    auto see = [&](int j, float sc) {
      if (!forced(j)) {
        const u32 key = order_key(sc);
        kmx = max(kmx, key);
        kmn_inv = max(kmn_inv, ~key);
      }
    };
    bool staged = false;  // uniform: topk_stage done with the whole row's keys
    {
      // the group's query rows at this lane's dims: loads issued now, summed inside the
      // scorer once its first key batch is in flight (one round trip for both)
      // (the same two loads on both q dtypes, no branch: f32 rows read their two
      // halves, bf16 rows their one slice twice)
      u32 qw[G][SDPL];
      const int q_es = p.q_f32 ? 4 : 2;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const int64_t qrow = (int64_t)b * p.q_batch_stride + (int64_t)(h * G + g) * p.q_row_stride + c16 * SDPL;
        const char* q0 = reinterpret_cast<const char*>(p.q) + qrow * q_es;
        load_words<SDPL / 2>(q0, qw[g]);
        load_words<SDPL / 2>(p.q_f32 ? q0 + SDPL * 2 : q0, qw[g] + SDPL / 2);
      }
      const int64_t kb_off = (int64_t)b * p.kb_batch_stride + (int64_t)h * p.kb_head_stride;
      // blocks [lo, hi): 32 per workgroup step (wave w, lane row r: block 32 t + 4 w + r)
      auto score_range = [&](int lo, int hi) {
        if (kSoloG && solo && n_it > 1) {
          if (p.score_quest) {
            if (p.kb_bf16) score_blocks<D, G, true, true, true>(p, kb_off, lo, hi, qw, fsc);
            else score_blocks<D, G, false, true, true>(p, kb_off, lo, hi, qw, fsc);
          } else {
            if (p.kb_bf16) score_blocks<D, G, true, false, true>(p, kb_off, lo, hi, qw, fsc);
            else score_blocks<D, G, false, false, true>(p, kb_off, lo, hi, qw, fsc);
          }
        } else if (p.score_quest) {
          if (p.kb_bf16) score_blocks<D, G, true, true, false>(p, kb_off, lo, hi, qw, fsc);
          else score_blocks<D, G, false, true, false>(p, kb_off, lo, hi, qw, fsc);
        } else {
          if (p.kb_bf16) score_blocks<D, G, true, false, false>(p, kb_off, lo, hi, qw, fsc);
          else score_blocks<D, G, false, false, false>(p, kb_off, lo, hi, qw, fsc);
        }
      };
      score_range(own_lo, own_hi);
      if (!solo) {
        if (threadIdx.x == 0) merge_todo[0] = 0u;
        __syncthreads();
        row_epoch = __builtin_amdgcn_readfirstlane(row_epoch_v);
        const u32 tag = partial_tag(bh, row_epoch);
        for (int j = own_lo + threadIdx.x; j < own_hi; j += kFinThreads) {
          const float sc = fsc[j];
          st_agent_u64(row_entries + j, ((unsigned long long)tag << 32) | __float_as_uint(sc));
          see(j, sc);
        }
        const unsigned long long t0 = clock_100mhz();
        bool missing = false;
        for (int j = threadIdx.x; j < nbs; j += kFinThreads) {
          if (j >= own_lo && j < own_hi) continue;
          unsigned long long v = ld_agent_u64(row_entries + j);
          while ((u32)(v >> 32) != tag && (long long)(clock_100mhz() - t0) <= p.wait_ticks) {
            __builtin_amdgcn_s_sleep(1);
            v = ld_agent_u64(row_entries + j);
          }
          if ((u32)(v >> 32) == tag) {
            const float sc = __uint_as_float((u32)v);
            fsc[j] = sc;
            see(j, sc);
          } else {
            missing = true;
          }
        }
        if (missing) merge_todo[0] = 1u;
        load_q(b, h);  // the stream's query operands: in flight during the selection
        topk_stage<kFinThreads>(ftk, kmx, kmn_inv);
        __syncthreads();
        staged = merge_todo[0] == 0u;
        if (!staged) {  // an entry missed the bound: the other items' blocks here
          if (threadIdx.x == 0) note_wait_fallback();
          score_range(0, own_lo);
          score_range(own_hi, nbs);
        }
      }
    }
    row_epoch = __builtin_amdgcn_readfirstlane(row_epoch_v);
    if (!staged) {  // one pass over the whole row in LDS
      if (solo) load_q(b, h);
      __syncthreads();
      kmx = 0u;
      kmn_inv = 0u;
      for (int t = threadIdx.x; t < nbs; t += kFinThreads) see(t, fsc[t]);
      topk_stage<kFinThreads>(ftk, kmx, kmn_inv);
      __syncthreads();
    }
    // the whole score row in LDS: the shared top-k rule
    const int n_chosen = topk_select<kFinThreads, true>(
        ftk, [&](int j) -> u32 { return order_key(fsc[j]); }, nbs, rule, [&](int pos, int j) { fsel[pos] = j; });
    if (item == 0 && p.idx_out) {
      for (int t = threadIdx.x; t < n_chosen; t += kFinThreads) p.idx_out[(int64_t)bh * p.k_cap + t] = fsel[t];
      if (threadIdx.x == 0) p.n_sel_out[bh] = n_chosen;
    }
    n_units = min(n_units, n_chosen);  // equal: the plan counts with the same rule
  } else if constexpr (SRC == kSrcLists) {
    // selected blocks of every route chunk (exclusive prefix in LDS), then the suffix tiles.
    // With few route chunks every list entry is staged in the same round trip as the
    // counts (entries past a chunk's count are never used).
    if (p.n_rc * kRouteChunk <= kSpecEntries) {
      const int32_t* src = p.rc_lists + (int64_t)bh * p.n_rc * kRouteChunk;
      for (int t = threadIdx.x; t < p.n_rc * kRouteChunk; t += kFinThreads) rc_entries[t] = src[t];
    }
    if (wave == 0) {
      int run = 0;
      for (int c0 = 0; c0 < p.n_rc; c0 += 64) {
        const int c = c0 + lane;
        const int v = c < p.n_rc ? max(p.rc_counts[(int64_t)bh * p.n_rc + c], 0) : 0;
        int inc = v;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
          const int o = __shfl_up(inc, off, 64);
          if (lane >= off) inc += o;
        }
        if (c < p.n_rc) rc_prefix[c] = run + inc - v;
        run += __shfl(inc, 63, 64);
      }
      if (lane == 0) rc_prefix[p.n_rc] = run;
    }
    __syncthreads();
    n_blk_units = rc_prefix[p.n_rc];
    sfx_len = p.sfx_len ? min(max(p.sfx_len[(int64_t)b * p.sfx_len_stride], 0), p.sfx_cap) : 0;
    n_units = n_blk_units + (sfx_len + kDenseTile - 1) / kDenseTile;
  } else if constexpr (SRC == kSrcCondFused) {
    // statistics, hand-off of the row's partials, routing and representatives of the
    // item's own blocks; then its selected blocks and (last item) the suffix
    row_epoch = __builtin_amdgcn_readfirstlane(row_epoch_v);
    n_blk_units = __builtin_amdgcn_readfirstlane(
        cond_fused_prologue<D, G>(p, cond_lds, b, h, item, n_items_row, row_epoch));
    sfx_len = (item == n_items_row - 1 && p.sfx_len)
                  ? min(max(p.sfx_len[(int64_t)b * p.sfx_len_stride], 0), p.sfx_cap)
                  : 0;
    n_units = n_blk_units + (sfx_len + kDenseTile - 1) / kDenseTile;
    slot_lo = 0;
    slot_hi = n_units * nsub_u;
  }
  bool split;
  int u_begin, nu;
  if constexpr (kBalanced) {
    // the plan's raw slots [slot_lo, slot_hi) lie in units [u_begin, u_begin + nu)
    split = n_items_row > 1;
    u_begin = slot_lo / nsub_u;
    nu = slot_hi > slot_lo ? cdiv_pos(slot_hi, nsub_u) - u_begin : 0;
    if (item == 0 && threadIdx.x == 0 && p.part_n) p.part_n[bh] = n_items_row;
  } else {
    // units are spread evenly over the row's items
    const int upi = max(1, (n_units + (int)gridDim.x - 1) / (int)gridDim.x);
    const int n_items = max(1, (n_units + upi - 1) / upi);
    split = gridDim.x > 1 || p.rep_ml != nullptr;  // partials + merge kernel
    if (item >= n_items) {
      // an empty slot: the merge reads every slot of the grid row, (m, l) = (-inf, 0)
      // and accumulators of zero (the merge weighs them by 0, so they must not be
      // left undefined: 0 x NaN is NaN)
      const int64_t slot = (int64_t)bh * p.max_items + item;
      for (int o = threadIdx.x; o < G * D; o += kFinThreads) p.part_acc[slot * (G * D) + o] = 0.f;
      if (threadIdx.x < G) {
        p.part_ml[(slot * G + threadIdx.x) * 2 + 0] = kNegInf;
        p.part_ml[(slot * G + threadIdx.x) * 2 + 1] = 0.f;
      }
      return;
    }
    u_begin = item * upi;
    nu = max(0, min(n_units, u_begin + upi) - u_begin);
    slot_lo = u_begin * nsub_u;
    slot_hi = (u_begin + nu) * nsub_u;
  }

  const ia_paged_kv& kv = p.kv;
  const int page_size = kv.page_size;
  const int32_t* bt_row = kv.block_table ? kv.block_table + (int64_t)b * kv.bt_stride : nullptr;
  // fp8 scales gathered per sequence: the (k, v) pairs of this row's logical pages
  const float* seq_sc =
      (kFp8 && kv.seq_scale) ? kv.seq_scale + (int64_t)b * kv.seq_scale_b_stride + (int64_t)h * kv.seq_scale_h_stride
                             : nullptr;

  // ---- prologue: token ranges of this item's units (the fused source computes them
  // from its LDS selection where they are used), then one page id per subtile
  auto fused_range = [&](int ul, int& lo, int& hi) {
    const int u = u_begin + ul;
    const int j = u >= n_units ? -1 : fsel[u];
    lo = 0;
    hi = 0;
    if (j >= 0 && (int64_t)j * p.unit_tokens < seq_len) {
      lo = j * p.unit_tokens;
      hi = min(lo + p.unit_tokens, seq_len);
    }
  };
  for (int t = threadIdx.x; SRC != kSrcTopkFused && t < nu; t += kFinThreads) {
    const int u = u_begin + t;
    int lo = 0, hi = 0, sfx = 0;
    if constexpr (SRC == kSrcTopk || SRC == kSrcTopkFused) {
      const int j = u >= n_units ? -1 : (SRC == kSrcTopkFused) ? fsel[u] : p.idx[(int64_t)bh * p.k_cap + u];
      if (j >= 0 && (int64_t)j * p.unit_tokens < seq_len) {
        lo = j * p.unit_tokens;
        hi = min(lo + p.unit_tokens, seq_len);
      }
    } else if constexpr (SRC == kSrcDense) {
      lo = u * p.unit_tokens;
      hi = min(lo + p.unit_tokens, seq_len);
    } else if constexpr (SRC == kSrcCondFused) {
      if (u < n_blk_units) {  // entry = block id | valid tokens << 16
        const int e = cond_lds.list[u];
        lo = (e & 0xffff) * p.unit_tokens;
        hi = lo + max(0, min(e >> 16, p.unit_tokens));
      } else {
        lo = (u - n_blk_units) * kDenseTile;
        hi = min(lo + kDenseTile, sfx_len);
        sfx = 1;
      }
    } else {
      if (u < n_blk_units) {
        int lo_c = 0, hi_c = p.n_rc - 1;  // last chunk whose prefix <= u
        while (lo_c < hi_c) {
          const int mid = (lo_c + hi_c + 1) >> 1;
          if (rc_prefix[mid] <= u) lo_c = mid;
          else hi_c = mid - 1;
        }
        // entry = block id | valid tokens << 16 (written by the route kernel)
        const int idx = lo_c * kRouteChunk + (u - rc_prefix[lo_c]);
        const int e = (p.n_rc * kRouteChunk <= kSpecEntries) ? rc_entries[idx]
                                                            : p.rc_lists[(int64_t)bh * p.n_rc * kRouteChunk + idx];
        const int j = e & 0xffff;
        if (e >= 0 && j < p.nb_max) {
          lo = j * p.unit_tokens;
          hi = lo + max(0, min(e >> 16, p.unit_tokens));
        }
      } else {
        lo = (u - n_blk_units) * kDenseTile;
        hi = min(lo + kDenseTile, sfx_len);
        sfx = 1;
      }
    }
    unit_lo[t] = lo;
    unit_hi[t] = sfx ? -hi - 1 : hi;  // suffix units carry a negative end
  }
  if constexpr (SRC != kSrcTopkFused) __syncthreads();  // fused: fsel is synchronised
  // valid subtiles of the item's raw slots in ascending order, compacted (ballots +
  // per-wave counts)
  int n_sub = 0;  // uniform
  const int raw0 = u_begin * nsub_u;
  for (int t0 = 0; t0 < nu * nsub_u; t0 += kFinThreads) {
    const int t = t0 + threadIdx.x;
    int pg = kNoPage, info = 0, sc = 0;
    if (t < nu * nsub_u && raw0 + t >= slot_lo && raw0 + t < slot_hi) {
      const int u = t / nsub_u;
      int lo, hi_raw;
      if constexpr (SRC == kSrcTopkFused) {
        fused_range(u, lo, hi_raw);
      } else {
        lo = unit_lo[u];
        hi_raw = unit_hi[u];
      }
      const bool sfx = hi_raw < 0;
      const int hi = sfx ? -hi_raw - 1 : hi_raw;
      const int tok = lo + 16 * (t - u * nsub_u);
      if (tok < hi) {
        const int nv = min(16, hi - tok);
        if (sfx) {
          pg = kSfxPage;
          info = (tok << 5) | nv;
        } else {
          const int lp = tok / page_size;
          if (!bt_row) {
            pg = lp;
          } else if (lp < kv.bt_cols) {
            pg = bt_row[lp];
          }
          if (pg < 0 || (int64_t)pg >= kv.n_pages) pg = kNoPage;
          info = ((tok - lp * page_size) << 5) | nv;
          sc = 2 * lp;
        }
      }
    }
    const bool ok = pg != kNoPage;
    const unsigned long long bal = __ballot(ok);
    if (lane == 0) wcnt_p[wave] = __popcll(bal);
    __syncthreads();
    int off = n_sub;
    for (int w = 0; w < wave; ++w) off += wcnt_p[w];
    if (ok) {
      const int k = off + __popcll(bal & ((1ull << lane) - 1ull));
      sub_pg[k] = pg;
      sub_info[k] = info;
      if constexpr (kFp8) sub_sc[k] = sc;
    }
#pragma unroll
    for (int w = 0; w < kFinWaves; ++w) n_sub += wcnt_p[w];
    __syncthreads();  // also publishes the last pass's sub_pg / sub_info to the stream
  }
  n_sub = __builtin_amdgcn_readfirstlane(n_sub);

  const char* kbase = reinterpret_cast<const char*>(kv.k) + (int64_t)h * kv.k_head_stride * KV::kBytes;
  const char* vbase = reinterpret_cast<const char*>(kv.v) + (int64_t)h * kv.v_head_stride * KV::kBytes;
  const int lane_off = c16 * DPL * KV::kBytes;

  // ---- subtile iterator: wave w takes the item's valid subtiles w, w + 4, ...
  struct Sub {
    int k;    // index in the compacted list; >= n_sub when exhausted
    int pg;   // page id (kSfxPage: suffix)
    int row;  // first row within the page (suffix: first suffix token)
    int nv;   // valid rows, 1..16
    int sc;   // fp8: 2 x logical page (the pair's offset in the sequence scales)
  };
  // (wave-uniform: kept in scalar registers).  Past the list the iterator names row 0
  // of subtile 0 with no valid rows: the ring's loads stay unconditional (the same
  // count on every path, so the compiler's memory-counter waits stay exact) and
  // touch one row already read.  Requires n_sub >= 1.
  auto seek = [&](int k) -> Sub {
    const int kc = k < n_sub ? k : 0;
    const int info = __builtin_amdgcn_readfirstlane(sub_info[kc]);
    const int pg = __builtin_amdgcn_readfirstlane(sub_pg[kc]);
    const int sc = kFp8 ? __builtin_amdgcn_readfirstlane(sub_sc[kc]) : 0;
    return k < n_sub ? Sub{k, pg, info >> 5, info & 31, sc} : Sub{n_sub, pg, info >> 5, 0, sc};
  };
  auto next = [&](const Sub& c) -> Sub { return seek(c.k + kFinWaves); };

  // K and V row pointers of a subtile and their row strides in bytes
  auto sub_rows = [&](const Sub& sb, const char*& kp, const char*& vp, int64_t& kts, int64_t& vts) {
    if (kListUnits && sb.pg == kSfxPage) {
      kts = p.sfx_k_token_stride * KV::kBytes;
      vts = p.sfx_v_token_stride * KV::kBytes;
      kp = reinterpret_cast<const char*>(p.sfx_k) +
           ((int64_t)b * p.sfx_k_batch_stride + (int64_t)h * p.sfx_k_head_stride) * KV::kBytes + (int64_t)sb.row * kts;
      vp = reinterpret_cast<const char*>(p.sfx_v) +
           ((int64_t)b * p.sfx_v_batch_stride + (int64_t)h * p.sfx_v_head_stride) * KV::kBytes + (int64_t)sb.row * vts;
    } else {
      kts = kv.k_token_stride * KV::kBytes;
      vts = kv.v_token_stride * KV::kBytes;
      kp = kbase + (int64_t)sb.pg * kv.k_page_stride * KV::kBytes + (int64_t)sb.row * kts;
      vp = vbase + (int64_t)sb.pg * kv.v_page_stride * KV::kBytes + (int64_t)sb.row * vts;
    }
  };

  // fp8 pages: the (K, V) scales of the subtile's page, loaded unconditionally (the
  // suffix source, which has none, reads a word of its own row; consume uses 1).
  // With sequence scales both words come from the row's pair for the logical page
  // (a block's pages share one line); else from the per-page arrays (two lines).
  auto page_scales = [&](const Sub& sb, const char* kp, u32 (&xb)[2]) {
    if constexpr (kFp8) {
      const bool paged = sb.pg >= 0;
      const int64_t at = (int64_t)sb.pg * kv.scale_page_stride + h;
      const float* ks = seq_sc ? seq_sc + sb.sc : kv.k_scale + at;
      const float* vs = seq_sc ? seq_sc + sb.sc + 1 : kv.v_scale + at;
      xb[0] = *(paged ? reinterpret_cast<const u32*>(ks) : reinterpret_cast<const u32*>(kp));
      xb[1] = *(paged ? reinterpret_cast<const u32*>(vs) : reinterpret_cast<const u32*>(kp));
    }
  };

  // ---- software pipeline over a ring of NBUF register buffers: while subtile n
  // is consumed, subtiles n+1 .. n+NBUF-1 are in flight.  Everything a subtile
  // reads from memory (rows, and an fp8 page's two scales in xbuf) is loaded by its
  // issue: a load issued by consume would make the wave wait for every load in
  // flight (the vector memory counter drains in order).
  auto stream = [&](auto&& issue, auto&& consume) {
    // The one-launch top-k call's long streams whose consume is the longer one (keys
    // through LDS, fp8 codes widened) keep one subtile in flight per wave: a CU then
    // streams faster than with two (C3 -1.0 to -1.2 us, C5 -1.2 us; same bits).  The
    // condition-rule calls' short streams keep the deeper ring for their start.
    constexpr int NBUF = (SRC == kSrcTopkFused && (KROWS || kFp8)) ? 2 : KV::kRing;
    // the priority feedback below stays in the fp8 and key-row top-k calls (measured
    // faster with it) and in the finalizes of the multi-launch paths; the uniform bf16
    // top-k call (C4 -0.4, C2 -0.15 us) and the one-launch condition calls (-0.1 to
    // -0.3 us) run without it
    constexpr bool kPrioFeedback = !(SRC == kSrcCondFused || (SRC == kSrcTopkFused && !KROWS && kBf16));
    u32 kbuf[NBUF][4][NWD], vbuf[NBUF][4][NWD], xbuf[NBUF][2];
    Sub ring[NBUF];
    if (n_sub == 0) return;
    if constexpr (SRC == kSrcCondFused)  // a wave with no subtile of the item's list
      if (wave >= n_sub) return;
    ring[0] = seek(wave);
    issue(ring[0], kbuf[0], vbuf[0], xbuf[0]);
    // the loads stay in ring order and ahead of the work on older subtiles (no
    // instruction crosses a scheduling barrier): the wait for subtile n then leaves
    // the loads of n+1 .. in flight
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 1; k < NBUF - 1; ++k) {
      ring[k] = next(ring[k - 1]);
      issue(ring[k], kbuf[k], vbuf[k], xbuf[k]);
      __builtin_amdgcn_sched_barrier(0);
    }
    // The wave's subtiles (k = wave, wave + 8, ... < n_sub) in whole rotations of the
    // ring, then the remainder: the loop has one exit, at its latch.  (An exit from
    // the middle of a rotation would reach the loop head through a flag, and the
    // compiler's wait counts there, merged over both edges, drained the loads in
    // flight once per rotation.)
    static_assert(NBUF >= 2 && NBUF <= 4, "ring of 2 to 4 buffers");
    int n_done = 0;
    auto step = [&](auto kc) {
      constexpr int k = decltype(kc)::value;
      constexpr int fk = (k + NBUF - 1) % NBUF;  // free buffer
      constexpr int pk = (k + NBUF - 2) % NBUF;  // most recently issued
      ring[fk] = next(ring[pk]);
      issue(ring[fk], kbuf[fk], vbuf[fk], xbuf[fk]);
      __builtin_amdgcn_sched_barrier(0);
      consume(ring[k], kbuf[k], vbuf[k], xbuf[k]);
      // the two waves of a SIMD (w, w ^ 4) stream equal shares, but issue
      // arbitration favours the older one; the wave ahead yields priority so
      // both finish together (the assignment, hence the result, is unchanged)
      ++n_done;
      if constexpr (kPrioFeedback) {
        wprog[wave] = n_done;
        const int other = wprog[wave ^ (kFinWaves / 2)];
        if (n_done > other) __builtin_amdgcn_s_setprio(0);
        else if (n_done < other) __builtin_amdgcn_s_setprio(2);
        else __builtin_amdgcn_s_setprio(1);
      }
    };
    const int n_my = wave < n_sub ? (n_sub - wave + kFinWaves - 1) / kFinWaves : 0;
    const int n_rot = n_my / NBUF, rem = n_my - n_rot * NBUF;
    for (int rot = 0; rot < n_rot; ++rot) {
      step(std::integral_constant<int, 0>{});
      step(std::integral_constant<int, 1>{});
      if constexpr (NBUF > 2) step(std::integral_constant<int, 2>{});
      if constexpr (NBUF > 3) step(std::integral_constant<int, 3>{});
    }
    if (rem > 0) step(std::integral_constant<int, 0>{});
    if constexpr (NBUF > 2)
      if (rem > 1) step(std::integral_constant<int, 1>{});
    if constexpr (NBUF > 3)
      if (rem > 2) step(std::integral_constant<int, 2>{});
  };

  if constexpr (kMfma) {
    // ================= bf16 / fp8 caches: both products on MFMA, one subtile at a time
    // Q.K: S^T = K Q^T with v_mfma_f32_16x16x32_bf16 per 32-dim k-slice.  A = the 16
    // token rows (lane (r, c16) feeds A row c16 with token rho = c16/4 + 4 (c16%4) of
    // the subtile, 8 dims of k-slice kk at mfma_kslice(kk, r)); B = the G query rows
    // replicated over the 16 columns (column c <-> query row c % G).  Accumulator i
    // of lane (r, c16) then holds the score of token r + 4i for query row c16 % G.
    // P.V: O += P V with v_mfma_f32_16x16x16_bf16 per dim group n < DPL.  A = P: row
    // c16 (query row c16 % G), k = 4r + i <-> token r + 4i, i.e. the lane's own four
    // weights; B = V: column c16 <-> dim c16*DPL + n, k = 4r + i <-> token 4i + r, the
    // lane's own row loads of steps i = 0..3 interleaved by v_perm.  Accumulator i of
    // lane (r, c16) holds O[row 4r + i][dim c16*DPL + n], row 4r + i <-> query row
    // (4r + i) % G.  Scores and weights never leave the lane.
    const int rho = (c16 >> 2) + 4 * (c16 & 3);
    u32 qop[kMfmaK][4];
#pragma unroll
    for (int kk = 0; kk < kMfmaK; ++kk)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        qop[kk][e] = p.q_f32 ? pack_bf16x2(__uint_as_float(qraw[kk][2 * e]), __uint_as_float(qraw[kk][2 * e + 1]))
                             : qraw[kk][e];
    f32x4_t acc[DPL];
#pragma unroll
    for (int n = 0; n < DPL; ++n) acc[n] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    float m_run = kNegInf, l_run = 0.f;

    auto issue = [&](auto kl, const Sub& sb, u32 (&kb)[4][NWD], u32 (&vb)[4][NWD], u32 (&xb)[2]) {
      constexpr bool kKeyLds = decltype(kl)::value;
      // (the one-launch condition call streams a few subtiles per item: past its list
      // a wave issues nothing rather than the placeholder loads)
      if constexpr (SRC == kSrcCondFused)
        if (sb.k >= n_sub) return;
      const char* kp;
      const char* vp;
      int64_t kts, vts;
      sub_rows(sb, kp, vp, kts, vts);
      page_scales(sb, kp, xb);
      if constexpr (kKeyLds) {
        // K as whole rows, like V (step i: token 4i + r, dims c16*DPL ..): each load
        // instruction reads four full 256-byte rows, where the operand layout below
        // would read 64 bytes of sixteen rows (half lines, which cap a CU's stream
        // rate); consume passes them through LDS to the operand layout
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int tl = (4 * i + r < sb.nv) ? 4 * i + r : 0;
          load_words<NWD>(kp + (int64_t)tl * kts + lane_off, kb[i]);
        }
      } else {
        // K: token rho (row 0 past the valid rows), NWD 16-byte pieces at 64*pc + 16*r
        const char* kr = kp + (int64_t)(rho < sb.nv ? rho : 0) * kts + 16 * r;
#pragma unroll
        for (int pc = 0; pc < NWD; ++pc) {
          const u32x4_t a = ld_stream16(kr + 64 * pc);
          const u32 w4[4] = {a[0], a[1], a[2], a[3]};
#pragma unroll
          for (int e = 0; e < 4; ++e) kb[(4 * pc + e) / NWD][(4 * pc + e) % NWD] = w4[e];
        }
      }
      // V: step i, token 4i + r, dims c16*DPL ..
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int tl = (4 * i + r < sb.nv) ? 4 * i + r : 0;
        load_words<NWD>(vp + (int64_t)tl * vts + lane_off, vb[i]);
      }
    };

    auto consume = [&](auto kl, const Sub& sb, const u32 (&kb)[4][NWD], const u32 (&vb)[4][NWD], const u32 (&xb)[2]) {
      constexpr bool kKeyLds = decltype(kl)::value;
      auto kword = [&](int fw) -> u32 { return kb[fw / NWD][fw % NWD]; };
      // bf16 keys through LDS: row t's 16-byte piece c at slot 16 t + (c ^ sw(t)),
      // sw(t) = (t >> 2) | (t & 3) << 2; the lane then reads piece 4 kk + r of token
      // rho, its operand for k-slice kk (the same words the operand-layout loads
      // gave).  sw(4 i + r) = i + 4 r and sw(rho) = c16, so both the writes and the
      // reads of any 8 consecutive lanes touch 8 distinct 16-byte bank groups (with
      // sw(t) = t the reads of lanes c16 and c16 + 2 met in one group)
      u32x4_t kop[kKeyLds ? kMfmaK : 1];
      if constexpr (kKeyLds) {
        u32x4_t* kl = key_lds[wave];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t = 4 * i + r;
          kl[16 * t + (c16 ^ (i + 4 * r))] = u32x4_t{kb[i][0], kb[i][1], kb[i][2], kb[i][3]};
        }
        wave_lds_sync();
#pragma unroll
        for (int kk = 0; kk < kMfmaK; ++kk) kop[kk] = kl[16 * rho + ((4 * kk + r) ^ c16)];
        wave_lds_sync();  // (every lane's reads before the next subtile's writes)
      }
      // ---------------- scores: token r + 4i, query row c16 % G, in accumulator i
      f32x4_t s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < kMfmaK; ++kk) {
        u32 w[4];
        if constexpr (kKeyLds) {
#pragma unroll
          for (int e = 0; e < 4; ++e) w[e] = kop[kk][e];
        } else if constexpr (kFp8) {  // piece kk/2, half kk%2: 8 codes widened to bf16 (exact)
          const u32 c0 = kword(4 * (kk >> 1) + 2 * (kk & 1)), c1 = kword(4 * (kk >> 1) + 2 * (kk & 1) + 1);
          w[0] = fp8x2_to_bf16x2<false>(c0);
          w[1] = fp8x2_to_bf16x2<true>(c0);
          w[2] = fp8x2_to_bf16x2<false>(c1);
          w[3] = fp8x2_to_bf16x2<true>(c1);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) w[e] = kword(4 * kk + e);
        }
        s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(w), as_bf16x8(qop[kk]), s, 0, 0, 0);
      }
      float sc = p.scale_log2;
      float vsc = 1.f;
      if constexpr (kFp8) {
        if (sb.pg >= 0) {
          sc *= __uint_as_float(xb[0]);
          vsc = __uint_as_float(xb[1]);
        }
      }
      // ---------------- online softmax, one update per subtile (max over the 16
      // tokens: in-lane over i, then over the four lane rows with permlane swaps)
      float sv[4];
      float mt = kNegInf;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sv[i] = (r + 4 * i < sb.nv) ? s[i] * sc : kNegInf;
        mt = fmaxf(mt, sv[i]);
      }
      mt = rows_max(mt);
      const float m_new = fmaxf(m_run, mt);
      float pw[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) pw[i] = (sv[i] == kNegInf) ? 0.f : exp2f(sv[i] - m_new);
      if (__any(m_new > m_run)) {
        const float alpha = (m_new == kNegInf) ? 1.f : exp2f(m_run - m_new);
        l_run *= alpha;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float a = mfma_row_alpha<G>(alpha, i, lane);
#pragma unroll
          for (int n = 0; n < DPL; ++n) acc[n][i] *= a;
        }
      }
      m_run = m_new;
      l_run += (pw[0] + pw[1]) + (pw[2] + pw[3]);
      // ---------------- weighted values: bf16 weights (the reference's cast point);
      // an fp8 page's V scale is folded into the weight before the rounding
      const u32 pa0 = kFp8 ? pack_bf16x2(pw[0] * vsc, pw[1] * vsc) : pack_bf16x2(pw[0], pw[1]);
      const u32 pa1 = kFp8 ? pack_bf16x2(pw[2] * vsc, pw[3] * vsc) : pack_bf16x2(pw[2], pw[3]);
      const i16x4_t pa = as_i16x4(pa0, pa1);
      u32 vx[4][NWB];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (kFp8) {
#pragma unroll
          for (int w = 0; w < NWD; ++w) {
            vx[i][2 * w] = fp8x2_to_bf16x2<false>(vb[i][w]);
            vx[i][2 * w + 1] = fp8x2_to_bf16x2<true>(vb[i][w]);
          }
        } else {
#pragma unroll
          for (int w = 0; w < NWB; ++w) vx[i][w] = vb[i][w];
        }
      }
#pragma unroll
      for (int n = 0; n < DPL; ++n) {
        const u32 sel = (n & 1) ? 0x07060302u : 0x05040100u;
        const u32 b0 = __builtin_amdgcn_perm(vx[1][n >> 1], vx[0][n >> 1], sel);
        const u32 b1 = __builtin_amdgcn_perm(vx[3][n >> 1], vx[2][n >> 1], sel);
        acc[n] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pa, as_i16x4(b0, b1), acc[n], 0, 0, 0);
      }
    };

    auto run = [&](auto kl) {
      stream([&](const Sub& sb, u32 (&kb)[4][NWD], u32 (&vb)[4][NWD], u32 (&xb)[2]) { issue(kl, sb, kb, vb, xb); },
             [&](const Sub& sb, const u32 (&kb)[4][NWD], const u32 (&vb)[4][NWD], const u32 (&xb)[2]) {
               consume(kl, sb, kb, vb, xb);
             });
    };
    if constexpr (kKeyLdsAny) run(std::true_type{});
    else run(std::false_type{});

    // ---- fold the wave: l over the four lane rows; the query rows' accumulators sit
    // in lane rows r < max(1, G/4) (row 4r + i < G)
    l_run = rows_sum(l_run);
    if (r == 0 && c16 < G) {
      wm_lds[wave][c16] = m_run;
      wl_lds[wave][c16] = l_run;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 4 * r + i;
      if (row < G) {
#pragma unroll
        for (int n = 0; n < DPL; ++n) wacc_lds[wave][row * D + c16 * DPL + n] = acc[n][i];
      }
    }
  } else {

    constexpr int QW = kDot2 ? DPL / 2 : DPL;  // bf16 pairs or floats
    u32 qw[G][QW];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if (p.q_f32) {
        if constexpr (kDot2) {
#pragma unroll
          for (int e = 0; e < DPL / 2; ++e)
            qw[g][e] = pack_bf16x2(__uint_as_float(qraw[g][2 * e]), __uint_as_float(qraw[g][2 * e + 1]));
        } else {
#pragma unroll
          for (int e = 0; e < DPL; ++e) qw[g][e] = qraw[g][e];
        }
      } else {
        if constexpr (kDot2) {
#pragma unroll
          for (int e = 0; e < DPL / 2; ++e) qw[g][e] = qraw[g][e];
        } else {
#pragma unroll
          for (int e = 0; e < DPL / 2; ++e) {
            qw[g][2 * e] = __float_as_uint(bf16_lo(qraw[g][e]));
            qw[g][2 * e + 1] = __float_as_uint(bf16_hi(qraw[g][e]));
          }
        }
      }
    }

    if constexpr (kQLds) {
      if (wave == 0 && r == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int e = 0; e < DPL; ++e) q_lds[g * D + c16 * DPL + e] = __uint_as_float(qw[g][e]);
      }
      __syncthreads();
    }

    // Per-lane ownership of reduce-scattered scores: token step and query rows.
    const int my_step = c16 >> 2;
    int my_g[KG];
#pragma unroll
    for (int k = 0; k < KG; ++k) {
      if constexpr (G == 8) my_g[k] = 2 * (c16 & 3) + k;
      else if constexpr (G == 4) my_g[k] = c16 & 3;
      else if constexpr (G == 2) my_g[k] = (c16 >> 1) & 1;
      else my_g[k] = 0;
    }
    // For G < 4 several lanes hold copies of one score; only one copy counts in l.
    const bool l_owner = (G >= 4) || ((c16 & (G == 2 ? 1 : 3)) == 0);

    float m_run[KG], l_run[KG];
#pragma unroll
    for (int k = 0; k < KG; ++k) {
      m_run[k] = kNegInf;
      l_run[k] = 0.f;
    }
    float acc[G][DPL];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < DPL; ++e) acc[g][e] = 0.f;

    auto issue = [&](const Sub& sb, u32 (&kb)[4][NWD], u32 (&vb)[4][NWD], u32 (&xb)[2]) {
      // (the one-launch condition call streams a few subtiles per item: past its list
      // a wave issues nothing rather than the placeholder loads)
      if constexpr (SRC == kSrcCondFused)
        if (sb.k >= n_sub) return;
      const char* kp;
      const char* vp;
      int64_t kts, vts;
      sub_rows(sb, kp, vp, kts, vts);
      page_scales(sb, kp, xb);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // rows past the subtile's valid rows re-read its first row (always valid); their weights are zero
        const int tl = (4 * i + r < sb.nv) ? 4 * i + r : 0;
        load_words<NWD>(kp + (int64_t)tl * kts + lane_off, kb[i]);
        load_words<NWD>(vp + (int64_t)tl * vts + lane_off, vb[i]);
      }
    };

    auto consume = [&](const Sub& sb, const u32 (&kb)[4][NWD], const u32 (&vb)[4][NWD], const u32 (&xb)[2]) {
      // fp8 rows widened to bf16 pairs (exact: every e4m3 value is a bf16 value)
      u32 kx[4][NWB], vx[4][NWB];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (kFp8) {
#pragma unroll
          for (int w = 0; w < NWD; ++w) {
            kx[i][2 * w] = fp8x2_to_bf16x2<false>(kb[i][w]);
            kx[i][2 * w + 1] = fp8x2_to_bf16x2<true>(kb[i][w]);
            vx[i][2 * w] = fp8x2_to_bf16x2<false>(vb[i][w]);
            vx[i][2 * w + 1] = fp8x2_to_bf16x2<true>(vb[i][w]);
          }
        } else if constexpr (kBf16) {
#pragma unroll
          for (int w = 0; w < NWB; ++w) {
            kx[i][w] = kb[i][w];
            vx[i][w] = vb[i][w];
          }
        }
      }
      // ---------------- scores of the 16 tokens x G rows
      float part[NV];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (kDot2) {
#pragma unroll
          for (int g = 0; g < G; ++g) {
            float a = 0.f;
#pragma unroll
            for (int w = 0; w < NWB; ++w)
              a = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(qw[g][w]), as_bf16x2(kx[i][w]), a, false);
            part[i * G + g] = a;
          }
        } else if constexpr (!kQLds) {
#pragma unroll
          for (int g = 0; g < G; ++g) {
            float a = 0.f;
#pragma unroll
            for (int e = 0; e < DPL; ++e) a = fmaf(__uint_as_float(qw[g][e]), __uint_as_float(kb[i][e]), a);
            part[i * G + g] = a;
          }
        }
      }
      if constexpr (kQLds) {  // the same dot products, query row g read once per subtile
#pragma unroll
        for (int g = 0; g < G; ++g) {
          float qg[DPL];
#pragma unroll
          for (int e = 0; e < DPL; ++e) qg[e] = q_lds[g * D + c16 * DPL + e];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float a = 0.f;
#pragma unroll
            for (int e = 0; e < DPL; ++e) a = fmaf(qg[e], __uint_as_float(kb[i][e]), a);
            part[i * G + g] = a;
          }
        }
      }
      reduce_scatter16<NV>(part, lane);
      float sc = p.scale_log2;
      float vsc = 1.f;
      if constexpr (kFp8) {
        if (sb.pg >= 0) {
          sc *= __uint_as_float(xb[0]);
          vsc = __uint_as_float(xb[1]);
        }
      }
      const bool valid = 4 * my_step + r < sb.nv;

      // ---------------- online softmax, one update per subtile
      float pw[KG], m_new[KG];
      bool grow = false;
#pragma unroll
      for (int k = 0; k < KG; ++k) {
        const float sv = valid ? part[k] * sc : kNegInf;
        const float mt = fold_g<G, true>(sv);
        m_new[k] = fmaxf(m_run[k], mt);
        grow |= m_new[k] > m_run[k];
        pw[k] = (sv == kNegInf) ? 0.f : exp2f(sv - m_new[k]);
      }
      if (__any(grow)) {
        float alpha[KG];
#pragma unroll
        for (int k = 0; k < KG; ++k) {
          alpha[k] = (m_new[k] == kNegInf) ? 1.f : exp2f(m_run[k] - m_new[k]);
          l_run[k] *= alpha[k];
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float a = alpha_of_row<G>(alpha, g);
#pragma unroll
          for (int e = 0; e < DPL; ++e) acc[g][e] *= a;
        }
      }
#pragma unroll
      for (int k = 0; k < KG; ++k) {
        m_run[k] = m_new[k];
        l_run[k] += l_owner ? pw[k] : 0.f;
      }

      // ---------------- weighted values: weight of (token 4i + r, g) by row broadcast
      float pb[4][G];
      WeightBcast<G, 4 * G>::run(pw, pb);
      if constexpr (kDot2) {
        // bf16 weights (the reference's cast point); an fp8 page's V scale is folded
        // into the weight before the rounding
#pragma unroll
        for (int pr = 0; pr < 2; ++pr) {
          const int i1 = 2 * pr, i2 = 2 * pr + 1;
          u32 pp[G];
#pragma unroll
          for (int g = 0; g < G; ++g) pp[g] = kFp8 ? pack_bf16x2(pb[i1][g] * vsc, pb[i2][g] * vsc)
                                                   : pack_bf16x2(pb[i1][g], pb[i2][g]);
#pragma unroll
          for (int w = 0; w < NWB; ++w) {
            const u32 lo = __builtin_amdgcn_perm(vx[i2][w], vx[i1][w], 0x05040100u);
            const u32 hi = __builtin_amdgcn_perm(vx[i2][w], vx[i1][w], 0x07060302u);
#pragma unroll
            for (int g = 0; g < G; ++g) {
              acc[g][2 * w] = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(pp[g]), as_bf16x2(lo), acc[g][2 * w], false);
              acc[g][2 * w + 1] =
                  __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(pp[g]), as_bf16x2(hi), acc[g][2 * w + 1], false);
            }
          }
        }
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int g = 0; g < G; ++g)
#pragma unroll
            for (int e = 0; e < DPL; ++e) acc[g][e] = fmaf(pb[i][g], __uint_as_float(vb[i][e]), acc[g][e]);
      }
    };

    stream(issue, consume);

    // ---- fold the wave: rows (xor 16, 32) for acc, g-sharing lanes for l
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < DPL; ++e) {
        float v = acc[g][e];
        v += shfl_xor_f(v, 16);
        v += shfl_xor_f(v, 32);
        acc[g][e] = v;
      }
#pragma unroll
    for (int k = 0; k < KG; ++k) l_run[k] = fold_g<G, false>(l_run[k]);
    if (r == 0) {
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < DPL; ++e) wacc_lds[wave][g * D + c16 * DPL + e] = acc[g][e];
    }
    if (r == 0 && c16 < 4) {
#pragma unroll
      for (int k = 0; k < KG; ++k) {
        wm_lds[wave][my_g[k]] = m_run[k];
        wl_lds[wave][my_g[k]] = l_run[k];
      }
    }
  }
  __syncthreads();

  // ---- fold the waves: one (m, l, acc) per item, or the output when the item is alone
  // (a fused call writes its partials through to the coherence point: the row's
  // last item to finish merges them)
  // a fused call's item keeps its partial in its workgroup's slot (the row's items
  // are consecutive workgroups), others at (row, item)
  const int64_t pbase = src_fused(SRC) ? (int64_t)fused_slot : (int64_t)bh * p.max_items + item;
  for (int o = threadIdx.x; o < G * D; o += kFinThreads) {
    const int g = o / D;
    float M = kNegInf;
#pragma unroll
    for (int w = 0; w < kFinWaves; ++w) M = fmaxf(M, wm_lds[w][g]);
    if constexpr (SRC == kSrcCondFused) M = fmaxf(M, cond_lds.rep_m[g]);
    float a = 0.f, l = 0.f;
    if (M != kNegInf) {
#pragma unroll
      for (int w = 0; w < kFinWaves; ++w) {
        const float mw = wm_lds[w][g];
        const float f = (mw == kNegInf) ? 0.f : exp2f(mw - M);
        a += f * wacc_lds[w][o];
        l += f * wl_lds[w][g];
      }
      if constexpr (SRC == kSrcCondFused) {  // the representatives of the item's blocks
        const float mr = cond_lds.rep_m[g];
        if (mr != kNegInf) {
          float ra = 0.f;
#pragma unroll
          for (int w = 0; w < kFinWaves; ++w) ra += cond_lds.rep_acc[w][o];
          const float f = exp2f(mr - M);
          a += f * ra;
          l += f * cond_lds.rep_l[g];
        }
      }
    }
    if (!split) {
      store_decode_out<G, D>(p, b, h, o, a / fmaxf(l, 1e-30f));
    } else if (src_fused(SRC) && n_items_row <= kMergeGroup) {
      // tagged words: readable as soon as they land, no acknowledgement to wait for
      const unsigned long long tg = (unsigned long long)partial_tag(bh, row_epoch) << 32;
      unsigned long long* slot = p.tpart + pbase * (G * D + 2 * G);
      st_agent_u64(slot + o, tg | __float_as_uint(a));
      if (o % D == 0) {
        st_agent_u64(slot + G * D + 2 * g, tg | __float_as_uint(M));
        st_agent_u64(slot + G * D + 2 * g + 1, tg | __float_as_uint(l));
      }
    } else if (src_fused(SRC)) {
      st_agent(p.part_acc + pbase * (G * D) + o, a);
      if (o % D == 0) {
        st_agent(p.part_ml + (pbase * G + g) * 2 + 0, M);
        st_agent(p.part_ml + (pbase * G + g) * 2 + 1, l);
      }
    } else {
      p.part_acc[pbase * (G * D) + o] = a;
      if (o % D == 0) {
        p.part_ml[(pbase * G + g) * 2 + 0] = M;
        p.part_ml[(pbase * G + g) * 2 + 1] = l;
      }
    }
  }
  if constexpr (src_fused(SRC)) {
    if (split) {
      // the row's items count their finished partials; the one that brings the count
      // to n merges and resets the count for the next call.  Untagged partials (rows
      // of more than kMergeGroup items) are at the coherence point before the count
      // moves; tagged ones are read again until their tag arrives.  No item waits
      // for another's work, so nothing depends on which workgroups run together.
      if (n_items_row > kMergeGroup) wait_memory();
      __syncthreads();
      if (threadIdx.x == 0) {
        u32* ctr = p.rowctr + (int64_t)bh * kFlagStride;
        const u32 before = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const bool last = before == (u32)(n_items_row - 1);
        if (last) {  // every item has read the epoch: advance it for the next call
          st_agent_u32(ctr, 0u);
          st_agent_u32(ctr + 1, row_epoch + 1u);
        }
        merge_todo[0] = last ? 1u : 0u;
      }
      __syncthreads();
      if (merge_todo[0]) {
        if (n_items_row <= kMergeGroup)
          fused_merge_tagged<D, G>(p, b, h, (int64_t)fused_slot - item, n_items_row, partial_tag(bh, row_epoch));
        else if (n_items_row <= 2 * kMergeGroup)
          fused_merge<D, G, 2>(p, b, h, (int64_t)fused_slot - item, n_items_row);
        else if (n_items_row <= 4 * kMergeGroup)
          fused_merge<D, G, 4>(p, b, h, (int64_t)fused_slot - item, n_items_row);
        else
          fused_merge<D, G, kMergeGroups>(p, b, h, (int64_t)fused_slot - item, n_items_row);
      }
    }
  }
}

// Split-K merge, one workgroup per (sequence, kv head): out = sum_s f_s acc_s / sum_s f_s l_s
// with f_s = 2^(m_s - M) over the finalize items' partials and the route chunks'
// representative partials (CBT/legacy.py:765-794).  Up to kWaves x kMergeFastSlots
// slots are read in one round trip (one wave up to kMergeFastSlots, else every wave
// its eight, folded in LDS).  Beyond that, two
// dependent round trips: every slot's (m, l) is staged in LDS at once, then the
// accumulators of the non-empty slots are read with many loads in flight.
// n_slots: the items per (b, h) of a fixed-count launch; for a balanced launch
// (p.part_n set) each row's count is read from p.part_n and n_slots is the number
// of slots loaded before it arrives (at most kWaves x kMergeFastSlots and max_items);
// rows of one item are skipped (the finalize wrote their output).
template <int D, int G>
__global__ __launch_bounds__(kThreads) void ia_condition_block_splitk_merge(DecodeParams p, int n_slots) {
  __shared__ float m_lds[kMaxMergeSlots][G];
  __shared__ float l_lds[kMaxMergeSlots][G];
  __shared__ int list[kMaxMergeSlots];
  __shared__ float lsum[G];
  __shared__ int n_list;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int bh = blockIdx.x;
  const int b = bh / p.n_kv_heads;
  const int h = bh - b * p.n_kv_heads;
  const int n_rep = p.rep_ml ? p.n_rc : 0;
  // counted (balanced) launches: the row's item count comes from the finalize, and
  // wave 0 loads the first n_slots slots while it is in flight
  const bool counted = p.part_n != nullptr;
  constexpr int PER = G * D / 64;  // outputs per lane of one wave (all in query row o0 / D)
  const int o0 = lane * PER;
  const int g0 = o0 / D;
  // wave w holds slots 8 w .. 8 w + 7: up to kWaves * 8 slots in one round trip
  float mv[kMergeFastSlots], lv[kMergeFastSlots], av[kMergeFastSlots][PER];
  auto load_slot = [&](int j, const float* ml, const float* src) {
    mv[j] = ml[g0 * 2];
    lv[j] = ml[g0 * 2 + 1];
    if constexpr (PER % 4 == 0) {
#pragma unroll
      for (int e = 0; e < PER; e += 4) {
        const float4 w4 = *reinterpret_cast<const float4*>(src + o0 + e);
        av[j][e] = w4.x; av[j][e + 1] = w4.y; av[j][e + 2] = w4.z; av[j][e + 3] = w4.w;
      }
    } else {
#pragma unroll
      for (int e = 0; e < PER; ++e) av[j][e] = src[o0 + e];
    }
  };
  auto clear_slot = [&](int j) {
    mv[j] = kNegInf;
    lv[j] = 0.f;
#pragma unroll
    for (int e = 0; e < PER; ++e) av[j][e] = 0.f;
  };
#pragma unroll
  for (int j = 0; j < kMergeFastSlots; ++j) clear_slot(j);
  int n_fin = n_slots;
  if (counted) {
    // groups of kMergeGroup slots: wave w takes groups w and w + kWaves; the first
    // n_slots slots are loaded before the row's item count arrives
    n_fin = min(max(p.part_n[bh], 0), p.max_items);
    auto slot_ptrs = [&](int s, const float*& ml, const float*& acc) {
      const int64_t slot = (int64_t)bh * p.max_items + s;
      ml = p.part_ml + slot * G * 2;
      acc = p.part_acc + slot * (G * D);
    };
#pragma unroll
    for (int j = 0; j < kMergeFastSlots; ++j) {
      const int s = kMergeFastSlots * wave + j;
      if (s < n_slots) {
        const float *ml, *acc;
        slot_ptrs(s, ml, acc);
        load_slot(j, ml, acc);
      }
    }
    if (n_fin <= 1) return;  // a row of one item: the finalize wrote its output
    const int ng = (n_fin + kMergeGroup - 1) / kMergeGroup;
    if (ng == 1 && wave != 0) return;
    __shared__ float gm_lds[kMergeGroups][64];
    __shared__ float gl_lds[kMergeGroups][64];
    __shared__ float ga_lds[kMergeGroups][G * D];
    float gM = kNegInf, gL = 0.f, ga[PER];
    for (int g = wave; g < ng; g += kWaves) {
#pragma unroll
      for (int j = 0; j < kMergeGroup; ++j) {
        const int s = kMergeGroup * g + j;
        if (s >= n_fin) {
          clear_slot(j);
        } else if (g != wave || s >= n_slots) {
          const float *ml, *acc;
          slot_ptrs(s, ml, acc);
          load_slot(j, ml, acc);
        }
      }
      merge_group<PER>(mv, lv, av, gM, gL, ga);
      if (ng > 1) {
        gm_lds[g][lane] = gM;
        gl_lds[g][lane] = gL;
#pragma unroll
        for (int e = 0; e < PER; ++e) ga_lds[g][o0 + e] = ga[e];
      }
    }
    if (ng > 1) {
      __syncthreads();
      if (wave != 0) return;
    }
    merge_combine<PER>(
        ng, [&](int g) { return ng > 1 ? gm_lds[g][lane] : gM; }, [&](int g) { return ng > 1 ? gl_lds[g][lane] : gL; },
        [&](int g, int e) { return ng > 1 ? ga_lds[g][o0 + e] : ga[e]; },
        [&](int e, float v) { store_decode_out<G, D>(p, b, h, o0 + e, v); });
    return;
  }
  const int n_all = min(n_fin + n_rep, kMaxMergeSlots);
  auto ml_of = [&](int s) -> const float* {
    return s < n_fin ? p.part_ml + ((int64_t)bh * p.max_items + s) * G * 2
                     : p.rep_ml + ((int64_t)bh * p.n_rc + (s - n_fin)) * G * 2;
  };
  auto acc_of = [&](int s) -> const float* {
    return s < n_fin ? p.part_acc + ((int64_t)bh * p.max_items + s) * (G * D)
                     : p.rep_acc + ((int64_t)bh * p.n_rc + (s - n_fin)) * (G * D);
  };
  if (n_all <= kWaves * kMergeFastSlots) {
    // few slots: every slot's (m, l) and accumulators in one round trip (wave 0
    // alone up to 8 slots, else four waves folded in LDS)
    const bool solo = n_all <= kMergeFastSlots;
    if (solo && wave != 0) return;
    const int s_have = counted ? n_slots : 0;
#pragma unroll
    for (int j = 0; j < kMergeFastSlots; ++j) {
      const int s = kMergeFastSlots * wave + j;
      if (s >= s_have && s < n_all) load_slot(j, ml_of(s), acc_of(s));
      if (s >= n_all) clear_slot(j);  // speculative loads past the row's items
    }
    float M = kNegInf;
#pragma unroll
    for (int j = 0; j < kMergeFastSlots; ++j) M = fmaxf(M, mv[j]);
    float L = 0.f, a[PER];
#pragma unroll
    for (int e = 0; e < PER; ++e) a[e] = 0.f;
    if (M != kNegInf) {
#pragma unroll
      for (int j = 0; j < kMergeFastSlots; ++j) {
        const float f = (mv[j] == kNegInf) ? 0.f : exp2f(mv[j] - M);
        L += f * lv[j];
#pragma unroll
        for (int e = 0; e < PER; ++e) a[e] = fmaf(f, av[j][e], a[e]);
      }
    }
    if (!solo) {
      __shared__ float wm_f[kWaves][64];
      __shared__ float wl_f[kWaves][64];
      __shared__ float wa_f[kWaves][G * D];
      wm_f[wave][lane] = M;
      wl_f[wave][lane] = L;
#pragma unroll
      for (int e = 0; e < PER; ++e) wa_f[wave][o0 + e] = a[e];
      __syncthreads();
      if (wave != 0) return;
      M = kNegInf;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) M = fmaxf(M, wm_f[w][lane]);
      L = 0.f;
#pragma unroll
      for (int e = 0; e < PER; ++e) a[e] = 0.f;
      if (M != kNegInf) {
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
          const float mw = wm_f[w][lane];
          const float f = (mw == kNegInf) ? 0.f : exp2f(mw - M);
          L += f * wl_f[w][lane];
#pragma unroll
          for (int e = 0; e < PER; ++e) a[e] = fmaf(f, wa_f[w][o0 + e], a[e]);
        }
      }
    }
#pragma unroll
    for (int e = 0; e < PER; ++e) store_decode_out<G, D>(p, b, h, o0 + e, a[e] / fmaxf(L, 1e-30f));
    return;
  }
  for (int t = threadIdx.x; t < n_all * G; t += kThreads) {
    const int s = t / G, g = t - s * G;
    const float* ml = ml_of(s) + g * 2;
    m_lds[s][g] = ml[0];
    l_lds[s][g] = ml[1];
  }
  __syncthreads();
  // per row: M = max_s m_s, then f_s (kept in m_lds) and the denominator
  for (int g = wave; g < G; g += kWaves) {
    float M = kNegInf;
    for (int s = lane; s < n_all; s += 64) M = fmaxf(M, m_lds[s][g]);
    M = wave_max(M);
    float L = 0.f;
    for (int s = lane; s < n_all; s += 64) {
      const float m = m_lds[s][g];
      const float f = (m == kNegInf) ? 0.f : exp2f(m - M);
      m_lds[s][g] = f;
      L += f * l_lds[s][g];
    }
    L = wave_sum(L);
    if (lane == 0) lsum[g] = L;
  }
  __syncthreads();
  if (wave == 0) {  // slots with any weight, ascending
    int base = 0;
    for (int s0 = 0; s0 < n_all; s0 += 64) {
      const int s = s0 + lane;
      bool any = false;
      if (s < n_all) {
#pragma unroll
        for (int g = 0; g < G; ++g) any |= m_lds[s][g] != 0.f;
      }
      const unsigned long long bal = __ballot(any);
      if (any) list[base + __popcll(bal & ((1ull << lane) - 1ull))] = s;
      base += __popcll(bal);
    }
    if (lane == 0) n_list = base;
  }
  __syncthreads();
  // accumulators: wave w folds list entries w, w + 4, ...; lane owns PER consecutive
  // outputs of the slot's [G, D] block (vector loads), kU slots in flight
  constexpr int kU = 4;
  const int nl = n_list;
  float a[PER];
#pragma unroll
  for (int e = 0; e < PER; ++e) a[e] = 0.f;
  for (int i0 = wave; i0 < nl; i0 += kWaves * kU) {
    float v[kU][PER];
    float f[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int i = i0 + u * kWaves;
      const bool in = i < nl;
      const int s = in ? list[i] : 0;
      f[u] = in ? m_lds[s][g0] : 0.f;
      const float* src = acc_of(s) + o0;
      if (in) {
        if constexpr (PER % 4 == 0) {
#pragma unroll
          for (int e = 0; e < PER; e += 4) {
            const float4 w4 = *reinterpret_cast<const float4*>(src + e);
            v[u][e] = w4.x; v[u][e + 1] = w4.y; v[u][e + 2] = w4.z; v[u][e + 3] = w4.w;
          }
        } else {
#pragma unroll
          for (int e = 0; e < PER; ++e) v[u][e] = src[e];
        }
      } else {
#pragma unroll
        for (int e = 0; e < PER; ++e) v[u][e] = 0.f;
      }
    }
#pragma unroll
    for (int u = 0; u < kU; ++u)
#pragma unroll
      for (int e = 0; e < PER; ++e) a[e] = fmaf(f[u], v[u][e], a[e]);
  }
  __shared__ float wsum[kWaves][G * D];
#pragma unroll
  for (int e = 0; e < PER; ++e) wsum[wave][o0 + e] = a[e];
  __syncthreads();
  for (int o = threadIdx.x; o < G * D; o += kThreads) {
    float t = wsum[0][o];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) t += wsum[w][o];
    store_decode_out<G, D>(p, b, h, o, t / fmaxf(lsum[o / D], 1e-30f));
  }
}

// Per-instance launcher; returns IA_OK or an error code.
template <int D, int G, typename KV, int SRC, bool KROWS = false>
int launch_paged_finalize(const DecodeParams& p, dim3 grid, hipStream_t st) {
  hipLaunchKernelGGL((ia_condition_block_paged_finalize<D, G, KV, SRC, KROWS>), grid, dim3(kFinThreads), 0, st, p);
  int rc = check_launch("paged decode");
  if constexpr (src_fused(SRC)) {
    return rc;  // the row's last item merges inside the launch
  } else if constexpr (src_balanced(SRC)) {
    // a flat grid of at most n_rows workgroups gives every row a single item
    if (rc || (int)grid.x <= p.n_rows) return rc;
    const int even = ((int)grid.x + p.n_rows - 1) / p.n_rows;
    const int spec = std::min(kWaves * kMergeFastSlots, std::min(p.max_items, even));
    hipLaunchKernelGGL((ia_condition_block_splitk_merge<D, G>), dim3(p.n_rows), dim3(kThreads), 0, st, p, spec);
  } else {
    if (rc || (grid.x == 1 && !p.rep_ml)) return rc;
    hipLaunchKernelGGL((ia_condition_block_splitk_merge<D, G>), dim3(grid.y * grid.z), dim3(kThreads), 0, st, p,
                       (int)grid.x);
  }
  return check_launch("split-k merge");
}

// Resident workgroups of one instance on the current device, cached per device
// (relaxed atomics: concurrent first calls compute the same value).  0 on a query
// failure (the callers then assume 1024).
constexpr int kMaxCachedDevices = 64;
template <int D, int G, typename KV, int SRC, bool KROWS = false>
int resident_wgs() {
  static std::atomic<int> cached[kMaxCachedDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
  int n = dev < kMaxCachedDevices ? cached[dev].load(std::memory_order_relaxed) : 0;
  if (n == 0) {
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &per_cu, reinterpret_cast<const void*>(&ia_condition_block_paged_finalize<D, G, KV, SRC, KROWS>), kFinThreads,
            0) != hipSuccess)
      return 0;
    n = std::max(1, cus * per_cu);
    if (dev < kMaxCachedDevices) cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// Host helpers shared by the decode entry points (paged_decode.hip).
int units_cap_items(int64_t units);
size_t decode_ws_size(int batch, int hkv, int group, int d, int max_items);
void set_decode_ws(DecodeParams& p, char* ws, int64_t bh, int max_items, int group, int d);
int balanced_grid(const DecodeParams& p, int kv_dtype, int d, int g, int src, int64_t n_rows, int64_t units_max,
                  int nsub_u, int cap_items, hipStream_t st, int* grid_out, int* budget_out);
int check_kv(const ia_paged_kv* kv, int d);
int check_shape(const ia_decode_shape* s);
int dispatch_decode(const DecodeParams& p, int kv_dtype, int d, int g, int src, dim3 grid, hipStream_t st,
                    int* resident);
int decode_items(const DecodeParams& p, int kv_dtype, int d, int g, int src, int64_t bh, int64_t units_max,
                 int nsub_u, int cap_items, hipStream_t st, int* items_out);

// Fused top-k decode workspace: one 256-byte line per row first (the row's
// finished-partial count, zero between calls, and its epoch; max(rows, row_lines)
// lines), then the published score entries [row, nb_max] (8 bytes each), then the
// split-K partials, one slot per workgroup ((m, l) [slot, G, 2], acc [slot, G, D])
// and the items per row.  Zero-filled once; the row lines then carry the counts and
// epochs from call to call, and every published word carries its row's tag
// (partial_tag).  A buffer whose row lines stay at one place for every shape (a
// fixed row_lines at least every call's rows) may therefore serve calls of any shape
// in turn without another clear; with row_lines = 0 the later parts start where the
// shape's own rows end, so the buffer belongs to one shape.
struct FusedWs {
  size_t sbuf, part_ml, part_acc, part_n, tpart, total;
  int64_t slots;
};
FusedWs fused_ws_layout(int batch, int hkv, int g, int d, int nb_max, int k_cap, int block_size,
                        int64_t row_lines = 0);
int run_topk_decode(const ia_decode_shape* shape, const void* q, const ia_paged_kv* kv, const int32_t* seq_lens,
                    const ia_block_keys* keys, int32_t block_size, int32_t nb_max, int32_t k,
                    const int32_t* k_per_seq, int32_t forced_first, int32_t forced_last, int32_t forced_in_k,
                    int32_t k_cap, float scale, void* out, int32_t out_dtype, int32_t* idx_out, int32_t* n_sel_out,
                    void* workspace, size_t workspace_bytes, void* stream, int64_t row_lines = 0);

// Block-keys descriptor check and score scale (select_topk.hip); the hand-off wait
// bound of the fused top-k call (paged_decode.hip).
int check_block_keys(const ia_block_keys* keys, int G, int D, float* score_scale);
int64_t wait_limit_ticks();
int64_t set_wait_limit_ticks(int64_t ticks);

// Dispatch by kv dtype for one (D, G): defined in paged_decode_{bf16,f32,fp8}.hip.
int dispatch_bf16(const DecodeParams& p, int d, int g, int src, dim3 grid, hipStream_t st, int* resident);
int dispatch_f32(const DecodeParams& p, int d, int g, int src, dim3 grid, hipStream_t st, int* resident);
int dispatch_fp8(const DecodeParams& p, int d, int g, int src, dim3 grid, hipStream_t st, int* resident);
// Their translation units' wait-fallback counters (tu_wait_fallbacks).
uint64_t wait_fallbacks_bf16(bool reset);
uint64_t wait_fallbacks_f32(bool reset);
uint64_t wait_fallbacks_fp8(bool reset);

}  // namespace ia

