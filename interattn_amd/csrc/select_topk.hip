// Top-k block selection for gfx950: block scorer and per-(sequence, kv head)
// radix select fused in one launch, one 1024-thread workgroup per (sequence,
// kv head).  A whole score row stays inside one workgroup, so the launch needs
// no cross-workgroup synchronisation (an agent-scope fence writes back the
// XCD's L2 and costs far more than the work here).
//
//   scoring: score_j = (mean_g q_g) . k_bar_j / sqrt(D); one k_bar row per 16
//   lanes (4 rows per wave-wide load), 16 (bf16) or 8 (fp32) rows per lane in
//   flight, DPP row sums;
//   scores land in LDS (and in global memory when requested or too many).
//   selection:
//     * forced blocks: the first forced_first and last forced_last valid blocks;
//     * the k_eff largest remaining scores by an MSB-first 8-bit radix select
//       on order-preserving 32-bit keys (histograms in LDS), stopping as soon as
//       the threshold bin is taken whole; ties at the threshold go to the
//       lowest block indices;
//     * an ordered compaction (wave ballots + LDS offsets) writes the chosen
//       block ids in ascending order.
//   The rule is the group-mean score + torch.topk of CBG/methods/quest.py:91-103
//   with the mean key (k_bar) as the block representative.
#include "plan.hpp"
#include "topk_select.hpp"

namespace ia {

namespace {

constexpr int kSelThreads = 1024;
constexpr int kSelWaves = kSelThreads / 64;
constexpr int kMaxLdsScores = 8192;

struct SelectParams {
  const void* q;
  int64_t q_batch_stride, q_row_stride;
  const void* k_bar;  // mean-key score: k_bar; Quest score: k_max
  const void* k_min;  // Quest score
  int64_t kb_batch_stride, kb_head_stride;
  int32_t quest;
  const int32_t* seq_lens;
  int32_t block_size, nb_max, k, forced_first, forced_last, forced_in_k;
  const int32_t* k_per_seq;  // optional [batch]
  int32_t* idx;
  int32_t k_cap;
  int32_t* n_sel;
  float* scores;  // [batch*Hkv, nb_max] or null
  int32_t n_kv_heads;
  float score_scale;   // 1 / (G * sqrt(D)) (mean key) or 1 / G (Quest)
  int32_t lds_scores;  // score rows of up to this many blocks stay in LDS
};

template <int D, int G, bool QF32, bool KBF16, bool QUEST>
__global__ __launch_bounds__(kSelThreads) void ia_condition_block_select_topk(SelectParams p) {
  constexpr int DPL = D / 16;
  extern __shared__ float sc_lds[];  // p.lds_scores floats
  __shared__ TopkLds<kSelThreads> sel_lds;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c16 = lane & 15;
  const int r = lane >> 4;
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const int bh = b * p.n_kv_heads + h;
  const int seq_len = max(p.seq_lens[b], 0);
  const int nb = min((seq_len + p.block_size - 1) / p.block_size, p.nb_max);
  const bool in_lds = nb <= p.lds_scores;
  float* sc_row = p.scores ? p.scores + (int64_t)bh * p.nb_max : nullptr;

  // ---- q rows (loaded first, summed after the first k_bar loads are in flight)
  float qv[G][DPL];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int64_t row = (int64_t)b * p.q_batch_stride + (int64_t)(h * G + g) * p.q_row_stride + c16 * DPL;
#pragma unroll
    for (int e = 0; e < DPL; ++e) {
      if constexpr (QF32) qv[g][e] = reinterpret_cast<const float*>(p.q)[row + e];
      else qv[g][e] = __uint_as_float((u32)reinterpret_cast<const unsigned short*>(p.q)[row + e] << 16);
    }
  }
  float qm[DPL], qn[DPL];  // mean key: qm = sum_g q_g; Quest: qm = sum_g q_g+, qn = sum_g q_g-
  bool have_qm = false;

  // ---- scores: in step t, wave w handles row base + 64 t + 4 w + r; NS steps in
  // flight, their key words held in one vector value (registers, never memory); the
  // Quest score reads two key rows per block
  constexpr int EB = KBF16 ? 2 : 4;
  const char* kb = reinterpret_cast<const char*>(p.k_bar) +
                   ((int64_t)b * p.kb_batch_stride + (int64_t)h * p.kb_head_stride) * EB;
  const char* kn = reinterpret_cast<const char*>(QUEST ? p.k_min : p.k_bar) +
                   ((int64_t)b * p.kb_batch_stride + (int64_t)h * p.kb_head_stride) * EB;
  constexpr int NWR = DPL * EB / 4;                // words per lane per row
  constexpr int NW = D >= 128 && G * DPL < 64 ? 64 : 32;  // key words per lane in flight
  constexpr int NS = NW / NWR / (QUEST ? 2 : 1);   // steps in flight
  constexpr int kRowsPerStep = 4 * kSelWaves;
  typedef u32 __attribute__((ext_vector_type(NW))) words_t;
  for (int base = 0; base < nb; base += NS * kRowsPerStep) {
    words_t w;
    // loads without a per-lane condition (rows past nb re-read row nb - 1); steps
    // wholly past nb are skipped
#pragma unroll
    for (int t = 0; t < NS; ++t) {
      if (base + kRowsPerStep * t >= nb) break;  // uniform
      const int j = min(base + kRowsPerStep * t + 4 * wave + r, nb - 1);
#pragma unroll
      for (int q = 0; q < (QUEST ? 2 : 1); ++q) {
        const char* rowp = (q ? kn : kb) + ((int64_t)j * D + c16 * DPL) * EB;
        const int o = (QUEST ? 2 * t + q : t) * NWR;
        if constexpr (NWR >= 4) {
#pragma unroll
          for (int v4 = 0; v4 < NWR; v4 += 4) {
            const u32x4_t x = ld_stream16(rowp + 4 * v4);
            w[o + v4] = x[0];
            w[o + v4 + 1] = x[1];
            w[o + v4 + 2] = x[2];
            w[o + v4 + 3] = x[3];
          }
        } else {
          const u32x2_t x = ld_stream8(rowp);
          w[o] = x[0];
          w[o + 1] = x[1];
        }
      }
    }
    if (!have_qm) {
#pragma unroll
      for (int e = 0; e < DPL; ++e) {
        float a = 0.f, c = 0.f;
#pragma unroll
        for (int g = 0; g < G; ++g) {
          if constexpr (QUEST) {
            a += fmaxf(qv[g][e], 0.f);
            c += fminf(qv[g][e], 0.f);
          } else {
            a += qv[g][e];
          }
        }
        qm[e] = a;
        qn[e] = c;
      }
      have_qm = true;
    }
    if constexpr (NS >= 4 && NS <= 32) {
      // the NS steps' lane shares summed by one reduce-scatter over the 16-lane row
      // (the same pairs in the same tree as block_score's row sum, so the same bits)
      float v[NS];
#pragma unroll
      for (int t = 0; t < NS; ++t) {
        v[t] = 0.f;
        if (base + kRowsPerStep * t >= nb) continue;  // uniform
        u32 w1[NWR], w2[NWR];
#pragma unroll
        for (int e = 0; e < NWR; ++e) {
          w1[e] = w[(QUEST ? 2 * t : t) * NWR + e];
          w2[e] = QUEST ? w[(2 * t + 1) * NWR + e] : 0u;
        }
        v[t] = QUEST ? block_dot_quest<DPL, KBF16>(w1, w2, qm, qn) : block_dot<DPL, KBF16>(w1, qm);
      }
      reduce_scatter16<NS>(v, lane);
      constexpr int kHeld = NS >= 16 ? NS / 16 : 1;    // steps a lane holds
      constexpr int kCopies = NS >= 16 ? 1 : 16 / NS;  // lanes holding each step
#pragma unroll
      for (int k = 0; k < kHeld; ++k) {
        const int t = NS == 32 ? 2 * c16 + k : c16 / kCopies;
        const int j = base + kRowsPerStep * t + 4 * wave + r;
        if (c16 % kCopies == 0 && base + kRowsPerStep * t < nb && j < nb) {
          const float a = v[k] * p.score_scale;
          if (in_lds) sc_lds[j] = a;
          if (sc_row) sc_row[j] = a;
        }
      }
    } else {
#pragma unroll
      for (int t = 0; t < NS; ++t) {
        if (base + kRowsPerStep * t >= nb) break;  // uniform
        u32 w1[NWR], w2[NWR];
#pragma unroll
        for (int e = 0; e < NWR; ++e) {
          w1[e] = w[(QUEST ? 2 * t : t) * NWR + e];
          w2[e] = QUEST ? w[(2 * t + 1) * NWR + e] : 0u;
        }
        const float a = QUEST ? block_score_quest<DPL, KBF16>(w1, w2, qm, qn, p.score_scale)
                              : block_score<DPL, KBF16>(w1, qm, p.score_scale);
        const int j = base + kRowsPerStep * t + 4 * wave + r;
        if (c16 == 0 && j < nb) {
          if (in_lds) sc_lds[j] = a;
          if (sc_row) sc_row[j] = a;
        }
      }
    }
  }
  // blocks past this sequence's end read as -inf
  if (sc_row) {
    for (int j = nb + threadIdx.x; j < p.nb_max; j += kSelThreads) sc_row[j] = kNegInf;
  }
  __syncthreads();
  auto key_at = [&](int j) -> u32 { return order_key(in_lds ? sc_lds[j] : sc_row[j]); };

  // ---- selection (forced blocks, radix-select threshold, ordered compaction)
  const int k_b = p.k_per_seq ? max(p.k_per_seq[b], 0) : p.k;
  const TopkRule rule{p.forced_first, p.forced_last, k_b, p.forced_in_k, p.k_cap};
  int32_t* out_idx = p.idx + (int64_t)bh * p.k_cap;
  const int n = topk_select<kSelThreads>(sel_lds, key_at, nb, rule, [&](int pos, int j) { out_idx[pos] = j; });
  if (threadIdx.x == 0) p.n_sel[bh] = n;
}

size_t select_ws_size(int batch, int hkv, int nb_max) {
  const size_t bh = (size_t)batch * hkv;
  return bh * (size_t)std::max(nb_max, 1) * 4;
}

template <int D, int G>
int launch_select(const SelectParams& p, bool qf32, bool kbf16, dim3 grid, hipStream_t st) {
  const size_t lds = (size_t)p.lds_scores * sizeof(float);
  auto go = [&](auto kern) { hipLaunchKernelGGL(kern, grid, dim3(kSelThreads), lds, st, p); };
  if (p.quest) {
    if (qf32) kbf16 ? go(ia_condition_block_select_topk<D, G, true, true, true>)
                    : go(ia_condition_block_select_topk<D, G, true, false, true>);
    else kbf16 ? go(ia_condition_block_select_topk<D, G, false, true, true>)
               : go(ia_condition_block_select_topk<D, G, false, false, true>);
  } else {
    if (qf32) kbf16 ? go(ia_condition_block_select_topk<D, G, true, true, false>)
                    : go(ia_condition_block_select_topk<D, G, true, false, false>);
    else kbf16 ? go(ia_condition_block_select_topk<D, G, false, true, false>)
               : go(ia_condition_block_select_topk<D, G, false, false, false>);
  }
  return check_launch("select_topk");
}

}  // namespace

// Checks a block-keys descriptor and returns the score scale: 1 / (G sqrt(D)) for the
// mean-key score, 1 / G for the Quest score (CBG/methods/quest.py:97-101 takes the
// group mean and no 1/sqrt(D)).
int check_block_keys(const ia_block_keys* keys, int G, int D, float* score_scale) {
  if (!keys) return fail(IA_ERR_INVALID, "block keys are null");
  if (keys->dtype != IA_F32 && keys->dtype != IA_BF16) return fail(IA_ERR_INVALID, "key dtype must be IA_F32 or IA_BF16");
  const int eb = keys->dtype == IA_BF16 ? 2 : 4;
  if ((keys->batch_stride * eb) % 16 || (keys->head_stride * eb) % 16 || keys->batch_stride < 0 || keys->head_stride < 0)
    return fail(IA_ERR_INVALID, "key rows must be 16-byte aligned");
  const void* ptrs[2] = {nullptr, nullptr};
  if (keys->score == IA_SCORE_MEAN_KEY) {
    ptrs[0] = keys->k_bar;
    ptrs[1] = keys->k_bar;
    *score_scale = 1.0f / ((float)G * std::sqrt((float)D));
  } else if (keys->score == IA_SCORE_QUEST) {
    ptrs[0] = keys->k_max;
    ptrs[1] = keys->k_min;
    *score_scale = 1.0f / (float)G;
  } else {
    return fail(IA_ERR_INVALID, "score must be IA_SCORE_MEAN_KEY or IA_SCORE_QUEST");
  }
  for (const void* ptr : ptrs) {
    if (!ptr) return fail(IA_ERR_INVALID, "the score's key rows must be non-null (k_bar, or k_max and k_min)");
    if (reinterpret_cast<uintptr_t>(ptr) % 16) return fail(IA_ERR_INVALID, "key rows must be 16-byte aligned");
  }
  return IA_OK;
}

}  // namespace ia

namespace ia {

// Block mask [batch, Hkv, nb] of a top-k selection: one workgroup per (sequence, kv
// head) clears its row, then marks blocks idx[b, h, 0:n_sel] (ids outside [0, nb)
// are ignored).  Consumed by the fixed-mask hybrid decode (representatives for the
// unselected blocks).
__global__ __launch_bounds__(256) void ia_topk_block_mask_kernel(const int32_t* idx, const int32_t* n_sel,
                                                                 int32_t k_cap, int32_t nb, uint8_t* mask) {
  const int bh = blockIdx.y * gridDim.x + blockIdx.x;
  uint8_t* row = mask + (int64_t)bh * nb;
  for (int j = threadIdx.x; j < nb; j += 256) row[j] = 0;
  __syncthreads();
  const int n = min(max(n_sel[bh], 0), k_cap);
  for (int t = threadIdx.x; t < n; t += 256) {
    const int j = idx[(int64_t)bh * k_cap + t];
    if (j >= 0 && j < nb) row[j] = 1;
  }
}

}  // namespace ia

extern "C" {

int ia_topk_block_mask(const int32_t* idx, const int32_t* n_sel, int32_t k_cap, int32_t batch, int32_t n_kv_heads,
                       int32_t nb, uint8_t* mask, void* stream) {
  using namespace ia;
  if (batch < 0 || n_kv_heads <= 0 || nb < 0 || k_cap <= 0) return fail(IA_ERR_INVALID, "bad mask shape");
  if (batch == 0 || nb == 0) return IA_OK;
  if (!idx || !n_sel || !mask) return fail(IA_ERR_INVALID, "idx, n_sel and mask must be non-null");
  hipLaunchKernelGGL(ia_topk_block_mask_kernel, dim3(n_kv_heads, batch), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), idx, n_sel, k_cap, nb, mask);
  return check_launch("top-k block mask");
}

size_t ia_select_topk_workspace_size(int32_t batch, int32_t n_kv_heads, int32_t nb_max) {
  return ia::select_ws_size(batch, n_kv_heads, nb_max);
}

int ia_select_topk(const ia_decode_shape* shape, const void* q, const ia_block_keys* keys, const int32_t* seq_lens,
                   int32_t block_size, int32_t nb_max, int32_t k, const int32_t* k_per_seq, int32_t forced_first,
                   int32_t forced_last, int32_t forced_in_k, int32_t* idx, int32_t k_cap, int32_t* n_sel,
                   float* scores, void* workspace, size_t workspace_bytes, void* stream) {
  using namespace ia;
  if (!shape) return fail(IA_ERR_INVALID, "shape is null");
  if (shape->batch < 0 || shape->n_kv_heads <= 0 || shape->n_q_heads % shape->n_kv_heads != 0)
    return fail(IA_ERR_INVALID, "n_q_heads must be a positive multiple of n_kv_heads");
  const int G = shape->n_q_heads / shape->n_kv_heads;
  const int D = shape->head_dim;
  if (D != 64 && D != 128) return fail(IA_ERR_UNSUPPORTED, "head_dim must be 64 or 128");
  if (G != 1 && G != 2 && G != 4 && G != 8) return fail(IA_ERR_UNSUPPORTED, "GQA group size must be 1, 2, 4 or 8");
  if (shape->q_dtype != IA_F32 && shape->q_dtype != IA_BF16) return fail(IA_ERR_INVALID, "q dtype");
  float score_scale = 0.f;
  int rc = check_block_keys(keys, G, D, &score_scale);
  if (rc) return rc;
  if (!q || !seq_lens || !idx || !n_sel) return fail(IA_ERR_INVALID, "null pointer argument");
  if (block_size <= 0) return fail(IA_ERR_INVALID, "block_size must be positive");
  if (nb_max < 0 || k < 0 || forced_first < 0 || forced_last < 0 || k_cap <= 0)
    return fail(IA_ERR_INVALID, "nb_max, k, forced_* must be >= 0 and k_cap > 0");
  const size_t need = select_ws_size(shape->batch, shape->n_kv_heads, nb_max);
  if (!scores && nb_max > kMaxLdsScores && (!workspace || workspace_bytes < need))
    return fail(IA_ERR_WORKSPACE, "workspace too small: need " + std::to_string(need) + " bytes");
  if (shape->batch == 0) return IA_OK;
  const bool quest = keys->score == IA_SCORE_QUEST;
  SelectParams p{};
  p.q = q;
  p.q_batch_stride = shape->q_batch_stride;
  p.q_row_stride = shape->q_row_stride;
  p.k_bar = quest ? keys->k_max : keys->k_bar;
  p.k_min = keys->k_min;
  p.quest = quest;
  p.kb_batch_stride = keys->batch_stride;
  p.kb_head_stride = keys->head_stride;
  p.seq_lens = seq_lens;
  p.block_size = block_size;
  p.nb_max = nb_max;
  p.k = k;
  p.k_per_seq = k_per_seq;
  p.forced_first = forced_first;
  p.forced_last = forced_last;
  p.forced_in_k = forced_in_k;
  p.idx = idx;
  p.k_cap = k_cap;
  p.n_sel = n_sel;
  // scores go to global memory when asked for, or when a row does not fit in LDS
  p.scores = scores ? scores : (nb_max > kMaxLdsScores ? reinterpret_cast<float*>(workspace) : nullptr);
  p.n_kv_heads = shape->n_kv_heads;
  p.score_scale = score_scale;
  p.lds_scores = nb_max <= kMaxLdsScores ? nb_max : 0;
  dim3 grid(shape->n_kv_heads, shape->batch);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const bool qf32 = shape->q_dtype == IA_F32;
  const bool kbf16 = keys->dtype == IA_BF16;
#define IA_SEL(DD, GG) \
  if (D == DD && G == GG) return launch_select<DD, GG>(p, qf32, kbf16, grid, st);
  IA_SEL(128, 4) IA_SEL(128, 8) IA_SEL(128, 2) IA_SEL(128, 1)
  IA_SEL(64, 4) IA_SEL(64, 8) IA_SEL(64, 2) IA_SEL(64, 1)
#undef IA_SEL
  return fail(IA_ERR_UNSUPPORTED, "head_dim / group combination");
}

}  // extern "C"
