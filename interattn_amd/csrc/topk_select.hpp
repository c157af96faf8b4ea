// Per-(sequence, kv head) top-k block selection over a row of scores held by one
// workgroup (NT threads), shared by the standalone selector (select_topk.hip,
// 1024 threads) and the fused top-k finalize (paged_decode_kernel.hpp, 256 threads).
//
//   * forced blocks: the first forced_first and last forced_last valid blocks;
//   * the k_eff largest remaining scores by an MSB-first 8-bit radix select on
//     order-preserving 32-bit keys (histograms in LDS), stopping as soon as the
//     threshold bin is taken whole; ties at the threshold go to the lowest block
//     indices;
//   * an ordered compaction (wave ballots + LDS offsets) emits the chosen block
//     ids in ascending order.
// The rule is the group-mean score + torch.topk of CBG/methods/quest.py:91-103
// with the mean key (k_bar) as the block representative.
#pragma once

#include "ia_common.hpp"

namespace ia {

__device__ __forceinline__ u32 order_key(float s) {
  const u32 u = __float_as_uint(s);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Score of one block row held by a 16-lane row: lane c16 owns dims c16*DPL ..
// c16*DPL + DPL - 1 of k_bar (raw words: bf16 pairs or floats) and of the
// group-summed query qm; the DPP row sum gives every lane the full dot product.
// The standalone selector and the fused scorer share this arithmetic, so both
// produce bit-identical scores.
template <int DPL, bool KBF16>
__device__ __forceinline__ float block_score(const u32* w, const float* qm, float score_scale) {
  float a = 0.f;
  if constexpr (KBF16) {
#pragma unroll
    for (int e = 0; e < DPL / 2; ++e) {
      a = fmaf(qm[2 * e], bf16_lo(w[e]), a);
      a = fmaf(qm[2 * e + 1], bf16_hi(w[e]), a);
    }
  } else {
#pragma unroll
    for (int e = 0; e < DPL; ++e) a = fmaf(qm[e], __uint_as_float(w[e]), a);
  }
  return row16_sum(a) * score_scale;
}

constexpr int kTopkSubHist = 1;  // histogram copies (wave w counts into copy w % kTopkSubHist)

template <int NT>
struct TopkLds {
  u32 hist[kTopkSubHist][256];
  u32 red[2][NT / 64];
  int sh_int[4];
  int wave_cnt[2][NT / 64];
};

__device__ __forceinline__ u32 dpp_u32_max(u32 v) {
  v = max(v, (u32)__builtin_amdgcn_mov_dpp((int)v, kDppRowMirror, 0xf, 0xf, false));
  v = max(v, (u32)__builtin_amdgcn_mov_dpp((int)v, kDppRowHalfMirror, 0xf, 0xf, false));
  v = max(v, (u32)__builtin_amdgcn_mov_dpp((int)v, kDppXor2, 0xf, 0xf, false));
  v = max(v, (u32)__builtin_amdgcn_mov_dpp((int)v, kDppXor1, 0xf, 0xf, false));
  v = max(v, (u32)__shfl_xor((int)v, 16, 64));
  return max(v, (u32)__shfl_xor((int)v, 32, 64));
}

struct TopkRule {
  int forced_first, forced_last, k, forced_in_k, k_cap;
};

// Every thread of the workgroup calls this (it synchronises).  key_at(j) returns
// order_key(score_j) for 0 <= j < nb; emit(pos, j) is called for each chosen block,
// pos = 0, 1, ... in ascending block order (only pos < k_cap).  Returns the number
// of chosen blocks (clamped to k_cap).
template <int NT, typename KeyAt, typename Emit>
__device__ int topk_select(TopkLds<NT>& L, KeyAt key_at, int nb, const TopkRule& rule, Emit emit) {
  constexpr int kWv = NT / 64;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int ff = min(max(rule.forced_first, 0), nb);
  const int fl_start = max(nb - max(rule.forced_last, 0), 0);
  auto is_forced = [&](int j) { return j < ff || j >= fl_start; };
  const int n_forced = ff + (nb - max(fl_start, ff));  // |[0,ff) U [fl_start,nb)|
  const int n_cand = nb - n_forced;
  int k_eff = rule.forced_in_k ? rule.k - n_forced : rule.k;
  k_eff = max(k_eff, 0);
  k_eff = min(k_eff, max(rule.k_cap - n_forced, 0));

  u32 thr = 0u;       // threshold prefix; candidates with (key & thr_mask) > thr are taken
  u32 thr_mask = 0u;
  int take_ties = 0;  // candidates with (key & thr_mask) == thr taken, lowest indices first
  const bool take_all = k_eff >= n_cand;
  if (!take_all && k_eff > 0) {
    // the candidates' largest and smallest keys: the bytes they share are common to
    // every candidate, so the radix passes start at the first byte that differs
    u32 kmx = 0u, kmn_inv = 0u;  // max key, max of ~key
    for (int j = threadIdx.x; j < nb; j += NT) {
      if (is_forced(j)) continue;
      const u32 key = key_at(j);
      kmx = max(kmx, key);
      kmn_inv = max(kmn_inv, ~key);
    }
    kmx = dpp_u32_max(kmx);
    kmn_inv = dpp_u32_max(kmn_inv);
    if (lane == 0) {
      L.red[0][wave] = kmx;
      L.red[1][wave] = kmn_inv;
    }
    __syncthreads();
    kmx = 0u;
    kmn_inv = 0u;
#pragma unroll
    for (int w = 0; w < NT / 64; ++w) {
      kmx = max(kmx, L.red[0][w]);
      kmn_inv = max(kmn_inv, L.red[1][w]);
    }
    const u32 diff = kmx ^ ~kmn_inv;
    const int common_bytes = diff == 0u ? 4 : (__clz((int)diff) >> 3);
    u32 prefix = 0u, mask = 0u;
    if (common_bytes > 0) {
      mask = common_bytes == 4 ? 0xffffffffu : ~(0xffffffffu >> (8 * common_bytes));
      prefix = kmx & mask;
    }
    int remaining = k_eff;
    for (int shift = 24 - 8 * common_bytes; shift >= 0; shift -= 8) {
      for (int t = threadIdx.x; t < kTopkSubHist * 256; t += NT) (&L.hist[0][0])[t] = 0u;
      __syncthreads();
      u32* hist = L.hist[wave % kTopkSubHist];
      for (int j = threadIdx.x; j < nb; j += NT) {
        if (is_forced(j)) continue;
        const u32 key = key_at(j);
        if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
      }
      __syncthreads();
      if (wave == 0) {
        // bins in descending order: lane l owns bins 255-4l .. 252-4l
        u32 c[4];
        u32 tot = 0;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          c[t] = 0u;
#pragma unroll
          for (int h = 0; h < kTopkSubHist; ++h) c[t] += L.hist[h][255 - 4 * lane - t];
          tot += c[t];
        }
        u32 inc = tot;  // inclusive scan over lanes (descending-bin order)
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
          const u32 o = __shfl_up(inc, off, 64);
          if (lane >= off) inc += o;
        }
        const u32 exc = inc - tot;
        // the bin where the running count first reaches `remaining`
        if (exc < (u32)remaining && inc >= (u32)remaining) {
          u32 run = exc;
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            if (run + c[t] >= (u32)remaining) {
              L.sh_int[1] = 255 - 4 * lane - t;    // digit
              L.sh_int[2] = remaining - (int)run;  // still needed inside this bin
              L.sh_int[3] = (int)c[t];             // candidates inside this bin
              break;
            }
            run += c[t];
          }
        }
      }
      __syncthreads();
      const u32 digit = (u32)L.sh_int[1];
      remaining = L.sh_int[2];
      const int in_bin = L.sh_int[3];
      prefix |= digit << shift;
      mask |= 255u << shift;
      __syncthreads();
      if (remaining == in_bin) break;  // the whole bin is taken: the threshold is exact
    }
    thr = prefix;
    thr_mask = mask;
    take_ties = remaining;
  }

  // ordered compaction
  int base_sel = 0, base_tie = 0;
  for (int j0c = 0; j0c < nb; j0c += NT) {
    const int j = j0c + threadIdx.x;
    bool forced = false, above = false, tie = false;
    if (j < nb) {
      forced = is_forced(j);
      if (!forced) {
        if (take_all) {
          above = true;
        } else if (k_eff > 0) {
          const u32 key = key_at(j) & thr_mask;
          above = key > thr;
          tie = key == thr;
        }
      }
    }
    // tie rank in index order
    const unsigned long long tb = __ballot(tie);
    const int tie_rank_in_wave = __popcll(tb & ((1ull << lane) - 1ull));
    if (lane == 0) L.wave_cnt[1][wave] = __popcll(tb);
    __syncthreads();
    int tie_off = base_tie;
    for (int w = 0; w < wave; ++w) tie_off += L.wave_cnt[1][w];
    const bool take_tie = tie && (tie_off + tie_rank_in_wave < take_ties);
    const bool sel = forced || above || take_tie;
    const unsigned long long sb = __ballot(sel);
    const int sel_rank = __popcll(sb & ((1ull << lane) - 1ull));
    if (lane == 0) L.wave_cnt[0][wave] = __popcll(sb);
    __syncthreads();
    int sel_off = base_sel;
    for (int w = 0; w < wave; ++w) sel_off += L.wave_cnt[0][w];
    if (sel && sel_off + sel_rank < rule.k_cap) emit(sel_off + sel_rank, j);
    int tot_s = 0, tot_t = 0;
    for (int w = 0; w < kWv; ++w) {
      tot_s += L.wave_cnt[0][w];
      tot_t += L.wave_cnt[1][w];
    }
    base_sel += tot_s;
    base_tie += tot_t;
    __syncthreads();
  }
  return min(base_sel, rule.k_cap);
}

}  // namespace ia
