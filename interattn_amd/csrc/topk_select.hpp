// Per-(sequence, kv head) top-k block selection over a row of scores held by one
// workgroup (NT threads), shared by the standalone selector (select_topk.hip,
// 1024 threads) and the fused top-k finalize (paged_decode_kernel.hpp, 512 threads).
//
//   * forced blocks: the first forced_first and last forced_last valid blocks;
//   * the k_eff largest remaining scores, ties at the threshold going to the
//     lowest block indices.  The selection is fixed by its last member, the
//     threshold pair (kT, iT) in the order (score descending, index ascending):
//     a candidate j is chosen iff key_j > kT or (key_j == kT and j <= iT), with
//     key an order-preserving 32-bit image of the score.  The pair is found by
//       - a 256-bucket histogram over the candidates' score range [min, max]
//         (monotone float bucketing), whose prefix from the top names the bucket
//         holding the threshold, then the exact rank of each of that bucket's few
//         members (at most kTieCands of them); or, when the scores are not finite
//         or the bucket is crowded (many equal scores),
//       - an MSB-first 8-bit radix select on the keys (histograms in LDS),
//         stopping as soon as the threshold bin is taken whole;
//   * an ordered compaction (one block-wide scan of per-thread counts over
//     contiguous index ranges) emits the chosen block ids in ascending order.
// The rule is the group-mean score + torch.topk of CBG/methods/quest.py:91-103,
// with the mean key (k_bar) or Quest's page bound (k_max, k_min) scoring a block.
#pragma once

#include "ia_common.hpp"

namespace ia {

__device__ __forceinline__ u32 order_key(float s) {
  const u32 u = __float_as_uint(s);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float key_value(u32 key) {
  return __uint_as_float((key & 0x80000000u) ? (key & 0x7fffffffu) : ~key);
}

// Score of one block row held by a 16-lane row: lane c16 owns dims c16*DPL ..
// c16*DPL + DPL - 1 of k_bar (raw words: bf16 pairs or floats) and of the
// group-summed query qm; block_dot is the lane's share of the dot product and the
// DPP row sum gives every lane the full one.  The standalone selector and the fused
// scorer share this arithmetic, so both produce bit-identical scores (the fused
// scorer's reduce-scatter of many rows' shares adds the same pairs in the same tree
// as row16_sum).
template <int DPL, bool KBF16>
__device__ __forceinline__ float block_dot(const u32* w, const float* qm) {
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
  return a;
}

template <int DPL, bool KBF16>
__device__ __forceinline__ float block_score(const u32* w, const float* qm, float score_scale) {
  return row16_sum(block_dot<DPL, KBF16>(w, qm)) * score_scale;
}

// Quest score of one block (CBG/methods/quest.py:97-101): the group mean of
// sum_d max(q_gd k_max_d, q_gd k_min_d), which, since k_max >= k_min, equals
// (qa . k_max + qb . k_min) / G with qa = sum_g max(q_g, 0), qb = sum_g min(q_g, 0)
// (score_scale = 1 / G).  Key rows as for block_score.
template <int DPL, bool KBF16>
__device__ __forceinline__ float block_dot_quest(const u32* wx, const u32* wn, const float* qa, const float* qb) {
  float a = 0.f;
  if constexpr (KBF16) {
#pragma unroll
    for (int e = 0; e < DPL / 2; ++e) {
      a = fmaf(qa[2 * e], bf16_lo(wx[e]), a);
      a = fmaf(qb[2 * e], bf16_lo(wn[e]), a);
      a = fmaf(qa[2 * e + 1], bf16_hi(wx[e]), a);
      a = fmaf(qb[2 * e + 1], bf16_hi(wn[e]), a);
    }
  } else {
#pragma unroll
    for (int e = 0; e < DPL; ++e) {
      a = fmaf(qa[e], __uint_as_float(wx[e]), a);
      a = fmaf(qb[e], __uint_as_float(wn[e]), a);
    }
  }
  return a;
}

template <int DPL, bool KBF16>
__device__ __forceinline__ float block_score_quest(const u32* wx, const u32* wn, const float* qa, const float* qb,
                                                   float score_scale) {
  return row16_sum(block_dot_quest<DPL, KBF16>(wx, wn, qa, qb)) * score_scale;
}

constexpr int kTieCands = 128;  // threshold-bucket members ranked exactly
constexpr int kSegElems = 16;   // most consecutive indices per thread in one scan pass

template <int NT>
struct TopkLds {
  u32 hist[256];
  u32 red[2][NT / 64];
  int wsum[NT / 64];
  int sh_int[4];
  u32 tie_key[kTieCands];
  int tie_idx[kTieCands];
  int n_tie;
  u32 thr_key;
  int thr_idx;
};

// Maximum over the wave, all in DPP: row maxima, carried across rows by
// row_bcast15 / row_bcast31 into lane 63, read back as a uniform value.
__device__ __forceinline__ u32 wave_u32_max(u32 v) {
  v = max(v, (u32)__builtin_amdgcn_mov_dpp((int)v, kDppRowMirror, 0xf, 0xf, false));
  v = max(v, (u32)__builtin_amdgcn_mov_dpp((int)v, kDppRowHalfMirror, 0xf, 0xf, false));
  v = max(v, (u32)__builtin_amdgcn_mov_dpp((int)v, kDppXor2, 0xf, 0xf, false));
  v = max(v, (u32)__builtin_amdgcn_mov_dpp((int)v, kDppXor1, 0xf, 0xf, false));
  v = max(v, (u32)__builtin_amdgcn_update_dpp(0, (int)v, kDppRowBcast15, 0xa, 0xf, false));
  v = max(v, (u32)__builtin_amdgcn_update_dpp(0, (int)v, kDppRowBcast31, 0xc, 0xf, false));
  return (u32)__builtin_amdgcn_readlane((int)v, 63);
}

// Exclusive prefix sum of one int per thread over the workgroup (thread order);
// *total receives the sum.  Every thread calls it; two barriers.
template <int NT>
__device__ __forceinline__ int block_exclusive_scan(int v, int* wsum, int* total, bool reuse = true) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int inc = wave_inclusive_scan(v);
  if (lane == 63) wsum[wave] = inc;
  __syncthreads();
  int before = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < NT / 64; ++w) {
    const int s = wsum[w];
    tot += s;
    before += (w < wave) ? s : 0;
  }
  // reuse false (a uniform value): the caller synchronises before wsum is written again
  if (reuse) __syncthreads();
  *total = tot;
  return before + inc - v;
}

// Wave 0 of the workgroup: the histogram bin (scanned from the top) where the
// running count first reaches `remaining`; writes sh_int[1..3] = (bin, count still
// needed inside it, members of it).  The caller synchronises.
template <int NT>
__device__ __forceinline__ void threshold_bin(TopkLds<NT>& L, int remaining) {
  const int lane = threadIdx.x & 63;
  // bins in descending order: lane l owns bins 255-4l .. 252-4l
  u32 c[4];
  u32 tot = 0;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    c[t] = L.hist[255 - 4 * lane - t];
    tot += c[t];
  }
  const u32 inc = (u32)wave_inclusive_scan((int)tot);  // over lanes, descending-bin order
  const u32 exc = inc - tot;
  if (exc < (u32)remaining && inc >= (u32)remaining) {
    u32 run = exc;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      if (run + c[t] >= (u32)remaining) {
        L.sh_int[1] = 255 - 4 * lane - t;
        L.sh_int[2] = remaining - (int)run;
        L.sh_int[3] = (int)c[t];
        break;
      }
      run += c[t];
    }
  }
}

// The same bin computed by every wave for itself (no barrier, no LDS round trip):
// returns (bin, count still needed inside it, members of it) as uniform values.
__device__ __forceinline__ void threshold_bin_wave(const u32* hist, int remaining, int& bin, int& need, int& in_bin) {
  const int lane = threadIdx.x & 63;
  u32 c[4];
  u32 tot = 0;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    c[t] = hist[255 - 4 * lane - t];
    tot += c[t];
  }
  const u32 inc = (u32)wave_inclusive_scan((int)tot);
  const u32 exc = inc - tot;
  const bool here = exc < (u32)remaining && inc >= (u32)remaining;
  int b = 0, nd = 0, m = 0;
  if (here) {
    u32 run = exc;
    bool found = false;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      if (!found && run + c[t] >= (u32)remaining) {
        found = true;
        b = 255 - 4 * lane - t;
        nd = remaining - (int)run;
        m = (int)c[t];
      }
      run += c[t];
    }
  }
  const unsigned long long hit = __ballot(here);
  const int src = hit ? __ffsll((long long)hit) - 1 : 0;
  bin = __builtin_amdgcn_readlane(b, src);
  need = __builtin_amdgcn_readlane(nd, src);
  in_bin = __builtin_amdgcn_readlane(m, src);
}

struct TopkRule {
  int forced_first, forced_last, k, forced_in_k, k_cap;
};

// Blocks [0, ff) and [fl_start, nb) are forced in; the others are candidates.
struct TopkForced {
  int ff, fl_start;
  __device__ TopkForced(const TopkRule& rule, int nb)
      : ff(min(max(rule.forced_first, 0), nb)), fl_start(max(nb - max(rule.forced_last, 0), 0)) {}
  __device__ bool operator()(int j) const { return j < ff || j >= fl_start; }
};

// Sizes the rule fixes before any score is read: forced blocks, candidates and
// the number of candidates taken (k_eff).
struct TopkSizes {
  int ff, fl_start, n_forced, n_cand, k_eff;
};
__device__ __forceinline__ TopkSizes topk_sizes(int nb, const TopkRule& rule) {
  const TopkForced f(rule, nb);
  TopkSizes z;
  z.ff = f.ff;
  z.fl_start = f.fl_start;
  z.n_forced = f.ff + (nb - max(f.fl_start, f.ff));  // |[0,ff) U [fl_start,nb)|
  z.n_cand = nb - z.n_forced;
  int k_eff = rule.forced_in_k ? rule.k - z.n_forced : rule.k;
  k_eff = max(k_eff, 0);
  z.k_eff = min(k_eff, max(rule.k_cap - z.n_forced, 0));
  return z;
}

// Number of blocks topk_select chooses from a row of nb blocks (whatever the
// scores): every forced block, min(k_eff, candidates) others, clamped to k_cap.
__device__ __forceinline__ int topk_count(int nb, const TopkRule& rule) {
  const TopkSizes z = topk_sizes(nb, rule);
  return min(z.n_forced + min(z.k_eff, z.n_cand), rule.k_cap);
}

// Staged start of topk_select (for a caller that already walks the score row, e.g.
// while copying it to LDS): each thread passes the largest key and the largest ~key
// of the candidates it saw; the per-wave values land in L.red and the histogram is
// cleared.  The caller synchronises the workgroup before topk_select<..., staged>.
template <int NT>
__device__ __forceinline__ void topk_stage(TopkLds<NT>& L, u32 kmx, u32 kmn_inv) {
  const int wave = threadIdx.x >> 6;
  kmx = wave_u32_max(kmx);
  kmn_inv = wave_u32_max(kmn_inv);
  if ((threadIdx.x & 63) == 0) {
    L.red[0][wave] = kmx;
    L.red[1][wave] = kmn_inv;
  }
  for (int t = threadIdx.x; t < 256; t += NT) L.hist[t] = 0u;
  if (threadIdx.x == 0) L.n_tie = 0;
}

// Every thread of the workgroup calls this (it synchronises, also on return).  key_at(j) returns
// order_key(score_j) for 0 <= j < nb; emit(pos, j) is called for each chosen block,
// pos = 0, 1, ... in ascending block order (only pos < k_cap).  Returns the number
// of chosen blocks (clamped to k_cap).  STAGED: the caller ran topk_stage and a
// workgroup barrier (the first pass over the row is skipped).
template <int NT, bool STAGED = false, typename KeyAt, typename Emit>
__device__ __forceinline__ int topk_select(TopkLds<NT>& L, KeyAt key_at, int nb, const TopkRule& rule, Emit emit) {
  constexpr int kWv = NT / 64;
  const int wave = threadIdx.x >> 6;
  const TopkForced is_forced(rule, nb);
  const TopkSizes sizes = topk_sizes(nb, rule);
  const int n_cand = sizes.n_cand;
  const int k_eff = sizes.k_eff;
  // consecutive indices per thread in the scans over the row (all threads busy)
  const int seg = min(kSegElems, max(1, (nb + NT - 1) / NT));

  // threshold pair: every candidate when all are taken, none when k_eff == 0
  u32 kT = 0u;
  int iT = 0x7fffffff;
  if (k_eff == 0) {
    kT = 0xffffffffu;
    iT = -1;
  }
  if (k_eff > 0 && k_eff < n_cand) {
    // ---- the candidates' largest and smallest keys
    u32 kmx = 0u, kmn_inv = 0u;  // max key, max of ~key
    if constexpr (!STAGED) {
      for (int j = threadIdx.x; j < nb; j += NT) {
        if (is_forced(j)) continue;
        const u32 key = key_at(j);
        kmx = max(kmx, key);
        kmn_inv = max(kmn_inv, ~key);
      }
      topk_stage<NT>(L, kmx, kmn_inv);
      __syncthreads();
      kmx = 0u;
      kmn_inv = 0u;
    }
#pragma unroll
    for (int w = 0; w < kWv; ++w) {
      kmx = max(kmx, L.red[0][w]);
      kmn_inv = max(kmn_inv, L.red[1][w]);
    }
    const u32 kmn = ~kmn_inv;

    // ---- fast path: buckets over the finite score range, exact ranks in the
    // threshold bucket (the decision is uniform over the workgroup)
    const float fmax = key_value(kmx), fmin = key_value(kmn);
    const float bscale = 256.f / (fmax - fmin);
    bool fast = __builtin_isfinite(fmax) && __builtin_isfinite(fmin) && __builtin_isfinite(bscale) && bscale > 0.f;
    auto bucket = [&](u32 key) { return min(255, (int)((key_value(key) - fmin) * bscale)); };
    if (fast) {
      for (int j = threadIdx.x; j < nb; j += NT) {
        if (is_forced(j)) continue;
        atomicAdd(&L.hist[bucket(key_at(j))], 1u);
      }
      __syncthreads();
      int tb, need, in_bin;  // every wave finds the bin itself
      threshold_bin_wave(L.hist, k_eff, tb, need, in_bin);
      if (in_bin <= kTieCands) {
        for (int j = threadIdx.x; j < nb; j += NT) {
          if (is_forced(j)) continue;
          const u32 key = key_at(j);
          if (bucket(key) == tb) {
            const int s = atomicAdd(&L.n_tie, 1);
            L.tie_key[s] = key;
            L.tie_idx[s] = j;
          }
        }
        __syncthreads();
        // member i's rank among the bucket's members (key descending, then index
        // ascending: a strict order, so ranks are distinct); rank need - 1 is the threshold
        if (in_bin <= 64) {
          // every wave ranks the members from registers (lane i holds member i), so no
          // LDS round trip per member and no barrier before the threshold is known
          const int lane = threadIdx.x & 63;
          const bool mem = lane < in_bin;
          const u32 ki = mem ? L.tie_key[lane] : 0u;
          const int ji = mem ? L.tie_idx[lane] : 0;
          int rank = 0;
          for (int e = 0; e < in_bin; ++e) {
            const u32 ke = (u32)__builtin_amdgcn_readlane((int)ki, e);
            const int je = __builtin_amdgcn_readlane(ji, e);
            rank += (ke > ki || (ke == ki && je < ji)) ? 1 : 0;
          }
          const unsigned long long hit = __ballot(mem && rank == need - 1);
          const int src = __ffsll((long long)hit) - 1;
          kT = (u32)__builtin_amdgcn_readlane((int)ki, src);
          iT = __builtin_amdgcn_readlane(ji, src);
        } else {
          for (int i = threadIdx.x; i < in_bin; i += NT) {
            const u32 ki = L.tie_key[i];
            const int ji = L.tie_idx[i];
            int rank = 0;
            for (int e = 0; e < in_bin; ++e) {
              const u32 ke = L.tie_key[e];
              rank += (ke > ki || (ke == ki && L.tie_idx[e] < ji)) ? 1 : 0;
            }
            if (rank == need - 1) {
              L.thr_key = ki;
              L.thr_idx = ji;
            }
          }
          __syncthreads();
          kT = L.thr_key;
          iT = L.thr_idx;
        }
      } else {
        fast = false;
      }
    }

    if (!fast) {
      __syncthreads();  // every wave is done with the bucket histogram
      // ---- radix select on the keys: the bytes every candidate shares are skipped
      const u32 diff = kmx ^ kmn;
      const int common_bytes = diff == 0u ? 4 : (__clz((int)diff) >> 3);
      u32 prefix = 0u, mask = 0u;
      if (common_bytes > 0) {
        mask = common_bytes == 4 ? 0xffffffffu : ~(0xffffffffu >> (8 * common_bytes));
        prefix = kmx & mask;
      }
      int remaining = k_eff;
      int in_bin = n_cand;
      for (int shift = 24 - 8 * common_bytes; shift >= 0; shift -= 8) {
        for (int t = threadIdx.x; t < 256; t += NT) L.hist[t] = 0u;
        __syncthreads();
        for (int j = threadIdx.x; j < nb; j += NT) {
          if (is_forced(j)) continue;
          const u32 key = key_at(j);
          if ((key & mask) == prefix) atomicAdd(&L.hist[(key >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (wave == 0) threshold_bin<NT>(L, remaining);
        __syncthreads();
        const u32 digit = (u32)L.sh_int[1];
        remaining = L.sh_int[2];
        in_bin = L.sh_int[3];
        prefix |= digit << shift;
        mask |= 255u << shift;
        __syncthreads();
        if (remaining == in_bin) break;  // the whole bin is taken: the threshold is exact
      }
      kT = prefix;  // keys with (key & mask) >= prefix, i.e. key >= prefix (low bits zero)
      if (remaining != in_bin) {
        // mask is full: take the `remaining` lowest indices among keys equal to prefix
        int base = 0;
        for (int c0 = 0; c0 < nb; c0 += NT * seg) {
          const int j0 = c0 + threadIdx.x * seg;
          int cnt = 0;
          for (int e = 0; e < seg; ++e) {
            const int j = j0 + e;
            cnt += (j < nb && !is_forced(j) && key_at(j) == prefix) ? 1 : 0;
          }
          int total;
          const int before = base + block_exclusive_scan<NT>(cnt, L.wsum, &total);
          if (before < remaining && before + cnt >= remaining) {
            int run = before;
            for (int e = 0; e < seg; ++e) {
              const int j = j0 + e;
              if (j < nb && !is_forced(j) && key_at(j) == prefix && ++run == remaining) L.thr_idx = j;
            }
          }
          base += total;
          if (base >= remaining) break;  // uniform
        }
        __syncthreads();
        iT = L.thr_idx;
      }
    }
  }

  // ---- ordered compaction: each thread scans `seg` consecutive indices
  int base_sel = 0;
  for (int c0 = 0; c0 < nb; c0 += NT * seg) {
    const int j0 = c0 + threadIdx.x * seg;
    u32 bits = 0u;
    for (int e = 0; e < seg; ++e) {
      const int j = j0 + e;
      if (j < nb) {
        bool sel = is_forced(j);
        if (!sel) {
          const u32 key = key_at(j);
          sel = key > kT || (key == kT && j <= iT);
        }
        bits |= sel ? (1u << e) : 0u;
      }
    }
    int total;
    // the last chunk's scan needs no second barrier: the one below comes first
    int pos = base_sel + block_exclusive_scan<NT>(__popc(bits), L.wsum, &total, c0 + NT * seg < nb);
    while (bits) {
      const int e = __ffs((int)bits) - 1;
      bits &= bits - 1u;
      if (pos < rule.k_cap) emit(pos, j0 + e);
      ++pos;
    }
    base_sel += total;
  }
  __syncthreads();  // emitted entries (e.g. in LDS) are visible to the workgroup on return
  return min(base_sel, rule.k_cap);
}

}  // namespace ia
