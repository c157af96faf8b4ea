// Balanced split-K launch plan of the paged finalize.
//
// A balanced launch is one flat grid of workgroups over the (sequence, kv head)
// rows, r = b * Hkv + h.  With S_r = the row's units x subtiles per unit ("raw
// slots", unit-major), row r gets n_r items:
//   * every row alike (S_r = S): n = budget / rows items per row (budget = resident
//     workgroups), so the grid is used whole and workgroup w serves row
//     w / (grid / rows) (the guess the fused finalize loads ahead with); clamped to
//     at most max_items (the partial stride) and S / units-per-slot (items of at
//     least one unit), and to at least ceil(S / t_hi);
//   * otherwise n_r = max(1, ceil(S_r / t)) with t the smallest per-item slot budget
//     in [t_lo, t_hi] such that sum_r n_r <= budget (t_hi when none fits).  t_lo keeps
//     n_r <= max_items and items of at least one unit.
// Item i of a row covers q + 1 slots for i < rem and q slots after, q = S / n and
// rem = S - q n (never empty when S >= n); items are numbered row by row
// over the grid and the workgroups past the last item are idle.  t_hi keeps an
// item's unit ranges and subtile list within the finalize's LDS arrays.  Every
// function here runs in one wave, without barriers: the fused top-k launch computes
// the plan in every wave of every workgroup, the other launches in one wave of each
// finalize workgroup.  All evaluate the same code on the same S_r, so they agree
// bit for bit.
#pragma once

#include "topk_select.hpp"

namespace ia {

constexpr int kPlanRegRows = 4;        // rows per lane held in registers (256 rows)
constexpr int kPlanMaxUnits = 512;     // LDS unit ranges per finalize item
constexpr int kPlanMaxSubs = 2048;     // LDS subtiles per finalize item
constexpr int64_t kPlanMaxRows = 1 << 13;  // rows of one balanced launch (slot sums stay below 2^31)

// One finalize workgroup's share (32 bytes in memory).
struct PlanEntry {
  int row;  // -1: idle workgroup
  int item, n_items;
  int slot_lo, slot_hi;
  int n_units;  // units of the row
  int seq_len;  // the row's sequence length
  int k_row;    // the row's top-k k (fused source)
};

__host__ __device__ constexpr int plan_t_cap(int nsub_u) {
  return (kPlanMaxUnits - 1) * nsub_u < kPlanMaxSubs ? (kPlanMaxUnits - 1) * nsub_u : kPlanMaxSubs;
}

__device__ __forceinline__ int cdiv_pos(int a, int b) { return a / b + (a % b != 0); }

__device__ __forceinline__ int wave_sum_i(int v) { return __builtin_amdgcn_readlane(wave_inclusive_scan(v), 63); }

// ceil(s / t) for 0 <= s < 2^20 and t >= 1, from the float reciprocal rt of t: the
// product is within 1/4 of s / t, so one correction step gives the exact quotient.
__device__ __forceinline__ int ceil_div_rcp(int s, int t, float rt) {
  int q = (int)((float)s * rt);
  int rem = s - q * t;
  if (rem < 0) {
    --q;
    rem += t;
  } else if (rem >= t) {
    ++q;
    rem -= t;
  }
  return q + (rem > 0 ? 1 : 0);
}

// S_r of the rows one lane keeps in registers: rows lane + 64 k, k < kPlanRegRows.
struct PlanRows {
  int s[kPlanRegRows];
};

// The rule that sets each row's item count (see the top of this file).
struct PlanRule {
  int t;      // per-item slot budget (rows of unequal work)
  int n_all;  // items of every row when all rows have the same work, else 0
};

// The plan's rule, computed by one wave (every lane returns it).  slots_of(r) gives
// S_r for any row (rows past the register stage are read through it again).
template <typename SlotsOf>
__device__ __forceinline__ PlanRule plan_rule_wave(SlotsOf slots_of, int nrows, int budget, int max_items, int nsub_u,
                                   PlanRows& rows) {
  const int lane = threadIdx.x & 63;
  int ssum = 0, smax = 0;
#pragma unroll
  for (int k = 0; k < kPlanRegRows; ++k) {
    const int r = lane + 64 * k;
    rows.s[k] = r < nrows ? slots_of(r) : 0;
    ssum += rows.s[k];
    smax = max(smax, rows.s[k]);
  }
  for (int r = lane + 64 * kPlanRegRows; r < nrows; r += 64) {
    const int s = slots_of(r);
    ssum += s;
    smax = max(smax, s);
  }
  ssum = wave_sum_i(ssum);
  smax = (int)wave_u32_max((u32)smax);
  budget = max(budget, nrows);
  max_items = max(max_items, 1);
  const int t_cap = plan_t_cap(nsub_u);
  if ((int64_t)smax * nrows == (int64_t)ssum) {
    // every row alike: budget / rows items per row
    int n = min(budget / nrows, min(max_items, max(smax / nsub_u, 1)));
    n = max(n, max(cdiv_pos(smax, t_cap), 1));
    return PlanRule{0, n};
  }
  const int t_floor = min(max(nsub_u, cdiv_pos(smax, max_items)), t_cap);
  int lo = min(max(t_floor, cdiv_pos(ssum, budget)), t_cap);
  int hi = max(lo, min(smax, t_cap));
  // sum_r max(1, ceil(S_r / t)) <= ssum / t + nrows: this t always fits the budget
  if (budget > nrows) hi = max(lo, min(hi, cdiv_pos(ssum, budget - nrows)));
  auto items_at = [&](int t) -> int {
    const float rt = __builtin_amdgcn_rcpf((float)t);
    int a = 0;
#pragma unroll
    for (int k = 0; k < kPlanRegRows; ++k)
      if (lane + 64 * k < nrows) a += max(1, ceil_div_rcp(rows.s[k], t, rt));
    for (int r = lane + 64 * kPlanRegRows; r < nrows; r += 64) a += max(1, ceil_div_rcp(slots_of(r), t, rt));
    return wave_sum_i(a);
  };
  while (lo < hi) {  // the smallest t in [lo, hi] that fits (hi when none does)
    const int mid = (lo + hi) >> 1;
    if (items_at(mid) <= budget) hi = mid;
    else lo = mid + 1;
  }
  return PlanRule{lo, 0};
}

// Visit every row's items in grid order: visit(lane_active, r, S_r, n_r, first item's
// workgroup) is called by every lane for each 64-row chunk (lane_active false past
// nrows) and ends the walk by returning true (a uniform value); returns the number of
// workgroups the visited rows' items take.
template <typename SlotsOf, typename Visit>
__device__ __forceinline__ int plan_walk_wave(SlotsOf slots_of, const PlanRows& rows, int nrows, const PlanRule& rule, Visit visit) {
  const int lane = threadIdx.x & 63;
  const float rt = __builtin_amdgcn_rcpf((float)max(rule.t, 1));
  int base = 0;
  for (int r0 = 0; r0 < nrows; r0 += 64) {
    const int r = r0 + lane;
    const int k = r0 >> 6;
    int s = 0;
    if (r < nrows) {
      if (k < kPlanRegRows) {
#pragma unroll
        for (int kk = 0; kk < kPlanRegRows; ++kk)
          if (kk == k) s = rows.s[kk];
      } else {
        s = slots_of(r);
      }
    }
    const int n = r >= nrows ? 0 : rule.n_all > 0 ? rule.n_all : max(1, ceil_div_rcp(s, rule.t, rt));
    const int inc = wave_inclusive_scan(n);
    if (visit(r < nrows, r, s, n, base + inc - n)) return base;  // uniform stop
    base += __builtin_amdgcn_readlane(inc, 63);
  }
  return base;
}

// Row r's split: S_r = s slots in n items, q = s / n slots each and one more for the
// first rem = s - q n items.
struct PlanSplit {
  int r, s, n, q, rem, n_units;
};
__device__ __forceinline__ PlanSplit plan_split(int r, int s, int n, int nsub_u) {
  const int q = s / n;
  return PlanSplit{r, s, n, q, s - q * n, s / nsub_u};
}

// Fill the entry of item i of a split (no division: called once per workgroup).
__device__ __forceinline__ void plan_fill(PlanEntry& e, const PlanSplit& sp, int i) {
  e.row = sp.r;
  e.item = i;
  e.n_items = sp.n;
  e.slot_lo = i * sp.q + min(i, sp.rem);
  e.slot_hi = e.slot_lo + sp.q + (i < sp.rem ? 1 : 0);
  e.n_units = sp.n_units;
}

// The entry of workgroup w (one wave; every lane returns it; row -1 when idle).
// seq_len and k_row are left to the caller.
template <typename SlotsOf>
__device__ __forceinline__ PlanEntry plan_entry_wave(SlotsOf slots_of, const PlanRows& rows, int nrows, const PlanRule& rule, int w,
                                     int nsub_u) {
  PlanEntry e{};
  e.row = -1;
  plan_walk_wave(slots_of, rows, nrows, rule, [&](bool active, int r, int s, int n, int first) -> bool {
    const bool mine = active && w >= first && w < first + n;
    const unsigned long long bal = __ballot(mine);
    if (bal) {
      const int src = __ffsll((long long)bal) - 1;
      const int rr = __builtin_amdgcn_readlane(r, src);
      const int ss = __builtin_amdgcn_readlane(s, src);
      const int nn = __builtin_amdgcn_readlane(n, src);
      const int ff = __builtin_amdgcn_readlane(first, src);
      plan_fill(e, plan_split(rr, ss, nn, nsub_u), w - ff);
      return true;
    }
    return false;
  });
  return e;
}

}  // namespace ia
