// The condition (eps) rule inside the paged finalize's prologue (kSrcCondFused):
// one launch per layer call of the reference's fused path (CBT/core.py:1035-1155:
// statistics, routing with representatives, selected pages and suffix, merge).
//
// A row (sequence, kv head) has n items (workgroups, all resident at once); item i
// owns the row's blocks i, i + n, i + 2 n, ... (strided, so a run of neighbouring
// selected blocks spreads over the items instead of landing on one) and
//   1. computes s and delta of its blocks (CBT/core.py:747-814) into LDS and its
//      partials of the row statistics: per query row the max and sum exp of z and
//      of zc = z + log cosh(delta) over its blocks;
//   2. publishes them as tagged words (value bits | tag << 32) and reads the other
//      items' (waiting at most the wait limit; a partial still missing then is
//      recomputed here from the summaries, with the same code, so the same bits);
//   3. merges the n partials in item order into the row globals (every item the
//      same bits, CBT/core.py:817-847), routes its blocks with the condition
//      (CBT/page_attention.py:104-171), writes the selected flags when asked,
//      lists its selected blocks, and computes the representative partial of its
//      unselected blocks: logit z, value v_bar, weight beta (bf16-rounded with
//      v_bar for bf16 caches, CBT/page_attention.py:173-204);
//   4. streams its selected blocks (and, in the last item, the exact suffix) as the
//      route-list source does, folds the representative partial into its split-K
//      partial, and the row's last item merges the n partials in the launch.
// Included by paged_decode_kernel.hpp after DecodeParams, partial_tag and the
// reductions; not a standalone header.
#pragma once

namespace ia {

template <int D, int G>
struct CondLds {
  float s[G][kCondItemBlocks];       // s per (query row, own block); then the representatives' weights
  float dl[G][kCondItemBlocks];      // delta per (query row, own block)
  float lc[kCondItemBlocks];         // log(valid tokens) per own block, -inf for an empty one
  float part[kMaxItemsPerBh][4][G];  // the row's items' partials (z_m, z_l, c_m, c_l) per query row
  float own[4][G];                   // an item's partials, as computed by the waves
  float glob[4][G];                  // the row's globals
  float rep_acc[kFinWaves][G * D];   // representative partial per wave: sum of weight x v_bar
  float rep_m[G];                    //   its largest logit (log2 domain)
  float rep_l[G];                    //   and its weight sum
  int list[kCondItemBlocks];         // the own selected blocks, ascending: id | valid tokens << 16
  int wcnt[kFinWaves];
  u32 missing;
};

// 32-block steps of summary rows in flight per wave, and whether the item's first
// v_bar rows are loaded at the start (G = 8 has no registers to spare for either)
template <int G>
constexpr int cond_stat_steps() { return G <= 4 ? 2 : 1; }
template <int G>
constexpr bool cond_vbar_early() { return G <= 4; }

// Blocks of item i of n over a row of nb blocks (i < n <= nb): i, i + n, ..., so its
// local block j is row block i + j n.
__device__ __forceinline__ int cond_item_blocks(int i, int nb, int n) { return (nb - i + n - 1) / n; }

// Values per lane of the statistics' row reduce-scatter: s, A and B for G query rows
// (external-mask mode: s only), padded to a power of two.
template <int G, bool MASK>
constexpr int cond_nv() {
  return (MASK ? G : 3 * G) <= 4 ? 4 : (MASK ? G : 3 * G) <= 8 ? 8 : (MASK ? G : 3 * G) <= 16 ? 16 : 32;
}

// Steps 1-3 for item `item` of the n_it items of row (b, h).  SBF: the k_bar, bound
// and v_bar rows are all bf16 (one load per row slice); else their dtypes are read
// at run time.  MASK: the external-mask mode of fixed_mask_hybrid_attention
// (CBG/real_attention_benchmark/fixed_mask.py:38-239): the selection is the caller's
// mask [batch, Hkv, nb], there are no statistics to exchange, and a representative's
// logit is bf16(q) . bf16(k_bar) / sqrt(D) + log(count) for bf16 caches (q . k_bar /
// sqrt(D) + log(count) for fp32 caches), weighted against the largest of the item's
// representative logits.  Returns the number of selected blocks among the item's blocks (their
// list entries in L.list); the representative partial is left in L.rep_acc (one
// accumulator per wave, summed by the finalize's fold) / rep_m / rep_l.  Every
// thread of the workgroup calls it.
template <int D, int G, int SBF, bool MASK>
__device__ __forceinline__ int cond_fused_prologue_t(const DecodeParams& p, CondLds<D, G>& L, int b, int h, int item,
                                                     int n_it, u32 row_epoch) {
  constexpr int DPL = D / 16;
  constexpr int NV = cond_nv<G, MASK>();
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c16 = lane & 15;
  const int r = lane >> 4;
  const int t = threadIdx.x;
  const int nb = p.nb_max;
  const int bh = b * p.n_kv_heads + h;
  const int64_t vrow = (int64_t)bh * nb;  // summary row of block 0 of this (b, h)
  const int m = cond_item_blocks(item, nb, n_it);  // >= 1: the host keeps n_it <= nb
  const bool kbf = SBF || p.c_kbar_bf16, xbf = SBF || p.c_bounds_bf16, vbf = SBF || p.c_vbar_bf16;

  constexpr int kSteps = cond_stat_steps<G>();
  constexpr bool kEarlyV = cond_vbar_early<G>();
  // ---- issued first: the query rows for the statistics (row g at the lane's dims
  // c16 DPL ..), this thread's block (local t <-> item + t n_it): its count and norm
  // bound, and (G <= 4) the v_bar rows of the item's first two 32-block steps (every
  // local index clamped below m, so no load sits under a per-lane branch).  The query is
  // kept as raw words on both dtypes and converted after the summaries' loads are
  // issued: a conversion under a dtype branch would wait for the query first.
  SumRow<DPL> qw[G];
  const bool qbf = !p.q_f32;
#pragma unroll
  for (int g = 0; g < G; ++g)
    qw[g].load(p.q, (int64_t)b * p.q_batch_stride + (int64_t)(h * G + g) * p.q_row_stride + c16 * DPL, qbf);
  const bool mine = t < m;
  const int jt = item + min(t, m - 1) * n_it;
  const int cnt_ld = p.c_counts[(int64_t)b * nb + jt];
  const float bc_ld = MASK ? 0.f : p.c_vnorm_max[vrow + jt];
  const float b_all = MASK ? 0.f : p.c_vnorm_all[bh];
  const bool mask_ld = MASK && p.c_mask[vrow + jt] != 0;
  SumRow<DPL, SBF> vpre[kEarlyV ? 2 : 1];
  if constexpr (kEarlyV) {
#pragma unroll
    for (int u = 0; u < 2; ++u)
      vpre[u].load(p.c_vbar, (vrow + item + min(32 * u + 4 * wave + r, m - 1) * n_it) * D + c16 * DPL, vbf);
  }

  // ---- step 1: s and delta of item ri's blocks into L.s / L.dl, log(count) into
  // L.lc: its local block 32 step + 4 w + r on the 16 lanes of row r of wave w.  With
  // A = sum q (k_max + k_min) and B = sum |q| (k_max - k_min) (upper/lower = (A +- B)/2):
  // s = q.k_bar / sqrt(D), delta = |A/2 - s| + B/2 (in units of 1/sqrt(D)).  Each lane's
  // 3 G partial sums are reduce-scattered over its 16-lane row; lane c16 = g then
  // gathers s, A and B of query row g.
  auto item_stats = [&](int ri) {
    const int rm = cond_item_blocks(ri, nb, n_it);
    const int nsteps = (rm + 31) / 32;
    const int cl = t < rm ? p.c_counts[(int64_t)b * nb + ri + t * n_it] : 0;
    for (int s0 = 0; s0 < nsteps; s0 += kSteps) {
      SumRow<DPL, SBF> kb[kSteps];
      BoundRows<DPL, SBF> kx[MASK ? 1 : kSteps];
#pragma unroll
      for (int u = 0; u < kSteps; ++u) {
        const int64_t off = (vrow + ri + min(32 * (s0 + u) + 4 * wave + r, rm - 1) * n_it) * D + c16 * DPL;
        kb[u].load(p.c_kbar, off, kbf);
        if constexpr (!MASK) {
          kx[u].load(p.c_kmax, p.c_kmin, off, xbf, p.c_bounds_packed);
        }
      }
      if (s0 == 0 && t < kCondItemBlocks) L.lc[t] = cl > 0 ? __logf((float)cl) : kNegInf;
      // (external mask: bf16(q) and bf16(k_bar) for bf16 caches, fixed_mask.py:86-107)
      float qf[G][DPL];
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < DPL; ++e) qf[g][e] = MASK ? round_if(qw[g].at(e, qbf), p.c_rep_bf16) : qw[g].at(e, qbf);
#pragma unroll
      for (int u = 0; u < kSteps; ++u) {
        if (s0 + u >= nsteps) break;
        const int jl = 32 * (s0 + u) + 4 * wave + r;
        float ksum[DPL], kdif[DPL], kbv[DPL];
#pragma unroll
        for (int e = 0; e < DPL; ++e) {
          if constexpr (MASK) {
            kbv[e] = round_if(kb[u].at(e, kbf), p.c_rep_bf16 && !kbf);
            ksum[e] = kdif[e] = 0.f;
          } else {
            const float hx = kx[u].mx(e, xbf), ln = kx[u].mn(e, xbf);
            ksum[e] = hx + ln;
            kdif[e] = hx - ln;
            kbv[e] = kb[u].at(e, kbf);
          }
        }
        float v[NV];
#pragma unroll
        for (int i = 0; i < NV; ++i) v[i] = 0.f;
#pragma unroll
        for (int g = 0; g < G; ++g) {
          float a = 0.f, sa = 0.f, sb = 0.f;
#pragma unroll
          for (int e = 0; e < DPL; ++e) {
            const float qv = qf[g][e];
            a = fmaf(qv, kbv[e], a);
            if constexpr (!MASK) {
              sa = fmaf(qv, ksum[e], sa);
              sb = fmaf(fabsf(qv), kdif[e], sb);
            }
          }
          v[g] = a;
          if constexpr (!MASK) {
            v[G + g] = sa;
            v[2 * G + g] = sb;
          }
        }
        reduce_scatter16<NV>(v, lane);
        // value index x sits in lane src(x) of the row, in v[0] (v[x & 1] for NV = 32)
        auto fetch = [&](int x) -> float {
          const int src = (lane & ~15) + (NV == 32 ? x >> 1 : NV == 16 ? x : NV == 8 ? 2 * x : 4 * x);
          if constexpr (NV == 32) {
            const float a0 = __shfl(v[0], src, 64), a1 = __shfl(v[1], src, 64);
            return (x & 1) ? a1 : a0;
          } else {
            return __shfl(v[0], src, 64);
          }
        };
        const int gq = c16 < G ? c16 : 0;
        const float sv = fetch(gq) * p.c_scale;
        if constexpr (MASK) {
          if (c16 < G && jl < rm) L.s[c16][jl] = sv;
        } else {
          const float av = fetch(G + gq), bv = fetch(2 * G + gq);
          const float dl = fabsf(0.5f * av * p.c_scale - sv) + 0.5f * bv * p.c_scale;
          if (c16 < G && jl < rm) {
            L.s[c16][jl] = sv;
            L.dl[c16][jl] = dl;
          }
        }
      }
    }
  };

  // the partials of the item whose s, delta and log(count) are in L.s / L.dl / L.lc
  // (rm blocks): per query row the max and sum exp of z = s + log(count) and of zc.
  // Wave w takes (value, row) pairs w, w + 8, ...: each lane an online (max, sum) over
  // blocks lane, lane + 64, ..., then one (max, sum) reduction over the wave.  The
  // same code for any item, so a partial recomputed by another item has the same bits.
  // Leaves the partials in L.own (readable after its final barrier).
  auto item_partial = [&](int rm) {
    for (int pr = wave; pr < 2 * G; pr += kFinWaves) {
      const int wh = pr / G, g = pr - wh * G;
      float mx = kNegInf, sm = 0.f;
      for (int j = lane; j < rm; j += 64) {
        const float lcj = L.lc[j];
        float v = kNegInf;
        if (lcj != kNegInf) {
          v = L.s[g][j] + lcj;
          if (wh == 1) v += p.c_mass_exp ? L.dl[g][j] : log_cosh(L.dl[g][j]);
        }
        if (v > mx) {
          sm = (mx == kNegInf ? 0.f : sm * __expf(mx - v)) + 1.f;
          mx = v;
        } else if (v != kNegInf) {
          sm += __expf(v - mx);
        }
      }
      const float M = wave_max(mx);
      const float S = wave_sum(mx == kNegInf ? 0.f : sm * __expf(mx - M));
      if (lane == 0) {
        L.own[2 * wh][g] = M;
        L.own[2 * wh + 1][g] = S;
      }
    }
    __syncthreads();
  };

  item_stats(item);
  __syncthreads();
  if constexpr (!MASK) item_partial(m);
  if (MASK) {
  } else if (n_it > 1) {  // (a row of one item hands nothing over: every published word
                   // belongs to a call that advances the row's epoch)
    // ---- step 2: the own partial as tagged words, then the other items'
    const u32 tag = partial_tag(bh, row_epoch);
    unsigned long long* ent = p.sbuf + (int64_t)bh * (kMaxItemsPerBh * 4 * G);
    if (t < 4 * G) {
      const float x = L.own[t / G][t % G];
      st_agent_u64(ent + item * 4 * G + t, ((unsigned long long)tag << 32) | __float_as_uint(x));
      L.part[item][t / G][t % G] = x;
    }
    if (t == 0) L.missing = 0u;
    __syncthreads();
    const unsigned long long t0 = clock_100mhz();
    bool miss = false;
    for (int k = t; k < n_it * 4 * G; k += kFinThreads) {
      const int i = k / (4 * G);
      if (i == item) continue;
      unsigned long long v = ld_agent_u64(ent + k);
      while ((u32)(v >> 32) != tag && (long long)(clock_100mhz() - t0) <= p.wait_ticks) {
        __builtin_amdgcn_s_sleep(1);
        v = ld_agent_u64(ent + k);
      }
      if ((u32)(v >> 32) == tag) L.part[i][(k % (4 * G)) / G][k % G] = __uint_as_float((u32)v);
      else miss = true;
    }
    if (miss) L.missing = 1u;
    __syncthreads();
    if (L.missing) {  // a partner's partial missed the bound: every other item's here
      if (t == 0) note_wait_fallback();
      for (int i = 0; i < n_it; ++i) {
        if (i == item) continue;
        item_stats(i);
        __syncthreads();
        item_partial(cond_item_blocks(i, nb, n_it));
        if (t < 4 * G) L.part[i][t / G][t % G] = L.own[t / G][t % G];
        __syncthreads();
      }
      item_stats(item);  // the own blocks' s and delta again, for the routing
      __syncthreads();
    }
  } else if (t < 4 * G) {
    L.part[0][t / G][t % G] = L.own[t / G][t % G];
  }
  if constexpr (!MASK) __syncthreads();

  // ---- step 3: the row's globals, the items' partials merged in item order (wave w
  // takes (value, row) pairs w, w + 8, ...: lanes are items)
  for (int pr = wave; !MASK && pr < 2 * G; pr += kFinWaves) {
    const int v = pr / G, g = pr - v * G;
    const float mi = lane < n_it ? L.part[lane][2 * v][g] : kNegInf;
    const float li = lane < n_it ? L.part[lane][2 * v + 1][g] : 0.f;
    const float M = wave_max(mi);
    const float S = wave_sum(mi == kNegInf ? 0.f : li * __expf(mi - M));
    if (lane == 0) {
      L.glob[2 * v][g] = M;
      L.glob[2 * v + 1][g] = S;
    }
  }
  if constexpr (!MASK) __syncthreads();

  // routing of this thread's block: the group mean of the condition against eps (or
  // the caller's mask)
  const int cnt = mine ? cnt_ld : 0;  // this thread's block's valid tokens (0: none)
  const float b_c = mine ? bc_ld : 0.f;
  const bool act = cnt > 0;
  const float logc = __logf((float)max(cnt, 1));
  float zr[G];
  float mean = 0.f;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    zr[g] = act ? L.s[g][t] + logc : kNegInf;
    if (!MASK && act)
      mean += condition_value(L.dl[g][t], zr[g], L.glob[0][g], 1.f / L.glob[1][g], L.glob[2][g], 1.f / L.glob[3][g],
                              b_c, b_all, p.c_mass_exp);
  }
  mean /= (float)G;
  const bool sel = act && (MASK ? mask_ld : mean > p.c_eps);
  // external mask: the representatives' own largest logit per query row (no row
  // globals): the waves' maxima through LDS
  if constexpr (MASK) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float mx = wave_max(sel ? kNegInf : zr[g]);
      if (lane == 0) L.part[wave][0][g] = mx;
    }
    __syncthreads();
    if (t < G) {
      float mx = kNegInf;
#pragma unroll
      for (int w = 0; w < kFinWaves; ++w) mx = fmaxf(mx, L.part[w][0][t]);
      L.glob[0][t] = mx;
    }
    __syncthreads();
  }
  if (!MASK && p.c_selected && mine) {
#pragma unroll
    for (int g = 0; g < G; ++g)
      p.c_selected[((int64_t)b * p.n_kv_heads * G + h * G + g) * nb + jt] = sel ? 1 : 0;
  }
  const unsigned long long bal = __ballot(sel);
  if (lane == 0) L.wcnt[wave] = __popcll(bal);
  // representatives (the unselected blocks that exist, logit z): weights e^(z - z_m)
  // against the row's largest z, which bounds every representative logit (so no
  // reduction of their own maximum); L.s becomes the weight table (0 for selected,
  // empty or out-of-range blocks)
#pragma unroll
  for (int g = 0; g < G; ++g) L.s[g][t] = (sel || zr[g] == kNegInf) ? 0.f : __expf(zr[g] - L.glob[0][g]);
  __syncthreads();
  int off = 0, n_sel = 0;
#pragma unroll
  for (int w = 0; w < kFinWaves; ++w) {
    off += w < wave ? L.wcnt[w] : 0;
    n_sel += L.wcnt[w];
  }
  if (sel) L.list[off + __popcll(bal & ((1ull << lane) - 1ull))] = list_entry(jt, cnt);
  // the weights' sum per query row: wave g (in-lane sums, then one wave sum)
  if (wave < G) {
    float ls = 0.f;
    for (int j = lane; j < m; j += 64) ls += L.s[wave][j];
    ls = wave_sum(ls);
    if (lane == 0) {
      L.rep_l[wave] = ls;
      // the finalize's log2 domain; no weight at all: an empty partial
      L.rep_m[wave] = (ls == 0.f || L.glob[0][wave] == kNegInf) ? kNegInf : L.glob[0][wave] * kLog2e;
    }
  }
  // weighted v_bar: local block 32 step + 4 w + r on the 16 lanes of row r of wave w,
  // weight and value rounded to bf16 for bf16 caches
  float acc[G][DPL];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < DPL; ++e) acc[g][e] = 0.f;
  const int nst = (m + 31) / 32;
  for (int s0 = 0; s0 < nst; s0 += 2) {
    SumRow<DPL, SBF> vr[2];
    if (kEarlyV && s0 == 0) {
      vr[0] = vpre[0];
      vr[1] = vpre[kEarlyV ? 1 : 0];
    } else {
#pragma unroll
      for (int u = 0; u < 2; ++u)
        vr[u].load(p.c_vbar, (vrow + item + min(32 * (s0 + u) + 4 * wave + r, m - 1) * n_it) * D + c16 * DPL, vbf);
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      if (s0 + u >= nst) break;
      const int jl = 32 * (s0 + u) + 4 * wave + r;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float bw = round_if(L.s[g][jl], p.c_rep_bf16);
#pragma unroll
        for (int e = 0; e < DPL; ++e) acc[g][e] = fmaf(bw, round_if(vr[u].at(e, vbf), !vbf && p.c_rep_bf16), acc[g][e]);
      }
    }
  }
  // (each wave's accumulator stays in LDS; the fold after the stream, behind its
  // barrier, sums the waves')
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < DPL; ++e) {
      const float v = rows_sum(acc[g][e]);
      if (r == 0) L.rep_acc[wave][g * D + c16 * DPL + e] = v;
    }
  __syncthreads();  // the list entries, for the unit ranges
  return n_sel;
}

template <int D, int G>
__device__ __forceinline__ int cond_fused_prologue(const DecodeParams& p, CondLds<D, G>& L, int b, int h, int item,
                                                   int n_it, u32 row_epoch) {
  if (p.c_mask) {
    if (p.c_kbar_bf16 && p.c_vbar_bf16) return cond_fused_prologue_t<D, G, 1, true>(p, L, b, h, item, n_it, row_epoch);
    return cond_fused_prologue_t<D, G, 0, true>(p, L, b, h, item, n_it, row_epoch);
  }
  if (p.c_kbar_bf16 && p.c_bounds_bf16 && p.c_vbar_bf16)
    return cond_fused_prologue_t<D, G, 1, false>(p, L, b, h, item, n_it, row_epoch);
  return cond_fused_prologue_t<D, G, 0, false>(p, L, b, h, item, n_it, row_epoch);
}

}  // namespace ia
