// Paged decode attention for gfx950: the selected-block finalize (sparse) and
// the dense fallback share one kernel.
//
// Work decomposition
//   grid = (items, Hkv, batch); one 256-thread workgroup (4 waves) per split-K
//   item of one (sequence, kv head).  An item is a run of "units": selected
//   blocks (sparse) or 128-token tiles (dense).  Waves take units round-robin
//   and keep their own online-softmax state; the workgroup folds its four
//   waves in LDS and writes one (m, l, acc) partial.  The last workgroup of a
//   (sequence, kv head) -- found with a device-scope counter -- merges the
//   partials and writes the output row block, then re-arms the counter.
//
// Lane layout (head_dim D, DPL = D/16 dims per lane)
//   lane = 16*r + c.  A 16-token subtile (always inside one page) is read as
//   four steps i = 0..3; in step i, row r holds token 4i + r and lane c holds
//   dims [c*DPL, (c+1)*DPL).  Each step is one contiguous 4-token load per
//   wave (1 KiB for bf16 D=128).  Q.K partial sums for the 4 steps x G query
//   rows are reduce-scattered over the 16-lane row with DPP, leaving each lane
//   the complete score of one (token, query row) pair; V is read with the
//   same layout and weighted by softmax weights exchanged through LDS.
//
// Numerics follow the reference's fused kernel (CBT/page_attention.py):
//   bf16 K/V: scores = bf16(q) . K in fp32 (v_dot2_f32_bf16), fp32 online
//   softmax, weights rounded to bf16 for the P.V product (:248-252), fp32
//   normaliser (:253).  fp32 K/V: everything in fp32.  fp8 K/V: codes are
//   widened to fp32, the per-(page, head) scale multiplies the score and the
//   weight.
#include "ia_common.hpp"

namespace ia {

struct KvBf16 {
  static constexpr int kBytes = 2;
};
struct KvF32 {
  static constexpr int kBytes = 4;
};
struct KvFp8 {
  static constexpr int kBytes = 1;
};

template <int NWD>
__device__ __forceinline__ void load_words(const void* p, u32* w) {
  if constexpr (NWD == 8) {
    const uint4 a = reinterpret_cast<const uint4*>(p)[0];
    const uint4 b = reinterpret_cast<const uint4*>(p)[1];
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
    w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
  } else if constexpr (NWD == 4) {
    const uint4 a = *reinterpret_cast<const uint4*>(p);
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
  } else if constexpr (NWD == 2) {
    const uint2 a = *reinterpret_cast<const uint2*>(p);
    w[0] = a.x; w[1] = a.y;
  } else {
    w[0] = *reinterpret_cast<const u32*>(p);
  }
}

struct DecodeParams {
  const void* q;
  int64_t q_batch_stride, q_row_stride;
  ia_paged_kv kv;
  const int32_t* seq_lens;
  const int32_t* idx;  // sparse only
  const int32_t* n_sel;
  int32_t k_cap;
  int32_t block_size;  // sparse: tokens per selected block
  int32_t upi;         // units per item
  int32_t max_items;
  int32_t n_kv_heads;
  float scale_log2;    // softmax scale * log2(e)
  int32_t q_f32;       // q is fp32 (else bf16)
  int32_t out_f32;     // out is fp32 (else bf16)
  void* out;
  u32* counters;       // [batch * Hkv]
  float* part_ml;      // [batch*Hkv, max_items, G, 2]
  float* part_acc;     // [batch*Hkv, max_items, G, D]
};

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;

template <int D, int G, int NSUB, typename KV, bool SPARSE>
__global__ __launch_bounds__(kThreads) void ia_condition_block_paged_finalize(DecodeParams p) {
  constexpr int DPL = D / 16;
  constexpr int NWD = DPL * KV::kBytes / 4;
  constexpr int NV = 4 * G;
  constexpr int KG = NV >= 16 ? NV / 16 : 1;
  constexpr int TILE = NSUB * 16;
  constexpr bool kBf16 = KV::kBytes == 2;
  constexpr bool kFp8 = KV::kBytes == 1;

  __shared__ float p_lds[kWaves][TILE * G];
  __shared__ float alpha_lds[kWaves][G];
  __shared__ float wacc_lds[kWaves][G * D];
  __shared__ float wm_lds[kWaves][G];
  __shared__ float wl_lds[kWaves][G];
  __shared__ int last_flag;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c16 = lane & 15;
  const int r = lane >> 4;
  const int item = blockIdx.x;
  const int h = blockIdx.y;
  const int b = blockIdx.z;
  const int bh = b * p.n_kv_heads + h;

  const int seq_len = max(p.seq_lens[b], 0);
  int n_units;
  if constexpr (SPARSE) {
    n_units = min(max(p.n_sel[bh], 0), p.k_cap);
  } else {
    n_units = (seq_len + TILE - 1) / TILE;
  }
  const int n_items = max(1, min(p.max_items, (n_units + p.upi - 1) / p.upi));
  if (item >= n_items) return;

  // ---- query rows of this kv head, in the lane's dim slice
  constexpr int QW = kBf16 ? DPL / 2 : DPL;  // bf16 pairs or floats
  u32 qw[G][QW];
  {
    const int d0 = c16 * DPL;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int64_t row = (int64_t)b * p.q_batch_stride + (int64_t)(h * G + g) * p.q_row_stride;
      float qf[DPL];
      if (p.q_f32) {
        const float* qp = reinterpret_cast<const float*>(p.q) + row + d0;
#pragma unroll
        for (int e = 0; e < DPL; ++e) qf[e] = qp[e];
      } else {
        const unsigned short* qp = reinterpret_cast<const unsigned short*>(p.q) + row + d0;
#pragma unroll
        for (int e = 0; e < DPL; ++e) qf[e] = __uint_as_float((u32)qp[e] << 16);
      }
      if constexpr (kBf16) {
#pragma unroll
        for (int e = 0; e < DPL / 2; ++e) qw[g][e] = pack_bf16x2(qf[2 * e], qf[2 * e + 1]);
      } else {
#pragma unroll
        for (int e = 0; e < DPL; ++e) qw[g][e] = __float_as_uint(qf[e]);
      }
    }
  }

  const ia_paged_kv& kv = p.kv;
  const int page_size = kv.page_size;
  const int32_t* bt_row = kv.block_table ? kv.block_table + (int64_t)b * kv.bt_stride : nullptr;
  const char* kbase = reinterpret_cast<const char*>(kv.k);
  const char* vbase = reinterpret_cast<const char*>(kv.v);

  // Page of a (16-aligned) logical token; -1 when the table entry is out of range.
  auto page_of = [&](int tok) -> int64_t {
    const int lp = tok / page_size;
    if (bt_row && lp >= kv.bt_cols) return (int64_t)-1;
    const int64_t pg = bt_row ? (int64_t)bt_row[lp] : (int64_t)lp;
    return (pg >= 0 && pg < kv.n_pages) ? pg : (int64_t)-1;
  };

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

  float* my_p = p_lds[wave];

  auto process_tile = [&](int t0, int t_end) {
    // ---------------- scores
    float s[NSUB][KG];
#pragma unroll
    for (int sub = 0; sub < NSUB; ++sub) {
      const int ts = t0 + 16 * sub;
      int64_t pg = -1;
      if (ts < t_end) pg = page_of(ts);
      if (pg < 0) {
#pragma unroll
        for (int k = 0; k < KG; ++k) s[sub][k] = kNegInf;
        continue;
      }
      const int in_page = ts % page_size;
      const char* rowp = kbase + (pg * kv.k_page_stride + (int64_t)h * kv.k_head_stride +
                                  (int64_t)in_page * kv.k_token_stride) * KV::kBytes;
      u32 kw[4][NWD];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int tok = ts + 4 * i + r;
        if (tok < t_end) {
          load_words<NWD>(rowp + ((int64_t)(4 * i + r) * kv.k_token_stride + c16 * DPL) * KV::kBytes,
                          kw[i]);
        } else {
#pragma unroll
          for (int w = 0; w < NWD; ++w) kw[i][w] = 0u;
        }
      }
      float part[NV];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (kBf16) {
#pragma unroll
          for (int g = 0; g < G; ++g) {
            float a = 0.f;
#pragma unroll
            for (int w = 0; w < NWD; ++w)
              a = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(qw[g][w]), as_bf16x2(kw[i][w]), a, false);
            part[i * G + g] = a;
          }
        } else {
          float kf[DPL];
          if constexpr (kFp8) {
#pragma unroll
            for (int w = 0; w < NWD; ++w) fp8x4_to_f32(kw[i][w], kf + 4 * w);
          } else {
#pragma unroll
            for (int e = 0; e < DPL; ++e) kf[e] = __uint_as_float(kw[i][e]);
          }
#pragma unroll
          for (int g = 0; g < G; ++g) {
            float a = 0.f;
#pragma unroll
            for (int e = 0; e < DPL; ++e) a = fmaf(__uint_as_float(qw[g][e]), kf[e], a);
            part[i * G + g] = a;
          }
        }
      }
      reduce_scatter16<NV>(part, lane);
      float sc = p.scale_log2;
      if constexpr (kFp8) sc *= kv.k_scale[pg * kv.scale_page_stride + h];
      const bool valid = ts + 4 * my_step + r < t_end;
#pragma unroll
      for (int k = 0; k < KG; ++k) s[sub][k] = valid ? part[k] * sc : kNegInf;
    }

    // ---------------- online softmax update (per query row g)
    float alpha[KG];
#pragma unroll
    for (int k = 0; k < KG; ++k) {
      float mt = s[0][k];
#pragma unroll
      for (int sub = 1; sub < NSUB; ++sub) mt = fmaxf(mt, s[sub][k]);
      mt = fmaxf(mt, dpp<kDppRowRor4>(mt));
      mt = fmaxf(mt, dpp<kDppRowRor8>(mt));
      if constexpr (G < 4) {
        mt = fmaxf(mt, dpp<kDppXor1>(mt));
        mt = fmaxf(mt, dpp<kDppXor2>(mt));
      }
      mt = fmaxf(mt, shfl_xor_f(mt, 16));
      mt = fmaxf(mt, shfl_xor_f(mt, 32));
      const float m_new = fmaxf(m_run[k], mt);
      alpha[k] = (m_new == kNegInf) ? 1.f : exp2f(m_run[k] - m_new);
      m_run[k] = m_new;
      float lsum = 0.f;
#pragma unroll
      for (int sub = 0; sub < NSUB; ++sub) {
        const float pv = (s[sub][k] == kNegInf) ? 0.f : exp2f(s[sub][k] - m_new);
        lsum += pv;
        my_p[(16 * sub + 4 * my_step + r) * G + my_g[k]] = pv;
      }
      l_run[k] = l_run[k] * alpha[k] + (l_owner ? lsum : 0.f);
      alpha_lds[wave][my_g[k]] = alpha[k];
    }
    wave_lds_sync();
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float a = alpha_lds[wave][g];
#pragma unroll
      for (int e = 0; e < DPL; ++e) acc[g][e] *= a;
    }

    // ---------------- weighted values
#pragma unroll
    for (int sub = 0; sub < NSUB; ++sub) {
      const int ts = t0 + 16 * sub;
      if (ts >= t_end) break;
      const int64_t pg = page_of(ts);
      if (pg < 0) continue;
      const int in_page = ts % page_size;
      const char* rowp = vbase + (pg * kv.v_page_stride + (int64_t)h * kv.v_head_stride +
                                  (int64_t)in_page * kv.v_token_stride) * KV::kBytes;
      float vsc = 1.f;
      if constexpr (kFp8) vsc = kv.v_scale[pg * kv.scale_page_stride + h];
      if constexpr (kBf16) {
#pragma unroll
        for (int pr = 0; pr < 2; ++pr) {
          const int i1 = 2 * pr, i2 = 2 * pr + 1;
          const int tl1 = 4 * i1 + r, tl2 = 4 * i2 + r;
          u32 w1[NWD], w2[NWD];
          if (ts + tl1 < t_end) {
            load_words<NWD>(rowp + ((int64_t)tl1 * kv.v_token_stride + c16 * DPL) * 2, w1);
          } else {
#pragma unroll
            for (int w = 0; w < NWD; ++w) w1[w] = 0u;
          }
          if (ts + tl2 < t_end) {
            load_words<NWD>(rowp + ((int64_t)tl2 * kv.v_token_stride + c16 * DPL) * 2, w2);
          } else {
#pragma unroll
            for (int w = 0; w < NWD; ++w) w2[w] = 0u;
          }
          const float* p1 = my_p + (16 * sub + tl1) * G;
          const float* p2 = my_p + (16 * sub + tl2) * G;
          u32 pp[G];
#pragma unroll
          for (int g = 0; g < G; ++g) pp[g] = pack_bf16x2(p1[g], p2[g]);
#pragma unroll
          for (int w = 0; w < NWD; ++w) {
            const u32 lo = __builtin_amdgcn_perm(w2[w], w1[w], 0x05040100u);
            const u32 hi = __builtin_amdgcn_perm(w2[w], w1[w], 0x07060302u);
#pragma unroll
            for (int g = 0; g < G; ++g) {
              acc[g][2 * w] = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(pp[g]), as_bf16x2(lo), acc[g][2 * w], false);
              acc[g][2 * w + 1] = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(pp[g]), as_bf16x2(hi), acc[g][2 * w + 1], false);
            }
          }
        }
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int tl = 4 * i + r;
          u32 w1[NWD];
          if (ts + tl < t_end) {
            load_words<NWD>(rowp + ((int64_t)tl * kv.v_token_stride + c16 * DPL) * KV::kBytes, w1);
          } else {
#pragma unroll
            for (int w = 0; w < NWD; ++w) w1[w] = 0u;
          }
          float vf[DPL];
          if constexpr (kFp8) {
#pragma unroll
            for (int w = 0; w < NWD; ++w) fp8x4_to_f32(w1[w], vf + 4 * w);
          } else {
#pragma unroll
            for (int e = 0; e < DPL; ++e) vf[e] = __uint_as_float(w1[e]);
          }
          const float* pr = my_p + (16 * sub + tl) * G;
#pragma unroll
          for (int g = 0; g < G; ++g) {
            const float pw = pr[g] * vsc;
#pragma unroll
            for (int e = 0; e < DPL; ++e) acc[g][e] = fmaf(pw, vf[e], acc[g][e]);
          }
        }
      }
    }
    wave_lds_sync();
  };

  // ---- this wave's units
  const int u_begin = item * p.upi;
  const int u_end = min(n_units, u_begin + p.upi);
  for (int u = u_begin + wave; u < u_end; u += kWaves) {
    int tok_lo, tok_hi;
    if constexpr (SPARSE) {
      const int j = p.idx[(int64_t)bh * p.k_cap + u];
      if (j < 0) continue;
      tok_lo = j * p.block_size;
      if (tok_lo >= seq_len) continue;
      tok_hi = min(tok_lo + p.block_size, seq_len);
    } else {
      tok_lo = u * TILE;
      tok_hi = min(tok_lo + TILE, seq_len);
    }
    for (int t0 = tok_lo; t0 < tok_hi; t0 += TILE) process_tile(t0, min(t0 + TILE, tok_hi));
  }

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
  for (int k = 0; k < KG; ++k) {
    float v = l_run[k];
    v += dpp<kDppRowRor4>(v);
    v += dpp<kDppRowRor8>(v);
    if constexpr (G < 4) {
      v += dpp<kDppXor1>(v);
      v += dpp<kDppXor2>(v);
    }
    v += shfl_xor_f(v, 16);
    v += shfl_xor_f(v, 32);
    l_run[k] = v;
  }
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
  __syncthreads();

  // ---- fold the four waves; one (m, l, acc) per item
  constexpr int PER_T = (G * D + kThreads - 1) / kThreads;
  float it_acc[PER_T];
  float it_m[PER_T], it_l[PER_T];
#pragma unroll
  for (int t = 0; t < PER_T; ++t) {
    const int o = threadIdx.x + t * kThreads;
    it_acc[t] = 0.f;
    it_m[t] = kNegInf;
    it_l[t] = 0.f;
    if (o < G * D) {
      const int g = o / D;
      float M = kNegInf;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) M = fmaxf(M, wm_lds[w][g]);
      float a = 0.f, l = 0.f;
      if (M != kNegInf) {
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
          const float mw = wm_lds[w][g];
          const float f = (mw == kNegInf) ? 0.f : exp2f(mw - M);
          a += f * wacc_lds[w][o];
          l += f * wl_lds[w][g];
        }
      }
      it_acc[t] = a;
      it_m[t] = M;
      it_l[t] = l;
    }
  }

  auto store_out = [&](int o, float v) {
    const int g = o / D, d = o % D;
    const int64_t off = ((int64_t)b * (p.n_kv_heads * G) + h * G + g) * D + d;
    if (p.out_f32) {
      reinterpret_cast<float*>(p.out)[off] = v;
    } else {
      reinterpret_cast<unsigned short*>(p.out)[off] = f32_to_bf16_bits(v);
    }
  };

  if (n_items == 1) {
#pragma unroll
    for (int t = 0; t < PER_T; ++t) {
      const int o = threadIdx.x + t * kThreads;
      if (o < G * D) store_out(o, it_acc[t] / fmaxf(it_l[t], 1e-30f));
    }
    return;
  }

  const int64_t pbase = (int64_t)bh * p.max_items;
#pragma unroll
  for (int t = 0; t < PER_T; ++t) {
    const int o = threadIdx.x + t * kThreads;
    if (o < G * D) {
      p.part_acc[(pbase + item) * (G * D) + o] = it_acc[t];
      if (o % D == 0) {
        const int g = o / D;
        p.part_ml[((pbase + item) * G + g) * 2 + 0] = it_m[t];
        p.part_ml[((pbase + item) * G + g) * 2 + 1] = it_l[t];
      }
    }
  }
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const u32 prev = atomicAdd(&p.counters[bh], 1u);
    last_flag = (prev == (u32)(n_items - 1));
  }
  __syncthreads();
  if (!last_flag) return;
  __threadfence();

  // ---- last workgroup of this (sequence, kv head): merge the split-K partials
#pragma unroll
  for (int t = 0; t < PER_T; ++t) {
    const int o = threadIdx.x + t * kThreads;
    if (o < G * D) {
      const int g = o / D;
      float M = kNegInf;
      for (int c = 0; c < n_items; ++c) M = fmaxf(M, p.part_ml[((pbase + c) * G + g) * 2]);
      float a = 0.f, l = 0.f;
      if (M != kNegInf) {
        for (int c = 0; c < n_items; ++c) {
          const float mc = p.part_ml[((pbase + c) * G + g) * 2];
          const float f = (mc == kNegInf) ? 0.f : exp2f(mc - M);
          a += f * p.part_acc[(pbase + c) * (G * D) + o];
          l += f * p.part_ml[((pbase + c) * G + g) * 2 + 1];
        }
      }
      store_out(o, a / fmaxf(l, 1e-30f));
    }
  }
  if (threadIdx.x == 0) p.counters[bh] = 0u;
}

// ------------------------------------------------------------------ host side

namespace {

constexpr int kDenseTile = 128;
constexpr int kTargetWgs = 1024;

int pick_upi(int64_t total_units, int64_t units_per_bh_cap) {
  int64_t upi = (total_units + kTargetWgs - 1) / kTargetWgs;
  upi = std::max<int64_t>(upi, kWaves);
  upi = (upi + kWaves - 1) / kWaves * kWaves;
  if (units_per_bh_cap > 0) upi = std::min<int64_t>(upi, std::max<int64_t>(units_per_bh_cap, 1));
  return (int)std::max<int64_t>(upi, 1);
}

int sparse_upi(int batch, int hkv, int k_cap) { return pick_upi((int64_t)batch * hkv * k_cap, k_cap); }

int dense_upi(int batch, int hkv, int max_seq_len) {
  const int64_t tiles = (std::max(max_seq_len, 0) + kDenseTile - 1) / kDenseTile;
  return pick_upi((int64_t)batch * hkv * tiles, tiles);
}

size_t decode_ws_size(int batch, int hkv, int group, int d, int max_items) {
  const size_t bh = (size_t)batch * hkv;
  return align_up(bh * 4, 256) + align_up(bh * max_items * group * 2 * 4, 256) +
         bh * max_items * group * d * 4;
}

int check_kv(const ia_paged_kv* kv, int d) {
  if (!kv || !kv->k || !kv->v) return fail(IA_ERR_INVALID, "kv pool pointers must be non-null");
  if (kv->dtype != IA_F32 && kv->dtype != IA_BF16 && kv->dtype != IA_FP8_E4M3)
    return fail(IA_ERR_INVALID, "kv dtype must be IA_F32, IA_BF16 or IA_FP8_E4M3");
  if (kv->page_size <= 0 || kv->page_size % 16 != 0)
    return fail(IA_ERR_INVALID, "page_size must be a positive multiple of 16");
  const int eb = kv->dtype == IA_F32 ? 4 : (kv->dtype == IA_BF16 ? 2 : 1);
  const int64_t strides[6] = {kv->k_page_stride, kv->k_head_stride, kv->k_token_stride,
                              kv->v_page_stride, kv->v_head_stride, kv->v_token_stride};
  for (int64_t s : strides)
    if (s < 0 || (s * eb) % 16 != 0)
      return fail(IA_ERR_INVALID, "kv strides must be non-negative and 16-byte multiples");
  if (kv->k_token_stride < d || kv->v_token_stride < d)
    return fail(IA_ERR_INVALID, "kv token stride must be at least head_dim");
  if ((reinterpret_cast<uintptr_t>(kv->k) | reinterpret_cast<uintptr_t>(kv->v)) % 16 != 0)
    return fail(IA_ERR_INVALID, "kv base pointers must be 16-byte aligned");
  if (kv->dtype == IA_FP8_E4M3 && (!kv->k_scale || !kv->v_scale))
    return fail(IA_ERR_INVALID, "fp8 kv needs k_scale and v_scale");
  if (kv->block_table && (kv->bt_stride <= 0 || kv->bt_cols < 0 || kv->bt_cols > kv->bt_stride))
    return fail(IA_ERR_INVALID, "block table needs 0 <= bt_cols <= bt_stride and bt_stride > 0");
  return IA_OK;
}

int check_shape(const ia_decode_shape* s) {
  if (!s) return fail(IA_ERR_INVALID, "shape is null");
  if (s->batch < 0 || s->n_kv_heads <= 0 || s->n_q_heads <= 0)
    return fail(IA_ERR_INVALID, "batch must be >= 0 and head counts positive");
  if (s->n_q_heads % s->n_kv_heads != 0)
    return fail(IA_ERR_INVALID, "n_q_heads must be a multiple of n_kv_heads (grouped query attention)");
  const int g = s->n_q_heads / s->n_kv_heads;
  if (g != 1 && g != 2 && g != 4 && g != 8)
    return fail(IA_ERR_UNSUPPORTED, "GQA group size must be 1, 2, 4 or 8");
  if (s->head_dim != 64 && s->head_dim != 128) return fail(IA_ERR_UNSUPPORTED, "head_dim must be 64 or 128");
  if (s->q_dtype != IA_F32 && s->q_dtype != IA_BF16) return fail(IA_ERR_INVALID, "q dtype must be IA_F32 or IA_BF16");
  return IA_OK;
}

template <int D, int G, int NSUB, typename KV, bool SPARSE>
void launch_one(const DecodeParams& p, dim3 grid, hipStream_t st) {
  hipLaunchKernelGGL((ia_condition_block_paged_finalize<D, G, NSUB, KV, SPARSE>), grid, dim3(kThreads), 0, st, p);
}

template <int D, int G, int NSUB, bool SPARSE>
int dispatch_types(const DecodeParams& p, int kv_dtype, dim3 grid, hipStream_t st) {
  if (kv_dtype == IA_BF16) {
    launch_one<D, G, NSUB, KvBf16, SPARSE>(p, grid, st);
  } else if (kv_dtype == IA_F32) {
    if (!p.q_f32) return fail(IA_ERR_UNSUPPORTED, "fp32 kv needs fp32 q");
    launch_one<D, G, NSUB, KvF32, SPARSE>(p, grid, st);
  } else {
    if (p.q_f32) return fail(IA_ERR_UNSUPPORTED, "fp8 kv needs bf16 q");
    launch_one<D, G, NSUB, KvFp8, SPARSE>(p, grid, st);
  }
  return check_launch("paged decode");
}

template <int D, int G, bool SPARSE>
int dispatch_nsub(const DecodeParams& p, int nsub, int kv_dtype, dim3 grid, hipStream_t st) {
  if constexpr (!SPARSE) {
    return dispatch_types<D, G, 8, SPARSE>(p, kv_dtype, grid, st);
  } else {
    switch (nsub) {
      case 1: return dispatch_types<D, G, 1, SPARSE>(p, kv_dtype, grid, st);
      case 2: return dispatch_types<D, G, 2, SPARSE>(p, kv_dtype, grid, st);
      case 4: return dispatch_types<D, G, 4, SPARSE>(p, kv_dtype, grid, st);
      case 8: return dispatch_types<D, G, 8, SPARSE>(p, kv_dtype, grid, st);
    }
  }
  return fail(IA_ERR_UNSUPPORTED, "tile size");
}

template <bool SPARSE>
int dispatch(const DecodeParams& p, int d, int g, int nsub, int kv_dtype, dim3 grid, hipStream_t st) {
#define IA_DG(DD, GG) \
  if (d == DD && g == GG) return dispatch_nsub<DD, GG, SPARSE>(p, nsub, kv_dtype, grid, st);
  IA_DG(128, 4) IA_DG(128, 8) IA_DG(128, 2) IA_DG(128, 1)
  IA_DG(64, 4) IA_DG(64, 8) IA_DG(64, 2) IA_DG(64, 1)
#undef IA_DG
  return fail(IA_ERR_UNSUPPORTED, "head_dim / group combination");
}

int run_decode(bool sparse, const ia_decode_shape* shape, const void* q, const ia_paged_kv* kv,
               const int32_t* seq_lens, int32_t block_size, const int32_t* idx, int32_t k_cap,
               const int32_t* n_sel, int32_t max_seq_len, float scale, void* out, int32_t out_dtype,
               void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_shape(shape);
  if (rc) return rc;
  rc = check_kv(kv, shape->head_dim);
  if (rc) return rc;
  if (!q || !out || !seq_lens) return fail(IA_ERR_INVALID, "q, out and seq_lens must be non-null");
  if (out_dtype != IA_F32 && out_dtype != IA_BF16) return fail(IA_ERR_INVALID, "out dtype must be IA_F32 or IA_BF16");
  if (!(scale > 0.f) || !std::isfinite(scale)) return fail(IA_ERR_INVALID, "scale must be positive and finite");
  const int G = shape->n_q_heads / shape->n_kv_heads;
  const int D = shape->head_dim;
  int nsub = 8, upi = 1, max_items = 1;
  if (sparse) {
    if (!idx || !n_sel) return fail(IA_ERR_INVALID, "idx and n_sel must be non-null");
    if (block_size <= 0 || block_size % 16 != 0) return fail(IA_ERR_INVALID, "block_size must be a positive multiple of 16");
    if (k_cap <= 0) return fail(IA_ERR_INVALID, "k_cap must be positive");
    nsub = std::min(block_size, 128) / 16;
    if (nsub != 1 && nsub != 2 && nsub != 4 && nsub != 8)
      return fail(IA_ERR_UNSUPPORTED, "block_size below 128 must be 16, 32 or 64");
    upi = sparse_upi(shape->batch, shape->n_kv_heads, k_cap);
    max_items = (k_cap + upi - 1) / upi;
  } else {
    if (max_seq_len < 0) return fail(IA_ERR_INVALID, "max_seq_len must be >= 0");
    upi = dense_upi(shape->batch, shape->n_kv_heads, max_seq_len);
    const int tiles = (max_seq_len + kDenseTile - 1) / kDenseTile;
    max_items = std::max(1, (tiles + upi - 1) / upi);
  }
  const size_t need = decode_ws_size(shape->batch, shape->n_kv_heads, G, D, max_items);
  if (max_items > 1 && (!workspace || workspace_bytes < need))
    return fail(IA_ERR_WORKSPACE, "workspace too small: need " + std::to_string(need) + " bytes");
  if (shape->batch == 0) return IA_OK;

  DecodeParams p{};
  p.q = q;
  p.q_batch_stride = shape->q_batch_stride;
  p.q_row_stride = shape->q_row_stride;
  p.kv = *kv;
  p.seq_lens = seq_lens;
  p.idx = idx;
  p.n_sel = n_sel;
  p.k_cap = k_cap;
  p.block_size = block_size;
  p.upi = upi;
  p.max_items = max_items;
  p.n_kv_heads = shape->n_kv_heads;
  p.scale_log2 = scale * kLog2e;
  p.out = out;
  char* ws = reinterpret_cast<char*>(workspace);
  const size_t bh = (size_t)shape->batch * shape->n_kv_heads;
  if (ws) {
    p.counters = reinterpret_cast<u32*>(ws);
    p.part_ml = reinterpret_cast<float*>(ws + align_up(bh * 4, 256));
    p.part_acc = reinterpret_cast<float*>(ws + align_up(bh * 4, 256) + align_up(bh * max_items * G * 2 * 4, 256));
  }
  dim3 grid(max_items, shape->n_kv_heads, shape->batch);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  p.q_f32 = shape->q_dtype == IA_F32;
  p.out_f32 = out_dtype == IA_F32;
  if (sparse) return dispatch<true>(p, D, G, nsub, kv->dtype, grid, st);
  return dispatch<false>(p, D, G, 8, kv->dtype, grid, st);
}

}  // namespace
}  // namespace ia

extern "C" {

size_t ia_paged_decode_workspace_size(int32_t batch, int32_t n_kv_heads, int32_t group, int32_t head_dim,
                                      int32_t max_items) {
  return ia::decode_ws_size(batch, n_kv_heads, group, head_dim, std::max(max_items, 1));
}

int32_t ia_sparse_max_items(int32_t batch, int32_t n_kv_heads, int32_t k_cap) {
  const int upi = ia::sparse_upi(batch, n_kv_heads, k_cap);
  return std::max(1, (k_cap + upi - 1) / upi);
}

int32_t ia_dense_max_items(int32_t batch, int32_t n_kv_heads, int32_t max_seq_len) {
  const int upi = ia::dense_upi(batch, n_kv_heads, max_seq_len);
  const int tiles = (std::max(max_seq_len, 0) + ia::kDenseTile - 1) / ia::kDenseTile;
  return std::max(1, (tiles + upi - 1) / upi);
}

int ia_sparse_paged_decode(const ia_decode_shape* shape, const void* q, const ia_paged_kv* kv,
                           const int32_t* seq_lens, int32_t block_size, const int32_t* idx, int32_t k_cap,
                           const int32_t* n_sel, float scale, void* out, int32_t out_dtype, void* workspace,
                           size_t workspace_bytes, void* stream) {
  return ia::run_decode(true, shape, q, kv, seq_lens, block_size, idx, k_cap, n_sel, 0, scale, out, out_dtype,
                        workspace, workspace_bytes, stream);
}

int ia_paged_decode(const ia_decode_shape* shape, const void* q, const ia_paged_kv* kv, const int32_t* seq_lens,
                    int32_t max_seq_len, float scale, void* out, int32_t out_dtype, void* workspace,
                    size_t workspace_bytes, void* stream) {
  return ia::run_decode(false, shape, q, kv, seq_lens, 0, nullptr, 0, nullptr, max_seq_len, scale, out, out_dtype,
                        workspace, workspace_bytes, stream);
}

}  // extern "C"
