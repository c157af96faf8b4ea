// Per-block summaries of a paged K/V pool for gfx950 (the paged form of
// _build_prompt_blocks, CBT/core.py:449-500).
//
//   grid = (ceil(nb_max / 4), Hkv, batch), 256 threads; wave w summarises
//   logical block j = 4*blockIdx.x + w.  Tokens are read 16 at a time (one
//   page-resident subtile), 4 token rows per wave-wide load, 16 lanes per row
//   (DPL = D/16 dims per lane).  Sums are fp32 (the reference's
//   dtype=torch.float32 accumulation), extrema are exact copies, and the value
//   norm of each token is a DPP row sum of squares.  A second tiny kernel folds
//   v_norm_max into v_norm_all.
#include "ia_common.hpp"

namespace ia {
namespace {

struct SummaryParams {
  ia_paged_kv kv;
  const int32_t* seq_lens;
  int32_t n_kv_heads, block_size, nb_max;
  void* k_bar;
  void* v_bar;
  void* k_max;
  void* k_min;
  int32_t k_bar_dtype, v_bar_dtype, bounds_dtype;
  float* v_norm_max;
  float* v_norm_all;
  int32_t* counts;
  // incremental mode: blocks [old_seq_lens[b] / block_size, ceil(seq_lens[b] / block_size))
  // only, v_norm_all raised by atomic max (null: every block, full build)
  const int32_t* old_seq_lens;
};

__device__ __forceinline__ void store_elem(void* base, int64_t off, int dtype, float v) {
  if (dtype == IA_BF16) reinterpret_cast<unsigned short*>(base)[off] = f32_to_bf16_bits(v);
  else reinterpret_cast<float*>(base)[off] = v;
}

template <int DPL, int EB>
__device__ __forceinline__ void load_dims(const char* p, float* out) {
  if constexpr (EB == 4) {
#pragma unroll
    for (int e = 0; e < DPL; e += 4) {
      const u32x4_t a = ld_stream16(p + 4 * e);
      out[e] = __uint_as_float(a[0]); out[e + 1] = __uint_as_float(a[1]);
      out[e + 2] = __uint_as_float(a[2]); out[e + 3] = __uint_as_float(a[3]);
    }
  } else if constexpr (EB == 2) {
    u32 w[DPL / 2];
    if constexpr (DPL == 8) {
      const u32x4_t a = ld_stream16(p);
      w[0] = a[0]; w[1] = a[1]; w[2] = a[2]; w[3] = a[3];
    } else {
      const u32x2_t a = ld_stream8(p);
      w[0] = a[0]; w[1] = a[1];
    }
#pragma unroll
    for (int e = 0; e < DPL / 2; ++e) {
      out[2 * e] = bf16_lo(w[e]);
      out[2 * e + 1] = bf16_hi(w[e]);
    }
  } else {
    u32 w[DPL / 4];
    if constexpr (DPL == 8) {
      const u32x2_t a = ld_stream8(p);
      w[0] = a[0]; w[1] = a[1];
    } else {
      w[0] = ld_stream4(p);
    }
#pragma unroll
    for (int e = 0; e < DPL / 4; ++e) fp8x4_to_f32(w[e], out + 4 * e);
  }
}

template <int D, int EB>
__global__ __launch_bounds__(256) void ia_condition_block_summaries(SummaryParams p) {
  constexpr int DPL = D / 16;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c16 = lane & 15;
  const int r = lane >> 4;
  const int h = blockIdx.y;
  const int b = blockIdx.z;
  const int seq_len = max(p.seq_lens[b], 0);
  int j = blockIdx.x * 4 + wave;
  if (p.old_seq_lens) {
    j += max(p.old_seq_lens[b], 0) / p.block_size;
    if ((int64_t)j * p.block_size >= seq_len) return;  // only blocks holding tokens are refreshed
  }
  if (j >= p.nb_max) return;
  const ia_paged_kv& kv = p.kv;
  const int t_lo = j * p.block_size;
  const int t_hi = min(t_lo + p.block_size, seq_len);
  const int32_t* bt_row = kv.block_table ? kv.block_table + (int64_t)b * kv.bt_stride : nullptr;

  float ks[DPL], vs[DPL], kmx[DPL], kmn[DPL];
#pragma unroll
  for (int e = 0; e < DPL; ++e) {
    ks[e] = 0.f;
    vs[e] = 0.f;
    kmx[e] = kNegInf;
    kmn[e] = -kNegInf;
  }
  float vn = kNegInf;
  int cnt = 0;
  for (int ts = t_lo; ts < t_hi; ts += 16) {
    const int lp = ts / kv.page_size;
    if (bt_row && lp >= kv.bt_cols) break;
    const int64_t pg = bt_row ? (int64_t)bt_row[lp] : (int64_t)lp;
    if (pg < 0 || pg >= kv.n_pages) continue;
    const int in_page = ts % kv.page_size;
    float kscale = 1.f, vscale = 1.f;
    if constexpr (EB == 1) {
      kscale = kv.k_scale[pg * kv.scale_page_stride + h];
      vscale = kv.v_scale[pg * kv.scale_page_stride + h];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tl = 4 * i + r;
      const bool valid = ts + tl < t_hi;
      float kf[DPL], vf[DPL];
      if (valid) {
        const char* kp = reinterpret_cast<const char*>(kv.k) +
                         (pg * kv.k_page_stride + (int64_t)h * kv.k_head_stride +
                          (int64_t)(in_page + tl) * kv.k_token_stride + c16 * DPL) * EB;
        const char* vp = reinterpret_cast<const char*>(kv.v) +
                         (pg * kv.v_page_stride + (int64_t)h * kv.v_head_stride +
                          (int64_t)(in_page + tl) * kv.v_token_stride + c16 * DPL) * EB;
        load_dims<DPL, EB>(kp, kf);
        load_dims<DPL, EB>(vp, vf);
      } else {
#pragma unroll
        for (int e = 0; e < DPL; ++e) kf[e] = vf[e] = 0.f;
      }
      float sq = 0.f;
#pragma unroll
      for (int e = 0; e < DPL; ++e) {
        const float kx = kf[e] * kscale, vx = vf[e] * vscale;
        sq = fmaf(vx, vx, sq);
        if (valid) {
          ks[e] += kx;
          vs[e] += vx;
          kmx[e] = fmaxf(kmx[e], kx);
          kmn[e] = fminf(kmn[e], kx);
        }
      }
      sq = row16_sum(sq);
      if (valid) {
        vn = fmaxf(vn, sqrtf(sq));
        cnt += 1;
      }
    }
  }
  // fold the 4 token rows
#pragma unroll
  for (int e = 0; e < DPL; ++e) {
    ks[e] += shfl_xor_f(ks[e], 16);
    ks[e] += shfl_xor_f(ks[e], 32);
    vs[e] += shfl_xor_f(vs[e], 16);
    vs[e] += shfl_xor_f(vs[e], 32);
    kmx[e] = fmaxf(kmx[e], shfl_xor_f(kmx[e], 16));
    kmx[e] = fmaxf(kmx[e], shfl_xor_f(kmx[e], 32));
    kmn[e] = fminf(kmn[e], shfl_xor_f(kmn[e], 16));
    kmn[e] = fminf(kmn[e], shfl_xor_f(kmn[e], 32));
  }
  vn = fmaxf(vn, shfl_xor_f(vn, 16));
  vn = fmaxf(vn, shfl_xor_f(vn, 32));
  cnt += __shfl_xor(cnt, 16, 64);
  cnt += __shfl_xor(cnt, 32, 64);
  if (r != 0) return;
  const float inv = 1.0f / (float)max(cnt, 1);
  const int64_t row = (((int64_t)b * p.n_kv_heads + h) * p.nb_max + j) * D + c16 * DPL;
#pragma unroll
  for (int e = 0; e < DPL; ++e) {
    if (p.k_bar) store_elem(p.k_bar, row + e, p.k_bar_dtype, ks[e] * inv);
    if (p.v_bar) store_elem(p.v_bar, row + e, p.v_bar_dtype, vs[e] * inv);
    if (p.k_max) store_elem(p.k_max, row + e, p.bounds_dtype, kmx[e]);
    if (p.k_min) store_elem(p.k_min, row + e, p.bounds_dtype, kmn[e]);
  }
  if (c16 == 0) {
    if (p.v_norm_max) p.v_norm_max[((int64_t)b * p.n_kv_heads + h) * p.nb_max + j] = vn;
    if (h == 0) p.counts[(int64_t)b * p.nb_max + j] = cnt;
    // a refreshed block's norm only grows (tokens are appended), so the running
    // maximum stays exact; values are >= 0 or -inf, whose int32 bit patterns
    // order like the floats
    if (p.old_seq_lens && p.v_norm_all)
      atomicMax(reinterpret_cast<int*>(p.v_norm_all) + (int64_t)b * p.n_kv_heads + h, __float_as_int(vn));
  }
}

__global__ __launch_bounds__(256) void ia_condition_block_vnorm_all(const float* v_norm_max, float* v_norm_all,
                                                                    int32_t nb_max) {
  __shared__ float red[4];
  const int bh = blockIdx.x;
  float m = kNegInf;
  for (int j = threadIdx.x; j < nb_max; j += 256) m = fmaxf(m, v_norm_max[(int64_t)bh * nb_max + j]);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) v_norm_all[bh] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

template <int D>
void launch_summaries(const SummaryParams& p, int eb, dim3 grid, hipStream_t st) {
  if (eb == 4) hipLaunchKernelGGL((ia_condition_block_summaries<D, 4>), grid, dim3(256), 0, st, p);
  else if (eb == 2) hipLaunchKernelGGL((ia_condition_block_summaries<D, 2>), grid, dim3(256), 0, st, p);
  else hipLaunchKernelGGL((ia_condition_block_summaries<D, 1>), grid, dim3(256), 0, st, p);
}

}  // namespace
}  // namespace ia

namespace ia {
namespace {

int run_summaries(const ia_paged_kv* kv, const int32_t* old_seq_lens, const int32_t* seq_lens, int32_t batch,
                  int32_t n_kv_heads, int32_t head_dim, int32_t block_size, int32_t nb_max, int32_t window_blocks,
                  void* k_bar, int32_t k_bar_dtype, void* v_bar, int32_t v_bar_dtype, void* k_max, void* k_min,
                  int32_t bounds_dtype, float* v_norm_max, float* v_norm_all, int32_t* counts, void* stream) {
  if (!kv || !kv->k || !kv->v || !seq_lens || !counts) return fail(IA_ERR_INVALID, "null pointer argument");
  if (head_dim != 64 && head_dim != 128) return fail(IA_ERR_UNSUPPORTED, "head_dim must be 64 or 128");
  if (block_size <= 0 || block_size % 16) return fail(IA_ERR_INVALID, "block_size must be a positive multiple of 16");
  if (kv->page_size <= 0 || kv->page_size % 16) return fail(IA_ERR_INVALID, "page_size must be a positive multiple of 16");
  if (batch < 0 || n_kv_heads <= 0 || nb_max < 0) return fail(IA_ERR_INVALID, "batch/heads/nb_max");
  const int32_t dts[3] = {k_bar_dtype, v_bar_dtype, bounds_dtype};
  for (int32_t dt : dts)
    if (dt != IA_F32 && dt != IA_BF16) return fail(IA_ERR_INVALID, "summary dtypes must be IA_F32 or IA_BF16");
  if (kv->dtype == IA_FP8_E4M3 && (!kv->k_scale || !kv->v_scale)) return fail(IA_ERR_INVALID, "fp8 needs scales");
  if (v_norm_all && !v_norm_max) return fail(IA_ERR_INVALID, "v_norm_all needs v_norm_max");
  const int eb = kv->dtype == IA_F32 ? 4 : (kv->dtype == IA_BF16 ? 2 : 1);
  if ((kv->k_token_stride * eb) % 16 || (kv->v_token_stride * eb) % 16 || (kv->k_page_stride * eb) % 16 ||
      (kv->v_page_stride * eb) % 16 || (kv->k_head_stride * eb) % 16 || (kv->v_head_stride * eb) % 16)
    return fail(IA_ERR_INVALID, "kv strides must be 16-byte multiples");
  if (batch == 0 || nb_max == 0 || window_blocks == 0) return IA_OK;
  SummaryParams p{};
  p.kv = *kv;
  p.seq_lens = seq_lens;
  p.old_seq_lens = old_seq_lens;
  p.n_kv_heads = n_kv_heads;
  p.block_size = block_size;
  p.nb_max = nb_max;
  p.k_bar = k_bar;
  p.v_bar = v_bar;
  p.k_max = k_max;
  p.k_min = k_min;
  p.k_bar_dtype = k_bar_dtype;
  p.v_bar_dtype = v_bar_dtype;
  p.bounds_dtype = bounds_dtype;
  p.v_norm_max = v_norm_max;
  p.v_norm_all = v_norm_all;
  p.counts = counts;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  dim3 grid((window_blocks + 3) / 4, n_kv_heads, batch);
  if (head_dim == 128) launch_summaries<128>(p, eb, grid, st);
  else launch_summaries<64>(p, eb, grid, st);
  int rc = check_launch("block summaries");
  if (rc) return rc;
  if (v_norm_all && !old_seq_lens) {
    hipLaunchKernelGGL(ia_condition_block_vnorm_all, dim3(batch * n_kv_heads), dim3(256), 0, st, v_norm_max,
                       v_norm_all, nb_max);
    rc = check_launch("v_norm_all");
  }
  return rc;
}

}  // namespace
}  // namespace ia

extern "C" int ia_build_block_summaries(const ia_paged_kv* kv, const int32_t* seq_lens, int32_t batch,
                                        int32_t n_kv_heads, int32_t head_dim, int32_t block_size, int32_t nb_max,
                                        void* k_bar, int32_t k_bar_dtype, void* v_bar, int32_t v_bar_dtype,
                                        void* k_max, void* k_min, int32_t bounds_dtype, float* v_norm_max,
                                        float* v_norm_all, int32_t* counts, void* stream) {
  return ia::run_summaries(kv, nullptr, seq_lens, batch, n_kv_heads, head_dim, block_size, nb_max, nb_max, k_bar,
                           k_bar_dtype, v_bar, v_bar_dtype, k_max, k_min, bounds_dtype, v_norm_max, v_norm_all,
                           counts, stream);
}

extern "C" int ia_update_block_summaries(const ia_paged_kv* kv, const int32_t* old_seq_lens, const int32_t* seq_lens,
                                         int32_t batch, int32_t n_kv_heads, int32_t head_dim, int32_t block_size,
                                         int32_t nb_max, int32_t max_new_tokens, void* k_bar, int32_t k_bar_dtype,
                                         void* v_bar, int32_t v_bar_dtype, void* k_max, void* k_min,
                                         int32_t bounds_dtype, float* v_norm_max, float* v_norm_all, int32_t* counts,
                                         void* stream) {
  using namespace ia;
  if (!old_seq_lens) return fail(IA_ERR_INVALID, "old_seq_lens must be non-null");
  if (max_new_tokens < 0) return fail(IA_ERR_INVALID, "max_new_tokens must be >= 0");
  if (block_size <= 0) return fail(IA_ERR_INVALID, "block_size must be a positive multiple of 16");
  // the partial block at the old end plus every block the new tokens can reach
  const int64_t window = std::min<int64_t>((int64_t)nb_max, ((int64_t)max_new_tokens + block_size - 1) / block_size + 1);
  return run_summaries(kv, old_seq_lens, seq_lens, batch, n_kv_heads, head_dim, block_size, nb_max, (int32_t)window,
                       k_bar, k_bar_dtype, v_bar, v_bar_dtype, k_max, k_min, bounds_dtype, v_norm_max, v_norm_all,
                       counts, stream);
}
