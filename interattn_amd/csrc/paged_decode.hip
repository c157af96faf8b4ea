// Host side of the paged decode entry points: argument checks, split-K sizing
// and dispatch to the per-dtype kernel instances (paged_decode_{bf16,f32,fp8}.hip).
#include <algorithm>
#include <string>

#include "paged_decode_kernel.hpp"

namespace ia {

namespace {
// 200 us of the 100 MHz clock: a partner workgroup that runs alongside publishes within
// ~15 us of the launch; one that is not resident (the GPU shared with other work) costs
// the waiting item this bound and then its own computation of the missing data
constexpr int64_t kDefaultWaitTicks = 20000;
std::atomic<int64_t> g_wait_ticks{kDefaultWaitTicks};
}  // namespace

int64_t wait_limit_ticks() { return g_wait_ticks.load(std::memory_order_relaxed); }
int64_t set_wait_limit_ticks(int64_t ticks) {
  return g_wait_ticks.exchange(ticks < 0 ? kDefaultWaitTicks : ticks, std::memory_order_relaxed);
}

int units_cap_items(int64_t units) { return (int)std::max<int64_t>(1, std::min<int64_t>(units, kMaxItemsPerBh)); }

// Split-K workspace: (m, l) partials, accumulator partials, items per row.
size_t decode_ws_size(int batch, int hkv, int group, int d, int max_items) {
  const size_t bh = (size_t)batch * hkv;
  return align_up(bh * max_items * group * 2 * 4, 256) + align_up(bh * max_items * group * d * 4, 256) + bh * 4;
}

void set_decode_ws(DecodeParams& p, char* ws, int64_t bh, int max_items, int group, int d) {
  const size_t ml = align_up((size_t)bh * max_items * group * 2 * 4, 256);
  const size_t acc = align_up((size_t)bh * max_items * group * d * 4, 256);
  p.part_ml = reinterpret_cast<float*>(ws);
  p.part_acc = reinterpret_cast<float*>(ws + ml);
  p.part_n = reinterpret_cast<int32_t*>(ws + ml + acc);
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
  if (kv->seq_scale) {
    if (kv->dtype != IA_FP8_E4M3) return fail(IA_ERR_INVALID, "seq_scale is for fp8 kv only");
    if (kv->seq_scale_b_stride < 0 || kv->seq_scale_h_stride < 0 ||
        reinterpret_cast<uintptr_t>(kv->seq_scale) % 8 != 0 ||
        ((uintptr_t)kv->seq_scale_b_stride | (uintptr_t)kv->seq_scale_h_stride) % 2 != 0)
      return fail(IA_ERR_INVALID, "seq_scale pairs must be 8-byte aligned with non-negative even strides");
  }
  if (kv->block_table && (kv->bt_stride <= 0 || kv->bt_cols < 0 || kv->bt_cols > kv->bt_stride))
    return fail(IA_ERR_INVALID, "block table needs 0 <= bt_cols <= bt_stride and bt_stride > 0");
  if (kv->n_pages < 0) return fail(IA_ERR_INVALID, "n_pages must be >= 0");
  return IA_OK;
}

int check_shape(const ia_decode_shape* s) {
  if (!s) return fail(IA_ERR_INVALID, "shape is null");
  if (s->batch < 0 || s->n_kv_heads <= 0 || s->n_q_heads <= 0)
    return fail(IA_ERR_INVALID, "batch must be >= 0 and head counts positive");
  if (s->n_q_heads % s->n_kv_heads != 0)
    return fail(IA_ERR_INVALID, "n_q_heads must be a multiple of n_kv_heads (grouped query attention)");
  const int g = s->n_q_heads / s->n_kv_heads;
  if (g != 1 && g != 2 && g != 4 && g != 8) return fail(IA_ERR_UNSUPPORTED, "GQA group size must be 1, 2, 4 or 8");
  if (s->head_dim != 64 && s->head_dim != 128) return fail(IA_ERR_UNSUPPORTED, "head_dim must be 64 or 128");
  if (s->q_dtype != IA_F32 && s->q_dtype != IA_BF16) return fail(IA_ERR_INVALID, "q dtype must be IA_F32 or IA_BF16");
  return IA_OK;
}

int dispatch_decode(const DecodeParams& p, int kv_dtype, int d, int g, int src, dim3 grid, hipStream_t st,
                    int* resident) {
  if (kv_dtype == IA_BF16) return dispatch_bf16(p, d, g, src, grid, st, resident);
  if (kv_dtype == IA_F32) {
    if (!p.q_f32) return fail(IA_ERR_UNSUPPORTED, "fp32 kv needs fp32 q");
    return dispatch_f32(p, d, g, src, grid, st, resident);
  }
  if (p.q_f32) return fail(IA_ERR_UNSUPPORTED, "fp8 kv needs bf16 q");
  return dispatch_fp8(p, d, g, src, grid, st, resident);
}

int balanced_grid(const DecodeParams& p, int kv_dtype, int d, int g, int src, int64_t n_rows, int64_t units_max,
                  int nsub_u, int cap_items, hipStream_t st, int* grid_out, int* budget_out) {
  int resident = 0;
  int rc = dispatch_decode(p, kv_dtype, d, g, src, dim3(1), st, &resident);
  if (rc) return rc;
  if (resident <= 0) resident = 1024;
  // an item's unit ranges and subtile list live in LDS: at most t_cap raw slots
  const int64_t t_cap = plan_t_cap(nsub_u);
  const int64_t s_cap = units_max * nsub_u;
  if (s_cap > (int64_t)cap_items * t_cap)
    return fail(IA_ERR_UNSUPPORTED, "sequence too long for one launch: " + std::to_string(units_max) + " units");
  if (n_rows > kPlanMaxRows)
    return fail(IA_ERR_UNSUPPORTED, "batch x kv heads above " + std::to_string(kPlanMaxRows) + " rows for one launch");
  int64_t grid = n_rows;  // one item per row when the partials have a single slot
  if (cap_items > 1)
    grid = std::max<int64_t>(std::max<int64_t>(resident, n_rows), n_rows * ((s_cap + t_cap - 1) / t_cap));
  *grid_out = (int)grid;
  *budget_out = resident;
  return IA_OK;
}

int decode_items(const DecodeParams& p, int kv_dtype, int d, int g, int src, int64_t bh, int64_t units_max,
                 int nsub_u, int cap_items, hipStream_t st, int* items_out) {
  // about one resident round of workgroups over all (sequence, kv head)
  int resident = 0;
  int rc = dispatch_decode(p, kv_dtype, d, g, src, dim3(1), st, &resident);
  if (rc) return rc;
  if (resident <= 0) resident = 1024;
  int items = (int)std::max<int64_t>(1, resident / std::max<int64_t>(bh, 1));
  items = std::min(items, cap_items);
  // the item prologue stages unit ranges and page ids in LDS: bound the units per item
  const int upi_lds = std::min(kMaxUnitsPerItem, kMaxSubsPerItem / std::max(nsub_u, 1));
  if (upi_lds < 1) return fail(IA_ERR_UNSUPPORTED, "block_size too large for one work item");
  const int64_t need = (units_max + upi_lds - 1) / upi_lds;
  if (need > cap_items)
    return fail(IA_ERR_UNSUPPORTED, "sequence too long for one launch: " + std::to_string(units_max) + " units");
  items = (int)std::max<int64_t>(items, need);
  *items_out = std::max(items, 1);
  return IA_OK;
}

namespace {

int run_decode(bool sparse, const ia_decode_shape* shape, const void* q, const ia_paged_kv* kv,
               const int32_t* seq_lens, int32_t block_size, const int32_t* idx, int32_t k_cap, const int32_t* n_sel,
               int32_t max_seq_len, float scale, void* out, int32_t out_dtype, void* workspace,
               size_t workspace_bytes, void* stream) {
  int rc = check_shape(shape);
  if (rc) return rc;
  rc = check_kv(kv, shape->head_dim);
  if (rc) return rc;
  if (!q || !out || !seq_lens) return fail(IA_ERR_INVALID, "q, out and seq_lens must be non-null");
  if (out_dtype != IA_F32 && out_dtype != IA_BF16) return fail(IA_ERR_INVALID, "out dtype must be IA_F32 or IA_BF16");
  if (!(scale > 0.f) || !std::isfinite(scale)) return fail(IA_ERR_INVALID, "scale must be positive and finite");
  const int G = shape->n_q_heads / shape->n_kv_heads;
  const int D = shape->head_dim;
  int64_t units_max;
  int unit_tokens;
  if (sparse) {
    if (!idx || !n_sel) return fail(IA_ERR_INVALID, "idx and n_sel must be non-null");
    if (block_size <= 0 || block_size % 16 != 0)
      return fail(IA_ERR_INVALID, "block_size must be a positive multiple of 16");
    if (k_cap <= 0) return fail(IA_ERR_INVALID, "k_cap must be positive");
    units_max = k_cap;
    unit_tokens = block_size;
  } else {
    if (max_seq_len < 0) return fail(IA_ERR_INVALID, "max_seq_len must be >= 0");
    units_max = (max_seq_len + kDenseTile - 1) / kDenseTile;
    unit_tokens = kDenseTile;
  }
  const int cap_items = units_cap_items(units_max);
  const size_t need = decode_ws_size(shape->batch, shape->n_kv_heads, G, D, cap_items);
  if (cap_items > 1 && (!workspace || workspace_bytes < need))
    return fail(IA_ERR_WORKSPACE, "workspace too small: need " + std::to_string(need) + " bytes");
  if (reinterpret_cast<uintptr_t>(workspace) % 256)
    return fail(IA_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  if (shape->batch == 0) return IA_OK;

  DecodeParams p{};
  p.q = q;
  p.q_batch_stride = shape->q_batch_stride;
  p.q_row_stride = shape->q_row_stride;
  p.kv = *kv;
  p.seq_lens = seq_lens;
  p.idx = idx;
  p.n_sel = n_sel;
  p.k_cap = sparse ? k_cap : (int32_t)units_max;  // dense: tiles of max_seq_len
  p.unit_tokens = unit_tokens;
  p.n_kv_heads = shape->n_kv_heads;
  p.sfx_len_stride = 0;
  p.scale_log2 = scale * kLog2e;
  p.q_f32 = shape->q_dtype == IA_F32;
  p.out_f32 = out_dtype == IA_F32;
  p.out = out;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);

  const int64_t bh = (int64_t)shape->batch * shape->n_kv_heads;
  const int src = sparse ? kSrcTopk : kSrcDense;
  p.max_items = cap_items;  // stride of the partials; items per (b, h) never exceed it
  int grid = 0;
  rc = balanced_grid(p, kv->dtype, D, G, src, bh, units_max, (unit_tokens + 15) / 16, cap_items, st, &grid,
                     &p.plan_budget);
  if (rc) return rc;
  p.n_rows = (int)bh;
  if (workspace) set_decode_ws(p, reinterpret_cast<char*>(workspace), bh, cap_items, G, D);
  return dispatch_decode(p, kv->dtype, D, G, src, dim3(grid), st, nullptr);
}

}  // namespace

// Most workgroups a fused launch over `rows` rows may use: the largest resident count
// of its kernel over the kv dtypes, or rows x ceil(s_cap / t_cap) when LDS bounds
// force small items (balanced_grid's rule).
int64_t fused_grid_bound(int64_t rows, int g, int d, int k_cap, int block_size) {
  int resident = 0;
  const DecodeParams none{};
  for (auto run : {dispatch_bf16, dispatch_fp8, dispatch_f32}) {
    int r = 0;
    if (run(none, d, g, kSrcTopkFused, dim3(1), nullptr, &r) == IA_OK) resident = std::max(resident, r);
  }
  if (resident <= 0) resident = 1024;
  const int nsub_u = std::max(block_size / 16, 1);
  const int64_t t_cap = plan_t_cap(nsub_u);
  const int64_t s_cap = (int64_t)std::max(k_cap, 1) * nsub_u;
  return std::max<int64_t>(std::max<int64_t>(resident, rows), rows * ((s_cap + t_cap - 1) / t_cap));
}

FusedWs fused_ws_layout(int batch, int hkv, int g, int d, int nb_max, int k_cap, int block_size,
                        int64_t row_lines) {
  const int64_t rows = (int64_t)batch * hkv;
  FusedWs L;
  L.slots = fused_grid_bound(rows, g, d, k_cap, block_size);
  L.sbuf = align_up((size_t)std::max(rows, row_lines) * kFlagStride * 4, 256);
  L.part_ml = align_up(L.sbuf + (size_t)rows * std::max(nb_max, 1) * 8, 256);
  L.part_acc = align_up(L.part_ml + (size_t)L.slots * g * 2 * 4, 256);
  L.part_n = align_up(L.part_acc + (size_t)L.slots * g * d * 4, 256);
  L.tpart = align_up(L.part_n + (size_t)rows * 4, 256);
  L.total = align_up(L.tpart + (size_t)L.slots * (g * d + 2 * g) * 8, 256);
  return L;
}

int run_topk_decode(const ia_decode_shape* shape, const void* q, const ia_paged_kv* kv, const int32_t* seq_lens,
                    const ia_block_keys* keys, int32_t block_size, int32_t nb_max, int32_t k,
                    const int32_t* k_per_seq, int32_t forced_first, int32_t forced_last, int32_t forced_in_k,
                    int32_t k_cap, float scale, void* out, int32_t out_dtype, int32_t* idx_out, int32_t* n_sel_out,
                    void* workspace, size_t workspace_bytes, void* stream, int64_t row_lines) {
  int rc = check_shape(shape);
  if (rc) return rc;
  rc = check_kv(kv, shape->head_dim);
  if (rc) return rc;
  const int G = shape->n_q_heads / shape->n_kv_heads;
  const int D = shape->head_dim;
  float score_scale = 0.f;
  rc = check_block_keys(keys, G, D, &score_scale);
  if (rc) return rc;
  if (!q || !out || !seq_lens) return fail(IA_ERR_INVALID, "q, out and seq_lens must be non-null");
  if ((idx_out == nullptr) != (n_sel_out == nullptr)) return fail(IA_ERR_INVALID, "idx and n_sel go together");
  if (out_dtype != IA_F32 && out_dtype != IA_BF16) return fail(IA_ERR_INVALID, "out dtype must be IA_F32 or IA_BF16");
  if (!(scale > 0.f) || !std::isfinite(scale)) return fail(IA_ERR_INVALID, "scale must be positive and finite");
  if (block_size <= 0 || block_size % 16 != 0) return fail(IA_ERR_INVALID, "block_size must be a positive multiple of 16");
  if (nb_max < 0 || k < 0 || forced_first < 0 || forced_last < 0 || k_cap <= 0)
    return fail(IA_ERR_INVALID, "nb_max, k, forced_* must be >= 0 and k_cap > 0");
  if (nb_max > kFusedMaxBlocks || k_cap > kMaxUnitsPerItem)
    return fail(IA_ERR_UNSUPPORTED, "fused top-k decode takes nb_max <= " + std::to_string(kFusedMaxBlocks) +
                                        " and k_cap <= " + std::to_string(kMaxUnitsPerItem) +
                                        "; use ia_select_topk + ia_sparse_paged_decode");
  const FusedWs L = fused_ws_layout(shape->batch, shape->n_kv_heads, G, D, nb_max, k_cap, block_size, row_lines);
  if (!workspace || workspace_bytes < L.total)
    return fail(IA_ERR_WORKSPACE, "workspace too small: need " + std::to_string(L.total) + " bytes");
  if (reinterpret_cast<uintptr_t>(workspace) % 256) return fail(IA_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  if (shape->batch == 0) return IA_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  char* ws = reinterpret_cast<char*>(workspace);

  DecodeParams p{};
  p.q = q;
  p.q_batch_stride = shape->q_batch_stride;
  p.q_row_stride = shape->q_row_stride;
  p.kv = *kv;
  p.seq_lens = seq_lens;
  p.k_cap = k_cap;
  p.unit_tokens = block_size;
  p.nb_max = nb_max;
  p.k_per_seq = k_per_seq;
  // launches with per-sequence k (variable-length batches) load keys as whole rows: the
  // faster form where items differ in length and stream partly alone; uniform batches
  // keep the operand-layout loads (same results either way)
  p.key_rows = k_per_seq != nullptr;
  p.topk_k = k;
  p.forced_first = forced_first;
  p.forced_last = forced_last;
  p.forced_in_k = forced_in_k;
  p.idx_out = idx_out;
  p.n_sel_out = n_sel_out;
  p.n_kv_heads = shape->n_kv_heads;
  p.scale_log2 = scale * kLog2e;
  p.q_f32 = shape->q_dtype == IA_F32;
  p.out_f32 = out_dtype == IA_F32;
  p.out = out;
  const bool quest = keys->score == IA_SCORE_QUEST;
  p.kb = quest ? keys->k_max : keys->k_bar;
  p.kb2 = quest ? keys->k_min : keys->k_bar;
  p.kb_batch_stride = keys->batch_stride;
  p.kb_head_stride = keys->head_stride;
  p.kb_bf16 = keys->dtype == IA_BF16;
  p.score_quest = quest;
  p.score_scale = score_scale;
  p.rowctr = reinterpret_cast<u32*>(ws);
  p.sbuf = reinterpret_cast<unsigned long long*>(ws + L.sbuf);
  p.wait_ticks = wait_limit_ticks();
  const int cap_items = units_cap_items(k_cap);
  const int64_t bh = (int64_t)shape->batch * shape->n_kv_heads;
  p.max_items = cap_items;
  int grid = 0;
  rc = balanced_grid(p, kv->dtype, D, G, kSrcTopkFused, bh, k_cap, block_size / 16, cap_items, st, &grid,
                     &p.plan_budget);
  if (rc) return rc;
  if (grid > L.slots) return fail(IA_ERR_LAUNCH, "fused grid exceeds its workspace bound");
  p.n_rows = (int)bh;
  p.part_ml = reinterpret_cast<float*>(ws + L.part_ml);
  p.part_acc = reinterpret_cast<float*>(ws + L.part_acc);
  p.part_n = reinterpret_cast<int32_t*>(ws + L.part_n);
  p.tpart = reinterpret_cast<unsigned long long*>(ws + L.tpart);
  return dispatch_decode(p, kv->dtype, D, G, kSrcTopkFused, dim3(grid), st, nullptr);
}

}  // namespace ia

extern "C" {

size_t ia_sparse_topk_decode_workspace_size(int32_t batch, int32_t n_kv_heads, int32_t group, int32_t head_dim,
                                            int32_t nb_max, int32_t k_cap, int32_t block_size) {
  return ia::fused_ws_layout(batch, n_kv_heads, group, head_dim, nb_max, std::max(k_cap, 1), block_size).total;
}

int ia_sparse_topk_decode(const ia_decode_shape* shape, const void* q, const ia_paged_kv* kv, const int32_t* seq_lens,
                          const ia_block_keys* keys, int32_t block_size, int32_t nb_max, int32_t k,
                          const int32_t* k_per_seq, int32_t forced_first, int32_t forced_last, int32_t forced_in_k,
                          int32_t k_cap, float scale, void* out, int32_t out_dtype, int32_t* idx, int32_t* n_sel,
                          void* workspace, size_t workspace_bytes, void* stream) {
  return ia::run_topk_decode(shape, q, kv, seq_lens, keys, block_size, nb_max, k, k_per_seq, forced_first,
                             forced_last, forced_in_k, k_cap, scale, out, out_dtype, idx, n_sel, workspace,
                             workspace_bytes, stream);
}

int64_t ia_set_wait_limit(int64_t ticks) { return ia::set_wait_limit_ticks(ticks); }

int64_t ia_wait_fallbacks(int32_t reset) {
  const bool r = reset != 0;
  return (int64_t)(ia::wait_fallbacks_bf16(r) + ia::wait_fallbacks_f32(r) + ia::wait_fallbacks_fp8(r));
}

size_t ia_paged_decode_workspace_size(int32_t batch, int32_t n_kv_heads, int32_t group, int32_t head_dim,
                                      int32_t max_items) {
  return ia::decode_ws_size(batch, n_kv_heads, group, head_dim, std::max(max_items, 1));
}

int32_t ia_sparse_max_items(int32_t batch, int32_t n_kv_heads, int32_t k_cap) {
  (void)batch;
  (void)n_kv_heads;
  return ia::units_cap_items(k_cap);
}

int32_t ia_dense_max_items(int32_t batch, int32_t n_kv_heads, int32_t max_seq_len) {
  (void)batch;
  (void)n_kv_heads;
  return ia::units_cap_items((std::max(max_seq_len, 0) + ia::kDenseTile - 1) / ia::kDenseTile);
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
