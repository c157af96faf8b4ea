// Append one token per sequence into the paged K/V pool for gfx950: the write
// side of a serving decode step, so that a captured step (append, summary
// refresh, select, finalize) replays without host work.
//
//   ia_append_kv_rows: grid = (Hkv, batch), 64 threads; lane l copies 16-byte
//   chunks of the new K and V rows to pool[block_table[b, pos / page], h,
//   pos % page, :] with pos = seq_lens[b].
//   ia_append_kv_advance: seq_lens[b] += 1 where the row was written.  It is a
//   second launch so that no workgroup of the first can read a length that
//   another has already advanced.
#include "ia_common.hpp"

namespace ia {
namespace {

struct AppendParams {
  ia_paged_kv kv;
  const void* k_new;
  const void* v_new;
  int64_t new_batch_stride, new_head_stride;
  int32_t* seq_lens;
  int32_t head_bytes;  // D * element size
};

__device__ __forceinline__ int64_t page_of(const AppendParams& p, int b, int pos) {
  const ia_paged_kv& kv = p.kv;
  const int lp = pos / kv.page_size;
  int64_t pg = lp;
  if (kv.block_table) {
    if (lp >= kv.bt_cols) return -1;
    pg = kv.block_table[(int64_t)b * kv.bt_stride + lp];
  }
  return (pg < 0 || pg >= kv.n_pages) ? -1 : pg;
}

__global__ __launch_bounds__(64) void ia_append_kv_rows(AppendParams p, int eb) {
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const int pos = p.seq_lens[b];
  if (pos < 0) return;
  const int64_t pg = page_of(p, b, pos);
  if (pg < 0) return;
  const ia_paged_kv& kv = p.kv;
  const int in_page = pos % kv.page_size;
  char* kd = reinterpret_cast<char*>(const_cast<void*>(kv.k)) +
             (pg * kv.k_page_stride + (int64_t)h * kv.k_head_stride + (int64_t)in_page * kv.k_token_stride) * eb;
  char* vd = reinterpret_cast<char*>(const_cast<void*>(kv.v)) +
             (pg * kv.v_page_stride + (int64_t)h * kv.v_head_stride + (int64_t)in_page * kv.v_token_stride) * eb;
  const char* ks = reinterpret_cast<const char*>(p.k_new) + ((int64_t)b * p.new_batch_stride + (int64_t)h * p.new_head_stride) * eb;
  const char* vs = reinterpret_cast<const char*>(p.v_new) + ((int64_t)b * p.new_batch_stride + (int64_t)h * p.new_head_stride) * eb;
  for (int o = threadIdx.x * 16; o < p.head_bytes; o += 64 * 16) {
    *reinterpret_cast<uint4*>(kd + o) = *reinterpret_cast<const uint4*>(ks + o);
    *reinterpret_cast<uint4*>(vd + o) = *reinterpret_cast<const uint4*>(vs + o);
  }
}

__global__ __launch_bounds__(256) void ia_append_kv_advance(AppendParams p, int batch) {
  const int b = blockIdx.x * 256 + threadIdx.x;
  if (b >= batch) return;
  const int pos = p.seq_lens[b];
  if (pos >= 0 && page_of(p, b, pos) >= 0) p.seq_lens[b] = pos + 1;
}

}  // namespace
}  // namespace ia

extern "C" int ia_append_kv(const ia_paged_kv* kv, const void* k_new, const void* v_new, int64_t new_batch_stride,
                            int64_t new_head_stride, int32_t* seq_lens, int32_t batch, int32_t n_kv_heads,
                            int32_t head_dim, void* stream) {
  using namespace ia;
  if (!kv || !kv->k || !kv->v || !k_new || !v_new || !seq_lens) return fail(IA_ERR_INVALID, "null pointer argument");
  if (kv->dtype != IA_F32 && kv->dtype != IA_BF16) return fail(IA_ERR_UNSUPPORTED, "append takes bf16 or f32 pools");
  if (head_dim != 64 && head_dim != 128) return fail(IA_ERR_UNSUPPORTED, "head_dim must be 64 or 128");
  if (kv->page_size <= 0 || kv->page_size % 16) return fail(IA_ERR_INVALID, "page_size must be a positive multiple of 16");
  if (batch < 0 || n_kv_heads <= 0) return fail(IA_ERR_INVALID, "batch/heads");
  const int eb = kv->dtype == IA_F32 ? 4 : 2;
  const int64_t strides[8] = {kv->k_page_stride, kv->k_head_stride, kv->k_token_stride, kv->v_page_stride,
                              kv->v_head_stride, kv->v_token_stride, new_batch_stride, new_head_stride};
  for (int64_t s : strides)
    if (s < 0 || (s * eb) % 16) return fail(IA_ERR_INVALID, "strides must be non-negative 16-byte multiples");
  if ((reinterpret_cast<uintptr_t>(kv->k) | reinterpret_cast<uintptr_t>(kv->v) | reinterpret_cast<uintptr_t>(k_new) |
       reinterpret_cast<uintptr_t>(v_new)) % 16)
    return fail(IA_ERR_INVALID, "pointers must be 16-byte aligned");
  if (kv->block_table && (kv->bt_stride <= 0 || kv->bt_cols < 0 || kv->bt_cols > kv->bt_stride))
    return fail(IA_ERR_INVALID, "block table needs 0 <= bt_cols <= bt_stride and bt_stride > 0");
  if (batch == 0) return IA_OK;
  AppendParams p{};
  p.kv = *kv;
  p.k_new = k_new;
  p.v_new = v_new;
  p.new_batch_stride = new_batch_stride;
  p.new_head_stride = new_head_stride;
  p.seq_lens = seq_lens;
  p.head_bytes = head_dim * eb;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(ia_append_kv_rows, dim3(n_kv_heads, batch), dim3(64), 0, st, p, eb);
  int rc = check_launch("append kv");
  if (rc) return rc;
  hipLaunchKernelGGL(ia_append_kv_advance, dim3((batch + 255) / 256), dim3(256), 0, st, p, batch);
  return check_launch("append kv lengths");
}
