// ia_sparse_topk_decode_noalloc: the fused top-k decode call on a scratch buffer the
// library holds itself, for callers that cannot allocate device memory.
//
// The buffer is a file-scope device array (`scratch`, IA_NOALLOC_SCRATCH_BYTES),
// one copy per GPU, kept until the process ends.  In host code the array's name is
// only a stand-in for its device address: the address is looked up once per device
// with hipGetSymbolAddress (with that device current) and only that pointer is
// passed to kernels.  The part of the buffer that carries state from call to call
// (per-row counts and the published score entries, FusedWs up to part_ml) is
// cleared by a fill kernel on the caller's stream whenever the call shape differs
// from the previous call's on that device; the split-K partials are always written
// before they are read.  No hipMalloc, hipFree or allocating library routine is
// called.  Calls that overlap on one GPU share the buffer and race.
#include <mutex>
#include <string>

#include "paged_decode_kernel.hpp"

namespace ia {
namespace {

static __device__ __align__(256) unsigned char scratch[IA_NOALLOC_SCRATCH_BYTES];

// Zero n16 16-byte words (grid-stride; vector stores).
__global__ __launch_bounds__(256) void ia_fill_zero16(u32x4_t* p, int64_t n16) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (int64_t)gridDim.x * 256)
    p[i] = u32x4_t{0u, 0u, 0u, 0u};
}

struct ShapeKey {
  int32_t v[7];
  bool operator==(const ShapeKey& o) const {
    for (int i = 0; i < 7; ++i)
      if (v[i] != o.v[i]) return false;
    return true;
  }
};

struct DeviceScratch {
  void* ptr = nullptr;    // device address of `scratch` on this device
  bool have_key = false;  // the buffer's state belongs to `key`
  ShapeKey key{};
};

std::mutex g_mu;
DeviceScratch g_dev[kMaxCachedDevices];

// This device's scratch address (looked up on its first use) and, when the call
// shape changed, a clear of its first clear_bytes on the stream.
int device_scratch(const ShapeKey& key, size_t clear_bytes, hipStream_t st, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxCachedDevices)
    return fail(IA_ERR_LAUNCH, "no usable current device for the library scratch");
  std::lock_guard<std::mutex> lock(g_mu);
  DeviceScratch& s = g_dev[dev];
  if (!s.ptr) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return fail(IA_ERR_LAUNCH, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    s.ptr = ptr;
  }
  if (!s.have_key || !(s.key == key)) {
    const int64_t n16 = (int64_t)((clear_bytes + 15) / 16);
    const int blocks = (int)std::min<int64_t>(std::max<int64_t>((n16 + 255) / 256, 1), 1024);
    hipLaunchKernelGGL(ia_fill_zero16, dim3(blocks), dim3(256), 0, st, reinterpret_cast<u32x4_t*>(s.ptr), n16);
    const int rc = check_launch("scratch clear");
    if (rc) return rc;
    // under stream capture the clear is a node of the graph, not done yet: the next
    // call outside the graph clears again
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cap) != hipSuccess) cap = hipStreamCaptureStatusActive;
    s.have_key = cap == hipStreamCaptureStatusNone;
    s.key = key;
  }
  *out = s.ptr;
  return IA_OK;
}

}  // namespace
}  // namespace ia

extern "C" {

int ia_sparse_topk_decode_noalloc(const ia_decode_shape* shape, const void* q, const ia_paged_kv* kv,
                                  const int32_t* seq_lens, const ia_block_keys* keys, int32_t block_size,
                                  int32_t nb_max, int32_t k, const int32_t* k_per_seq, int32_t forced_first,
                                  int32_t forced_last, int32_t forced_in_k, int32_t k_cap, float scale, void* out,
                                  int32_t out_dtype, int32_t* idx, int32_t* n_sel, void* stream) {
  // the arguments that size the scratch are checked before it is touched (the launch
  // checks the rest)
  int rc = ia::check_shape(shape);
  if (rc) return rc;
  if (block_size <= 0 || block_size % 16 != 0) return ia::fail(IA_ERR_INVALID, "block_size must be a positive multiple of 16");
  if (nb_max < 0 || k_cap <= 0) return ia::fail(IA_ERR_INVALID, "nb_max must be >= 0 and k_cap > 0");
  if (shape->batch == 0) return IA_OK;
  const int G = shape->n_q_heads / shape->n_kv_heads;
  const ia::FusedWs L = ia::fused_ws_layout(shape->batch, shape->n_kv_heads, G, shape->head_dim, nb_max,
                                            std::max(k_cap, 1), block_size);
  if (L.total > (size_t)IA_NOALLOC_SCRATCH_BYTES)
    return ia::fail(IA_ERR_WORKSPACE, "ia_sparse_topk_decode_noalloc: this call needs " + std::to_string(L.total) +
                                          " bytes of scratch, above the library's " +
                                          std::to_string((size_t)IA_NOALLOC_SCRATCH_BYTES) +
                                          "; use ia_sparse_topk_decode with a workspace");
  const ia::ShapeKey key{{shape->batch, shape->n_kv_heads, G, shape->head_dim, nb_max, k_cap, block_size}};
  void* ws = nullptr;
  rc = ia::device_scratch(key, L.part_ml, reinterpret_cast<hipStream_t>(stream), &ws);
  if (rc) return rc;
  return ia::run_topk_decode(shape, q, kv, seq_lens, keys, block_size, nb_max, k, k_per_seq, forced_first,
                             forced_last, forced_in_k, k_cap, scale, out, out_dtype, idx, n_sel, ws,
                             (size_t)IA_NOALLOC_SCRATCH_BYTES, stream);
}

}  // extern "C"
