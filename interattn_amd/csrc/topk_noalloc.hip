// ia_sparse_topk_decode_noalloc: the fused top-k decode call on a scratch buffer the
// library holds itself, for callers that cannot allocate device memory.
//
// The buffer is a file-scope device array (`scratch`, IA_NOALLOC_SCRATCH_BYTES),
// one copy per GPU, kept until the process ends.  In host code the array's name is
// only a stand-in for its device address: the address is looked up once per device
// with hipGetSymbolAddress (with that device current) and only that pointer is
// passed to kernels.  The buffer carries state from call to call: per-row counts
// and epochs in row lines at a fixed place (kNoallocRowLines lines at its start,
// whatever the call shape), then the published score entries and partials, each
// tagged with its row and epoch.  It is cleared whole by a fill kernel on the
// caller's stream at its first use on a device, and never again: the epochs only
// grow, so a word left by an earlier call of any shape never carries the tag a later
// call waits for.  No hipMalloc, hipFree or allocating library routine is called.
// Calls that overlap on one GPU share the buffer and race.
#include <mutex>
#include <string>

#include "paged_decode_kernel.hpp"

namespace ia {
namespace {

static __device__ __align__(256) unsigned char scratch[IA_NOALLOC_SCRATCH_BYTES];

// (sequence, kv head) rows one call may have: their 256-byte lines (512 KiB) sit at
// the start of the scratch for every call shape
constexpr int64_t kNoallocRowLines = 2048;

// Zero n16 16-byte words (grid-stride; vector stores).
__global__ __launch_bounds__(256) void ia_fill_zero16(u32x4_t* p, int64_t n16) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (int64_t)gridDim.x * 256)
    p[i] = u32x4_t{0u, 0u, 0u, 0u};
}

struct DeviceScratch {
  void* ptr = nullptr;       // device address of `scratch` on this device
  bool initialised = false;  // the whole buffer has been cleared outside a graph capture
};

std::mutex g_mu;
DeviceScratch g_dev[kMaxCachedDevices];

// This device's scratch address (looked up on its first use) and, at its first use,
// a clear of the whole buffer on the stream.
int device_scratch(hipStream_t st, void** out) {
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
  if (!s.initialised) {
    constexpr int64_t n16 = (int64_t)IA_NOALLOC_SCRATCH_BYTES / 16;
    hipLaunchKernelGGL(ia_fill_zero16, dim3(1024), dim3(256), 0, st, reinterpret_cast<u32x4_t*>(s.ptr), n16);
    const int rc = check_launch("scratch clear");
    if (rc) return rc;
    // under stream capture the clear is a node of the graph (every replay clears the
    // buffer, epochs included), not done yet: the next call outside the graph clears
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cap) != hipSuccess) cap = hipStreamCaptureStatusActive;
    s.initialised = cap == hipStreamCaptureStatusNone;
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
  if ((int64_t)shape->batch * shape->n_kv_heads > ia::kNoallocRowLines)
    return ia::fail(IA_ERR_WORKSPACE, "ia_sparse_topk_decode_noalloc: the library's scratch holds at most " +
                                          std::to_string(ia::kNoallocRowLines) +
                                          " (sequence, kv head) rows; use ia_sparse_topk_decode with a workspace");
  const ia::FusedWs L = ia::fused_ws_layout(shape->batch, shape->n_kv_heads, G, shape->head_dim, nb_max,
                                            std::max(k_cap, 1), block_size, ia::kNoallocRowLines);
  if (L.total > (size_t)IA_NOALLOC_SCRATCH_BYTES)
    return ia::fail(IA_ERR_WORKSPACE, "ia_sparse_topk_decode_noalloc: this call needs " + std::to_string(L.total) +
                                          " bytes of scratch, above the library's " +
                                          std::to_string((size_t)IA_NOALLOC_SCRATCH_BYTES) +
                                          "; use ia_sparse_topk_decode with a workspace");
  void* ws = nullptr;
  rc = ia::device_scratch(reinterpret_cast<hipStream_t>(stream), &ws);
  if (rc) return rc;
  return ia::run_topk_decode(shape, q, kv, seq_lens, keys, block_size, nb_max, k, k_per_seq, forced_first,
                             forced_last, forced_in_k, k_cap, scale, out, out_dtype, idx, n_sel, ws,
                             (size_t)IA_NOALLOC_SCRATCH_BYTES, stream, ia::kNoallocRowLines);
}

}  // extern "C"
