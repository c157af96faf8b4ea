// Kernel instances of the paged decode for fp8 K/V (compiled separately so the
// instances build in parallel).
#include "paged_decode_kernel.hpp"

namespace ia {

namespace {
template <int D, int G>
int run_fp8(const DecodeParams& p, int src, dim3 grid, hipStream_t st, int* resident) {
  switch (src) {
    case kSrcTopk:
      if (resident) return *resident = resident_wgs<D, G, KvFp8, kSrcTopk>(), IA_OK;
      return launch_paged_finalize<D, G, KvFp8, kSrcTopk>(p, grid, st);
    case kSrcDense:
      if (resident) return *resident = resident_wgs<D, G, KvFp8, kSrcDense>(), IA_OK;
      return launch_paged_finalize<D, G, KvFp8, kSrcDense>(p, grid, st);
    case kSrcLists:
      if (resident) return *resident = resident_wgs<D, G, KvFp8, kSrcLists>(), IA_OK;
      return launch_paged_finalize<D, G, KvFp8, kSrcLists>(p, grid, st);
    case kSrcTopkFused:
      if (resident) return *resident = resident_wgs<D, G, KvFp8, kSrcTopkFused>(), IA_OK;
      return launch_paged_finalize<D, G, KvFp8, kSrcTopkFused>(p, grid, st);
  }
  return fail(IA_ERR_UNSUPPORTED, "unit source");
}
}  // namespace

int dispatch_fp8(const DecodeParams& p, int d, int g, int src, dim3 grid, hipStream_t st, int* resident) {
#define IA_CASE(DD, GG) \
  if (d == DD && g == GG) return run_fp8<DD, GG>(p, src, grid, st, resident);
  IA_CASE(128, 4) IA_CASE(128, 8) IA_CASE(128, 2) IA_CASE(128, 1)
  IA_CASE(64, 4) IA_CASE(64, 8) IA_CASE(64, 2) IA_CASE(64, 1)
#undef IA_CASE
  return fail(IA_ERR_UNSUPPORTED, "head_dim / group combination");
}

uint64_t wait_fallbacks_fp8(bool reset) { return tu_wait_fallbacks(reset); }

}  // namespace ia
