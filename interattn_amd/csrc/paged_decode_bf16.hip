// Kernel instances of the paged decode for bf16 K/V (compiled separately so the
// instances build in parallel).
#include "paged_decode_kernel.hpp"

namespace ia {

namespace {
template <int D, int G>
int run_bf16(const DecodeParams& p, int src, dim3 grid, hipStream_t st, int* resident) {
  switch (src) {
    case kSrcTopk:
      if (resident) return *resident = resident_wgs<D, G, KvBf16, kSrcTopk>(), IA_OK;
      return launch_paged_finalize<D, G, KvBf16, kSrcTopk>(p, grid, st);
    case kSrcDense:
      if (resident) return *resident = resident_wgs<D, G, KvBf16, kSrcDense>(), IA_OK;
      return launch_paged_finalize<D, G, KvBf16, kSrcDense>(p, grid, st);
    case kSrcLists:
      if (resident) return *resident = resident_wgs<D, G, KvBf16, kSrcLists>(), IA_OK;
      return launch_paged_finalize<D, G, KvBf16, kSrcLists>(p, grid, st);
    case kSrcTopkFused:
      if constexpr (D == 128) {
        if (p.key_rows) {  // keys as whole rows through LDS
          if (resident) return *resident = resident_wgs<D, G, KvBf16, kSrcTopkFused, true>(), IA_OK;
          return launch_paged_finalize<D, G, KvBf16, kSrcTopkFused, true>(p, grid, st);
        }
      }
      if (resident) return *resident = resident_wgs<D, G, KvBf16, kSrcTopkFused>(), IA_OK;
      return launch_paged_finalize<D, G, KvBf16, kSrcTopkFused>(p, grid, st);
    case kSrcCondFused:  // the one-launch condition call runs groups of up to 4 query rows
      if constexpr (G <= 4) {
        if (resident) return *resident = resident_wgs<D, G, KvBf16, kSrcCondFused>(), IA_OK;
        return launch_paged_finalize<D, G, KvBf16, kSrcCondFused>(p, grid, st);
      } else {
        return fail(IA_ERR_UNSUPPORTED, "one-launch condition call: GQA group above 4");
      }
  }
  return fail(IA_ERR_UNSUPPORTED, "unit source");
}
}  // namespace

int dispatch_bf16(const DecodeParams& p, int d, int g, int src, dim3 grid, hipStream_t st, int* resident) {
#define IA_CASE(DD, GG) \
  if (d == DD && g == GG) return run_bf16<DD, GG>(p, src, grid, st, resident);
  IA_CASE(128, 4) IA_CASE(128, 8) IA_CASE(128, 2) IA_CASE(128, 1)
  IA_CASE(64, 4) IA_CASE(64, 8) IA_CASE(64, 2) IA_CASE(64, 1)
#undef IA_CASE
  return fail(IA_ERR_UNSUPPORTED, "head_dim / group combination");
}

uint64_t wait_fallbacks_bf16(bool reset) { return tu_wait_fallbacks(reset); }

}  // namespace ia
