// Kernel instances of the paged decode for f32 K/V (compiled separately so the
// instances build in parallel).
#include "paged_decode_kernel.hpp"

namespace ia {

int dispatch_f32(const DecodeParams& p, int d, int g, bool sparse, dim3 grid, hipStream_t st, int* resident) {
#define IA_CASE(DD, GG)                                                             \
  if (d == DD && g == GG) {                                                         \
    if (sparse) {                                                                   \
      if (resident) return *resident = resident_wgs<DD, GG, KvF32, true>(), IA_OK;   \
      return launch_paged_finalize<DD, GG, KvF32, true>(p, grid, st);                \
    }                                                                               \
    if (resident) return *resident = resident_wgs<DD, GG, KvF32, false>(), IA_OK;    \
    return launch_paged_finalize<DD, GG, KvF32, false>(p, grid, st);                 \
  }
  IA_CASE(128, 4) IA_CASE(128, 8) IA_CASE(128, 2) IA_CASE(128, 1)
  IA_CASE(64, 4) IA_CASE(64, 8) IA_CASE(64, 2) IA_CASE(64, 1)
#undef IA_CASE
  return fail(IA_ERR_UNSUPPORTED, "head_dim / group combination");
}

}  // namespace ia
