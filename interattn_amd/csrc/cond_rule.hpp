// The reference's condition (eps) rule on the device: helpers shared by the
// standalone selection kernels (condition.hip) and the one-launch condition call
// (kSrcCondFused in paged_decode_kernel.hpp).
//
// Per block b of a (sequence, kv head) and query row g (CBT/core.py:509-555):
//   s = q.k_bar / sqrt(D), delta = max(|upper - s|, |lower - s|) from the
//   elementwise key extrema, z = s + log(max(count, 1)), zc = z + log cosh(delta)
//   (term1-mass-exp variant: z + delta); with the row globals z_m, z_l (max and
//   sum exp of z) and c_m, c_l (of zc),
//   cond = 2 B_all e^(z - c_m) (cosh(delta) - 1) / c_l + 2 b_c e^(z - z_m) tanh(delta / 2) / z_l
//   and a block is selected when the group mean of cond exceeds eps.
#pragma once

#include "ia_common.hpp"

namespace ia {

__device__ __forceinline__ float round_if(float x, bool rnd) {
  return rnd ? __uint_as_float((u32)f32_to_bf16_bits(x) << 16) : x;
}

// log cosh(d) = |d| + log(1 + e^{-2|d|}) - log 2, without overflow
__device__ __forceinline__ float log_cosh(float d) {
  const float a = fabsf(d);
  return a + __logf(1.f + __expf(-2.f * a)) - 0.69314718055994531f;
}

// Condition of one (row, block): term1 + term2 with
//   term1 = 2 B_all e^(z - c_m) (cosh(delta) - 1) / c_l   (mass_exp: 2 B_all e^(z + delta - c_m) / c_l)
//   term2 = 2 b_c e^(z - z_m) tanh(delta / 2) / z_l
// from one exponential of -delta (delta >= 0).  For delta >= 1/8
// e^(z - c_m) (cosh(delta) - 1) = (1 - e^-delta)^2 e^(z - c_m + delta) / 2, which cannot
// overflow before the product does; below it the Taylor series of cosh(delta) - 1 and
// tanh(delta / 2) avoid the cancellation of 1 - e^-delta.  inv_zl = 1/z_l, inv_cl = 1/c_l.
__device__ __forceinline__ float condition_value(float dl, float z, float zm, float inv_zl, float cm, float inv_cl,
                                                 float b_c, float b_all, bool mass_exp) {
  const float en = __expf(-dl);
  float tanh_half, term1;
  if (dl < 0.125f) {
    const float d2 = dl * dl;
    tanh_half = 0.5f * dl * (1.f - d2 * (1.f / 12.f) + d2 * d2 * (1.f / 120.f));
    term1 = mass_exp ? 2.f * b_all * __expf(z + dl - cm) * inv_cl
                     : b_all * __expf(z - cm) * d2 * (1.f + d2 * (1.f / 12.f) + d2 * d2 * (1.f / 360.f)) * inv_cl;
  } else {
    const float om = 1.f - en;
    tanh_half = om / (1.f + en);
    term1 = mass_exp ? 2.f * b_all * __expf(z + dl - cm) * inv_cl : b_all * om * om * __expf(z - cm + dl) * inv_cl;
  }
  return term1 + 2.f * b_c * __expf(z - zm) * tanh_half * inv_zl;
}

// Selected-block list entry for the finalize: block id in the low 16 bits, its
// valid-token count above (block ids < 65536 and counts <= 32767 are host-checked).
__device__ __forceinline__ int32_t list_entry(int j, int cnt) { return j | (cnt << 16); }

// One summary row slice of DPL elements as raw words.  BF16 = 1: bf16 rows, one
// load.  BF16 = 0: bf16 or fp32 chosen at run time, with the same two loads on both
// dtypes so no load sits under a branch (fp32 rows read their two halves, bf16 rows
// their one half twice, the second copy unused).  DPL = 8: 16-byte pieces; DPL = 4:
// 8-byte pieces.
template <int DPL, int BF16 = 0>
struct SumRow {
  static_assert(DPL == 8 || DPL == 4, "head_dim 64 or 128");
  u32 w[BF16 ? DPL / 2 : DPL];
  __device__ __forceinline__ void load(const void* base, int64_t off, bool bf16) {
    const char* p0 = reinterpret_cast<const char*>(base) + off * (BF16 || bf16 ? 2 : 4);
    if constexpr (BF16) {
      if constexpr (DPL == 8) {
        const u32x4_t a = ld_stream16(p0);
        w[0] = a[0]; w[1] = a[1]; w[2] = a[2]; w[3] = a[3];
      } else {
        const u32x2_t a = ld_stream8(p0);
        w[0] = a[0]; w[1] = a[1];
      }
    } else {
      constexpr int kPiece = DPL * 2;  // bytes of one piece
      const char* p1 = p0 + (bf16 ? 0 : kPiece);
      if constexpr (DPL == 8) {
        const u32x4_t a = ld_stream16(p0), c = ld_stream16(p1);
        w[0] = a[0]; w[1] = a[1]; w[2] = a[2]; w[3] = a[3];
        w[4] = c[0]; w[5] = c[1]; w[6] = c[2]; w[7] = c[3];
      } else {
        const u32x2_t a = ld_stream8(p0), c = ld_stream8(p1);
        w[0] = a[0]; w[1] = a[1]; w[2] = c[0]; w[3] = c[1];
      }
    }
  }
  __device__ __forceinline__ float at(int e, bool bf16) const {
    if constexpr (BF16) return (e & 1) ? bf16_hi(w[e >> 1]) : bf16_lo(w[e >> 1]);
    else return bf16 ? ((e & 1) ? bf16_hi(w[e >> 1]) : bf16_lo(w[e >> 1])) : __uint_as_float(w[e]);
  }
};

// The elementwise key bounds of one summary row slice (DPL elements at element offset
// off of a [.., D] row layout): k_max and k_min rows, or the packed k_bounds row of
// 2 D elements whose pair (k_max, k_min) of dimension e sits at [2e, 2e + 1] (the
// reference's layout, CBT/core.py:490-499).  Both forms take the same two loads of DPL
// elements, chosen without a branch (the two rows' slices, or the two halves of the
// lane's packed slice); mx(e) / mn(e) pick the elements.
template <int DPL, int BF16 = 0>
struct BoundRows {
  SumRow<DPL, BF16> a, b;
  bool packed;
  __device__ __forceinline__ void load(const void* kmax, const void* kmin, int64_t off, bool bf16, bool pk) {
    packed = pk;
    a.load(kmax, pk ? 2 * off : off, bf16);
    b.load(pk ? kmax : kmin, pk ? 2 * off + DPL : off, bf16);
  }
  // (each branch indexes within its row for the e it serves: no out-of-range index,
  // not even an unused one, so the rows stay in registers)
  __device__ __forceinline__ float mx(int e, bool bf16) const {
    if (e < DPL / 2) return packed ? a.at(2 * e, bf16) : a.at(e, bf16);
    return packed ? b.at(2 * e - DPL, bf16) : a.at(e, bf16);
  }
  __device__ __forceinline__ float mn(int e, bool bf16) const {
    if (e < DPL / 2) return packed ? a.at(2 * e + 1, bf16) : b.at(e, bf16);
    return packed ? b.at(2 * e + 1 - DPL, bf16) : b.at(e, bf16);
  }
};

}  // namespace ia
