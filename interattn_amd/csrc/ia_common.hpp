// Shared device helpers for the gfx950 kernels: element codecs, DPP
// cross-lane reductions inside 16-lane rows, and host-side error plumbing.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cmath>
#include <string>

#include "../../include/interattn_amd.h"

namespace ia {

typedef uint32_t u32;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
typedef __attribute__((ext_vector_type(2))) float f32x2_t;

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_huge_valf();

// ------------------------------------------------------------------ element codecs

__device__ __forceinline__ float bf16_lo(u32 w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(u32 w) { return __uint_as_float(w & 0xffff0000u); }

__device__ __forceinline__ bf16x2_t as_bf16x2(u32 w) { return __builtin_bit_cast(bf16x2_t, w); }

// Round-to-nearest-even float -> bf16 pair (lowers to v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ u32 pack_bf16x2(float lo, float hi) {
  bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(u32, v);
}

__device__ __forceinline__ unsigned short f32_to_bf16_bits(float x) {
  __bf16 h = (__bf16)x;
  return __builtin_bit_cast(unsigned short, h);
}

// Four OCP e4m3fn codes in one word -> four floats (v_cvt_pk_f32_fp8).
__device__ __forceinline__ void fp8x4_to_f32(u32 w, float* out) {
  f32x2_t a = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
  f32x2_t b = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
  out[0] = a[0];
  out[1] = a[1];
  out[2] = b[0];
  out[3] = b[1];
}

// Two OCP e4m3fn codes (byte pair HI of w) widened to a bf16 pair: exact, since
// every e4m3 value is a bf16 value (scale 1.0).
template <bool HI>
__device__ __forceinline__ u32 fp8x2_to_bf16x2(u32 w) {
  return __builtin_bit_cast(u32, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, HI));
}

// ------------------------------------------------------------------ MFMA operands

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;  // 16x16x32 bf16 A/B operand
typedef __attribute__((ext_vector_type(4))) short i16x4_t;    // 16x16x16 bf16 A/B operand
typedef __attribute__((ext_vector_type(4))) float f32x4_t;    // 16x16 f32 accumulator
typedef __attribute__((ext_vector_type(4))) u32 u32x4_t;
typedef __attribute__((ext_vector_type(2))) u32 u32x2_t;

__device__ __forceinline__ bf16x8_t as_bf16x8(const u32* w) {
  return __builtin_bit_cast(bf16x8_t, u32x4_t{w[0], w[1], w[2], w[3]});
}
__device__ __forceinline__ i16x4_t as_i16x4(u32 lo, u32 hi) {
  return __builtin_bit_cast(i16x4_t, u32x2_t{lo, hi});
}

// ------------------------------------------------------------------ streaming loads

// Loads of data read once per call (K/V pages, summary rows): the nontemporal hint
// (`nt` on the global load) keeps them from displacing reusable lines in L2 and the
// MALL.  Measured at C4 (537 MB of K/V gathered in 4 KiB pages): 113 -> 107 us.
__device__ __forceinline__ u32x4_t ld_stream16(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
}
__device__ __forceinline__ u32x2_t ld_stream8(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(p));
}
__device__ __forceinline__ u32 ld_stream4(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32*>(p));
}

// ------------------------------------------------------------------ hand-offs between workgroups

// Workgroups of one launch hand data to each other (score ranges, split-K partials)
// through memory at the device's coherence point: agent-scope relaxed atomics
// (`sc1` on the global store / load), so a store is written through the XCD's L2
// and a load never returns another XCD's stale copy, with no L2 writeback or
// invalidate.  A publisher stores its data, waits until the stores are acknowledged
// (s_waitcnt vmcnt(0)) and only then raises a flag; a consumer reads the data after
// it has seen the flag (or a tag carried in the data word itself).  Measured on MI355X: ~1.75 us from a 2 KB publish to its
// observation on another XCD (a kernel boundary after a streaming kernel costs
// ~4.5 us).
__device__ __forceinline__ void st_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ u32 ld_agent_u32(const u32* p) {
  return __hip_atomic_load(const_cast<u32*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent_u32(u32* p, u32 v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent_u64(unsigned long long* p, unsigned long long v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long ld_agent_u64(const unsigned long long* p) {
  return __hip_atomic_load(const_cast<unsigned long long*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ u32 fetch_add_agent_u32(u32* p, u32 v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// every memory operation this wave issued has completed (stores acknowledged)
__device__ __forceinline__ void wait_memory() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// the 100 MHz constant clock
__device__ __forceinline__ unsigned long long clock_100mhz() {
  unsigned long long t;
  asm volatile("s_memrealtime %0\n\ts_waitcnt lgkmcnt(0)" : "=s"(t)::"memory");
  return t;
}

// ------------------------------------------------------------------ DPP within 16-lane rows

constexpr int kDppRowMirror = 0x140;
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppXor2 = 0x4E;  // quad_perm [2,3,0,1]
constexpr int kDppXor1 = 0xB1;  // quad_perm [1,0,3,2]
constexpr int kDppRowRor4 = 0x124;
constexpr int kDppRowRor8 = 0x128;

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}

constexpr int kDppRowShr1 = 0x111;     // row_shr:n = 0x110 + n
constexpr int kDppRowBcast15 = 0x142;  // lane 15 of each row to the next row
constexpr int kDppRowBcast31 = 0x143;  // lane 31 to rows 2 and 3

// Inclusive prefix sum over the 64 lanes in lane order, all in DPP (no LDS):
// row_shr 1, 2, 4, 8 scan each 16-lane row, then the row totals are carried by
// row_bcast15 (rows 1, 3) and row_bcast31 (rows 2, 3).
__device__ __forceinline__ int wave_inclusive_scan(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, kDppRowShr1, 0xf, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, kDppRowShr1 + 1, 0xf, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, kDppRowShr1 + 3, 0xf, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, kDppRowShr1 + 7, 0xf, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, kDppRowBcast15, 0xa, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, kDppRowBcast31, 0xc, 0xf, false);
  return v;
}

// Maximum / sum over the four 16-lane rows (lanes c, c+16, c+32, c+48), every lane
// receiving the result, on the VALU (gfx950 permlane swaps; no LDS crossbar):
// swapping a register with itself leaves lane l the pair {v[l], v[l ^ 32]}, then
// {v[l], v[l ^ 16]}.
__device__ __forceinline__ float rows_max(float v) {
  auto t = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(t[0]), __uint_as_float(t[1]));
  t = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(t[0]), __uint_as_float(t[1]));
}
__device__ __forceinline__ float rows_sum(float v) {
  auto t = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(t[0]) + __uint_as_float(t[1]);
  t = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(t[0]) + __uint_as_float(t[1]);
}

// Sum over the 16 lanes of a row; every lane receives the total.  Partner sets
// of mirror, half-mirror, xor2, xor1 are disjoint at each step.
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp<kDppRowMirror>(v);
  v += dpp<kDppRowHalfMirror>(v);
  v += dpp<kDppXor2>(v);
  v += dpp<kDppXor1>(v);
  return v;
}

template <int N, int CTRL>
__device__ __forceinline__ void rs_step(float* v, bool sel) {
#pragma unroll
  for (int k = 0; k < N / 2; ++k) {
    const float lo = v[k], hi = v[k + N / 2];
    const float keep = sel ? hi : lo;
    const float send = sel ? lo : hi;
    v[k] = keep + dpp<CTRL>(send);
  }
}

// Reduce-scatter of NV per-lane partial sums over the 16 lanes of a row.
// On return v[0 .. max(1, NV/16)) holds complete sums; with b = lane & 15 the
// value index held in v[k] is
//   NV=32: 2b + k,  NV=16: b,  NV=8: b >> 1,  NV=4: b >> 2.
template <int NV>
__device__ __forceinline__ void reduce_scatter16(float* v, int lane) {
  static_assert(NV == 4 || NV == 8 || NV == 16 || NV == 32, "NV");
  const int b = lane & 15;
  rs_step<NV, kDppRowMirror>(v, b & 8);
  rs_step<NV / 2, kDppRowHalfMirror>(v, b & 4);
  if constexpr (NV >= 8) {
    rs_step<NV / 4, kDppXor2>(v, b & 2);
  } else {
    v[0] += dpp<kDppXor2>(v[0]);
  }
  if constexpr (NV >= 16) {
    rs_step<NV / 8, kDppXor1>(v, b & 1);
  } else {
    v[0] += dpp<kDppXor1>(v[0]);
  }
}

__device__ __forceinline__ float shfl_xor_f(float v, int m) { return __shfl_xor(v, m, 64); }

__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp<kDppRowMirror>(v));
  v = fmaxf(v, dpp<kDppRowHalfMirror>(v));
  v = fmaxf(v, dpp<kDppXor2>(v));
  v = fmaxf(v, dpp<kDppXor1>(v));
  return v;
}

// Reductions over the 64 lanes of a wave; every lane receives the result.
__device__ __forceinline__ float wave_sum(float v) { return rows_sum(row16_sum(v)); }
__device__ __forceinline__ float wave_max(float v) { return rows_max(row16_max(v)); }

// Wave-level barrier for LDS traffic that stays inside one wavefront.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ------------------------------------------------------------------ host error plumbing

void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int check_launch(const char* what);

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

}  // namespace ia
