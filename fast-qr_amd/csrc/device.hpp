// device.hpp — shared gfx950 device helpers for the batched QR kernels.
//
// Wave64 only (CDNA4).  Cross-lane moves use DPP row/quad permutes and
// ds_swizzle where a fixed xor pattern fits inside 32 lanes, and gfx950's
// v_permlane32_swap for the xor-32 step.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fastqr {

constexpr int kWave = 64;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float v32 __attribute__((ext_vector_type(32)));

// Householder reflector in the reference's convention (LAPACK slarfg without
// the safmin rescaling loop; submissions/candidate.py:654-668, 2084-2098).
// `inv` scales x into v (v = x * inv); the reference divides by
// (alpha - beta), LAPACK multiplies by its reciprocal — the latter is used.
// The square root and both reciprocals are the hardware v_sqrt_f32 /
// v_rcp_f32 (<= 1 ulp each; the arguments are far from the denormal range for
// any input whose squared column norms are representable).
struct Reflector {
  float beta;
  float tau;
  float inv;
};

__device__ __forceinline__ Reflector make_reflector(float alpha, float sigma) {
  Reflector r;
  if (sigma > 0.0f) {
    const float norm = __builtin_amdgcn_sqrtf(fmaf(alpha, alpha, sigma));
    r.beta = (alpha >= 0.0f) ? -norm : norm;
    r.tau = (r.beta - alpha) * __builtin_amdgcn_rcpf(r.beta);
    r.inv = __builtin_amdgcn_rcpf(alpha - r.beta);
  } else {
    r.beta = alpha;
    r.tau = 0.0f;
    r.inv = 0.0f;  // inactive: v below the diagonal is written as 0
  }
  return r;
}

// value of lane (lane ^ OFF), OFF a power of two < 64.
template <int OFF>
__device__ __forceinline__ float xor_lane(float v) {
  static_assert(OFF >= 1 && OFF <= 32 && (OFF & (OFF - 1)) == 0, "power of two");
  if constexpr (OFF == 1) {
    // quad_perm [1,0,3,2]
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true));
  } else if constexpr (OFF == 2) {
    // quad_perm [2,3,0,1]
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true));
  } else if constexpr (OFF == 8) {
    // row_ror:8 inside each 16-lane row == xor 8
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xF, 0xF, true));
  } else if constexpr (OFF == 4 || OFF == 16) {
    // ds_swizzle bit-mask mode inside 32-lane halves: and 0x1f, or 0, xor OFF
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x1F | (OFF << 10)));
  } else {
    // xor 32 with v_permlane32_swap(v, v): the first result keeps lanes 0-31
    // and receives lanes 0-31 into 32-63; the second receives lanes 32-63 into
    // 0-31 and keeps 32-63.
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float((__lane_id() < 32) ? r[1] : r[0]);
  }
}

// v(lane) + v(lane ^ 32) in every lane: the two results of one
// v_permlane32_swap are exactly {v_l, v_(l^32)} in some order per half.
__device__ __forceinline__ float xor32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// v(lane) + v(lane ^ 16): the two results of one v_permlane16_swap(v, v) are
// {v_l, v_(l^16)} in some order in every lane.
__device__ __forceinline__ float xor16_sum(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Totals over the four 16-lane rows of two values at once, in every lane
// (a(l) + a(l^16) + a(l^32) + a(l^48), same for b, in the same order of
// additions as xor16_sum then xor32_sum).  v_permlane16_swap(a, b) leaves
// rows (a0,b0,a2,b2) and (a1,b1,a3,b3), whose sum holds the a pairs in rows 0
// and 2 and the b pairs in rows 1 and 3; a v_permlane32_swap of that with
// itself adds the halves, and a v_permlane16_swap with itself spreads row 0
// (a) and row 1 (b) to all rows: three exchanges instead of four.
__device__ __forceinline__ void pair_row_sums(float& a, float& b) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  const float s = __uint_as_float(p[0]) + __uint_as_float(p[1]);
  const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(s), __float_as_uint(s), false, false);
  const float t = __uint_as_float(h[0]) + __uint_as_float(h[1]);
  const auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(t), __float_as_uint(t), false, false);
  a = __uint_as_float(q[0]);
  b = __uint_as_float(q[1]);
}

// Reflector without branches (alpha, sigma wave-uniform): the same values as
// make_reflector, selected instead of branched on so a column step has no
// scalar branch.
__device__ __forceinline__ Reflector make_reflector_sel(float alpha, float sigma) {
  const float nrm = __builtin_amdgcn_sqrtf(fmaf(alpha, alpha, sigma));
  const float bt = (alpha >= 0.0f) ? -nrm : nrm;
  const bool act = sigma > 0.0f;
  Reflector r;
  r.tau = act ? (bt - alpha) * __builtin_amdgcn_rcpf(bt) : 0.0f;
  r.inv = act ? __builtin_amdgcn_rcpf(alpha - bt) : 0.0f;
  r.beta = act ? bt : alpha;
  return r;
}

// Sum over all 64 lanes, result in every lane.
__device__ __forceinline__ float wave_sum(float v) {
  v = xor32_sum(v);
  v += xor_lane<16>(v);
  v += xor_lane<8>(v);
  v += xor_lane<4>(v);
  v += xor_lane<2>(v);
  v += xor_lane<1>(v);
  return v;
}

// One halving step of the transpose-reduction: lanes whose bit log2(OFF) is
// set keep the upper half of the live values, the others the lower half, and
// each adds its partner's copy of the half it keeps.
template <int OFF, int LIVE>
__device__ __forceinline__ void halve_step(float* p, int lane) {
  const bool hi = (lane & OFF) != 0;
#pragma unroll
  for (int i = 0; i < LIVE / 2; ++i) {
    const float lo_v = p[i];
    const float hi_v = p[i + LIVE / 2];
    const float send = hi ? lo_v : hi_v;
    const float keep = hi ? hi_v : lo_v;
    p[i] = keep + xor_lane<OFF>(send);
  }
}

// Reduce NB per-lane partials over the 64 lanes of a wave with
// NB-1 + 6 - log2(NB) shuffles (instead of 6 * NB).  On return lane l holds,
// in p[0], the wave total of value index  l >> (6 - log2 NB)  (every lane in
// a group of 64/NB lanes holds the same total).
template <int NB>
__device__ __forceinline__ float wave_transpose_reduce(float* p, int lane) {
  static_assert(NB == 1 || NB == 2 || NB == 4 || NB == 8 || NB == 16 || NB == 32 || NB == 64, "NB");
  if constexpr (NB >= 2) halve_step<32, NB>(p, lane);
  if constexpr (NB >= 4) halve_step<16, NB / 2>(p, lane);
  if constexpr (NB >= 8) halve_step<8, NB / 4>(p, lane);
  if constexpr (NB >= 16) halve_step<4, NB / 8>(p, lane);
  if constexpr (NB >= 32) halve_step<2, NB / 16>(p, lane);
  if constexpr (NB >= 64) halve_step<1, NB / 32>(p, lane);
  float v = p[0];
  // plain butterfly over the lane bits not used for value selection
  if constexpr (NB <= 1) v += xor_lane<32>(v);
  if constexpr (NB <= 2) v += xor_lane<16>(v);
  if constexpr (NB <= 4) v += xor_lane<8>(v);
  if constexpr (NB <= 8) v += xor_lane<4>(v);
  if constexpr (NB <= 16) v += xor_lane<2>(v);
  if constexpr (NB <= 32) v += xor_lane<1>(v);
  return v;
}

template <int NB>
__device__ __forceinline__ constexpr int reduce_shift() {
  return NB == 1 ? 6 : NB == 2 ? 5 : NB == 4 ? 4 : NB == 8 ? 3 : NB == 16 ? 2 : NB == 32 ? 1 : 0;
}

// ---- buffer addressing: one SGPR descriptor per matrix, 32-bit byte offsets
// per lane.  An offset at or beyond `bytes` reads 0 and drops stores
// (hardware range check), so masked lanes use kOffNone instead of a branch.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr uint32_t kOffNone = 0x80000000u;
// descriptor word 3 for raw (untyped) access on GFX9-family parts
constexpr int kRsrcWord3 = 0x00020000;

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kRsrcWord3);
}
__device__ __forceinline__ float buf_load(rsrc_t r, uint32_t off) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0));
}
__device__ __forceinline__ f32x4 buf_load4(rsrc_t r, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
  f32x4 out;
  out[0] = __uint_as_float(v[0]);
  out[1] = __uint_as_float(v[1]);
  out[2] = __uint_as_float(v[2]);
  out[3] = __uint_as_float(v[3]);
  return out;
}
__device__ __forceinline__ void buf_store(rsrc_t r, uint32_t off, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, (int)off, 0, 0);
}
__device__ __forceinline__ void buf_store4(rsrc_t r, uint32_t off, f32x4 v) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  u32x4 u = {__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])};
  __builtin_amdgcn_raw_buffer_store_b128(u, r, (int)off, 0, 0);
}

// Order this wave's LDS writes before its later LDS reads (no workgroup barrier).
__device__ __forceinline__ void wave_sync_lds() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ float readlane(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

}  // namespace fastqr
