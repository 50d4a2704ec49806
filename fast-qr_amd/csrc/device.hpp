// device.hpp — shared gfx950 device helpers for the batched QR kernels.
//
// Wave64 only (CDNA4).  Cross-lane moves use DPP row/quad permutes and
// ds_swizzle where a fixed xor pattern fits inside 32 lanes, ds_bpermute
// (__shfl_xor) for the xor-32 step.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fastqr {

constexpr int kWave = 64;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// Householder reflector in the reference's convention (LAPACK slarfg without
// the safmin rescaling loop; submissions/candidate.py:654-668, 2084-2098).
// `inv` scales x into v (v = x * inv); the reference divides by
// (alpha - beta), LAPACK multiplies by its reciprocal — the latter is used.
struct Reflector {
  float beta;
  float tau;
  float inv;
};

__device__ __forceinline__ Reflector make_reflector(float alpha, float sigma) {
  Reflector r;
  if (sigma > 0.0f) {
    const float norm = sqrtf(alpha * alpha + sigma);
    r.beta = (alpha >= 0.0f) ? -norm : norm;
    r.tau = (r.beta - alpha) / r.beta;
    r.inv = 1.0f / (alpha - r.beta);
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
    return __shfl_xor(v, OFF, kWave);
  }
}

// Sum over all 64 lanes, result in every lane.
__device__ __forceinline__ float wave_sum(float v) {
  v += xor_lane<32>(v);
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

__device__ __forceinline__ float readlane(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

}  // namespace fastqr
