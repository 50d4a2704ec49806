// qr_mixed.hip — the reduced-precision variant of the blocked QR: trailing
// update with rounded operands, and the block copies of its repair steps.
//
// Reference counterpart: the experimental mixed-precision direction of
// tools/blocked_qr_reference.py:25-122 (precision modes "tf32-input" and
// "fp16-input" round the operands of each update product, panels stay fp32)
// and its CUDA prototype submissions/candidate.py:539-554 (update_operand_352),
// 2240-2402 (panel refresh and R repair kernels).  The update here is
//
//   P = r(V)^T r(X),   M = r(T)^T r(P),   X <- X - r(V) r(M)
//
// with r() the operand rounding of the mode, every product accumulated in
// fp32: fp32 (no rounding, v_mfma_f32_32x32x2f32), tf32-input (round to 10
// stored mantissa bits, nearest-even, then the fp32 MFMA: products of such
// values are exact in fp32; gfx950 has no xf32 MFMA), fp16-input and
// bf16-input (the operands converted round-to-nearest-even and multiplied by
// v_mfma_f32_32x32x8_f16 / _bf16 with fp32 accumulation).
#include "device.hpp"
#include "kernels.hpp"

namespace fastqr {

namespace {

typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));

// Operand rounding of each mode, round to nearest, ties to even.
template <int PREC>
__device__ __forceinline__ float round_operand(float x) {
  if constexpr (PREC == kPrecTf32) {
    uint32_t u = __float_as_uint(x);
    u += 0xFFFu + ((u >> 13) & 1u);
    return __uint_as_float(u & 0xFFFFE000u);
  } else if constexpr (PREC == kPrecBf16) {
    uint32_t u = __float_as_uint(x);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return __uint_as_float(u & 0xFFFF0000u);
  } else if constexpr (PREC == kPrecF16) {
    return (float)(_Float16)x;
  } else {
    return x;
  }
}

__device__ __forceinline__ short bf16_bits(float x) {
  uint32_t u = __float_as_uint(x);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (short)(u >> 16);
}

// acc += A B over one 32-deep slice of the contraction: a[4s+t] and b[4s+t]
// (lane (h, l32)) are A[l32][8s+4h+t] and B[8s+4h+t][l32]; the rounding of
// the mode is applied to both operands here.
template <int PREC>
__device__ __forceinline__ void mma32(f32x16& acc, const float (&a)[16], const float (&b)[16]) {
  if constexpr (PREC == kPrecF16) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      f16x4 av, bv;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        av[t] = (_Float16)a[4 * s + t];
        bv[t] = (_Float16)b[4 * s + t];
      }
      acc = __builtin_amdgcn_mfma_f32_32x32x8f16(av, bv, acc, 0, 0, 0);
    }
  } else if constexpr (PREC == kPrecBf16) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      s16x4 av, bv;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        av[t] = bf16_bits(a[4 * s + t]);
        bv[t] = bf16_bits(b[4 * s + t]);
      }
      acc = __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(av, bv, acc, 0, 0, 0);
    }
  } else {
    // K = 2 per instruction: instruction j contracts rows {8(j/4)+(j%4), +4}
    // (lane halves h = 0, 1), the same pairing for both operands
#pragma unroll
    for (int j = 0; j < 16; ++j)
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(round_operand<PREC>(a[j]), round_operand<PREC>(b[j]), acc, 0, 0, 0);
  }
}

constexpr int kMixedWaves = 4;

// One workgroup per (32-column strip of the trailing columns, matrix): the
// update of columns [c_begin + 32*strip, +32) ∩ [c_begin, n), rows [k0, n),
// by the panel of width w at column k0 (V below its diagonal in H, T in
// workspace slot 0 of the matrix).  Wave wv owns the 32-row tiles wv, wv+4, ...
// Tiles are read in the accumulator layout (lane (h, l32): rows 8s+4h .. +3
// of column l32, 16 bytes per lane with VEC); the apply phase needs V by
// rows, which it gets through a per-wave LDS transpose.
template <int PREC, bool VEC>
__global__ void __launch_bounds__(kMixedWaves * 64)
mixed_update_kernel(float* __restrict__ H, int64_t hs0, int ldh, const float* __restrict__ Tws, int n, int k0,
                    int w, int c_begin) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int h = lane >> 5, l32 = lane & 31;
  const int64_t b = blockIdx.y;
  const int m = n - k0;
  const int ntiles = (m + 31) >> 5;
  const int col = c_begin + 32 * (int)blockIdx.x + l32;
  const bool colok = col < n;
  const rsrc_t rs = make_rsrc(H + b * hs0, (uint32_t)(4 * (int64_t)ldh * n));
  // element (row r, column c) of the panel-relative block: rows from k0
  auto off = [&](int r, int c) -> uint32_t { return 4u * (uint32_t)((k0 + c) * ldh + k0 + r); };
  // rows r0 .. r0+3 of column c (VEC: m is a multiple of 4, so r0 < m covers all four)
  auto load4 = [&](int r0, int c, bool ok) -> f32x4 {
    if constexpr (VEC) return buf_load4(rs, (ok && r0 < m) ? off(r0, c) : kOffNone);
    f32x4 v;
#pragma unroll
    for (int t = 0; t < 4; ++t) v[t] = buf_load(rs, (ok && r0 + t < m) ? off(r0 + t, c) : kOffNone);
    return v;
  };
  auto store4 = [&](int r0, int c, bool ok, f32x4 v) {
    if constexpr (VEC) {
      buf_store4(rs, (ok && r0 < m) ? off(r0, c) : kOffNone, v);
    } else {
#pragma unroll
      for (int t = 0; t < 4; ++t) buf_store(rs, (ok && r0 + t < m) ? off(r0 + t, c) : kOffNone, v[t]);
    }
  };
  // V of tile rt in the accumulator layout: va[4s+t] = V[32 rt + 8s+4h+t][l32]
  // (zero above the diagonal, one on it, H below; columns >= w zero)
  auto v_tile = [&](int rt, float (&va)[16]) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int r0 = 32 * rt + 8 * s + 4 * h;
      const f32x4 x = load4(r0, l32, l32 < w && r0 + 3 > l32);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int r = r0 + t;
        va[4 * s + t] = (l32 >= w || r < l32) ? 0.0f : (r == l32 ? 1.0f : x[t]);
      }
    }
  };

  __shared__ float Ts[32][33];
  __shared__ float Pp[kMixedWaves][16][64];
  __shared__ float Vt[kMixedWaves][32][33];
  for (int idx = threadIdx.x; idx < 32 * 32; idx += kMixedWaves * 64) {
    const int r = idx >> 5, c = idx & 31;
    Ts[r][c] = (r < w && c < w) ? Tws[b * kMaxSlots * 1024 + r * 32 + c] : 0.0f;
  }

  // P = V^T X over this wave's tiles
  f32x16 P;
#pragma unroll
  for (int j = 0; j < 16; ++j) P[j] = 0.0f;
  for (int rt = wave; rt < ntiles; rt += kMixedWaves) {
    float va[16], xb[16];
    v_tile(rt, va);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const f32x4 x = load4(32 * rt + 8 * s + 4 * h, col - k0, colok);
#pragma unroll
      for (int t = 0; t < 4; ++t) xb[4 * s + t] = x[t];
    }
    mma32<PREC>(P, va, xb);  // A[l32][row] = V[row][l32], B = X
  }
#pragma unroll
  for (int j = 0; j < 16; ++j) Pp[wave][j][lane] = P[j];
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    float sum = 0.0f;
#pragma unroll
    for (int wv = 0; wv < kMixedWaves; ++wv) sum += Pp[wv][j][lane];
    P[j] = sum;
  }

  // M = T^T P: A[l32][kk] = T[kk][l32], B = P in accumulator layout
  float ta[16], pb[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    ta[j] = Ts[8 * (j >> 2) + 4 * h + (j & 3)][l32];
    pb[j] = P[j];
  }
  f32x16 Mw;
#pragma unroll
  for (int j = 0; j < 16; ++j) Mw[j] = 0.0f;
  mma32<PREC>(Mw, ta, pb);
  float mb[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) mb[j] = Mw[j];

  // X <- X - V M, tile by tile: A[l32][kk] = V[row l32][kk], from the
  // accumulator-layout tile through LDS
  for (int rt = wave; rt < ntiles; rt += kMixedWaves) {
    float va[16];
    v_tile(rt, va);
#pragma unroll
    for (int j = 0; j < 16; ++j) Vt[wave][8 * (j >> 2) + 4 * h + (j & 3)][l32] = va[j];
    wave_sync_lds();
#pragma unroll
    for (int j = 0; j < 16; ++j) va[j] = Vt[wave][l32][8 * (j >> 2) + 4 * h + (j & 3)];
    wave_sync_lds();  // this tile's reads before the next tile's writes
    f32x16 D;
#pragma unroll
    for (int j = 0; j < 16; ++j) D[j] = 0.0f;
    mma32<PREC>(D, va, mb);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int r0 = 32 * rt + 8 * s + 4 * h;
      f32x4 x = load4(r0, col - k0, colok);
#pragma unroll
      for (int t = 0; t < 4; ++t) x[t] -= D[4 * s + t];
      store4(r0, col - k0, colok, x);
    }
  }
}

// dst[b, dr0 + i, dc0 + j] = src[b, i, j] for i < rows, j < cols (src and
// dst pre-offset to their first element); with `upper` only where
// dr0 + i <= dc0 + j.
__global__ void __launch_bounds__(256)
block_copy_kernel(const float* __restrict__ src, int64_t s0, int64_t s1, int64_t s2, float* __restrict__ dst,
                  int64_t d0, int64_t d1, int64_t d2, int rows, int cols, int dr0, int dc0, int upper) {
  const int64_t b = blockIdx.y;
  const int64_t total = (int64_t)rows * cols;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
    const int i = (int)(e % rows), j = (int)(e / rows);
    if (upper && dr0 + i > dc0 + j) continue;
    dst[b * d0 + i * d1 + j * d2] = src[b * s0 + i * s1 + j * s2];
  }
}

}  // namespace

hipError_t launch_mixed_update(int prec, float* H, int64_t batch, int64_t hs0, int64_t ldh, const float* Tws, int n,
                               int k0, int w, int c_begin, bool vec, hipStream_t stream) {
  if (c_begin >= n || w < 1 || w > 32 || batch < 1 || batch > kMaxGridY) return hipErrorInvalidValue;
  // the 16-byte form needs 4-row groups that never straddle the last row
  if (vec && ((n - k0) % 4 != 0 || ldh % 4 != 0 || k0 % 4 != 0)) return hipErrorInvalidValue;
  const dim3 grid((unsigned)((n - c_begin + 31) / 32), (unsigned)batch);
  const dim3 block(kMixedWaves * 64);
#define FASTQR_MIXED_LAUNCH(P)                                                                                  \
  if (vec)                                                                                                      \
    hipLaunchKernelGGL((mixed_update_kernel<P, true>), grid, block, 0, stream, H, hs0, (int)ldh, Tws, n, k0, w,  \
                       c_begin);                                                                                \
  else                                                                                                          \
    hipLaunchKernelGGL((mixed_update_kernel<P, false>), grid, block, 0, stream, H, hs0, (int)ldh, Tws, n, k0, w, \
                       c_begin);
  switch (prec) {
    case kPrecF32:
      FASTQR_MIXED_LAUNCH(kPrecF32);
      break;
    case kPrecTf32:
      FASTQR_MIXED_LAUNCH(kPrecTf32);
      break;
    case kPrecF16:
      FASTQR_MIXED_LAUNCH(kPrecF16);
      break;
    case kPrecBf16:
      FASTQR_MIXED_LAUNCH(kPrecBf16);
      break;
    default:
      return hipErrorInvalidValue;
  }
#undef FASTQR_MIXED_LAUNCH
  return hipGetLastError();
}

hipError_t launch_block_copy(const float* src, int64_t batch, int64_t s0, int64_t s1, int64_t s2, float* dst,
                             int64_t d0, int64_t d1, int64_t d2, int rows, int cols, int dr0, int dc0, bool upper,
                             hipStream_t stream) {
  if (rows <= 0 || cols <= 0 || batch <= 0) return hipSuccess;
  if (batch > kMaxGridY) return hipErrorInvalidValue;
  const int64_t total = (int64_t)rows * cols;
  const int64_t wgs = (total + 255) / 256;
  const dim3 grid((unsigned)(wgs < 1024 ? wgs : 1024), (unsigned)batch);
  hipLaunchKernelGGL(block_copy_kernel, grid, dim3(256), 0, stream, src, s0, s1, s2, dst, d0, d1, d2, rows, cols, dr0,
                     dc0, upper ? 1 : 0);
  return hipGetLastError();
}

}  // namespace fastqr
