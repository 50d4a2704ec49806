// wy.hpp — MFMA building blocks of the compact-WY trailing update (fp32,
// v_mfma_f32_32x32x2f32), shared by the strip-resident update (qr_blocked.hip)
// and the row-split update (qr_update.hip).
//
// A 32-row tile of one column strip is held in the MFMA accumulator layout:
// lane (h = lane/32, l32 = lane%32) holds, in register 4q+i, row r0 + 8q + 4h + i
// of column (strip start + l32).
#pragma once

#include "device.hpp"

namespace fastqr {

// Column-major matrix accessed through a buffer descriptor: element (row, col)
// at byte offset 4 * (col * ldh + row); the host keeps 4 * ldh * n below 2^31,
// so every offset fits in 32 bits.
struct MatBuf {
  rsrc_t r;
  int ldh;
  int n;
  __device__ __forceinline__ uint32_t off(int row, int col) const { return 4u * (uint32_t)(col * ldh + row); }
};

// 32-row tile of column `col` (rows r0.., MFMA accumulator layout: register
// 4q+i <- row r0 + 8q + 4h + i); rows >= n and !ok read as 0.
template <bool VEC>
__device__ __forceinline__ f32x16 tile_load(const MatBuf& M, int r0, int col, bool ok, int h) {
  f32x16 x;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int rb = r0 + 8 * q + 4 * h;
    if constexpr (VEC) {
      const f32x4 v = buf_load4(M.r, (ok && rb < M.n) ? M.off(rb, col) : kOffNone);
#pragma unroll
      for (int i = 0; i < 4; ++i) x[4 * q + i] = v[i];
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) x[4 * q + i] = buf_load(M.r, (ok && rb + i < M.n) ? M.off(rb + i, col) : kOffNone);
    }
  }
  return x;
}

// The same tile from a row-major matrix (element (row, col) at byte offset
// 4 * (row * lda + col) of descriptor r, n rows): the 32 lanes of a half read
// 32 consecutive columns of one row per load (128 contiguous bytes).
__device__ __forceinline__ f32x16 tile_load_rm(rsrc_t r, int lda, int n, int r0, int col, bool ok, int h) {
  f32x16 x;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = r0 + 8 * q + 4 * h + i;
      x[4 * q + i] = buf_load(r, (ok && row < n) ? 4u * (uint32_t)(row * lda + col) : kOffNone);
    }
  }
  return x;
}

template <bool VEC>
__device__ __forceinline__ void tile_store(const MatBuf& M, int r0, int col, bool ok, int h, const f32x16& x) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int rb = r0 + 8 * q + 4 * h;
    if constexpr (VEC) {
      f32x4 v = {x[4 * q + 0], x[4 * q + 1], x[4 * q + 2], x[4 * q + 3]};
      buf_store4(M.r, (ok && rb < M.n) ? M.off(rb, col) : kOffNone, v);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) buf_store(M.r, (ok && rb + i < M.n) ? M.off(rb + i, col) : kOffNone, x[4 * q + i]);
    }
  }
}

// V of the transform whose reflectors start at row/column kw (width nb <= 32)
// for the 32-row tile at r0, with the unit diagonal and the zeros above it
// applied; `ok` false loads zeros.
//   pattern A (P = V^T X): lane holds rows r0 + 8q + 4h + i of reflector l32;
//   pattern B (X += V W):  lane holds row r0 + l32 of reflector 8q + 4h + i.
// Only a tile that starts above row kw + nb meets the triangle; every other
// tile (and, for nb = 32, every reflector index) needs no per-element mask,
// which the uniform branches below exploit.
template <bool VEC>
__device__ __forceinline__ f32x16 wy_load_va(const MatBuf& M, int kw, int nb, int r0, int h, int l32, bool ok) {
  const int refl = l32;
  f32x16 va;
  if (r0 >= kw + nb && nb == 32) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int rb = r0 + 8 * q + 4 * h;
      f32x4 v;
      if constexpr (VEC) {
        v = buf_load4(M.r, (ok && rb < M.n) ? M.off(rb, kw + refl) : kOffNone);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = buf_load(M.r, (ok && rb + i < M.n) ? M.off(rb + i, kw + refl) : kOffNone);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) va[4 * q + i] = v[i];
    }
    return va;
  }
  const bool active = ok && refl < nb;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int rb = r0 + 8 * q + 4 * h;
    f32x4 v;
    if constexpr (VEC) {
      v = buf_load4(M.r, (active && rb < M.n) ? M.off(rb, kw + refl) : kOffNone);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = buf_load(M.r, (active && rb + i < M.n) ? M.off(rb + i, kw + refl) : kOffNone);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int rr = rb + i - kw;
      va[4 * q + i] = (rr < refl) ? 0.0f : (rr == refl ? 1.0f : v[i]);
    }
  }
  return va;
}

__device__ __forceinline__ f32x16 wy_load_vb(const MatBuf& M, int kw, int nb, int r0, int h, int l32, bool ok) {
  const int row = r0 + l32;
  f32x16 vb;
  if (r0 >= kw + nb && nb == 32) {
    const bool okr = ok && row < M.n;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int refl = 8 * (j >> 2) + 4 * h + (j & 3);
      vb[j] = buf_load(M.r, okr ? M.off(row, kw + refl) : kOffNone);
    }
    return vb;
  }
  const int rr = row - kw;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int refl = 8 * (j >> 2) + 4 * h + (j & 3);
    const bool load = ok && refl < nb && rr > refl && row < M.n;
    const float v = buf_load(M.r, load ? M.off(row, kw + refl) : kOffNone);
    vb[j] = (refl < nb && rr == refl) ? 1.0f : v;
  }
  return vb;
}

__device__ __forceinline__ void wy_mfma_p(f32x16& P, const f32x16& va, const f32x16& X) {
#pragma unroll
  for (int j = 0; j < 16; ++j) P = __builtin_amdgcn_mfma_f32_32x32x2f32(va[j], X[j], P, 0, 0, 0);
}

__device__ __forceinline__ void wy_mfma_apply(f32x16& X, const f32x16& vb, const f32x16& W) {
#pragma unroll
  for (int j = 0; j < 16; ++j) X = __builtin_amdgcn_mfma_f32_32x32x2f32(vb[j], W[j], X, 0, 0, 0);
}

// Pattern B of a tile from its pattern A registers, transposed through a
// per-wave LDS tile VT[32 reflectors][32 rows (+4 pad)]: the float4 writes
// (8 lanes, 36-word stride) and the row-contiguous reads are conflict-free.
// Replaces 16 strided global loads per lane by one LDS round trip.
__device__ __forceinline__ f32x16 wy_transpose_va(float (*VT)[36], const f32x16& va, int h, int l32) {
#pragma unroll
  for (int q = 0; q < 4; ++q)
    *reinterpret_cast<f32x4*>(&VT[l32][8 * q + 4 * h]) = f32x4{va[4 * q], va[4 * q + 1], va[4 * q + 2], va[4 * q + 3]};
  wave_sync_lds();
  f32x16 vb;
#pragma unroll
  for (int j = 0; j < 16; ++j) vb[j] = VT[8 * (j >> 2) + 4 * h + (j & 3)][l32];
  wave_sync_lds();
  return vb;
}

// P += V^T X for one 32-row tile at r0.
template <bool VEC>
__device__ __forceinline__ void wy_accumulate(f32x16& P, const f32x16& X, const MatBuf& M, int kw, int nb, int r0,
                                              int h, int l32) {
  const f32x16 va = wy_load_va<VEC>(M, kw, nb, r0, h, l32, true);
  wy_mfma_p(P, va, X);
}

// X += V W for one tile.
__device__ __forceinline__ void wy_apply(f32x16& X, const f32x16& W, const MatBuf& M, int kw, int nb, int r0, int h,
                                         int l32) {
  const f32x16 vb = wy_load_vb(M, kw, nb, r0, h, l32, true);
  wy_mfma_apply(X, vb, W);
}

}  // namespace fastqr
