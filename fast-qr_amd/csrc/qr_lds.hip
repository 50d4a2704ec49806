// qr_lds.hip — small-n path (64 < n <= 176): one workgroup per matrix with the
// whole matrix resident in LDS for the entire factorisation.
//
// Reference counterpart: geqrf176_kernel (submissions/candidate.py:356-504),
// one CTA per matrix with the 176 x 176 matrix column-major in shared memory,
// one block reduction per (column, column tile) pair and a thread-0 reflector.
//
// Here the matrix (column-major, leading dimension LDM = n rounded up to a
// multiple of 4, plus 4 so that the 32 lanes of an MFMA tile load, one column
// each, fall in different banks) is read once from HBM, factored in LDS, and
// written once.  Per 32-column panel:
//   * panel_body (panel.hpp) factors the panel from LDS in registers on one
//     wave (no barriers), with wavefront DPP / permlane reductions, while the
//     other three waves apply the previous panel's transform to the strips
//     right of this panel;
//   * the panel's compact-WY transform is applied to the next strip with
//     v_mfma_f32_32x32x2f32, every operand read from LDS,
//     X <- X - V (T^T (V^T X)), its tiles split over the four waves.
// Rows between n and LDM stay zero throughout (the reflectors never touch
// them), so 4-row groups need no per-row masking.
#include "kernels.hpp"
#include "panel.hpp"

namespace fastqr {

namespace {

constexpr int kLdsWaves = 4;
constexpr int kCritWaves = 4;  // waves sharing the next strip's update (LDS for their partials)
constexpr int kLdsMaxTiles = (kLdsMaxN + 31) / 32;          // 32-row MFMA tiles of a strip
constexpr int kLdsMaxLd = ((kLdsMaxN + 3) & ~3) + 4;         // leading dimension for n = kLdsMaxN

__device__ __forceinline__ int lds_ld(int n) { return ((n + 3) & ~3) + 4; }

// The panel at column k0 of the LDS matrix: element (r, c) at M[(k0 + c) * ldm + k0 + r].
template <int NWP>
struct LdsPanelIO {
  float* M;
  int ldm;
  int k0;
  float (*T)[33];
  float* tau;
  int64_t ts1;
  __device__ __forceinline__ int idx(int r, int c) const { return (k0 + c) * ldm + k0 + r; }
  __device__ __forceinline__ f32x4 load4(int r, int c, bool ok) const {
    return ok ? *reinterpret_cast<const f32x4*>(M + idx(r, c)) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }
  __device__ __forceinline__ float load1(int r, int c, bool ok) const { return ok ? M[idx(r, c)] : 0.0f; }
  __device__ __forceinline__ void store4(int r, int c, bool ok, f32x4 v) const {
    if (ok) *reinterpret_cast<f32x4*>(M + idx(r, c)) = v;
  }
  __device__ __forceinline__ void store1(int r, int c, bool ok, float v) const {
    if (ok) M[idx(r, c)] = v;
  }
  __device__ __forceinline__ void store_T(int /*slot*/, int r, int c, float v) const { T[r][c] = v; }
  __device__ __forceinline__ void store_tau(int c, float v) const { tau[(int64_t)(k0 + c) * ts1] = v; }
  __device__ __forceinline__ void barrier() const {
    if constexpr (NWP == 1) {
      wave_sync_lds();
    } else {
      __syncthreads();
    }
  }
};

// Loads and stores below are branch-free: a masked lane reads a valid address
// (element 0) and discards the value, so a whole strip update is one basic
// block and the compiler can issue the LDS reads of a tile ahead of the MFMAs
// of the previous one.
__device__ __forceinline__ f32x4 lds_load4(const float* M, int idx, bool ok) {
  const f32x4 v = *reinterpret_cast<const f32x4*>(M + (ok ? idx : 0));
  return ok ? v : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
}
__device__ __forceinline__ float lds_load1(const float* M, int idx, bool ok) {
  const float v = M[ok ? idx : 0];
  return ok ? v : 0.0f;
}

// Apply the panel at k0 (32 reflectors, T in Tk) to the 32-column strip at
// column c0 (columns >= n masked), rows [k0, k0 + 32 NT), NT = ceil((n - k0) /
// 32): P = V^T X, W = -T^T P, X += V W.  One wave; V, X and T come from LDS.
// Only the first tile holds V's unit diagonal and the zeros above it, and only
// the last tile can reach rows >= npad, so the masks are confined to those.
template <int NT>
__device__ __forceinline__ void lds_update_strip(float* M, int ldm, int n, int npad, int k0, const float (*Tk)[33],
                                                 int c0, int h, int l32) {
  const int col = c0 + l32;
  const bool colok = col < n;
  f32x16 X[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int rb = k0 + 32 * t + 8 * q + 4 * h;
      const f32x4 v = lds_load4(M, col * ldm + rb, colok && (t + 1 < NT || rb < npad));
#pragma unroll
      for (int i = 0; i < 4; ++i) X[t][4 * q + i] = v[i];
    }
  }
  f32x16 P;
#pragma unroll
  for (int j = 0; j < 16; ++j) P[j] = 0.0f;
  const float* Vc = M + (k0 + l32) * ldm;  // pattern A: this lane's reflector
#pragma unroll
  for (int t = 0; t < NT; ++t) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int rb = k0 + 32 * t + 8 * q + 4 * h;
      const f32x4 v = (t + 1 < NT) ? *reinterpret_cast<const f32x4*>(Vc + rb) : lds_load4(Vc, rb, rb < npad);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float vv = v[i];
        if (t == 0) {
          const int rr = 8 * q + 4 * h + i;  // row within the panel
          vv = (rr < l32) ? 0.0f : (rr == l32 ? 1.0f : vv);
        }
        P = __builtin_amdgcn_mfma_f32_32x32x2f32(vv, X[t][4 * q + i], P, 0, 0, 0);
      }
    }
  }
  f32x16 W;
#pragma unroll
  for (int j = 0; j < 16; ++j) W[j] = 0.0f;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int kk = 8 * (j >> 2) + 4 * h + (j & 3);
    W = __builtin_amdgcn_mfma_f32_32x32x2f32(Tk[kk][l32], P[j], W, 0, 0, 0);
  }
#pragma unroll
  for (int j = 0; j < 16; ++j) W[j] = -W[j];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int row = k0 + 32 * t + l32;  // pattern B: this lane's row
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float vb[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int rf = 8 * q + 4 * h + i;
        const int idx = (k0 + rf) * ldm + row;
        float v;
        if (t == 0) {
          v = lds_load1(M, idx, l32 > rf);
          v = (l32 == rf) ? 1.0f : v;
        } else if (t + 1 == NT) {
          v = lds_load1(M, idx, row < npad);
        } else {
          v = M[idx];
        }
        vb[i] = v;
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) X[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(vb[i], W[4 * q + i], X[t], 0, 0, 0);
    }
  }
#pragma unroll
  for (int t = 0; t < NT; ++t) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int rb = k0 + 32 * t + 8 * q + 4 * h;
      if (colok && (t + 1 < NT || rb < npad))
        *reinterpret_cast<f32x4*>(M + col * ldm + rb) = f32x4{X[t][4 * q + 0], X[t][4 * q + 1], X[t][4 * q + 2],
                                                              X[t][4 * q + 3]};
    }
  }
}

// The next strip's update after a panel (the critical path), its tiles split
// over the first kCritWaves waves (wave w takes tiles w, w + kCritWaves, ...):
// each forms the partial P of its tiles, the partials meet in LDS (summed in
// wave order, bitwise reproducible), every splitting wave forms W = -T^T P and
// applies it to its own tiles.  All kLdsWaves waves pass the two barriers.
template <int NT>
__device__ __forceinline__ void lds_update_strip_split(float* M, int ldm, int n, int npad, int k0,
                                                       const float (*Tk)[33], int c0, int wave, int h, int l32,
                                                       float (*Pp)[16][64]) {
  constexpr int TW = (NT + kCritWaves - 1) / kCritWaves;  // tiles per splitting wave, at most
  const int col = c0 + l32;
  const bool colok = col < n;
  const bool active = wave < kCritWaves;
  const int lane = 32 * h + l32;
  f32x16 X[TW];
  f32x16 P;
#pragma unroll
  for (int j = 0; j < 16; ++j) P[j] = 0.0f;
  const float* Vc = M + (k0 + l32) * ldm;  // pattern A: this lane's reflector
#pragma unroll
  for (int i = 0; i < TW; ++i) {
    const int t = wave + kCritWaves * i;
    const bool tok = active && t < NT;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int rb = k0 + 32 * t + 8 * q + 4 * h;
      const f32x4 v = lds_load4(M, col * ldm + rb, tok && colok && rb < npad);
#pragma unroll
      for (int e = 0; e < 4; ++e) X[i][4 * q + e] = v[e];
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int rb = k0 + 32 * t + 8 * q + 4 * h;
      const f32x4 v = lds_load4(Vc, rb, tok && rb < npad);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int rr = 32 * t + 8 * q + 4 * h + e;  // row within the panel
        const float vv = (rr < l32) ? 0.0f : (rr == l32 ? 1.0f : v[e]);
        P = __builtin_amdgcn_mfma_f32_32x32x2f32(vv, X[i][4 * q + e], P, 0, 0, 0);
      }
    }
  }
  if (active) {
#pragma unroll
    for (int j = 0; j < 16; ++j) Pp[wave][j][lane] = P[j];
  }
  __syncthreads();
  if (active) {
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      float acc = Pp[0][j][lane];
#pragma unroll
      for (int w = 1; w < kCritWaves; ++w) acc += Pp[w][j][lane];
      P[j] = acc;
    }
    f32x16 W;
#pragma unroll
    for (int j = 0; j < 16; ++j) W[j] = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int kk = 8 * (j >> 2) + 4 * h + (j & 3);
      W = __builtin_amdgcn_mfma_f32_32x32x2f32(Tk[kk][l32], P[j], W, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) W[j] = -W[j];
#pragma unroll
    for (int i = 0; i < TW; ++i) {
      const int t = wave + kCritWaves * i;
      if (t >= NT) continue;
      const int row = k0 + 32 * t + l32;  // pattern B: this lane's row
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float vb[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int rf = 8 * q + 4 * h + e;
          const float v = lds_load1(M, (k0 + rf) * ldm + row, 32 * t + l32 > rf && row < npad);
          vb[e] = (32 * t + l32 == rf) ? 1.0f : v;
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) X[i] = __builtin_amdgcn_mfma_f32_32x32x2f32(vb[e], W[4 * q + e], X[i], 0, 0, 0);
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int rb = k0 + 32 * t + 8 * q + 4 * h;
        if (colok && rb < npad)
          *reinterpret_cast<f32x4*>(M + col * ldm + rb) = f32x4{X[i][4 * q + 0], X[i][4 * q + 1], X[i][4 * q + 2],
                                                                X[i][4 * q + 3]};
      }
    }
  }
  __syncthreads();
}

// The far strips (from column c_first) of the panel at k0, one strip per wave,
// round robin over `nw` waves starting with wave `w0`; this wave is `wave`.
__device__ __forceinline__ void lds_update_far(float* M, int ldm, int n, int npad, int k0, const float (*Tk)[33],
                                               int c_first, int wave, int w0, int nw, int h, int l32) {
  const int nstrips = (n - c_first + 31) >> 5;
  const int nt = (n - k0 + 31) >> 5;
  for (int s = wave - w0; s < nstrips; s += nw) {
    const int c0 = c_first + 32 * s;
    switch (nt) {
      case 6: lds_update_strip<6>(M, ldm, n, npad, k0, Tk, c0, h, l32); break;
      case 5: lds_update_strip<5>(M, ldm, n, npad, k0, Tk, c0, h, l32); break;
      case 4: lds_update_strip<4>(M, ldm, n, npad, k0, Tk, c0, h, l32); break;
      case 3: lds_update_strip<3>(M, ldm, n, npad, k0, Tk, c0, h, l32); break;
      default: lds_update_strip<2>(M, ldm, n, npad, k0, Tk, c0, h, l32); break;
    }
  }
}

}  // namespace

__global__ void __launch_bounds__(kLdsWaves * 64) qr_lds_kernel(const float* __restrict__ A, int64_t as0, int64_t as1,
                                                                int64_t as2, float* __restrict__ H, int64_t hs0,
                                                                int64_t hs1, int64_t hs2, float* __restrict__ tau,
                                                                int64_t ts0, int64_t ts1, int n) {
  __shared__ __attribute__((aligned(16))) float M[kLdsMaxN * kLdsMaxLd];
  __shared__ float Tk[2][32][33];  // T of the current and the previous panel
  __shared__ float Pp[kCritWaves][16][64];
  __shared__ PanelLds<1, 2> Lp;  // shared by the panel forms below
  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int ldm = lds_ld(n);
  const int npad = (n + 3) & ~3;

  // A -> LDS.  Lanes take consecutive columns and four consecutive rows each,
  // so every global load instruction covers 64 columns of one row and every
  // LDS store is one 16-byte column segment (the bank pattern of an MFMA tile
  // load); 16 rows per wave and pass keep 48 loads in flight per lane.
  const float* Ab = A + b * as0;
  const bool a_vec = as1 == 1 && (as2 & 3) == 0 && (as0 & 3) == 0 && ((uintptr_t)A & 15) == 0;
  if (a_vec) {
    // column-major source: a wave reads whole columns, lanes taking four
    // consecutive rows each (16-byte global loads and LDS stores); eight
    // columns per wave and pass keep eight loads in flight per lane
    const int r = 4 * lane;
    for (int c0 = 8 * wave; c0 < n; c0 += 8 * kLdsWaves) {
      f32x4 v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int c = c0 + j;
        if (c < n && r + 3 < n) {
          v[j] = *reinterpret_cast<const f32x4*>(Ab + (int64_t)c * as2 + r);
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) v[j][i] = (c < n && r + i < n) ? Ab[(int64_t)c * as2 + r + i] : 0.0f;
        }
      }
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (c0 + j < n && r < npad) *reinterpret_cast<f32x4*>(M + (c0 + j) * ldm + r) = v[j];
    }
  }
  for (int r0 = 16 * wave; !a_vec && r0 < npad; r0 += 16 * kLdsWaves) {
    f32x4 v[kLdsMaxTiles / 2][4];
#pragma unroll
    for (int cc = 0; cc < kLdsMaxTiles / 2; ++cc) {
      const int c = 64 * cc + lane;
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = r0 + 4 * g + i;
          v[cc][g][i] = (c < n && r < n) ? Ab[r * as1 + c * as2] : 0.0f;
        }
    }
#pragma unroll
    for (int cc = 0; cc < kLdsMaxTiles / 2; ++cc) {
      const int c = 64 * cc + lane;
#pragma unroll
      for (int g = 0; g < 4; ++g)
        if (c < n && r0 + 4 * g < npad) *reinterpret_cast<f32x4*>(M + c * ldm + r0 + 4 * g) = v[cc][g];
    }
  }
  __syncthreads();

  // Per 32-column panel at k0 (panel p), two phases:
  //   B: wave 0 factors the panel (one wave: no barriers in its column loop)
  //      while waves 1-3 apply the previous panel's transform to the strips
  //      right of this panel (those columns wait for nothing else);
  //   A: all waves apply this panel's transform to the next strip, the next
  //      panel's columns, its tiles split over kCritWaves waves.
  // Phase B's two parts touch disjoint columns and T buffers (T of panel p
  // in Tk[p & 1]), so only a barrier between the phases is needed.
  float* tb = tau + b * ts0;
  for (int k0 = 0, p = 0; k0 < n; k0 += 32, ++p) {
    // lane-derived values are recomputed per panel from an opaque copy of the
    // thread id: hoisted out of this loop they would exceed the SGPR budget
    int t = tid;
    asm volatile("" : "+v"(t));
    const int m = n - k0;
    const int w = m < 32 ? m : 32;
    const int wv = __builtin_amdgcn_readfirstlane(t >> 6);
    if (wv == 0) {
      // one form per height class: the column loop runs over every tile of
      // the form, so a form no taller than the panel saves the masked tiles
      LdsPanelIO<1> io{M, ldm, k0, Tk[p & 1], tb, ts1};
      if (m > 144) {
        panel_body_lds<1, (kLdsMaxN + 15) / 16, 2, true>(io, m, t, Lp);
      } else if (m > 112) {
        panel_body_lds<1, 9, 2, true>(io, m, t, Lp);
      } else if (m > 80) {
        panel_body_lds<1, 7, 2, true>(io, m, t, Lp);
      } else if (m > 64) {
        panel_body_lds<1, 5, 2, true>(io, m, t, Lp);
      } else {
        panel_body_lds<1, 4, 2, true>(io, m, t, Lp);
      }
    } else if (k0 > 0 && k0 + 32 < n) {
      lds_update_far(M, ldm, n, npad, k0 - 32, Tk[(p - 1) & 1], k0 + 32, wv, 1, kLdsWaves - 1, (t >> 5) & 1, t & 31);
    }
    __syncthreads();
    if (w == 32 && k0 + 32 < n) {
      const int nt = (m + 31) >> 5;
      const int h = (t >> 5) & 1, l32 = t & 31;
      switch (nt) {
        case 6: lds_update_strip_split<6>(M, ldm, n, npad, k0, Tk[p & 1], k0 + 32, wv, h, l32, Pp); break;
        case 5: lds_update_strip_split<5>(M, ldm, n, npad, k0, Tk[p & 1], k0 + 32, wv, h, l32, Pp); break;
        case 4: lds_update_strip_split<4>(M, ldm, n, npad, k0, Tk[p & 1], k0 + 32, wv, h, l32, Pp); break;
        case 3: lds_update_strip_split<3>(M, ldm, n, npad, k0, Tk[p & 1], k0 + 32, wv, h, l32, Pp); break;
        default: lds_update_strip_split<2>(M, ldm, n, npad, k0, Tk[p & 1], k0 + 32, wv, h, l32, Pp); break;
      }
    }
  }

  // LDS -> H.  Columns contiguous in H: a wave writes whole columns, lanes
  // taking four consecutive rows each (16-byte LDS reads and global stores).
  float* Hb = H + b * hs0;
  const bool h_vec = hs1 == 1 && (hs2 & 3) == 0 && (hs0 & 3) == 0 && ((uintptr_t)H & 15) == 0;
  if (h_vec) {
    const int r = 4 * lane;
    for (int c = wave; c < n; c += kLdsWaves) {
      if (r < n) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(M + c * ldm + r);
        if (r + 3 < n) {
          *reinterpret_cast<f32x4*>(Hb + (int64_t)c * hs2 + r) = v;
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (r + i < n) Hb[(int64_t)c * hs2 + r + i] = v[i];
        }
      }
    }
  } else {
    // any strides: lanes along columns, four rows each
    for (int r0 = 4 * wave; r0 < n; r0 += 4 * kLdsWaves) {
#pragma unroll
      for (int cc = 0; cc < kLdsMaxTiles / 2; ++cc) {
        const int c = 64 * cc + lane;
        if (c < n) {
          const f32x4 v = *reinterpret_cast<const f32x4*>(M + c * ldm + r0);
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (r0 + i < n) Hb[(int64_t)(r0 + i) * hs1 + (int64_t)c * hs2] = v[i];
        }
      }
    }
  }
}

hipError_t launch_qr_lds(const float* A, int64_t batch, int n, int64_t as0, int64_t as1, int64_t as2, float* H,
                         int64_t hs0, int64_t hs1, int64_t hs2, float* tau, int64_t ts0, int64_t ts1,
                         hipStream_t stream) {
  if (n <= 64 || n > kLdsMaxN) return hipErrorInvalidValue;
  hipLaunchKernelGGL(qr_lds_kernel, dim3((unsigned)batch), dim3(kLdsWaves * 64), 0, stream, A, as0, as1, as2, H, hs0,
                     hs1, hs2, tau, ts0, ts1, n);
  return hipGetLastError();
}

}  // namespace fastqr
