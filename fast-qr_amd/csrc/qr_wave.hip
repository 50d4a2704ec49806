// qr_wave.hip — batched QR for n <= 64: one wave64 per matrix, no LDS.
//
// Reference counterpart: geqrf32_kernel, submissions/candidate.py:146-226
// (one warp32 per 32x32 matrix, the matrix transposed in shared memory, one
// warp reduction per (k, j) pair).
//
// Layout: the matrix is cut into 16x16 tiles held in the accumulator layout
// of v_mfma_f32_16x16x4f32: lane (kq = lane/16, cn = lane%16) holds, in
// X[tr][tc], rows 16tr + 4kq .. +3 of column 16tc + cn.  A 16-lane row of the
// wave therefore holds four rows of all sixteen columns of a tile column, and
// at step j the pivot column is broadcast to every lane of its row by the DPP
// row_newbcast modifier of the FMAs that use it.  Each lane then forms, for its own
// columns c >= j,
//     g_c = sum_{r>j} x_r a_r[c]        (c == j gives sigma)
// over its four rows per tile; the four 16-lane rows are summed with
// v_permlane16_swap / v_permlane32_swap (two exchanges, no LDS, no barrier).
// Row j of every column travels with the same two exchanges, so each lane
// ends up with  z_c = a_j[c] + g_c / (alpha - beta) = v^T a_c  and applies
// a_r[c] -= tau z_c v_r to its registers.
#include "device.hpp"
#include "kernels.hpp"

namespace fastqr {

namespace {

// 16-lane row R of v in every row: v_permlane32_swap(v, v) returns rows
// (0,1,0,1) and (2,3,2,3); v_permlane16_swap(w, w) then returns (w0,w0,w2,w2)
// and (w1,w1,w3,w3).  Two exchanges, no selects, no arithmetic.
template <int R>
__device__ __forceinline__ float row_broadcast(float v) {
  const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  const unsigned w = R < 2 ? h[0] : h[1];
  const auto q = __builtin_amdgcn_permlane16_swap(w, w, false, false);
  return __uint_as_float((R & 1) ? q[1] : q[0]);
}

// DPP rows (16-lane groups kq) whose register i holds a row below row JJ of
// the tile (rows 4kq + i); all four rows for a tile below the diagonal tile.
constexpr int below_rows(int jj, int i, bool diag) {
  int m = 0;
  for (int kq = 0; kq < 4; ++kq)
    if (!diag || 4 * kq + i > jj) m |= 1 << kq;
  return m;
}

// The pivot broadcast (row_newbcast:J, lane J of each 16-lane row) fused into
// v_fmac_f32_dpp, and the rows at or above the pivot skipped by the DPP row
// mask (a masked lane keeps its destination).  The compiler does not fold a
// row_newbcast move into an FMA, so the forms are written out; each block
// opens with the two wait states a DPP read needs after a VALU write of its
// source register ("s_nop 1"), which the compiler cannot see across asm.
//   g0 += b(x0) y0 + b(x2) y2,  g1 += b(x1) y1 + b(x3) y3
template <int J, int M0, int M1, int M2, int M3>
__device__ __forceinline__ void bdot4(float& g0, float& g1, const f32x4& x, const f32x4& y) {
  asm("s_nop 1\n\t"
      "v_fmac_f32_dpp %0, %2, %6 row_newbcast:%c10 row_mask:%c11 bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %1, %3, %7 row_newbcast:%c10 row_mask:%c12 bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %0, %4, %8 row_newbcast:%c10 row_mask:%c13 bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %1, %5, %9 row_newbcast:%c10 row_mask:%c14 bank_mask:0xf"
      : "+v"(g0), "+v"(g1)
      : "v"(x[0]), "v"(x[1]), "v"(x[2]), "v"(x[3]), "v"(y[0]), "v"(y[1]), "v"(y[2]), "v"(y[3]), "i"(J), "i"(M0),
        "i"(M1), "i"(M2), "i"(M3));
}

//   d_i += b(x_i) a
template <int J, int M0, int M1, int M2, int M3>
__device__ __forceinline__ void baxpy4(f32x4& d, const f32x4& x, float a) {
  float d0 = d[0], d1 = d[1], d2 = d[2], d3 = d[3];
  asm("s_nop 1\n\t"
      "v_fmac_f32_dpp %0, %4, %8 row_newbcast:%c9 row_mask:%c10 bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %1, %5, %8 row_newbcast:%c9 row_mask:%c11 bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %2, %6, %8 row_newbcast:%c9 row_mask:%c12 bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %3, %7, %8 row_newbcast:%c9 row_mask:%c13 bank_mask:0xf"
      : "+v"(d0), "+v"(d1), "+v"(d2), "+v"(d3)
      : "v"(x[0]), "v"(x[1]), "v"(x[2]), "v"(x[3]), "v"(a), "i"(J), "i"(M0), "i"(M1), "i"(M2), "i"(M3));
  d = f32x4{d0, d1, d2, d3};
}

//   x_i += b(x_i) a  (the pivot column's own tile: lane J keeps its value, a = 0 there)
template <int J, int M0, int M1, int M2, int M3>
__device__ __forceinline__ void baxpy4_self(f32x4& x, float a) {
  float x0 = x[0], x1 = x[1], x2 = x[2], x3 = x[3];
  asm("s_nop 1\n\t"
      "v_fmac_f32_dpp %0, %0, %4 row_newbcast:%c5 row_mask:%c6 bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %1, %1, %4 row_newbcast:%c5 row_mask:%c7 bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %2, %2, %4 row_newbcast:%c5 row_mask:%c8 bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %3, %3, %4 row_newbcast:%c5 row_mask:%c9 bank_mask:0xf"
      : "+v"(x0), "+v"(x1), "+v"(x2), "+v"(x3)
      : "v"(a), "i"(J), "i"(M0), "i"(M1), "i"(M2), "i"(M3));
  x = f32x4{x0, x1, x2, x3};
}

template <int... I>
struct seq {};
template <int N, int... I>
struct make_seq : make_seq<N - 1, N - 1, I...> {};
template <int... I>
struct make_seq<0, I...> {
  using type = seq<I...>;
};

}  // namespace

template <int NT>
struct WaveQR {
  f32x4 X[NT][NT];
  float tv[NT];   // lane cn: tau of column 16 tc + cn
  float inv[NT];  // lane cn: 1 / (alpha - beta) of column 16 tc + cn (applied after the last step)
  int kq, cn;

  // one Householder step on column J (compile-time), for n > J
  template <int J>
  __device__ __forceinline__ void step() {
    constexpr int TJ = J / 16, JJ = J % 16, KQJ = JJ / 4, IJ = JJ % 4;
    // row J of every column (register IJ of tile row TJ in DPP row KQJ),
    // broadcast to every row; alpha straight from its owner lane
    float rt[NT];
#pragma unroll
    for (int tc = TJ; tc < NT; ++tc) rt[tc] = row_broadcast<KQJ>(X[TJ][tc][IJ]);
    const float alpha = readlane(X[TJ][TJ][IJ], 16 * KQJ + JJ);
    // g_c = sum_{r > J} x_r a_r[c]: the pivot column broadcast along each
    // 16-lane row, rows <= J skipped by the row masks of the diagonal tile row
    constexpr int D0 = below_rows(JJ, 0, true), D1 = below_rows(JJ, 1, true);
    constexpr int D2 = below_rows(JJ, 2, true), D3 = below_rows(JJ, 3, true);
    float g[NT];
#pragma unroll
    for (int tc = TJ; tc < NT; ++tc) {
      float a0 = 0.0f, a1 = 0.0f;
      bdot4<JJ, D0, D1, D2, D3>(a0, a1, X[TJ][TJ], X[TJ][tc]);
#pragma unroll
      for (int tr = TJ + 1; tr < NT; ++tr) bdot4<JJ, 15, 15, 15, 15>(a0, a1, X[tr][TJ], X[tr][tc]);
      g[tc] = a0 + a1;
    }
#pragma unroll
    for (int tc = TJ; tc + 1 < NT; tc += 2) pair_row_sums(g[tc], g[tc + 1]);
    if constexpr (((NT - TJ) & 1) != 0) g[NT - 1] = xor32_sum(xor16_sum(g[NT - 1]));
    // lane JJ holds column J's totals
    const float sigma = readlane(g[TJ], JJ);
    const Reflector rf = make_reflector_sel(alpha, sigma);
    float alp[NT], s[NT];
#pragma unroll
    for (int tc = TJ; tc < NT; ++tc) {
      const float z = fmaf(g[tc], rf.inv, rt[tc]);
      s[tc] = (tc > TJ || cn > JJ) ? rf.tau * z : 0.0f;
      alp[tc] = -s[tc] * rf.inv;
    }
    // a_r[c] -= tau z_c v_r,  v_r = x_r * inv below row J (x is 0 at rows <= J);
    // the pivot column (s = 0) keeps its unscaled x: v = x * inv is applied
    // once after the last step
#pragma unroll
    for (int tc = TJ + 1; tc < NT; ++tc) {
      baxpy4<JJ, D0, D1, D2, D3>(X[TJ][tc], X[TJ][TJ], alp[tc]);
#pragma unroll
      for (int tr = TJ + 1; tr < NT; ++tr) baxpy4<JJ, 15, 15, 15, 15>(X[tr][tc], X[tr][TJ], alp[tc]);
    }
    baxpy4_self<JJ, D0, D1, D2, D3>(X[TJ][TJ], alp[TJ]);
#pragma unroll
    for (int tr = TJ + 1; tr < NT; ++tr) baxpy4_self<JJ, 15, 15, 15, 15>(X[tr][TJ], alp[TJ]);
    // row J: a_J[c] - s_c for c > J, beta on the diagonal
    {
      const bool row_j = kq == KQJ;  // selects, not a branch: a branch here makes
                                     // the compiler copy whole register quads
#pragma unroll
      for (int tc = TJ; tc < NT; ++tc) {
        const float a = X[TJ][tc][IJ];
        const float nv = (tc == TJ && cn == JJ) ? rf.beta : a - s[tc];
        X[TJ][tc][IJ] = row_j ? nv : a;
      }
    }
    tv[TJ] = (cn == JJ) ? rf.tau : tv[TJ];
    inv[TJ] = (cn == JJ) ? rf.inv : inv[TJ];
  }

  // v = x * inv below the diagonal of every column
  __device__ __forceinline__ void scale_reflectors() {
#pragma unroll
    for (int tr = 0; tr < NT; ++tr)
#pragma unroll
      for (int tc = 0; tc <= tr; ++tc)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = 16 * tr + 4 * kq + i, c = 16 * tc + cn;
          if (r > c) X[tr][tc][i] *= inv[tc];
        }
  }

  template <int... J>
  __device__ __forceinline__ void run(int n, seq<J...>) {
    // steps J < n in order (n here: the number of steps); the fold stops at
    // the first J >= n
    (void)((J < n ? (step<J>(), true) : false) && ...);
  }
};

// CM: A is column-major with 16-byte aligned columns (chosen on the host, so
// the row-major kernel carries no extra branch).
template <int NT, bool CM>
__global__ void __launch_bounds__(64) qr_wave_kernel(const float* __restrict__ A, int64_t as0, int64_t as1,
                                                      int64_t as2, float* __restrict__ H, int64_t hs0, int64_t hs1,
                                                      int64_t hs2, float* __restrict__ tau, int64_t ts0, int64_t ts1,
                                                      int n) {
  const int64_t b = blockIdx.x;
  const int lane = threadIdx.x;
  WaveQR<NT> q;
  q.kq = lane >> 4;
  q.cn = lane & 15;
  const float* Ab = A + b * as0;
  // Column-major source (CM): a lane's four rows of a column are one 16-byte
  // load (four lanes cover 64 contiguous bytes of each column).  Otherwise one
  // element per load, lanes along the columns of a row.
#pragma unroll
  for (int tr = 0; tr < NT; ++tr) {
#pragma unroll
    for (int tc = 0; tc < NT; ++tc) {
      const int c = 16 * tc + q.cn;
      const int r0 = 16 * tr + 4 * q.kq;
      if (CM && c < n && r0 + 3 < n) {
        q.X[tr][tc] = *reinterpret_cast<const f32x4*>(Ab + c * as2 + r0);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = r0 + i;
          q.X[tr][tc][i] = (r < n && c < n) ? Ab[r * as1 + c * as2] : 0.0f;
        }
      }
    }
    q.tv[tr] = 0.0f;
    q.inv[tr] = 0.0f;
  }

  // steps 0 .. n-2: the last column has no rows below its diagonal, so its
  // reflector is the identity (tau 0, R_nn = alpha), which the registers
  // already hold (tau and the scale start at 0; LAPACK's slarfg(1, ...) alike)
  q.run(n - 1, typename make_seq<16 * NT>::type{});
  q.scale_reflectors();

  float* Hb = H + b * hs0;
  const bool vec = hs1 == 1 && (hs2 & 3) == 0 && (hs0 & 3) == 0 && ((uintptr_t)H & 15) == 0;
#pragma unroll
  for (int tr = 0; tr < NT; ++tr) {
#pragma unroll
    for (int tc = 0; tc < NT; ++tc) {
      const int c = 16 * tc + q.cn;
      const int r0 = 16 * tr + 4 * q.kq;
      if (c < n) {
        if (vec && r0 + 3 < n) {
          *reinterpret_cast<f32x4*>(Hb + c * hs2 + r0) = q.X[tr][tc];
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (r0 + i < n) Hb[(r0 + i) * hs1 + c * hs2] = q.X[tr][tc][i];
        }
      }
    }
    const int c = 16 * tr + q.cn;
    if (q.kq == 0 && c < n) tau[b * ts0 + c * ts1] = q.tv[tr];
  }
}

hipError_t launch_qr_wave(const float* A, int64_t batch, int n, int64_t as0, int64_t as1, int64_t as2, float* H,
                          int64_t hs0, int64_t hs1, int64_t hs2, float* tau, int64_t ts0, int64_t ts1,
                          hipStream_t stream) {
  const dim3 grid((unsigned)batch);
  const dim3 block(64);
  const bool cm = as1 == 1 && (as2 & 3) == 0 && (as0 & 3) == 0 && ((uintptr_t)A & 15) == 0;
#define FASTQR_WAVE_LAUNCH(NT)                                                                                  \
  if (cm)                                                                                                       \
    hipLaunchKernelGGL((qr_wave_kernel<NT, true>), grid, block, 0, stream, A, as0, as1, as2, H, hs0, hs1, hs2, \
                       tau, ts0, ts1, n);                                                                       \
  else                                                                                                          \
    hipLaunchKernelGGL((qr_wave_kernel<NT, false>), grid, block, 0, stream, A, as0, as1, as2, H, hs0, hs1, hs2, \
                       tau, ts0, ts1, n)
  if (n <= 16) {
    FASTQR_WAVE_LAUNCH(1);
  } else if (n <= 32) {
    FASTQR_WAVE_LAUNCH(2);
  } else if (n <= 48) {
    FASTQR_WAVE_LAUNCH(3);
  } else if (n <= 64) {
    FASTQR_WAVE_LAUNCH(4);
  } else {
    return hipErrorInvalidValue;
  }
#undef FASTQR_WAVE_LAUNCH
  return hipGetLastError();
}

}  // namespace fastqr
