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
// at step j the pivot column is broadcast to every lane of its row with one
// DPP row_newbcast move per register.  Each lane then forms, for its own
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

// lane J of this lane's 16-lane row
template <int J>
__device__ __forceinline__ float row_bcast(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x150 + J, 0xF, 0xF, false));
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
    // row J of every column: register IJ of tile row TJ in DPP row KQJ, zero
    // in the other rows, so the cross-row sums that total the dot products
    // also broadcast it to every lane
    float rt[NT];
#pragma unroll
    for (int tc = TJ; tc < NT; ++tc) rt[tc] = (kq == KQJ) ? X[TJ][tc][IJ] : 0.0f;
    // pivot column, broadcast along each 16-lane row; rows <= J masked
    f32x4 xb[NT];
#pragma unroll
    for (int tr = TJ; tr < NT; ++tr) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float v = row_bcast<JJ>(X[tr][TJ][i]);
        xb[tr][i] = (tr > TJ || 4 * kq + i > JJ) ? v : 0.0f;
      }
    }
    float g[NT];
#pragma unroll
    for (int tc = TJ; tc < NT; ++tc) {
      float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
      for (int tr = TJ; tr < NT; ++tr) {
        a0 = fmaf(xb[tr][0], X[tr][tc][0], a0);
        a1 = fmaf(xb[tr][1], X[tr][tc][1], a1);
        a0 = fmaf(xb[tr][2], X[tr][tc][2], a0);
        a1 = fmaf(xb[tr][3], X[tr][tc][3], a1);
      }
      g[tc] = a0 + a1;
    }
#pragma unroll
    for (int tc = TJ; tc < NT; ++tc) g[tc] = xor16_sum(g[tc]), rt[tc] = xor16_sum(rt[tc]);
#pragma unroll
    for (int tc = TJ; tc < NT; ++tc) g[tc] = xor32_sum(g[tc]), rt[tc] = xor32_sum(rt[tc]);
    const float alpha = readlane(rt[TJ], JJ);
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
    for (int tr = TJ; tr < NT; ++tr) {
#pragma unroll
      for (int tc = TJ; tc < NT; ++tc) {
#pragma unroll
        for (int i = 0; i < 4; ++i) X[tr][tc][i] = fmaf(alp[tc], xb[tr][i], X[tr][tc][i]);
      }
    }
    // row J: a_J[c] - s_c for c > J, beta on the diagonal
    if (kq == KQJ) {
#pragma unroll
      for (int tc = TJ; tc < NT; ++tc)
        X[TJ][tc][IJ] = (tc == TJ && cn == JJ) ? rf.beta : X[TJ][tc][IJ] - s[tc];
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
    // steps J < n in order; the fold stops at the first J >= n
    (void)((J < n ? (step<J>(), true) : false) && ...);
  }
};

template <int NT>
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
#pragma unroll
  for (int tr = 0; tr < NT; ++tr) {
#pragma unroll
    for (int tc = 0; tc < NT; ++tc) {
      const int c = 16 * tc + q.cn;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 16 * tr + 4 * q.kq + i;
        q.X[tr][tc][i] = (r < n && c < n) ? Ab[r * as1 + c * as2] : 0.0f;
      }
    }
    q.tv[tr] = 0.0f;
    q.inv[tr] = 0.0f;
  }

  q.run(n, typename make_seq<16 * NT>::type{});
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
#define FASTQR_WAVE_LAUNCH(NT) \
  hipLaunchKernelGGL((qr_wave_kernel<NT>), grid, block, 0, stream, A, as0, as1, as2, H, hs0, hs1, hs2, tau, ts0, ts1, n)
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
