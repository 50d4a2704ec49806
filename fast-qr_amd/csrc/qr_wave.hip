// qr_wave.hip — batched QR for n <= 64: one wave64 per matrix.
//
// Reference counterpart: geqrf32_kernel, submissions/candidate.py:146-226
// (one warp32 per 32x32 matrix, rows across lanes, one warp reduction per
// (k, j) pair).  Here lane j owns column j in NR VGPRs, so no per-column
// reduction is needed: at step k lane k publishes its column through LDS and
// every lane forms, in registers,
//     sigma = sum_{i>k} x_i^2,   g_j = sum_{i>k} x_i a_j[i]
// and updates its own column with w_j = a_j[k] + g_j / (alpha - beta), which
// is v^T a_j for the reflector v = (1, x / (alpha - beta)).
#include "device.hpp"
#include "kernels.hpp"

namespace fastqr {

template <int NR, bool EXACT>
__global__ void __launch_bounds__(64) qr_wave_kernel(const float* __restrict__ A, int64_t as0,
                                                      int64_t as1, int64_t as2, float* __restrict__ H,
                                                      int64_t hs0, int64_t hs1, int64_t hs2,
                                                      float* __restrict__ tau, int64_t ts0, int64_t ts1,
                                                      int n_rt) {
  constexpr int UNROLL_K = EXACT ? NR : 1;
  const int n = EXACT ? NR : n_rt;
  const int64_t b = blockIdx.x;
  const int lane = threadIdx.x;
  __shared__ float xs[NR];
  __shared__ float tile[NR * (NR + 1)];

  float a[NR];
  const float* Ab = A + b * as0;
  const bool own = lane < n;
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    a[i] = (own && i < n) ? Ab[i * as1 + lane * as2] : 0.0f;
  }
  float my_tau = 0.0f;

#pragma unroll UNROLL_K
  for (int k = 0; k < n; ++k) {
    if (lane == k) {
#pragma unroll
      for (int i = 0; i < NR; ++i) xs[i] = a[i];
    }
    __syncthreads();
    float x[NR];
#pragma unroll
    for (int i = 0; i < NR; ++i) x[i] = (i > k) ? xs[i] : 0.0f;
    const float alpha = xs[k];
    float sigma = 0.0f;
    float g = 0.0f;
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      sigma = fmaf(x[i], x[i], sigma);
      g = fmaf(x[i], a[i], g);
    }
    const Reflector r = make_reflector(alpha, sigma);
    if (lane > k) {
      const float s = r.tau * fmaf(g, r.inv, a[k]);
#pragma unroll
      for (int i = 0; i < NR; ++i) {
        const float v = (i > k) ? x[i] * r.inv : (i == k ? 1.0f : 0.0f);
        a[i] = fmaf(-s, v, a[i]);
      }
    } else if (lane == k) {
#pragma unroll
      for (int i = 0; i < NR; ++i) {
        if (i > k) a[i] = x[i] * r.inv;
        if (i == k) a[i] = r.beta;
      }
      my_tau = r.tau;
    }
    __syncthreads();
  }

  if (own) tau[b * ts0 + lane * ts1] = my_tau;
  float* Hb = H + b * hs0;
  if (hs1 == 1) {
    // column-contiguous H: transpose through LDS so a store covers whole columns
    if (lane < NR) {
#pragma unroll
      for (int i = 0; i < NR; ++i) tile[lane * (NR + 1) + i] = a[i];
    }
    __syncthreads();
    constexpr int CPI = 64 / NR;  // columns per store instruction
    const int ri = lane % NR;
    const int cj = lane / NR;
#pragma unroll
    for (int it = 0; it < NR / CPI; ++it) {
      const int j = it * CPI + cj;
      if (ri < n && j < n) Hb[j * hs2 + ri] = tile[j * (NR + 1) + ri];
    }
  } else if (own) {
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      if (i < n) Hb[i * hs1 + lane * hs2] = a[i];
    }
  }
}

hipError_t launch_qr_wave(const float* A, int64_t batch, int n, int64_t as0, int64_t as1,
                          int64_t as2, float* H, int64_t hs0, int64_t hs1, int64_t hs2, float* tau,
                          int64_t ts0, int64_t ts1, hipStream_t stream) {
  const dim3 grid((unsigned)batch);
  const dim3 block(64);
#define FASTQR_WAVE_LAUNCH(NR, EX)                                                                   \
  hipLaunchKernelGGL((qr_wave_kernel<NR, EX>), grid, block, 0, stream, A, as0, as1, as2, H, hs0, hs1, \
                     hs2, tau, ts0, ts1, n)
  if (n == 32) {
    FASTQR_WAVE_LAUNCH(32, true);
  } else if (n == 16) {
    FASTQR_WAVE_LAUNCH(16, true);
  } else if (n == 64) {
    FASTQR_WAVE_LAUNCH(64, true);
  } else if (n < 16) {
    FASTQR_WAVE_LAUNCH(16, false);
  } else if (n < 32) {
    FASTQR_WAVE_LAUNCH(32, false);
  } else {
    FASTQR_WAVE_LAUNCH(64, false);
  }
#undef FASTQR_WAVE_LAUNCH
  return hipGetLastError();
}

}  // namespace fastqr
