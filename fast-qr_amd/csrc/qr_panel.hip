// qr_panel.hip — 32-column panel factorisation for panels of up to 2048 rows.
//
// Reference counterpart: blocked{n}_panel_factor_kernel and the T formation of
// blocked{n}_trailing_update_kernel (submissions/candidate.py:2404-2505,
// 2544-2584; T recurrence tools/blocked_qr_reference.py:98-109).
//
// Layout.  The panel's rows are split into 16-row tiles held in the
// v_mfma_f32_16x16x4f32 accumulator layout: lane (kq = lane/16, cn = lane%16)
// holds, for each tile it owns, rows 4kq..4kq+3 of column cn of block 0
// (panel columns 0-15) and of block 1 (columns 16-31).  Wave w owns tiles
// w, w+NW, ...  A 16-lane DPP row therefore holds 4 rows of all 16 columns of
// a block, so the pivot column j of a block is broadcast to its row with the
// row_newbcast:j DPP modifier fused into the FMAs (v_fmac_f32_dpp): no LDS
// traffic and no extra moves for the Householder vector.
//
// Block 0 is factored column by column (one reduction per column, as the
// wider kernel in qr_blocked.hip); its compact-WY transform is then applied
// to block 1 with MFMAs inside the kernel (P = V0^T X1 and W = T0^T P take
// both operands straight from registers through the contraction-index
// permutation; X1 += V0 W reads V0 transposed through LDS); block 1 is
// factored; G = V0^T V1 (MFMA) joins the two 16x16 T factors into the panel's
// 32x32 T = [[T0, -T0 G T1], [0, T1]].
#include <utility>

#include "device.hpp"
#include "kernels.hpp"

namespace fastqr {

typedef float f32x4v __attribute__((ext_vector_type(4)));

// The compiler's DPP combiner does not fold a row_newbcast move into an FMA, so
// the two fused forms the column loop needs are written out.  Each block opens
// with "s_nop 1": the two wait states a DPP read needs after a VALU write of its
// source register, which the compiler's hazard tracking cannot see across asm.
// row_newbcast:J reads lane J of each 16-lane row; every lane is written.

// g0 += b(x0) y0 + b(x2) y2,  g1 += b(x1) y1 + b(x3) y3,  b = row_newbcast:J
template <int J>
__device__ __forceinline__ void bcast_dot4(float& g0, float& g1, f32x4v x, f32x4v y) {
  asm("s_nop 1\n\t"
      "v_fmac_f32_dpp %0, %2, %6 row_newbcast:%c10 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %1, %3, %7 row_newbcast:%c10 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %0, %4, %8 row_newbcast:%c10 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %1, %5, %9 row_newbcast:%c10 row_mask:0xf bank_mask:0xf"
      : "+v"(g0), "+v"(g1)
      : "v"(x[0]), "v"(x[1]), "v"(x[2]), "v"(x[3]), "v"(y[0]), "v"(y[1]), "v"(y[2]), "v"(y[3]), "i"(J));
}

// x_i += b(x_i) a_i,  b = row_newbcast:J
template <int J>
__device__ __forceinline__ void bcast_axpy4(f32x4v& x, float a0, float a1, float a2, float a3) {
  float x0 = x[0], x1 = x[1], x2 = x[2], x3 = x[3];
  asm("s_nop 1\n\t"
      "v_fmac_f32_dpp %0, %0, %4 row_newbcast:%c8 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %1, %1, %5 row_newbcast:%c8 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %2, %2, %6 row_newbcast:%c8 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %3, %3, %7 row_newbcast:%c8 row_mask:0xf bank_mask:0xf"
      : "+v"(x0), "+v"(x1), "+v"(x2), "+v"(x3)
      : "v"(a0), "v"(a1), "v"(a2), "v"(a3), "i"(J));
  x = f32x4v{x0, x1, x2, x3};
}

template <class F, int... I>
__device__ __forceinline__ void unroll_seq(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}

__device__ __forceinline__ f32x4v mfma16(float a, float b, f32x4v c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

template <int NW, int TPW>
__global__ void __launch_bounds__(NW * 64) panel32_kernel(float* __restrict__ H, int64_t hs0, int64_t ldh,
                                                          float* __restrict__ tau, int64_t ts0, int64_t ts1,
                                                          float* __restrict__ Tws, int n, int k0, int slot) {
  const int64_t b = blockIdx.x;
  const int m = n - k0;
  const int w = m < 32 ? m : 32;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int kq = lane >> 4;
  const int cn = lane & 15;
  // panel element (row r, column c) at byte offset 4 * ((k0 + c) * ldh + k0 + r) of matrix b
  const rsrc_t rs = make_rsrc(H + b * hs0, (uint32_t)(4 * ldh * n));
  const uint32_t base = 4u * (uint32_t)(k0 * ldh + k0);
  auto off = [&](int r, int c) -> uint32_t { return base + 4u * (uint32_t)(c * ldh + r); };

  __shared__ float2 red[2][NW][16];
  __shared__ float ys[2][16][17];
  __shared__ float taus[32];
  __shared__ float Ts[32][33];
  __shared__ float Gs[16][17];
  __shared__ float Mt[16][17];
  __shared__ f32x4v Pp[NW][64];
  __shared__ float Vt[NW][16][17];

  f32x4v X[2][TPW];
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      const int r = 16 * (wave + NW * t) + 4 * kq;
      const int c = 16 * blk + cn;
      const bool ok = c < w && r < m;
      // rows r..r+3 are either all < m or all >= m when m % 4 == 0; otherwise per element
      if ((m & 3) == 0) {
        X[blk][t] = buf_load4(rs, ok ? off(r, c) : kOffNone);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) X[blk][t][i] = buf_load(rs, (c < w && r + i < m) ? off(r + i, c) : kOffNone);
      }
    }
  }
  float my_inv[2] = {0.0f, 0.0f};

  // ---- factor one 16-column block ------------------------------------------
  auto factor_block = [&](auto blk_c) {
    constexpr int BLK = decltype(blk_c)::value;
    unroll_seq(
        [&](auto jj_c) {
          constexpr int JJ = decltype(jj_c)::value;
          constexpr int JG = 16 * BLK + JJ;  // column within the panel
          if (JG >= w) return;
          constexpr int PAR = JJ & 1;
          // partial  sum_{r > JG} x_r a_r[cn]  over this lane's rows
          // (rows <= JG lie only in the first tile of each wave; they are masked there)
          const int rb0 = 16 * wave + 4 * kq;
          float g0 = 0.0f, g1 = 0.0f;
          {
            f32x4v y;
#pragma unroll
            for (int i = 0; i < 4; ++i) y[i] = (rb0 + i > JG) ? X[BLK][0][i] : 0.0f;
            bcast_dot4<JJ>(g0, g1, X[BLK][0], y);
          }
#pragma unroll
          for (int t = 1; t < TPW; ++t) bcast_dot4<JJ>(g0, g1, X[BLK][t], X[BLK][t]);
          float g = g0 + g1;
          // row JG of my column: tile BLK, row 4*(JJ/4) + JJ%4 of it
          constexpr int T_OWN = BLK / NW;
          float rowv = (wave == BLK % NW && kq == JJ / 4) ? X[BLK][T_OWN][JJ & 3] : 0.0f;
          g += xor_lane<16>(g);
          rowv += xor_lane<16>(rowv);
          g = xor32_sum(g);
          rowv = xor32_sum(rowv);
          float tot = g, rowt = rowv;
          if constexpr (NW > 1) {
            if (kq == 0) red[PAR][wave][cn] = make_float2(g, rowv);
            __syncthreads();
            tot = 0.0f;
            rowt = 0.0f;
#pragma unroll
            for (int wv = 0; wv < NW; ++wv) {
              const float2 p = red[PAR][wv][cn];
              tot += p.x;
              rowt += p.y;
            }
          }
          const float sigma = readlane(tot, JJ);
          const float alpha = readlane(rowt, JJ);
          const Reflector rf = make_reflector(alpha, sigma);
          const float z = fmaf(tot, rf.inv, rowt);
          const float s = (cn > JJ && 16 * BLK + cn < w) ? rf.tau * z : 0.0f;
          if (wave == 0 && kq == 0) {
            ys[BLK][cn][JJ] = (cn < JJ) ? my_inv[BLK] * z : z;
            if (cn == JJ) taus[JG] = rf.tau;
          }
          if (cn == JJ) my_inv[BLK] = rf.inv;
          const float alp = -s * rf.inv;
          bcast_axpy4<JJ>(X[BLK][0], (rb0 > JG) ? alp : 0.0f, (rb0 + 1 > JG) ? alp : 0.0f,
                          (rb0 + 2 > JG) ? alp : 0.0f, (rb0 + 3 > JG) ? alp : 0.0f);
#pragma unroll
          for (int t = 1; t < TPW; ++t) bcast_axpy4<JJ>(X[BLK][t], alp, alp, alp, alp);
          if (wave == BLK % NW && kq == JJ / 4) {
            const float a = X[BLK][T_OWN][JJ & 3];
            X[BLK][T_OWN][JJ & 3] = (cn == JJ) ? rf.beta : a - s;
          }
        },
        std::make_integer_sequence<int, 16>{});
    // v = x * inv below the diagonal
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      const int rbase = 16 * (wave + NW * t) + 4 * kq;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (rbase + i > 16 * BLK + cn) X[BLK][t][i] *= my_inv[BLK];
    }
  };

  // V of a block as an MFMA operand: unit diagonal, zeros above it
  auto vval = [&](int blk, int t, int i) -> float {
    const int r = 16 * (wave + NW * t) + 4 * kq + i;
    const int c = 16 * blk + cn;
    return r > c ? X[blk][t][i] : (r == c ? 1.0f : 0.0f);
  };

  // T of a block (16 x 16, slarft recurrence) into Ts at (16*blk, 16*blk)
  auto build_t = [&](int blk) {
    if (wave == 0 && lane < 16) {
      float trow[16];
#pragma unroll
      for (int jj = 0; jj < 16; ++jj) {
        float acc = 0.0f;
#pragma unroll
        for (int p = 0; p < jj; ++p) acc = fmaf(trow[p], ys[blk][p][jj], acc);
        const float tj = (16 * blk + jj < w) ? taus[16 * blk + jj] : 0.0f;
        trow[jj] = (lane < jj) ? -tj * acc : (lane == jj ? tj : 0.0f);
      }
#pragma unroll
      for (int jj = 0; jj < 16; ++jj) Ts[16 * blk + lane][16 * blk + jj] = trow[jj];
    }
  };

  // sum an MFMA accumulator over the waves (result in every wave)
  auto wave_allreduce = [&](f32x4v v) -> f32x4v {
    if constexpr (NW == 1) {
      return v;
    } else {
      Pp[wave][lane] = v;
      __syncthreads();
      f32x4v s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int wv = 0; wv < NW; ++wv) s += Pp[wv][lane];
      __syncthreads();
      return s;
    }
  };

  factor_block(std::integral_constant<int, 0>{});
  __syncthreads();
  build_t(0);

  if (w > 16) {
    __syncthreads();  // T0 in LDS
    // P = V0^T X1 (16 x 16)
    f32x4v P = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int t = 0; t < TPW; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) P = mfma16(vval(0, t, j), X[1][t][j], P);
    P = wave_allreduce(P);
    // W = -(T0^T P)
    f32x4v W = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < 4; ++j) W = mfma16(Ts[4 * kq + j][cn], P[j], W);
    W = -W;
    // X1 += V0 W, V0 transposed through a per-wave LDS tile
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
#pragma unroll
      for (int i = 0; i < 4; ++i) Vt[wave][4 * kq + i][cn] = vval(0, t, i);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int j = 0; j < 4; ++j) X[1][t] = mfma16(Vt[wave][cn][4 * kq + j], W[j], X[1][t]);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    factor_block(std::integral_constant<int, 1>{});
    __syncthreads();
    build_t(1);
    // G = V0^T V1
    f32x4v G = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int t = 0; t < TPW; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) G = mfma16(vval(0, t, j), vval(1, t, j), G);
    G = wave_allreduce(G);
    if (wave == 0) {
#pragma unroll
      for (int j = 0; j < 4; ++j) Gs[4 * kq + j][cn] = G[j];
    }
    __syncthreads();  // Gs and T1 visible
    // T01 = -(T0 G) T1 by wave 0, 4 entries per lane
    if (wave == 0) {
      const int i = lane >> 2, j0 = 4 * (lane & 3);
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < 16; ++k) acc = fmaf(Ts[i][k], Gs[k][j0 + jj], acc);
        Mt[i][j0 + jj] = acc;
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < 16; ++k) acc = fmaf(Mt[i][k], Ts[16 + k][16 + j0 + jj], acc);
        Ts[i][16 + j0 + jj] = -acc;
      }
    }
  } else {
    // a narrow last panel: the other quadrants of T are zero
    for (int idx = threadIdx.x; idx < 32 * 32; idx += NW * 64) {
      const int r = idx >> 5, c = idx & 31;
      if (r >= 16 || c >= 16) Ts[r][c] = 0.0f;
    }
  }
  if (w > 16) {
    for (int idx = threadIdx.x; idx < 16 * 16; idx += NW * 64) Ts[16 + (idx >> 4)][idx & 15] = 0.0f;
  }
  __syncthreads();

  // write the panel, T and tau
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      const int r = 16 * (wave + NW * t) + 4 * kq;
      const int c = 16 * blk + cn;
      if ((m & 3) == 0) {
        buf_store4(rs, (c < w && r < m) ? off(r, c) : kOffNone, X[blk][t]);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) buf_store(rs, (c < w && r + i < m) ? off(r + i, c) : kOffNone, X[blk][t][i]);
      }
    }
  }
  float* Tb = Tws + (b * kMaxSlots + slot) * 32 * 32;
  for (int idx = threadIdx.x; idx < 32 * 32; idx += NW * 64) Tb[idx] = Ts[idx >> 5][idx & 31];
  if (threadIdx.x < w) tau[b * ts0 + (int64_t)(k0 + threadIdx.x) * ts1] = taus[threadIdx.x];
}

hipError_t launch_panel32(float* H, int64_t batch, int64_t hs0, int64_t ldh, float* tau, int64_t ts0, int64_t ts1,
                          float* Tws, int n, int k0, int slot, hipStream_t stream) {
  const int m = n - k0;
  const dim3 grid((unsigned)batch);
#define FASTQR_P32(NW, TPW)                                                                                      \
  hipLaunchKernelGGL((panel32_kernel<NW, TPW>), grid, dim3(NW * 64), 0, stream, H, hs0, ldh, tau, ts0, ts1, Tws, n, \
                     k0, slot)
  // rows covered = 16 * NW * TPW
  if (m <= 128) {
    FASTQR_P32(2, 4);
  } else if (m <= 256) {
    FASTQR_P32(4, 4);
  } else if (m <= 512) {
    FASTQR_P32(4, 8);
  } else if (m <= 1024) {
    FASTQR_P32(8, 8);
  } else if (m <= 2048) {
    FASTQR_P32(16, 8);
  } else {
    return hipErrorInvalidValue;
  }
#undef FASTQR_P32
  return hipGetLastError();
}

}  // namespace fastqr
