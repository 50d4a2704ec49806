// panel.hpp — panel factorisation (16- or 32-column panels), shared by the
// blocked path (qr_panel.hip: one workgroup per matrix, panel in global H) and
// the LDS-resident small-n path (qr_lds.hip: panel in LDS).
//
// Reference counterpart: blocked{n}_panel_factor_kernel and the T formation of
// blocked{n}_trailing_update_kernel (submissions/candidate.py:2404-2505,
// 2544-2584; T recurrence tools/blocked_qr_reference.py:98-109).
//
// Layout.  The panel's rows are split into 16-row tiles held in the
// v_mfma_f32_16x16x4f32 accumulator layout: lane (kq = lane/16, cn = lane%16)
// holds, for each tile it owns, rows 4kq..4kq+3 of column cn of block 0
// (panel columns 0-15) and, for 32-column panels, of block 1 (columns 16-31).
// Wave w owns tiles w, w+NW, ...  A 16-lane DPP row therefore holds 4 rows of
// all 16 columns of a block, so the pivot column j is broadcast along its row
// with the row_newbcast:j DPP modifier fused into the FMAs (v_fmac_f32_dpp).
//
// Column step j (one reduction for every column of the block):
//   lane (kq, cn) forms  sum_{r > j} x_r a_r[cn]  over its rows;  the four
//   16-lane rows of a wave are summed with v_permlane16_swap and
//   v_permlane32_swap and, with several waves, the waves through one LDS
//   exchange and one barrier (a one-wave panel has no LDS traffic and no
//   barrier in its column loop).  The total is sigma for cn == j, v^T a_cn
//   for cn > j (update scale) and v_cn^T v_j for cn < j.  Row j of every
//   column travels in the same exchange.  The reflector is formed without
//   branches and every lane updates its rows.  Column j of the block's T
//   factor is formed in the same step from the v_cn^T v_j values (slarft
//   recurrence, one DPP-broadcast FMA per earlier column), so no serial T
//   pass follows the loop.
//
// Block 0 is factored column by column; for 32-column panels its compact-WY
// transform is then applied to block 1 with MFMAs inside the kernel
// (P = V0^T X1 and W = T0^T P take both operands straight from registers
// through the contraction-index permutation; X1 += V0 W reads V0 transposed
// through LDS), block 1 is factored, and G = V0^T V1 joins the two 16x16 T
// factors into the panel's T = [[T0, -T0 G T1], [0, T1]].
#pragma once

#include <utility>

#include "device.hpp"

namespace fastqr {

namespace {

// The compiler's DPP combiner does not fold a row_newbcast move into an FMA, so
// the fused forms the column loop needs are written out.  Each block opens
// with "s_nop 1": the two wait states a DPP read needs after a VALU write of its
// source register, which the compiler's hazard tracking cannot see across asm.
// row_newbcast:J reads lane J of each 16-lane row; every lane is written.

// g0 += b(x0) y0 + b(x2) y2,  g1 += b(x1) y1 + b(x3) y3,  b = row_newbcast:J
template <int J>
__device__ __forceinline__ void bcast_dot4(float& g0, float& g1, f32x4 x, f32x4 y) {
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
__device__ __forceinline__ void bcast_axpy4(f32x4& x, float a0, float a1, float a2, float a3) {
  float x0 = x[0], x1 = x[1], x2 = x[2], x3 = x[3];
  asm("s_nop 1\n\t"
      "v_fmac_f32_dpp %0, %0, %4 row_newbcast:%c8 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %1, %1, %5 row_newbcast:%c8 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %2, %2, %6 row_newbcast:%c8 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %3, %3, %7 row_newbcast:%c8 row_mask:0xf bank_mask:0xf"
      : "+v"(x0), "+v"(x1), "+v"(x2), "+v"(x3)
      : "v"(a0), "v"(a1), "v"(a2), "v"(a3), "i"(J));
  x = f32x4{x0, x1, x2, x3};
}

// Two tiles per block (one "s_nop 1" for eight FMAs; inside a block no DPP
// source is written):  g0,g1 += tile a as above, g2,g3 += tile b
template <int J>
__device__ __forceinline__ void bcast_dot8(float& g0, float& g1, float& g2, float& g3, f32x4 xa, f32x4 ya,
                                           f32x4 xb, f32x4 yb) {
  asm("s_nop 1\n\t"
      "v_fmac_f32_dpp %0, %4, %8 row_newbcast:%c20 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %1, %5, %9 row_newbcast:%c20 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %2, %12, %16 row_newbcast:%c20 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %3, %13, %17 row_newbcast:%c20 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %0, %6, %10 row_newbcast:%c20 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %1, %7, %11 row_newbcast:%c20 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %2, %14, %18 row_newbcast:%c20 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %3, %15, %19 row_newbcast:%c20 row_mask:0xf bank_mask:0xf"
      : "+v"(g0), "+v"(g1), "+v"(g2), "+v"(g3)
      : "v"(xa[0]), "v"(xa[1]), "v"(xa[2]), "v"(xa[3]), "v"(ya[0]), "v"(ya[1]), "v"(ya[2]), "v"(ya[3]),
        "v"(xb[0]), "v"(xb[1]), "v"(xb[2]), "v"(xb[3]), "v"(yb[0]), "v"(yb[1]), "v"(yb[2]), "v"(yb[3]), "i"(J));
}

// xa_i += b(xa_i) a,  xb_i += b(xb_i) a
template <int J>
__device__ __forceinline__ void bcast_axpy8(f32x4& xa, f32x4& xb, float a) {
  float a0 = xa[0], a1 = xa[1], a2 = xa[2], a3 = xa[3];
  float b0 = xb[0], b1 = xb[1], b2 = xb[2], b3 = xb[3];
  asm("s_nop 1\n\t"
      "v_fmac_f32_dpp %0, %0, %8 row_newbcast:%c9 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %1, %1, %8 row_newbcast:%c9 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %2, %2, %8 row_newbcast:%c9 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %3, %3, %8 row_newbcast:%c9 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %4, %4, %8 row_newbcast:%c9 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %5, %5, %8 row_newbcast:%c9 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %6, %6, %8 row_newbcast:%c9 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %7, %7, %8 row_newbcast:%c9 row_mask:0xf bank_mask:0xf"
      : "+v"(a0), "+v"(a1), "+v"(a2), "+v"(a3), "+v"(b0), "+v"(b1), "+v"(b2), "+v"(b3)
      : "v"(a), "i"(J));
  xa = f32x4{a0, a1, a2, a3};
  xb = f32x4{b0, b1, b2, b3};
}

// acc += b(y) t,  b = row_newbcast:P
template <int P>
__device__ __forceinline__ void bcast_fma(float& acc, float y, float t) {
  asm("s_nop 1\n\t"
      "v_fmac_f32_dpp %0, %1, %2 row_newbcast:%c3 row_mask:0xf bank_mask:0xf"
      : "+v"(acc)
      : "v"(y), "v"(t), "i"(P));
}

template <class F, int... I>
__device__ __forceinline__ void unroll_seq(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}

__device__ __forceinline__ f32x4 mfma16(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}


}  // namespace

// The LDS a panel factorisation works in (NW waves, NBLK 16-column blocks).
// It does not depend on the tile count, so a kernel that factors panels of
// several heights with forms of different tile counts gives them one copy
// (panel_body_lds); panel_body declares its own.
template <int NW, int NBLK>
struct PanelLds {
  static constexpr int NWR = NW > 1 ? NW : 2;
  static constexpr int NPAIR = NBLK > 1 ? NBLK / 2 : 1;
  static constexpr int NW2 = NBLK > 1 ? NW : 1;
  static constexpr int PCH = NBLK > 4 ? 4 : (NBLK > 1 ? NBLK - 1 : 1);
  // red[parity][column][wave]: per-wave partials (sum, row j) of one column step
  __attribute__((aligned(16))) float2 red[2][16][NWR];
  // T of each 32-column slot (blocks 2p and 2p+1): [[T_2p, T_2p,2p+1], [0, T_2p+1]]
  float Ts[NPAIR][32][33];
  float Gs[16][17];
  float Mt[16][17];
  // block updates: partial products of up to PCH later blocks are summed over
  // the waves in one LDS round
  __attribute__((aligned(16))) f32x4 Pp[NW2][PCH][64];
  float Vt[NW2][16][17];
};

// Factor the panel described by `io` (m rows, up to 16 * NBLK columns) with NW
// waves (threads 0 .. NW*64-1 of the workgroup), TPW 16-row tiles per wave
// (rows covered: 16 * NW * TPW), NBLK 16-column blocks.  VEC: rows are loaded
// and stored four at a time.  `io` supplies the panel's storage (global H
// through a buffer descriptor, or LDS), where its T factor and tau go, and the
// barrier among the NW waves.  `tid` is the thread's index in the workgroup
// (a caller that factors many panels in one kernel passes it through an
// opaque copy, so that the lane masks derived from it are recomputed per
// panel instead of being held live across the caller's loop).
// L: the panel's LDS, which the caller may share between forms.
template <int NW, int TPW, int NBLK, bool VEC, class IO>
__device__ __forceinline__ void panel_body_lds(IO& io, int m, int tid, PanelLds<NW, NBLK>& L) {
  static_assert(NW == 1 || NW % 2 == 0, "wave count");
  static_assert(NBLK == 1 || NBLK == 2 || NBLK == 4 || NBLK == 8, "16-, 32-, 64- or 128-column panels");
  static_assert(NW * TPW >= NBLK, "the panel's diagonal tiles must exist");
  constexpr int NB = 16 * NBLK;
  const int w = m < NB ? m : NB;
  const int lane = tid & 63;
  const int wave = NW == 1 ? 0 : __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kq = lane >> 4;
  const int cn = lane & 15;

  constexpr int NPAIR = PanelLds<NW, NBLK>::NPAIR;
  constexpr int PCH = PanelLds<NW, NBLK>::PCH;
  auto& red = L.red;
  auto& Ts = L.Ts;
  auto& Gs = L.Gs;
  auto& Mt = L.Mt;
  auto& Pp = L.Pp;
  auto& Vt = L.Vt;
  for (int idx = tid; idx < NPAIR * 32 * 33; idx += NW * 64) (&Ts[0][0][0])[idx] = 0.0f;

  f32x4 X[NBLK][TPW];
#pragma unroll
  for (int blk = 0; blk < NBLK; ++blk) {
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      const int r = 16 * (wave + NW * t) + 4 * kq;
      const int c = 16 * blk + cn;
      if constexpr (VEC) {
        X[blk][t] = io.load4(r, c, c < w && r < m);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) X[blk][t][i] = io.load1(r + i, c, c < w && r + i < m);
      }
    }
  }
  float my_inv[NBLK], my_tau[NBLK];
#pragma unroll
  for (int blk = 0; blk < NBLK; ++blk) my_inv[blk] = my_tau[blk] = 0.0f;

  // ---- factor one 16-column block; lane cn returns row cn of the block's T --
  auto factor_block = [&](auto blk_c, float (&trow)[16]) {
    constexpr int BLK = decltype(blk_c)::value;
    // tile t may hold rows <= 16*BLK + 15 only if its first row 16*(wave + NW*t) <= 16*BLK
    constexpr int T_OWN = BLK / NW;  // tile of the owner wave holding the block's diagonal rows
    constexpr int W_OWN = BLK % NW;
#pragma unroll
    for (int jj = 0; jj < 16; ++jj) trow[jj] = 0.0f;  // columns past the panel width stay zero
    unroll_seq(
        [&](auto jj_c) {
          constexpr int JJ = decltype(jj_c)::value;
          constexpr int JG = 16 * BLK + JJ;  // column within the panel
          if (JG >= w) return;
          constexpr int PAR = JJ & 1;
          float g[4] = {0.0f, 0.0f, 0.0f, 0.0f};
          // tiles t < TD may hold rows <= JG (masked); the rest two per block
          constexpr int TD = (BLK / NW + 1 < TPW) ? BLK / NW + 1 : TPW;
#pragma unroll
          for (int t = 0; t < TD; ++t) {
            float* acc = g + 2 * (t & 1);
            const int rb = 16 * (wave + NW * t) + 4 * kq;
            f32x4 y;
#pragma unroll
            for (int i = 0; i < 4; ++i) y[i] = (rb + i > JG) ? X[BLK][t][i] : 0.0f;
            bcast_dot4<JJ>(acc[0], acc[1], X[BLK][t], y);
          }
#pragma unroll
          for (int t = TD; t + 1 < TPW; t += 2)
            bcast_dot8<JJ>(g[0], g[1], g[2], g[3], X[BLK][t], X[BLK][t], X[BLK][t + 1], X[BLK][t + 1]);
          if constexpr (((TPW - TD) & 1) != 0) bcast_dot4<JJ>(g[0], g[1], X[BLK][TPW - 1], X[BLK][TPW - 1]);
          float tot = (g[0] + g[1]) + (g[2] + g[3]);
          // row JG of my column: tile T_OWN of wave W_OWN, register JJ % 4 of lane row JJ / 4
          const bool row_owner = (wave == W_OWN) && (kq == JJ / 4);
          float rowt = row_owner ? X[BLK][T_OWN][JJ & 3] : 0.0f;
          pair_row_sums(tot, rowt);
          if constexpr (NW > 1) {
            if (kq == 0) red[PAR][cn][wave] = make_float2(tot, rowt);
            io.barrier();
            const float4* rp = reinterpret_cast<const float4*>(&red[PAR][cn][0]);
            float4 q[NW / 2];
#pragma unroll
            for (int k = 0; k < NW / 2; ++k) q[k] = rp[k];
            float2 s2[NW / 2];
#pragma unroll
            for (int k = 0; k < NW / 2; ++k) s2[k] = make_float2(q[k].x + q[k].z, q[k].y + q[k].w);
#pragma unroll
            for (int h = NW / 4; h >= 1; h >>= 1) {
#pragma unroll
              for (int k = 0; k < h; ++k) s2[k] = make_float2(s2[k].x + s2[k + h].x, s2[k].y + s2[k + h].y);
            }
            tot = s2[0].x;
            rowt = s2[0].y;
          }
          const float sigma = readlane(tot, JJ);
          const float alpha = readlane(rowt, JJ);
          const Reflector rf = make_reflector_sel(alpha, sigma);
          const float z = fmaf(tot, rf.inv, rowt);
          const float s = (cn > JJ) ? rf.tau * z : 0.0f;
          const float alp = -s * rf.inv;
#pragma unroll
          for (int t = 0; t < TD; ++t) {
            const int rb = 16 * (wave + NW * t) + 4 * kq;
            bcast_axpy4<JJ>(X[BLK][t], (rb > JG) ? alp : 0.0f, (rb + 1 > JG) ? alp : 0.0f,
                            (rb + 2 > JG) ? alp : 0.0f, (rb + 3 > JG) ? alp : 0.0f);
          }
#pragma unroll
          for (int t = TD; t + 1 < TPW; t += 2) bcast_axpy8<JJ>(X[BLK][t], X[BLK][t + 1], alp);
          if constexpr (((TPW - TD) & 1) != 0) bcast_axpy4<JJ>(X[BLK][TPW - 1], alp, alp, alp, alp);
          {
            const float a = X[BLK][T_OWN][JJ & 3];
            const float nv = (cn == JJ) ? rf.beta : a - s;
            X[BLK][T_OWN][JJ & 3] = row_owner ? nv : a;
          }
          // T column JJ:  T[i][JJ] = -tau * sum_{i <= p < JJ} T[i][p] y_p,  y_p = v_p^T v_JJ
          // (lane p holds y_p = inv_p * z_p; T[i][p] = 0 for p < i)
          const float y = my_inv[BLK] * z;
          float acc = 0.0f;
          unroll_seq([&](auto p_c) { bcast_fma<decltype(p_c)::value>(acc, y, trow[decltype(p_c)::value]); },
                     std::make_integer_sequence<int, JJ>{});
          trow[JJ] = (cn < JJ) ? -rf.tau * acc : (cn == JJ ? rf.tau : 0.0f);
          my_inv[BLK] = (cn == JJ) ? rf.inv : my_inv[BLK];
          my_tau[BLK] = (cn == JJ) ? rf.tau : my_tau[BLK];
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

  // sum an MFMA accumulator over the waves (result in every wave)
  auto wave_allreduce = [&](f32x4 v) -> f32x4 {
    if constexpr (NW == 1) {
      return v;
    } else {
      Pp[wave][0][lane] = v;
      io.barrier();
      f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int wv = 0; wv < NW; ++wv) s += Pp[wv][0][lane];
      io.barrier();
      return s;
    }
  };

  auto store_trow = [&](int blk, const float (&trow)[16]) {
    if (wave == 0 && kq == 0) {
      const int o = 16 * (blk & 1);
#pragma unroll
      for (int jj = 0; jj < 16; ++jj) Ts[blk >> 1][o + cn][o + jj] = trow[jj];
    }
  };

  // Apply block B's transform to every later block (right-looking inside the
  // panel): P_c = V_B^T X_c, W_c = -(T_B^T P_c), X_c += V_B W_c, with 16x16x4
  // MFMAs on the registers; V_B is transposed through a per-wave LDS tile once
  // per tile for all later blocks.
  auto apply_block = [&](auto b_c) {
    constexpr int B = decltype(b_c)::value;
    constexpr int NL = NBLK - 1 - B;  // later blocks
    constexpr int PO = B >> 1, OO = 16 * (B & 1);
    io.barrier();  // T_B in LDS
    f32x4 W[NL];
    unroll_seq(
        [&](auto c0_c) {
          constexpr int C0 = decltype(c0_c)::value * PCH;  // first later block of this chunk
          if constexpr (C0 < NL) {
            constexpr int NC = (NL - C0) < PCH ? (NL - C0) : PCH;
            f32x4 P[NC];
#pragma unroll
            for (int k = 0; k < NC; ++k) P[k] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int t = 0; t < TPW; ++t)
#pragma unroll
              for (int j = 0; j < 4; ++j) {
                const float v = vval(B, t, j);
#pragma unroll
                for (int k = 0; k < NC; ++k) P[k] = mfma16(v, X[B + 1 + C0 + k][t][j], P[k]);
              }
            if constexpr (NW > 1) {
#pragma unroll
              for (int k = 0; k < NC; ++k) Pp[wave][k][lane] = P[k];
              io.barrier();
#pragma unroll
              for (int k = 0; k < NC; ++k) {
                f32x4 sum = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int wv = 0; wv < NW; ++wv) sum += Pp[wv][k][lane];
                P[k] = sum;
              }
              io.barrier();
            }
#pragma unroll
            for (int k = 0; k < NC; ++k) {
              f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
              for (int j = 0; j < 4; ++j) acc = mfma16(Ts[PO][OO + 4 * kq + j][OO + cn], P[k][j], acc);
              W[C0 + k] = -acc;
            }
          }
        },
        std::make_integer_sequence<int, (NL + PCH - 1) / PCH>{});
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
#pragma unroll
      for (int i = 0; i < 4; ++i) Vt[wave][4 * kq + i][cn] = vval(B, t, i);
      wave_sync_lds();
      float vt[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) vt[j] = Vt[wave][cn][4 * kq + j];
#pragma unroll
      for (int k = 0; k < NL; ++k)
#pragma unroll
        for (int j = 0; j < 4; ++j) X[B + 1 + k][t] = mfma16(vt[j], W[k][j], X[B + 1 + k][t]);
      wave_sync_lds();
    }
  };

  // Join the T factors of blocks B-1 and B (B odd) into their 32-column slot:
  // T_{B-1,B} = -T_{B-1} G T_B with G = V_{B-1}^T V_B.
  auto join_pair = [&](auto b_c) {
    constexpr int B = decltype(b_c)::value;
    constexpr int PO = B >> 1;
    f32x4 G = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int t = 0; t < TPW; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) G = mfma16(vval(B - 1, t, j), vval(B, t, j), G);
    G = wave_allreduce(G);
    if (wave == 0) {
#pragma unroll
      for (int j = 0; j < 4; ++j) Gs[4 * kq + j][cn] = G[j];
    }
    io.barrier();  // Gs and T_B visible
    if (wave == 0) {
      const int i = lane >> 2, j0 = 4 * (lane & 3);
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < 16; ++k) acc = fmaf(Ts[PO][i][k], Gs[k][j0 + jj], acc);
        Mt[i][j0 + jj] = acc;
      }
      wave_sync_lds();
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < 16; ++k) acc = fmaf(Mt[i][k], Ts[PO][16 + k][16 + j0 + jj], acc);
        Ts[PO][i][16 + j0 + jj] = -acc;
      }
    }
  };

  io.barrier();  // zeroed T slots visible before any block writes its T
  unroll_seq(
      [&](auto b_c) {
        constexpr int B = decltype(b_c)::value;
        if (16 * B >= w) return;
        {
          float trow[16];
          factor_block(b_c, trow);
          store_trow(B, trow);
        }
        if constexpr ((B & 1) == 1) join_pair(b_c);
        if constexpr (B + 1 < NBLK) {
          if (16 * (B + 1) < w) apply_block(b_c);
        }
      },
      std::make_integer_sequence<int, NBLK>{});
  io.barrier();

  // write the panel, T (one 32 x 32 slot per 32 columns; a 16-column panel
  // fills the upper-left quarter of one slot) and tau.  For scalar loads and
  // for 16- and 32-column panels the lane's row and column go through an
  // opaque copy: the store offsets and bounds are then recomputed here instead
  // of being kept live (spilled, with scalar loads) since the loads.  64- and
  // 128-column panels keep them (measured on MI355X: 40 x 352 3% slower
  // otherwise).
  int kq_s = kq, cn_s = cn;
  if constexpr (!VEC || NBLK <= 2) asm volatile("" : "+v"(kq_s), "+v"(cn_s));
#pragma unroll
  for (int blk = 0; blk < NBLK; ++blk) {
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      const int r = 16 * (wave + NW * t) + 4 * kq_s;
      const int c = 16 * blk + cn_s;
      if constexpr (VEC) {
        io.store4(r, c, c < w && r < m, X[blk][t]);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) io.store1(r + i, c, c < w && r + i < m, X[blk][t][i]);
      }
    }
  }
  for (int idx = tid; idx < NPAIR * 32 * 32; idx += NW * 64) {
    const int p = idx >> 10, r = (idx >> 5) & 31, c = idx & 31;
    io.store_T(p, r, c, Ts[p][r][c]);
  }
  if (wave == 0 && kq == 0) {
#pragma unroll
    for (int blk = 0; blk < NBLK; ++blk) {
      const int c = 16 * blk + cn;
      if (c < w) io.store_tau(c, my_tau[blk]);
    }
  }
}

template <int NW, int TPW, int NBLK, bool VEC, class IO>
__device__ __forceinline__ void panel_body(IO& io, int m, int tid) {
  __shared__ PanelLds<NW, NBLK> L;
  panel_body_lds<NW, TPW, NBLK, VEC>(io, m, tid, L);
}

}  // namespace fastqr
