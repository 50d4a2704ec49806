// qr_update.hip — row-split compact-WY trailing update for tall matrices and
// small batches.
//
// Reference counterpart: blocked{n}_trailing_update_kernel,
// submissions/candidate.py:2507-2716 (compact-WY mode, 2586-2672), which gives
// each CTA whole columns of the trailing matrix; with a batch of 2 or 8 that
// leaves most of the GPU idle, and a 4096-row strip does not fit in one
// workgroup's registers.  Here the rows are split too:
//
//   X <- X - V (T^T (V^T X))      V: m x k (k <= 128 reflectors of up to four
//                                 consecutive panels), T: k x k, X: m x c
//
//   wyr_partial_kernel  grid (32-column strips, row-block groups, batch), one
//                       wave per row block: P_rb = V_rb^T X_rb (fp32 MFMA
//                       32x32x2, X tiles as the B operand in accumulator
//                       layout); from 8 row blocks on, four per workgroup,
//                       their partials summed in LDS into one.  Strips inside
//                       the group's own columns are read as V (unit diagonal,
//                       zeros above), which gives the Gram matrix V^T V the
//                       group T needs.
//   wyr_tg_kernel       one workgroup per matrix: sums the Gram partials and
//                       joins the panels' T factors into the group T
//                       (T_[1:j] = [[T_[1:j-1], -T_[1:j-1] G_[1:j-1,j] T_j], [0, T_j]]).
//   wyr_w_kernel        four waves per strip: W = -T^T sum_rb P_rb.
//   wyr_apply_kernel    grid (strips, row blocks, batch), one wave: X_rb += V_rb W.
//
// Partial products are summed in a fixed order (no atomics), so results are
// bitwise reproducible.
#include "device.hpp"
#include "kernels.hpp"
#include "wy.hpp"

namespace fastqr {

namespace {

// Partial-product layout: one 32x32 block = 16 accumulator registers x 64
// lanes, quad-major: registers 4q .. 4q+3 of lane l at floats 256 q + 4 l ..
// +3, so every access instruction moves one contiguous KiB, 16 bytes per lane
// (a wave can hold at most 63 loads in flight: with 16-byte loads that is
// 16 blocks).
__device__ __forceinline__ int acc_off(int j, int lane) { return 256 * (j >> 2) + 4 * lane + (j & 3); }

__device__ __forceinline__ void store_acc(float* __restrict__ dst, const f32x16& v, int lane) {
#pragma unroll
  for (int q = 0; q < 4; ++q)
    *reinterpret_cast<f32x4*>(dst + acc_off(4 * q, lane)) = f32x4{v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
}

__device__ __forceinline__ f32x16 load_acc(const float* __restrict__ src, int lane) {
  f32x16 v;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const f32x4 x = *reinterpret_cast<const f32x4*>(src + acc_off(4 * q, lane));
#pragma unroll
    for (int i = 0; i < 4; ++i) v[4 * q + i] = x[i];
  }
  return v;
}

// row within a 32x32 block held by register j of a lane in half h
__device__ __forceinline__ int acc_row(int j, int h) { return 8 * (j >> 2) + 4 * h + (j & 3); }

}  // namespace

// Ppart index of (matrix b, strip s, row block rb, reflector block blk)
__device__ __forceinline__ int64_t pp_index(int64_t b, int s, int rb, int blk, int nstrips, int nrb) {
  return (((b * nstrips + s) * nrb + rb) * kWyrMaxBlk + blk) * 1024;
}

// Tiles of a row block are software-pipelined: the X and V loads of tile t+1
// are issued before the MFMAs of tile t (loads past the block read zeros
// through the buffer range check).
//
// SEPX: the updated columns are a matrix X of their own (xcols columns,
// leading dimension ldx, H's rows) (ormqr).  H holds vcols columns.
//
// PG waves per workgroup, one row block each (rb = PG * blockIdx.y + wave):
// with PG = 4 the four partials meet in LDS (added in wave order, so the sum
// is bitwise reproducible) and one partial per group of four row blocks is
// stored -- whoever forms W then sums a quarter as many (nrp = gridDim.y).
template <int NBLK, bool VEC, bool SEPX, int PG>
__global__ void __launch_bounds__(64 * PG) wyr_partial_kernel(const float* __restrict__ H, int64_t hs0, int ldh,
                                                              int n, int kv, int k, int c_begin, int c_end,
                                                              int gram_end, int rows_per_blk,
                                                              float* __restrict__ Ppart, int nstrips, int nrp, int hi,
                                                              const float* __restrict__ X_, int64_t xs0, int ldx,
                                                              int xcols, int vcols) {
  static_assert(PG == 1 || PG == 4, "row blocks per partial");
  if (hi) __builtin_amdgcn_s_setprio(2);
  const int wave = PG == 1 ? 0 : __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int s = blockIdx.x, rb = PG * (int)blockIdx.y + wave;
  const int64_t b = blockIdx.z;
  const int lane = threadIdx.x & 63, h = lane >> 5, l32 = lane & 31;
  const int col = c_begin + 32 * s + l32;
  const bool colok = col < c_end;
  const bool is_v = !SEPX && c_begin + 32 * s < gram_end;  // strip of the group's own columns: read as V
  const MatBuf M{make_rsrc(H + b * hs0, (uint32_t)(4 * ldh * vcols)), ldh, n};
  const MatBuf Mx = SEPX ? MatBuf{make_rsrc(X_ + b * xs0, (uint32_t)(4 * ldx * xcols)), ldx, n} : M;
  const int r_lo = kv + rb * rows_per_blk;
  const int r_hi = min(n, r_lo + rows_per_blk);

  auto load_x = [&](int r0) -> f32x16 {
    f32x16 x = tile_load<VEC>(Mx, r0, col, colok && r0 < r_hi, h);
    if (is_v) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int row = r0 + acc_row(j, h);
        x[j] = row < col ? 0.0f : (row == col ? 1.0f : x[j]);
      }
    }
    return x;
  };
  auto load_v = [&](int r0, f32x16 (&v)[NBLK]) {
#pragma unroll
    for (int blk = 0; blk < NBLK; ++blk) {
      const int kw = kv + 32 * blk;
      v[blk] = wy_load_va<VEC>(M, kw, min(32, k - 32 * blk), r0, h, l32, r0 < r_hi && r0 + 32 > kw);
    }
  };

  f32x16 P[NBLK];
#pragma unroll
  for (int blk = 0; blk < NBLK; ++blk)
#pragma unroll
    for (int j = 0; j < 16; ++j) P[blk][j] = 0.0f;

  f32x16 X = load_x(r_lo);
  f32x16 V[NBLK];
  load_v(r_lo, V);
  for (int r0 = r_lo; r0 < r_hi; r0 += 32) {
    const f32x16 Xn = load_x(r0 + 32);
    f32x16 Vn[NBLK];
    load_v(r0 + 32, Vn);
#pragma unroll
    for (int blk = 0; blk < NBLK; ++blk)
      if (r0 + 32 > kv + 32 * blk) wy_mfma_p(P[blk], V[blk], X);
    X = Xn;
#pragma unroll
    for (int blk = 0; blk < NBLK; ++blk) V[blk] = Vn[blk];
  }
  if constexpr (PG == 1) {
#pragma unroll
    for (int blk = 0; blk < NBLK; ++blk)
      store_acc(Ppart + pp_index(b, s, (int)blockIdx.y, blk, nstrips, nrp), P[blk], lane);
  } else {
    // one reflector block at a time through LDS; wave w adds and stores
    // register quarter w (one contiguous KiB of the partial's layout)
    __shared__ __attribute__((aligned(16))) float red[PG][1024];
#pragma unroll
    for (int blk = 0; blk < NBLK; ++blk) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<f32x4*>(&red[wave][256 * q + 4 * lane]) =
            f32x4{P[blk][4 * q], P[blk][4 * q + 1], P[blk][4 * q + 2], P[blk][4 * q + 3]};
      __syncthreads();
      f32x4 sum = *reinterpret_cast<const f32x4*>(&red[0][256 * wave + 4 * lane]);
#pragma unroll
      for (int v = 1; v < PG; ++v) sum += *reinterpret_cast<const f32x4*>(&red[v][256 * wave + 4 * lane]);
      *reinterpret_cast<f32x4*>(Ppart + pp_index(b, s, (int)blockIdx.y, blk, nstrips, nrp) + 256 * wave + 4 * lane) =
          sum;
      __syncthreads();  // every wave's reads before the next block's writes
    }
  }
}

// Sum of the row-block partials of one (strip, reflector block) by the four
// waves of a workgroup: wave w adds row blocks w, w + 4, ... with independent
// loads in flight, the four sums meet in LDS.  The order of additions is fixed
// (bitwise reproducible).  Returns the total in wave 0's registers.
constexpr int kSumWaves = 4;

__device__ __forceinline__ f32x16 wave_partial_sum(const float* __restrict__ Ppart, int64_t b, int s, int blk,
                                                   int nstrips, int nrb, int wave, int lane) {
  f32x16 acc;
#pragma unroll
  for (int j = 0; j < 16; ++j) acc[j] = 0.0f;
  int rb = wave;
  for (; rb + 3 * kSumWaves < nrb; rb += 4 * kSumWaves) {
    f32x16 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = load_acc(Ppart + pp_index(b, s, rb + u * kSumWaves, blk, nstrips, nrb), lane);
#pragma unroll
    for (int u = 0; u < 4; ++u) acc += v[u];
  }
  for (; rb < nrb; rb += kSumWaves) acc += load_acc(Ppart + pp_index(b, s, rb, blk, nstrips, nrb), lane);
  return acc;
}

// Sum the row-block partials of strips [0, gridDim.x) into Gsum (the Gram
// matrix V^T V of the group's own strips): one workgroup per (strip, block,
// matrix).
__global__ void __launch_bounds__(kSumWaves * 64) wyr_reduce_kernel(const float* __restrict__ Ppart, int nstrips,
                                                                    int nrb, float* __restrict__ Gsum, int hi) {
  if (hi) __builtin_amdgcn_s_setprio(2);
  const int s = blockIdx.x, blk = blockIdx.y;
  const int64_t b = blockIdx.z;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  __shared__ float red[kSumWaves][16][64];
  const f32x16 acc = wave_partial_sum(Ppart, b, s, blk, nstrips, nrb, wave, lane);
#pragma unroll
  for (int j = 0; j < 16; ++j) red[wave][j][lane] = acc[j];
  __syncthreads();
  if (wave == 0) {
    f32x16 tot;
#pragma unroll
    for (int j = 0; j < 16; ++j) tot[j] = (red[0][j][lane] + red[1][j][lane]) + (red[2][j][lane] + red[3][j][lane]);
    store_acc(Gsum + ((b * kWyrMaxBlk + blk) * kWyrMaxBlk + s) * 1024, tot, lane);
  }
}

// Group T (k x k, leading dimension kWyrTgLd) from the Gram matrix (Gsum) and
// the panels' T factors (q panels of width nb, 16 or 32, in workspace slots
// slot0 ..).
__global__ void __launch_bounds__(1024) wyr_tg_kernel(const float* __restrict__ Gsum, const float* __restrict__ Tws,
                                                      int slot0, int q, int nb, int k, float* __restrict__ Tg,
                                                      int hi) {
  if (hi) __builtin_amdgcn_s_setprio(2);
  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x;
  __shared__ float Gs[kWyrMaxK][kWyrMaxK + 1];
  __shared__ float Ts[kWyrMaxK][kWyrMaxK + 1];
  __shared__ float Mt[kWyrMaxK][33];
  const int nblk = (k + 31) / 32;
  // block (blk, s) of G = V_blk^T V_s, accumulator layout; the loads of a
  // thread's (up to 16) elements are all in flight before the LDS writes
  constexpr int kG = kWyrMaxBlk * kWyrMaxBlk;
  float gv[kG];
#pragma unroll
  for (int u = 0; u < kG; ++u) {
    const int idx = tid + u * 1024;
    const int pair = idx >> 10;
    const int blk = pair % nblk, s = pair / nblk;
    gv[u] = (idx < nblk * nblk * 1024) ? Gsum[((b * kWyrMaxBlk + blk) * kWyrMaxBlk + s) * 1024 + (idx & 1023)] : 0.0f;
  }
  // the panels' T factors on the diagonal (nb * nb <= 1024: one element per
  // thread and panel)
  float tv[kWyrMaxK / 16];
#pragma unroll
  for (int i = 0; i < kWyrMaxK / 16; ++i) {
    const int r = tid / nb, c = tid % nb;
    tv[i] = (i < q && tid < nb * nb && i * nb + r < k && i * nb + c < k)
                ? Tws[(b * kMaxSlots + slot0 + i) * 1024 + r * 32 + c]
                : 0.0f;
  }
#pragma unroll
  for (int u = 0; u < kG; ++u) {
    const int idx = tid + u * 1024;
    // float idx & 1023 of the block holds register j of lane `lane` (acc_off)
    const int lane = (idx >> 2) & 63, j = 4 * ((idx >> 8) & 3) + (idx & 3), pair = idx >> 10;
    const int blk = pair % nblk, s = pair / nblk;
    if (idx < nblk * nblk * 1024) Gs[32 * blk + acc_row(j, lane >> 5)][32 * s + (lane & 31)] = gv[u];
  }
  for (int idx = tid; idx < kWyrMaxK * kWyrMaxK; idx += 1024) Ts[idx / kWyrMaxK][idx % kWyrMaxK] = 0.0f;
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kWyrMaxK / 16; ++i) {
    const int r = tid / nb, c = tid % nb;
    if (i < q && tid < nb * nb && r <= c && i * nb + r < k && i * nb + c < k) Ts[i * nb + r][i * nb + c] = tv[i];
  }
  __syncthreads();
  // T join, one panel at a time, on v_mfma_f32_16x16x4f32 with both operands
  // read from LDS (lane l supplies A(l % 16, l / 16) and B(l / 16, l % 16);
  // accumulator register i of lane l is C(4 (l / 16) + i, l % 16)), one 16 x 16
  // output tile per wave and round:
  //   Mt = G[0:c0, c0:c0+nb] T_j,   T[0:c0, c0:c0+nb] = -T[0:c0, 0:c0] Mt.
  // Ts is zero below its diagonal and beyond k, so the products run over
  // whole 4-deep slices without masks (nb and c0 are multiples of 16).
  {
    const int wave = tid >> 6, lane = tid & 63;
    const int li = lane & 15, lk = lane >> 4;
    for (int j = 1; j < q; ++j) {
      const int c0 = j * nb;
      if (c0 >= k) break;
      const int tc = nb / 16, ntile = (c0 / 16) * tc;
      for (int t = wave; t < ntile; t += 16) {
        const int r0 = 16 * (t / tc), cc = 16 * (t % tc);
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int p = 0; p < nb; p += 4)
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(Gs[r0 + li][c0 + p + lk], Ts[c0 + p + lk][c0 + cc + li], acc, 0,
                                                     0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) Mt[r0 + 4 * lk + i][cc + li] = acc[i];
      }
      __syncthreads();
      for (int t = wave; t < ntile; t += 16) {
        const int r0 = 16 * (t / tc), cc = 16 * (t % tc);
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int p = r0; p < c0; p += 4)  // T(r, p) = 0 for p < r
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(Ts[r0 + li][p + lk], Mt[p + lk][cc + li], acc, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) Ts[r0 + 4 * lk + i][c0 + cc + li] = -acc[i];
      }
      __syncthreads();
    }
  }
  float* Tb = Tg + b * kWyrTgStride;
  for (int idx = tid; idx < kWyrMaxK * kWyrMaxK; idx += 1024) {
    const int r = idx / kWyrMaxK, c = idx % kWyrMaxK;
    Tb[r * kWyrTgLd + c] = (r < k && c < k) ? Ts[r][c] : 0.0f;
  }
}

// W = -T^T sum_rb P_rb for the strips [s0, s0 + gridDim.x) of Ppart; T is the
// k x k matrix at Tsrc (+ b * t_stride, leading dimension ldt).  Four waves:
// the row-block sums of every reflector block are split over the waves and
// combined in LDS; wave w then forms W block w (T upper triangular:
// W_w = sum_{p <= w} T(p, w)^T P_p), its T values loaded before its MFMAs.
template <int NBLK>
__global__ void __launch_bounds__(kSumWaves * 64) wyr_w_kernel(const float* __restrict__ Ppart, int nstrips, int nrb,
                                                               int s0, const float* __restrict__ Tsrc,
                                                               int64_t t_stride, int ldt, int k,
                                                               float* __restrict__ Wbuf, int nstrips_w, int hi,
                                                               int t_trans) {
  if (hi) __builtin_amdgcn_s_setprio(2);
  const int s = blockIdx.x;
  const int64_t b = blockIdx.y;
  const int lane = threadIdx.x & 63, h = lane >> 5, l32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  __shared__ float red[kSumWaves][NBLK][16][64];
#pragma unroll
  for (int blk = 0; blk < NBLK; ++blk) {
    const f32x16 acc = wave_partial_sum(Ppart, b, s0 + s, blk, nstrips, nrb, wave, lane);
#pragma unroll
    for (int j = 0; j < 16; ++j) red[wave][blk][j][lane] = acc[j];
  }
  __syncthreads();
  if (wave >= NBLK) return;
  const int blk = wave;
  const float* Tb = Tsrc + b * t_stride;
  f32x16 W;
#pragma unroll
  for (int j = 0; j < 16; ++j) W[j] = 0.0f;
#pragma unroll
  for (int bp = 0; bp < NBLK; ++bp) {
    // T upper triangular: block (bp, blk) of T (of T^T with t_trans) is zero for bp > blk (bp < blk)
    if (t_trans ? bp < blk : bp > blk) continue;
    float t[16];
    f32x16 P;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int kk = 32 * bp + acc_row(j, h);
      const int cc = 32 * blk + l32;
      // t_trans: W = -T P (T stored, read as T^T)
      t[j] = (kk < k && cc < k) ? Tb[t_trans ? cc * ldt + kk : kk * ldt + cc] : 0.0f;
      P[j] = (red[0][bp][j][lane] + red[1][bp][j][lane]) + (red[2][bp][j][lane] + red[3][bp][j][lane]);
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) W = __builtin_amdgcn_mfma_f32_32x32x2f32(t[j], P[j], W, 0, 0, 0);
  }
#pragma unroll
  for (int j = 0; j < 16; ++j) W[j] = -W[j];
  store_acc(Wbuf + ((b * nstrips_w + s) * kWyrMaxBlk + blk) * 1024, W, lane);
}

// W of one strip formed by a single wave (the fused variant of the apply
// kernel): the row-block partials summed in row-block order, then W = -T^T P
// as in wyr_w_kernel.  These launches hold one wave per CU or fewer, so the
// wave spends registers on latency: up to 16 partials (4 KiB each) are in
// flight at once (a 4096-row narrow update sums 32 of them).
template <int NBLK>
__device__ __forceinline__ void wave_form_w(f32x16 (&W)[NBLK], const float* __restrict__ Ppart, int64_t b, int s,
                                            int nstrips, int nrb, const float* __restrict__ Tb, int ldt, int k,
                                            int lane) {
  const int h = lane >> 5, l32 = lane & 31;
  constexpr int kInFlight = NBLK == 1 ? 16 : 8;
  f32x16 P[NBLK];
#pragma unroll
  for (int blk = 0; blk < NBLK; ++blk) {
#pragma unroll
    for (int j = 0; j < 16; ++j) P[blk][j] = 0.0f;
    int rb = 0;
    for (; rb + kInFlight <= nrb; rb += kInFlight) {
      f32x16 v[kInFlight];
#pragma unroll
      for (int u = 0; u < kInFlight; ++u) v[u] = load_acc(Ppart + pp_index(b, s, rb + u, blk, nstrips, nrb), lane);
#pragma unroll
      for (int u = 0; u < kInFlight; ++u) P[blk] += v[u];
    }
    for (; rb + 3 < nrb; rb += 4) {
      f32x16 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = load_acc(Ppart + pp_index(b, s, rb + u, blk, nstrips, nrb), lane);
#pragma unroll
      for (int u = 0; u < 4; ++u) P[blk] += v[u];
    }
    for (; rb < nrb; ++rb) P[blk] += load_acc(Ppart + pp_index(b, s, rb, blk, nstrips, nrb), lane);
  }
#pragma unroll
  for (int blk = 0; blk < NBLK; ++blk) {
    f32x16 acc;
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[j] = 0.0f;
#pragma unroll
    for (int bp = 0; bp <= blk; ++bp) {
      float t[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int kk = 32 * bp + acc_row(j, h);
        const int cc = 32 * blk + l32;
        t[j] = (kk < k && cc < k) ? Tb[kk * ldt + cc] : 0.0f;
      }
#pragma unroll
      for (int j = 0; j < 16; ++j) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(t[j], P[bp][j], acc, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) W[blk][j] = -acc[j];
  }
}

// FW: W formed in the kernel from the partials (Ppart, strips s0 + s) and T
// instead of read from Wbuf; every row block's wave repeats it, which costs
// less than the separate W launch on the critical path.
template <int NBLK, bool VEC, bool FW, bool SEPX>
__global__ void __launch_bounds__(64) wyr_apply_kernel(float* __restrict__ H, int64_t hs0, int ldh, int n, int kv,
                                                       int k, int c_begin, int c_end, int rows_per_blk,
                                                       const float* __restrict__ Wbuf, int nstrips_w, int hi,
                                                       const float* __restrict__ Ppart, int nstrips, int nrb, int s0,
                                                       const float* __restrict__ Tsrc, int64_t t_stride, int ldt,
                                                       float* __restrict__ X_, int64_t xs0, int ldx, int xcols,
                                                       int vcols) {
  if (hi) __builtin_amdgcn_s_setprio(2);
  const int s = blockIdx.x, rb = blockIdx.y;
  const int64_t b = blockIdx.z;
  const int lane = threadIdx.x, h = lane >> 5, l32 = lane & 31;
  const int col = c_begin + 32 * s + l32;
  const bool colok = col < c_end;
  const MatBuf M{make_rsrc(H + b * hs0, (uint32_t)(4 * ldh * vcols)), ldh, n};
  const MatBuf Mx = SEPX ? MatBuf{make_rsrc(X_ + b * xs0, (uint32_t)(4 * ldx * xcols)), ldx, n} : M;
  const int r_lo = kv + rb * rows_per_blk;
  const int r_hi = min(n, r_lo + rows_per_blk);
  f32x16 W[NBLK];
  if constexpr (FW) {
    wave_form_w<NBLK>(W, Ppart, b, s0 + s, nstrips, nrb, Tsrc + b * t_stride, ldt, k, lane);
  } else {
#pragma unroll
    for (int blk = 0; blk < NBLK; ++blk)
      W[blk] = load_acc(Wbuf + ((b * nstrips_w + s) * kWyrMaxBlk + blk) * 1024, lane);
  }

  auto load_v = [&](int r0, f32x16 (&v)[NBLK]) {
#pragma unroll
    for (int blk = 0; blk < NBLK; ++blk) {
      const int kw = kv + 32 * blk;
      v[blk] = wy_load_vb(M, kw, min(32, k - 32 * blk), r0, h, l32, r0 < r_hi && r0 + 32 > kw);
    }
  };
  f32x16 X = tile_load<VEC>(Mx, r_lo, col, colok, h);
  f32x16 V[NBLK];
  load_v(r_lo, V);
  for (int r0 = r_lo; r0 < r_hi; r0 += 32) {
    const f32x16 Xn = tile_load<VEC>(Mx, r0 + 32, col, colok && r0 + 32 < r_hi, h);
    f32x16 Vn[NBLK];
    load_v(r0 + 32, Vn);
#pragma unroll
    for (int blk = 0; blk < NBLK; ++blk)
      if (r0 + 32 > kv + 32 * blk) wy_mfma_apply(X, V[blk], W[blk]);
    tile_store<VEC>(Mx, r0, col, colok, h, X);
    X = Xn;
#pragma unroll
    for (int blk = 0; blk < NBLK; ++blk) V[blk] = Vn[blk];
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
// Partials stored per launch of nrb row blocks: one per four row blocks from
// 8 row blocks on (summed in the partial kernel's LDS), else one each.
static int wyr_partial_groups(int nrb) { return nrb >= 8 ? (nrb + 3) / 4 : nrb; }

int wyr_rows_per_block(int m, int64_t batch, int cols) {
  // enough waves to fill the GPU (about 1024 (strip, row block) pairs per
  // launch) with as few row blocks as possible (each adds a partial to sum)
  const int64_t strips = (cols + 31) / 32;
  int r = 512;
  while (r > 128 && batch * strips * ((m + r - 1) / r) < 1024) r >>= 1;
  // A batch of a few matrices still under that count at 128 rows: 32-row
  // blocks, one tile per wave (measured on MI355X, 2 x 4096: 128-row blocks
  // 13.3 ms, 64-row 12.9, 32-row with the partials grouped by four 12.2; for
  // 8 x 2048 smaller blocks gain nothing).  Only where the partials fit the
  // area wyr_workspace_floats sizes for 128-row blocks at m rows.
  if (batch <= 4 && batch * strips * ((m + 127) / 128) < 1024) {
    const int64_t nrp = wyr_partial_groups((m + 31) / 32);
    if (strips * nrp <= ((int64_t)(m + 31) / 32 + kWyrMaxBlk) * ((m + 127) / 128)) r = 32;
  }
  return r;
}

size_t wyr_workspace_floats(int64_t batch, int n) {
  const int64_t nstrips = (n + 31) / 32 + kWyrMaxBlk;
  const int64_t nrb = (n + 127) / 128;
  const int64_t pp = batch * nstrips * nrb * kWyrMaxBlk * 1024;
  const int64_t w = batch * nstrips * kWyrMaxBlk * 1024;
  const int64_t g = batch * kWyrMaxBlk * kWyrMaxBlk * 1024;
  return (size_t)(pp + w + g);
}

hipError_t launch_wyr(const WyrCall& c, hipStream_t stream) {
  const int m = c.n - c.kv;
  if (c.c_end <= c.c_begin || m <= 0 || c.k <= 0 || c.k > kWyrMaxK) return hipSuccess;
  if (c.gram && (c.nb % 16 != 0 || c.nb > 32 || c.q * c.nb > kWyrMaxK)) return hipErrorInvalidValue;  // the T join's tiles
  const int nblk = (c.k + 31) / 32;
  const int nrb = (m + c.rows_per_blk - 1) / c.rows_per_blk;
  // partials per four row blocks once there are 8 or more: W is formed (by
  // every apply wave on the critical path) from a quarter as many
  const int nrp = wyr_partial_groups(nrb);
  const int pg = nrp == nrb ? 1 : 4;
  const int nstrips = (c.c_end - c.c_begin + 31) / 32;
  const int gram_strips = c.gram ? nblk : 0;  // the first strips of [c_begin, c_end) are the group's own columns
  const int gram_end = c.gram ? c.kv + c.k : 0;
  const int hi = c.hi_prio ? 1 : 0;
  float* Ppart = c.scratch;
  float* Wbuf = c.scratch + (size_t)c.batch * nstrips * nrp * kWyrMaxBlk * 1024;
  const dim3 gp((unsigned)nstrips, (unsigned)nrp, (unsigned)c.batch);
  const bool sepx = c.X != nullptr;
  const int vcols = c.vcols > 0 ? c.vcols : c.n;
#define WYR_PARTIAL3(NB_, VEC_, SEPX_, PG_)                                                                       \
  hipLaunchKernelGGL((wyr_partial_kernel<NB_, VEC_, SEPX_, PG_>), gp, dim3(64 * PG_), 0, stream, c.H, c.hs0, c.ldh, \
                     c.n, c.kv, c.k, c.c_begin, c.c_end, gram_end, c.rows_per_blk, Ppart, nstrips, nrp, hi, c.X,     \
                     c.xs0, c.ldx, c.xcols, vcols)
#define WYR_PARTIAL2(NB_, VEC_, SEPX_)    \
  do {                                    \
    if (pg == 4)                          \
      WYR_PARTIAL3(NB_, VEC_, SEPX_, 4);  \
    else                                  \
      WYR_PARTIAL3(NB_, VEC_, SEPX_, 1);  \
  } while (0)
#define WYR_PARTIAL(NB_)                                                                                           \
  do {                                                                                                             \
    if (sepx) {                                                                                                    \
      if (c.vec)                                                                                                   \
        WYR_PARTIAL2(NB_, true, true);                                                                             \
      else                                                                                                         \
        WYR_PARTIAL2(NB_, false, true);                                                                            \
    } else if (c.vec) {                                                                                            \
      WYR_PARTIAL2(NB_, true, false);                                                                              \
    } else {                                                                                                       \
      WYR_PARTIAL2(NB_, false, false);                                                                             \
    }                                                                                                              \
  } while (0)
  switch (nblk) {
    case 1: WYR_PARTIAL(1); break;
    case 2: WYR_PARTIAL(2); break;
    case 3: WYR_PARTIAL(3); break;
    default: WYR_PARTIAL(4); break;
  }
#undef WYR_PARTIAL
#undef WYR_PARTIAL2
#undef WYR_PARTIAL3
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;

  const float* Tsrc = c.Tslot;
  int64_t t_stride = (int64_t)kMaxSlots * 1024;
  int ldt = 32;
  if (c.gram) {
    // Gram strips: sum the partials, then join the panels' T factors
    float* Gsum = Wbuf + (size_t)c.batch * nstrips * kWyrMaxBlk * 1024;
    hipLaunchKernelGGL(wyr_reduce_kernel, dim3((unsigned)gram_strips, (unsigned)nblk, (unsigned)c.batch),
                       dim3(kSumWaves * 64), 0,
                       stream, Ppart, nstrips, nrp, Gsum, hi);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL(wyr_tg_kernel, dim3((unsigned)c.batch), dim3(1024), 0, stream, Gsum, c.Tws, c.slot0, c.q, c.nb,
                       c.k, c.Tg, hi);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  if (c.use_tg) {
    Tsrc = c.Tg;
    t_stride = kWyrTgStride;
    ldt = kWyrTgLd;
  }
  const int nx = nstrips - gram_strips;  // strips that are updated
  if (nx <= 0) return hipSuccess;
  // critical-path updates form W inside the apply kernel (one launch fewer)
  const bool fw = c.hi_prio && !sepx && !c.t_trans;
  const dim3 gw((unsigned)nx, (unsigned)c.batch);
  if (!fw) switch (nblk) {
    case 1:
      hipLaunchKernelGGL((wyr_w_kernel<1>), gw, dim3(kSumWaves * 64), 0, stream, Ppart, nstrips, nrp, gram_strips, Tsrc, t_stride,
                         ldt, c.k, Wbuf, nx, hi, c.t_trans ? 1 : 0);
      break;
    case 2:
      hipLaunchKernelGGL((wyr_w_kernel<2>), gw, dim3(kSumWaves * 64), 0, stream, Ppart, nstrips, nrp, gram_strips, Tsrc, t_stride,
                         ldt, c.k, Wbuf, nx, hi, c.t_trans ? 1 : 0);
      break;
    case 3:
      hipLaunchKernelGGL((wyr_w_kernel<3>), gw, dim3(kSumWaves * 64), 0, stream, Ppart, nstrips, nrp, gram_strips, Tsrc, t_stride,
                         ldt, c.k, Wbuf, nx, hi, c.t_trans ? 1 : 0);
      break;
    default:
      hipLaunchKernelGGL((wyr_w_kernel<4>), gw, dim3(kSumWaves * 64), 0, stream, Ppart, nstrips, nrp, gram_strips, Tsrc, t_stride,
                         ldt, c.k, Wbuf, nx, hi, c.t_trans ? 1 : 0);
      break;
  }
  if ((e = hipGetLastError()) != hipSuccess) return e;
  const int xc_begin = c.c_begin + 32 * gram_strips;
  const dim3 ga((unsigned)nx, (unsigned)nrb, (unsigned)c.batch);
#define WYR_APPLY_FW(NB_, VEC_, FW_, SEPX_)                                                                        \
  hipLaunchKernelGGL((wyr_apply_kernel<NB_, VEC_, FW_, SEPX_>), ga, dim3(64), 0, stream, c.H, c.hs0, c.ldh, c.n, c.kv, \
                     c.k, xc_begin, c.c_end, c.rows_per_blk, Wbuf, nx, hi, Ppart, nstrips, nrp, gram_strips, Tsrc,   \
                     t_stride, ldt, c.X, c.xs0, c.ldx, c.xcols, vcols)
#define WYR_APPLY(NB_)                                                                                             \
  do {                                                                                                             \
    if (sepx && c.vec)                                                                                             \
      WYR_APPLY_FW(NB_, true, false, true);                                                                        \
    else if (sepx)                                                                                                 \
      WYR_APPLY_FW(NB_, false, false, true);                                                                       \
    else if (c.vec && fw)                                                                                          \
      WYR_APPLY_FW(NB_, true, true, false);                                                                        \
    else if (c.vec)                                                                                                \
      WYR_APPLY_FW(NB_, true, false, false);                                                                       \
    else if (fw)                                                                                                   \
      WYR_APPLY_FW(NB_, false, true, false);                                                                       \
    else                                                                                                           \
      WYR_APPLY_FW(NB_, false, false, false);                                                                      \
  } while (0)
  switch (nblk) {
    case 1: WYR_APPLY(1); break;
    case 2: WYR_APPLY(2); break;
    case 3: WYR_APPLY(3); break;
    default: WYR_APPLY(4); break;
  }
#undef WYR_APPLY
#undef WYR_APPLY_FW
  return hipGetLastError();
}

}  // namespace fastqr
