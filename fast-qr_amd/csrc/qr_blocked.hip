// qr_blocked.hip — blocked compact-WY Householder QR for n > 64: the copy of A
// into H and the trailing update.  The panel factorisation is in qr_panel.hip.
//
// Reference counterpart: geqrf{n}_blocked_cuda_impl and its kernels,
// submissions/candidate.py:2100-2161 (copy), 2507-2716 (trailing update),
// restricted to the full fp32 factorisation (factor_cols = n, no tail
// projection, no repair).
//
//   wy_update_kernel  grid = (32-column strips, batch).  A2 <- A2 - V (T^T (V^T A2))
//                     with v_mfma_f32_32x32x2f32.  A2 tiles are held in the MFMA
//                     accumulator layout and reused directly as the B operand of
//                     V^T A2 by permuting the contraction index (any order of
//                     the row sum is valid), so no register shuffles are needed.
#include <unordered_map>

#include "device.hpp"
#include "kernels.hpp"
#include "wy.hpp"

namespace fastqr {

// ---------------------------------------------------------------------------
// A (any strides) -> H (columns contiguous, leading dimension ldh)
// ---------------------------------------------------------------------------
// Copy modes: element loads (any strides), 16-byte row segments transposed
// through LDS (row-major source), 16-byte column segments (column-major).
constexpr int kCopyScalar = 0, kCopyRowVec = 1, kCopyColVec = 2;
// One 64 x 64 tile (row block ti, column block tj) of matrix b; columns >= c1
// are left alone.
__device__ __forceinline__ void copy_tile(const float* __restrict__ A, int64_t as0, int64_t as1, int64_t as2,
                                          float* __restrict__ H, int64_t hs0, int64_t ldh, int n, int c1, int mode,
                                          int64_t b, int ti, int tj, float (*tile)[65]) {
  const float* Ab = A + b * as0;
  float* Hb = H + b * hs0;
  const int tid = threadIdx.x;
  if (mode == kCopyColVec) {
    // column-major source, columns 16-byte aligned and n a multiple of 4: no
    // transpose, each thread moves four 16-byte column segments straight
    // through (16 threads cover 256 contiguous bytes of a column)
    const int i4 = 4 * (tid & 15);
    f32x4 v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int j = (tid >> 4) + 16 * k;
      const int gi = ti * 64 + i4, gj = tj * 64 + j;
      if (gi < n && gj < c1) v[k] = *reinterpret_cast<const f32x4*>(Ab + (int64_t)gj * as2 + gi);
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int j = (tid >> 4) + 16 * k;
      const int gi = ti * 64 + i4, gj = tj * 64 + j;
      if (gi < n && gj < c1) *reinterpret_cast<f32x4*>(Hb + (int64_t)gj * ldh + gi) = v[k];
    }
    return;
  }
  if (mode == kCopyRowVec) {
    // row-major source, every row and column a multiple of 16 bytes: each
    // thread moves four 16-byte row segments in and four column segments out
    const int c4 = 4 * (tid & 15);
    f32x4 v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int i = (tid >> 4) + 16 * k;
      const int gi = ti * 64 + i, gj = tj * 64 + c4;
      v[k] = (gi < n && gj < c1) ? *reinterpret_cast<const f32x4*>(Ab + (int64_t)gi * as1 + gj)
                                : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int i = (tid >> 4) + 16 * k;
#pragma unroll
      for (int e = 0; e < 4; ++e) tile[i][c4 + e] = v[k][e];
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int j = (tid >> 4) + 16 * k;
      const int gi = ti * 64 + c4, gj = tj * 64 + j;
      if (gi < n && gj < c1)
        *reinterpret_cast<f32x4*>(Hb + (int64_t)gj * ldh + gi) =
            f32x4{tile[c4][j], tile[c4 + 1][j], tile[c4 + 2][j], tile[c4 + 3][j]};
    }
    return;
  }
  if (as1 != 1) {
    // consecutive threads walk along j (row-major-like source)
    for (int idx = tid; idx < 64 * 64; idx += 256) {
      const int i = idx >> 6, j = idx & 63;
      const int gi = ti * 64 + i, gj = tj * 64 + j;
      tile[i][j] = (gi < n && gj < c1) ? Ab[gi * as1 + gj * as2] : 0.0f;
    }
  } else {
    for (int idx = tid; idx < 64 * 64; idx += 256) {
      const int j = idx >> 6, i = idx & 63;
      const int gi = ti * 64 + i, gj = tj * 64 + j;
      tile[i][j] = (gi < n && gj < c1) ? Ab[gi + gj * as2] : 0.0f;
    }
  }
  __syncthreads();
  for (int idx = tid; idx < 64 * 64; idx += 256) {
    const int j = idx >> 6, i = idx & 63;
    const int gi = ti * 64 + i, gj = tj * 64 + j;
    if (gi < n && gj < c1) Hb[(int64_t)gj * ldh + gi] = tile[i][j];
  }
}

// Tiles (matrix, row block, column block from tj0) in order, workgroup L
// taking tiles L, L + gridDim.x, ...: a grid smaller than the tile count
// leaves the CUs' other slots to kernels on another stream (an HBM-bound copy
// does not need them all).
__global__ void __launch_bounds__(256) copy_to_colmajor_kernel(const float* __restrict__ A, int64_t as0,
                                                                int64_t as1, int64_t as2,
                                                                float* __restrict__ H, int64_t hs0,
                                                                int64_t ldh, int n, int c1, int ntile, int ntj,
                                                                int tj0, int mode, int64_t total) {
  __shared__ float tile[64][65];
  const int per_matrix = ntile * ntj;
  for (int64_t L = blockIdx.x; L < total; L += gridDim.x) {
    const int64_t b = L / per_matrix;
    const int t = (int)(L - b * per_matrix);
    copy_tile(A, as0, as1, as2, H, hs0, ldh, n, c1, mode, b, t % ntile, tj0 + t / ntile, tile);
    __syncthreads();  // the next tile rewrites `tile`
  }
}

// ---------------------------------------------------------------------------
// Trailing update  A2 <- A2 - V T^T V^T A2  (fp32 MFMA 32x32x2)
// ---------------------------------------------------------------------------
// Applies `nwy` consecutive compact-WY transforms (last to first when `rev`),
// transform i starting at
// row and column kw = k0 + i*nb with width nb (<= 32) and T factor in
// workspace slot (slot0 + i), to the 32-column strip
// [c_begin + 32*strip, +32) of [c_begin, c_end), rows [k0, n).  The strip
// is split into 32-row tiles; wave w owns tiles w, w+NW, ...  With RES the
// tiles stay in VGPRs (MFMA accumulator layout) across all transforms: one
// load and one store per element.  Without RES (taller strips) each transform
// streams them twice.  Per transform: P = V^T X (the X registers are the B
// operand, the contraction index permuted to match the accumulator layout),
// P summed over waves in LDS, W = -(T^T P), X += V W.
//
// SEPX: the updated columns live in a matrix X of their own (xcols columns,
// leading dimension ldx, rows as H's) instead of H, and V is read from H's
// first vcols columns (ormqr: Q C or Q^T C with V, T from a factorisation).
//
// LOADA (strip-resident only): the strip's tiles are first read from the
// row-major input A (leading dimension lda, a_bytes per matrix) instead of H
// -- the first update of columns the blocked path did not copy -- and stored
// to H as usual.
template <int NW, int TPW, bool RES, bool VEC, bool SEPX, bool LOADA>
__device__ __forceinline__ void wy_update_item(float* __restrict__ H, int64_t hs0, int64_t ldh, int vcols,
                                               float* __restrict__ X_, int64_t xs0, int64_t ldx, int xcols,
                                               const float* __restrict__ Tws, int n, int k0, int nb, int slot0,
                                               int nwy, int rev, int c_begin, int c_end, int64_t b, int strip,
                                               const float* __restrict__ A, int64_t as0, int lda, uint32_t a_bytes) {
  static_assert(!LOADA || (RES && !SEPX), "A is read by the strip-resident geqrf update only");
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: scalar branches on tiles
  const int h = lane >> 5;
  const int l32 = lane & 31;
  const int m = n - k0;
  const int ntiles = (m + 31) >> 5;
  const int col = c_begin + 32 * strip + l32;
  const bool colok = col < c_end;
  const MatBuf M{make_rsrc(H + b * hs0, (uint32_t)(4 * ldh * (SEPX ? vcols : n))), (int)ldh, n};
  // the updated columns (H itself unless SEPX)
  const MatBuf Mx = SEPX ? MatBuf{make_rsrc(X_ + b * xs0, (uint32_t)(4 * ldx * xcols)), (int)ldx, n} : M;

  __shared__ float Ts[kMaxWY][32][33];
  __shared__ float Pt[16][64];
  // Per-wave LDS region: the wave's P partial (16 x 64) during the reduction
  // over waves, then (up to 8 waves) the transpose tile through which the
  // apply phase gets V from its pattern A registers.  A wave writes its
  // region only after the barrier that ends every wave's reads of the
  // partials, so the two uses never overlap.
  constexpr bool LT = RES && NW <= 8;
  constexpr int REG = LT ? 32 * 36 : 16 * 64;
  __shared__ __attribute__((aligned(16))) float Wreg[NW > 1 || LT ? NW : 1][REG];
  auto Pp = [&](int wv, int j) -> float* { return &Wreg[wv][j * 64]; };
  auto VTs = [&](int wv) { return reinterpret_cast<float (*)[36]>(&Wreg[wv][0]); };

  // The strip's tiles first, then the T factors with a chunk of loads in
  // flight before their LDS writes: the latencies overlap instead of one
  // global load per LDS write in turn.
  f32x16 X[TPW];
  if constexpr (LOADA) {
    const rsrc_t ra = make_rsrc(A + b * as0, a_bytes);
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      const int rt = wave + NW * t;
      X[t] = tile_load_rm(ra, lda, n, k0 + 32 * rt, col, colok && rt < ntiles, h);
    }
  } else if constexpr (RES) {
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      const int rt = wave + NW * t;
      X[t] = tile_load<VEC>(Mx, k0 + 32 * rt, col, colok && rt < ntiles, h);
    }
  }
  constexpr int kTChunk = 8;
  for (int base = threadIdx.x; base < nwy * 32 * 32; base += kTChunk * NW * 64) {
    float tv[kTChunk];
#pragma unroll
    for (int u = 0; u < kTChunk; ++u) {
      const int idx = base + u * NW * 64;
      const int i = idx >> 10, r = (idx >> 5) & 31, cc = idx & 31;
      tv[u] = (idx < nwy * 32 * 32 && r < nb && cc < nb) ? Tws[((b * kMaxSlots + slot0 + i) * 32 + r) * 32 + cc]
                                                         : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < kTChunk; ++u) {
      const int idx = base + u * NW * 64;
      if (idx < nwy * 32 * 32) Ts[idx >> 10][(idx >> 5) & 31][idx & 31] = tv[u];
    }
  }
  __syncthreads();

  for (int step = 0; step < nwy; ++step) {
    // rev: last transform first (backward accumulation of Q)
    const int i = rev ? nwy - 1 - step : step;
    const int kw = k0 + i * nb;
    const int rt_first = (kw - k0) >> 5;  // tiles above this transform are untouched
    // Row base made opaque per transform: the per-tile row indices and offsets
    // are then recomputed (one add each) instead of being hoisted out of this
    // loop and spilled.
    int kb = k0;
    asm volatile("" : "+v"(kb));
    f32x16 P;
#pragma unroll
    for (int j = 0; j < 16; ++j) P[j] = 0.0f;
    // V prefetch depth: 0 = each tile's V loads next to its MFMAs, 2 = the V
    // of all of this wave's tiles in flight at once, loaded before the P
    // MFMAs and kept (vb) for the apply phase, at the cost of TPW more tiles
    // of registers.  Measured on MI355X: it pays with
    // 8 waves per workgroup (tall strips, few workgroups per CU); the 4-wave
    // variants (short strips, many workgroups) gain more from the occupancy
    // the registers would cost, and 16 waves (128 registers each) leave no
    // room for it.
    constexpr int PFM = (RES && TPW > 1 && TPW <= 4 && NW == 8) ? 2 : 0;
    f32x16 vb[PFM == 2 ? TPW : 1];
    if constexpr (RES && PFM == 0) {
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        const int rt = wave + NW * t;
        if (rt < ntiles && rt >= rt_first) wy_accumulate<VEC>(P, X[t], M, kw, nb, kb + 32 * rt, h, l32);
        __builtin_amdgcn_sched_barrier(0);
      }
    } else if constexpr (RES) {
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        const int rt = wave + NW * t;
        vb[t] = wy_load_va<VEC>(M, kw, nb, kb + 32 * rt, h, l32, rt < ntiles && rt >= rt_first);
      }
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        const int rt = wave + NW * t;
        if (rt < ntiles && rt >= rt_first) wy_mfma_p(P, vb[t], X[t]);
      }
    } else {
      for (int rt = wave; rt < ntiles; rt += NW) {
        if (rt < rt_first) continue;
        const f32x16 Xs = tile_load<VEC>(Mx, k0 + 32 * rt, col, colok, h);
        wy_accumulate<VEC>(P, Xs, M, kw, nb, k0 + 32 * rt, h, l32);
      }
    }
    if constexpr (NW > 1) {
      // sum over waves: each wave reduces 16/NW of the registers
#pragma unroll
      for (int j = 0; j < 16; ++j) Pp(wave, j)[lane] = P[j];
      __syncthreads();
      constexpr int SL = 16 / NW;
#pragma unroll
      for (int jj = 0; jj < SL; ++jj) {
        const int j = wave * SL + jj;
        float acc = 0.0f;
#pragma unroll
        for (int wv = 0; wv < NW; ++wv) acc += Pp(wv, j)[lane];
        Pt[j][lane] = acc;
      }
      __syncthreads();
#pragma unroll
      for (int j = 0; j < 16; ++j) P[j] = Pt[j][lane];
    }
    f32x16 W;
#pragma unroll
    for (int j = 0; j < 16; ++j) W[j] = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int kk = 8 * (j >> 2) + 4 * h + (j & 3);
      W = __builtin_amdgcn_mfma_f32_32x32x2f32(Ts[i][kk][l32], P[j], W, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) W[j] = -W[j];
    if constexpr (RES && PFM == 0 && !LT) {
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        const int rt = wave + NW * t;
        if (rt < ntiles && rt >= rt_first) wy_apply(X[t], W, M, kw, nb, kb + 32 * rt, h, l32);
        __builtin_amdgcn_sched_barrier(0);
      }
    } else if constexpr (RES && PFM == 0) {
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        const int rt = wave + NW * t;
        if (rt < ntiles && rt >= rt_first) {
          const f32x16 va = wy_load_va<VEC>(M, kw, nb, kb + 32 * rt, h, l32, true);
          wy_mfma_apply(X[t], wy_transpose_va(VTs(wave), va, h, l32), W);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    } else if constexpr (RES) {
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        const int rt = wave + NW * t;
        if (rt < ntiles && rt >= rt_first) wy_mfma_apply(X[t], wy_transpose_va(VTs(wave), vb[t], h, l32), W);
      }
    } else {
      for (int rt = wave; rt < ntiles; rt += NW) {
        if (rt < rt_first) continue;
        f32x16 C = tile_load<VEC>(Mx, k0 + 32 * rt, col, colok, h);
        wy_apply(C, W, M, kw, nb, k0 + 32 * rt, h, l32);
        tile_store<VEC>(Mx, k0 + 32 * rt, col, colok, h, C);
      }
      // the next transform reloads what this wave stored
      __syncthreads();
    }
  }

  if constexpr (RES) {
    // recompute the store offsets rather than keeping the load offsets alive
    int kb = k0, cs = col;
    asm volatile("" : "+v"(kb), "+v"(cs));
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      const int rt = wave + NW * t;
      tile_store<VEC>(Mx, kb + 32 * rt, cs, colok && rt < ntiles, h, X[t]);
    }
  }
}

// One work item = one (matrix, 32-column strip).  Items are taken in an
// XCD-aware order: workgroups are dispatched round-robin over the 8 XCDs, so
// workgroup L runs on XCD L % 8, and item L goes to matrix (L % 8) + 8 k, so
// all strips of a matrix land on one XCD and the matrix's reflectors V, which
// every strip reads, are fetched into that XCD's L2 once.  A grid smaller
// than the item count loops (stride a multiple of 8, so each workgroup stays
// on its XCD's matrices): the caller uses it to leave CUs free for the
// critical-path kernels on the other stream.
template <int NW, int TPW, bool RES, bool VEC, bool SEPX, bool LOADA>
__global__ void __launch_bounds__(NW * 64)
__attribute__((amdgpu_waves_per_eu((TPW >= 2 && NW >= 4) || (TPW >= 4 && NW <= 4) ? 2 : 4, 8)))
wy_update_kernel(float* __restrict__ H, int64_t hs0, int64_t ldh, int vcols, float* __restrict__ X, int64_t xs0,
                 int64_t ldx, int xcols, const float* __restrict__ Tws, int n, int k0, int nb, int slot0, int nwy,
                 int rev, int c_begin, int c_end, int hi_prio, int nstrips, int batch, const float* __restrict__ A,
                 int64_t as0, int lda, uint32_t a_bytes) {
  // updates on the critical path (the rest of a panel group, the next group's
  // columns) win issue arbitration against the wide update they overlap
  if (hi_prio) __builtin_amdgcn_s_setprio(2);
  const int total = 8 * ((batch + 7) >> 3) * nstrips;
  for (int L = blockIdx.x; L < total; L += gridDim.x) {
    const int xk = L >> 3;
    const int64_t b = (L & 7) + 8 * (xk / nstrips);
    const int strip = xk % nstrips;
    if (b < batch)
      wy_update_item<NW, TPW, RES, VEC, SEPX, LOADA>(H, hs0, ldh, vcols, X, xs0, ldx, xcols, Tws, n, k0, nb, slot0,
                                                     nwy, rev, c_begin, c_end, b, strip, A, as0, lda, a_bytes);
    __syncthreads();  // the next item rewrites the LDS buffers
  }
}

// ---------------------------------------------------------------------------
// Host-side launchers
// ---------------------------------------------------------------------------
hipError_t launch_copy_colmajor(const float* A, int64_t batch, int n, int64_t as0, int64_t as1, int64_t as2,
                                float* H, int64_t hs0, int64_t ldh, int c0, int c1, hipStream_t stream, int max_wgs) {
  if (c0 < 0 || (c0 & 63) != 0 || c1 > n) return hipErrorInvalidValue;
  if (c1 <= c0) return hipSuccess;
  const int ntile = (n + 63) / 64;
  const int tj0 = c0 / 64, ntj = (c1 - c0 + 63) / 64;
  const bool h_vec = (ldh & 3) == 0 && (hs0 & 3) == 0 && ((uintptr_t)H & 15) == 0 && (n & 3) == 0 &&
                     (as0 & 3) == 0 && ((uintptr_t)A & 15) == 0;
  const int mode = (h_vec && as2 == 1 && (as1 & 3) == 0)   ? kCopyRowVec
                   : (h_vec && as1 == 1 && (as2 & 3) == 0) ? kCopyColVec
                                                           : kCopyScalar;
  const int64_t total = batch * ntile * ntj;
  int64_t grid = total < ((int64_t)1 << 30) ? total : ((int64_t)1 << 30);
  if (max_wgs > 0 && grid > max_wgs) grid = max_wgs;
  hipLaunchKernelGGL(copy_to_colmajor_kernel, dim3((unsigned)grid), dim3(256), 0, stream, A, as0, as1, as2, H, hs0, ldh,
                     n, c1, ntile, ntj, tj0, mode, total);
  return hipGetLastError();
}

namespace {

// Workgroups of `kernel` resident per CU (queried once per kernel and thread).
template <class K>
int wgs_per_cu(K kernel, int threads) {
  thread_local std::unordered_map<const void*, int> cache;
  const void* key = reinterpret_cast<const void*>(kernel);
  auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  int v = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, kernel, threads, 0) != hipSuccess || v < 1) v = 1;
  cache.emplace(key, v);
  return v;
}

// Compute units of the current device (queried once per device and thread).
int device_cus() {
  thread_local std::unordered_map<int, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 1;
  auto it = cache.find(dev);
  if (it != cache.end()) return it->second;
  int v = 0;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v < 1) v = 1;
  cache.emplace(dev, v);
  return v;
}

}  // namespace

// Shared by launch_wy_update (X = H) and launch_wy_apply (X a matrix of its
// own, SEPX): picks the (waves, tiles per wave) variant and the grid.
template <bool SEPX>
static hipError_t launch_wy(float* H, int64_t batch, int64_t hs0, int64_t ldh, int vcols, float* X, int64_t xs0,
                            int64_t ldx, int xcols, const float* Tws, int n, int k0, int nb, int slot0, int nwy,
                            int c_begin, int c_end, bool vec, bool hi_prio, int max_cus, hipStream_t stream,
                            bool reverse, const float* A = nullptr, int64_t as0 = 0, int64_t lda = 0) {
  const int cols = c_end - c_begin;
  if (cols <= 0 || nwy <= 0) return hipSuccess;
  const int ntiles = (n - k0 + 31) / 32;
  const int64_t strips = (cols + 31) / 32;
  const int64_t groups8 = (batch + 7) / 8;
  const int64_t items = 8 * groups8 * strips;
  if (items > 0x7fffffffLL) return hipErrorInvalidValue;
  const int ns = (int)strips, nbatch = (int)batch;
  // grid: every item, or at most max_cus CUs' worth of resident workgroups
  auto grid_for = [&](auto kernel, int threads) -> dim3 {
    int64_t g = items;
    int64_t cap = 0;
    if (max_cus > 0) {
      cap = ((int64_t)max_cus * wgs_per_cu(kernel, threads)) & ~(int64_t)7;
    } else if (max_cus == kWyLeaveOneSlot) {
      const int w = wgs_per_cu(kernel, threads);
      cap = ((int64_t)device_cus() * (w > 1 ? w - 1 : 1)) & ~(int64_t)7;
    }
    if (cap >= 8 && cap < g) g = cap;
    return dim3((unsigned)g);
  };
  // Tiles per wave: as few as the launch's size allows, so that a strip's
  // MFMA work is spread over several SIMDs when there are few strips (small
  // batches, narrow updates), and 4 per wave once the launch alone holds
  // about four waves per SIMD of the GPU.
  constexpr int64_t kWaveBudget = 4096;
  // At most 8 waves: 16-wave workgroups (128 registers a wave) spill and have
  // no room for the LDS transpose of V (measured on MI355X: 8 waves of 2-4
  // tiles make 40 x 352 7% and 60 x 1024 3% faster); taller strips use 8
  // waves of up to 8 tiles.
  int nw = 0, tpw = 0;
  for (int t = 1; t <= 4; t *= 2) {
    int w = 1;
    while (w * t < ntiles) w *= 2;
    if (w <= 8 && strips * batch * w <= kWaveBudget) {
      nw = w, tpw = t;
      break;
    }
  }
  if (nw == 0 && ntiles <= 32) {
    tpw = 4;
    nw = 1;
    while (nw * 4 < ntiles) nw *= 2;
  } else if (nw == 0) {
    nw = 8, tpw = 8;
  }
  const bool res = nw * tpw >= ntiles;
  const int prio = hi_prio ? 1 : 0;
  const int rv = reverse ? 1 : 0;
  const bool loada = !SEPX && A != nullptr;
  if (loada && !res) return hipErrorInvalidValue;  // only the strip-resident forms read A
  const uint32_t a_bytes = loada ? (uint32_t)(4 * ((int64_t)(n - 1) * lda + n)) : 0u;
  auto go = [&](auto kernel, int threads) -> hipError_t {
    hipLaunchKernelGGL(kernel, grid_for(kernel, threads), dim3(threads), 0, stream, H, hs0, ldh, vcols, X, xs0, ldx,
                       xcols, Tws, n, k0, nb, slot0, nwy, rv, c_begin, c_end, prio, ns, nbatch, A, as0, (int)lda,
                       a_bytes);
    return hipGetLastError();
  };
#define FASTQR_WY(NW, TPW, RES)                                                                     \
  if (nw == NW && tpw == TPW && res == RES) {                                                       \
    if constexpr (!SEPX) {                                                                          \
      if (loada)                                                                                    \
        return vec ? go(wy_update_kernel<NW, TPW, RES, true, SEPX, true>, NW * 64)                  \
                   : go(wy_update_kernel<NW, TPW, RES, false, SEPX, true>, NW * 64);                \
    }                                                                                               \
    return vec ? go(wy_update_kernel<NW, TPW, RES, true, SEPX, false>, NW * 64)                     \
               : go(wy_update_kernel<NW, TPW, RES, false, SEPX, false>, NW * 64);                   \
  }
  FASTQR_WY(1, 1, true)
  FASTQR_WY(2, 1, true)
  FASTQR_WY(4, 1, true)
  FASTQR_WY(8, 1, true)
  FASTQR_WY(1, 2, true)
  FASTQR_WY(2, 2, true)
  FASTQR_WY(4, 2, true)
  FASTQR_WY(8, 2, true)
  FASTQR_WY(1, 4, true)
  FASTQR_WY(2, 4, true)
  FASTQR_WY(4, 4, true)
  FASTQR_WY(8, 4, true)
  FASTQR_WY(8, 8, true)
#undef FASTQR_WY
  // strips taller than 8 waves x 8 tiles: stream the tiles
  return vec ? go(wy_update_kernel<16, 1, false, true, SEPX, false>, 1024)
             : go(wy_update_kernel<16, 1, false, false, SEPX, false>, 1024);
}

hipError_t launch_wy_update(float* H, int64_t batch, int64_t hs0, int64_t ldh, const float* Tws, int n,
                            int k0, int nb, int slot0, int nwy, int c_begin, int c_end, bool vec, bool hi_prio,
                            int max_cus, hipStream_t stream, bool reverse, const float* A, int64_t as0, int64_t lda) {
  return launch_wy<false>(H, batch, hs0, ldh, n, H, hs0, ldh, n, Tws, n, k0, nb, slot0, nwy, c_begin, c_end, vec,
                          hi_prio, max_cus, stream, reverse, A, as0, lda);
}

hipError_t launch_wy_apply(const float* V, int64_t batch, int64_t vs0, int64_t ldv, int vcols, float* C, int64_t cs0,
                           int64_t ldc, int ccols, const float* Tws, int m, int k0, int nb, int slot0, int nwy,
                           bool vec, hipStream_t stream, bool reverse) {
  return launch_wy<true>(const_cast<float*>(V), batch, vs0, ldv, vcols, C, cs0, ldc, ccols, Tws, m, k0, nb, slot0,
                         nwy, 0, ccols, vec, false, 0, stream, reverse);
}

}  // namespace fastqr
