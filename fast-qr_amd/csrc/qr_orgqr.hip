// qr_orgqr.hip — explicit Q from the compact-Householder output (H, tau):
// Q = H_0 H_1 ... H_{n-1}, the product torch.linalg.householder_product forms
// for the reference's checker (official/reference.py:199).
//
// Backward accumulation over 32-column panels, in place in Q (LAPACK sorgqr's
// order): Q starts as the reflectors V below the diagonal and zeros above it;
// for panel p = last .. 0 at column k0 the panel's block reflector
// B = I - V T V^T = H_k0 ... H_{k0+nb-1} is applied to the columns right of
// the panel (rows k0..n, where the later panels have already formed their part
// of Q), then the panel's own columns become B [I; 0] = [I; 0] - V (T V1^T),
// V1 the panel's top nb x nb unit lower triangle.
//
//   orgqr_init_kernel   Q <- strictly lower part of H (any strides), 0 above
//   orgqr_larft_kernel  per (panel, matrix): G = V^T V, T by the slarft
//                       recurrence, Y = T V1^T; T is stored transposed, so the
//                       trailing-update kernels (which apply A - V T_s^T V^T A
//                       with the stored T_s) apply B itself
//   orgqr_panel_kernel  the panel's own columns, Q[r, k0+c] = d(r-k0, c) - V[r,:] Y[:, c]
//   orgqr_small_kernel  n <= 32: all of the above for one matrix in one workgroup
#include "device.hpp"
#include "kernels.hpp"

namespace fastqr {

// One workgroup per (column, matrix): Q(i, j) = H(i, j) for i > j, else 0.
// Each element is read and written by the same thread, so Q may be H itself.
__global__ void __launch_bounds__(256) orgqr_init_kernel(const float* __restrict__ H, int64_t hs0, int64_t hs1,
                                                         int64_t hs2, float* __restrict__ Q, int64_t qs0,
                                                         int64_t ldq, int n) {
  const int j = blockIdx.x;
  const int64_t b = blockIdx.y;
  const float* hc = H + b * hs0 + (int64_t)j * hs2;
  float* qc = Q + b * qs0 + (int64_t)j * ldq;
  for (int i = threadIdx.x; i < n; i += 256) qc[i] = (i > j) ? hc[(int64_t)i * hs1] : 0.0f;
}

// T and Y of one 32-column panel.  Rows are staged through LDS 64 at a time
// (the next chunk's loads in flight while the current one is used); the four
// waves split each chunk's rows and accumulate G = V^T V with
// v_mfma_f32_32x32x2f32: for rows (r, r+1) lane (h, c) holds V(r+h, c), which
// is both its A element (V^T) and its B element (V).  The slarft recurrence
// T(i, j) = -tau_j sum_{i <= l < j} T(i, l) G(l, j) needs only row i of T, so
// lane i runs it alone.  The panel's reflectors are columns k0.. of the first
// nrefl (rows k0..n).  t_trans: store T^T (orgqr) or T itself (ormqr's Q^T C);
// Y is formed only when Yws is given.
__global__ void __launch_bounds__(256) orgqr_larft_kernel(const float* __restrict__ Q, int64_t qs0, int ldq, int n,
                                                          int nrefl, const float* __restrict__ tau, int64_t ts0,
                                                          int64_t ts1, int64_t batch, float* __restrict__ Tws,
                                                          float* __restrict__ Yws, int t_trans, int p_off) {
  const int p = p_off + blockIdx.x;
  const int64_t b = blockIdx.y;
  const int k0 = 32 * p;
  const int nb = min(32, nrefl - k0);
  const int m = n - k0;
  const float* Qb = Q + b * qs0;
  const int t = threadIdx.x;
  const int lane = t & 63, h = lane >> 5, l32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);

  __shared__ float Vs[64][33];
  __shared__ float V1s[32][33];
  __shared__ float Gs[32][33];
  __shared__ float Ts[32][33];
  __shared__ float Gp[4][16][64];
  __shared__ float taus[32];
  if (t < 32) taus[t] = (t < nb) ? tau[b * ts0 + (int64_t)(k0 + t) * ts1] : 0.0f;

  // element u of this thread's share of a 64 x 32 chunk: column c, chunk row rr
  auto fetch = [&](int r0, float (&v)[8]) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int idx = t + 256 * u;
      const int c = idx >> 6, r = r0 + (idx & 63);
      float x = 0.0f;
      if (c < nb && r < m) x = (r == c) ? 1.0f : (r < c ? 0.0f : Qb[(int64_t)(k0 + c) * ldq + k0 + r]);
      v[u] = x;
    }
  };
  f32x16 acc;
#pragma unroll
  for (int j = 0; j < 16; ++j) acc[j] = 0.0f;
  float nxt[8];
  fetch(0, nxt);
  for (int r0 = 0; r0 < m; r0 += 64) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int idx = t + 256 * u;
      Vs[idx & 63][idx >> 6] = nxt[u];
    }
    __syncthreads();
    if (r0 == 0) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int idx = t + 256 * u;
        V1s[idx >> 5][idx & 31] = Vs[idx >> 5][idx & 31];
      }
    }
    if (r0 + 64 < m) fetch(r0 + 64, nxt);
    // rows past m were staged as zeros: the whole chunk can be summed
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float v = Vs[16 * wave + 2 * k + h][l32];
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(v, v, acc, 0, 0, 0);
    }
    __syncthreads();
  }
#pragma unroll
  for (int j = 0; j < 16; ++j) Gp[wave][j][lane] = acc[j];
  __syncthreads();
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int e = t + 256 * u;
    const int j = e >> 6, ln = e & 63;
    const float g = (Gp[0][j][ln] + Gp[1][j][ln]) + (Gp[2][j][ln] + Gp[3][j][ln]);
    Gs[8 * (j >> 2) + 4 * (ln >> 5) + (j & 3)][ln & 31] = g;
  }
  __syncthreads();

  // Row i of T in registers, every loop unrolled: the G loads of a step do not
  // wait on its FMA chain (T(i, l) = 0 for l < i, so the sum over l < j only
  // picks up l >= i; G is symmetric, so row j of Gs is column j of G).
  if (t < 32) {
    const int i = t;
    float trow[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      float acc_s = 0.0f;
#pragma unroll
      for (int l = 0; l < j; ++l) acc_s = fmaf(trow[l], Gs[j][l], acc_s);
      const float tj = taus[j];  // 0 for j >= nb
      trow[j] = (i == j) ? tj : (i < j ? -tj * acc_s : 0.0f);
    }
#pragma unroll
    for (int j = 0; j < 32; ++j) Ts[i][j] = trow[j];
  }
  __syncthreads();

  const int64_t slot = ((int64_t)(p / kMaxSlots) * batch + b) * kMaxSlots + (p % kMaxSlots);
  float* To = Tws + slot * 1024;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int idx = t + 256 * u;
    const int r = idx >> 5, c = idx & 31;
    To[idx] = t_trans ? Ts[c][r] : Ts[r][c];
  }
  if (Yws == nullptr) return;
  float* Yo = Yws + slot * 1024;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int idx = t + 256 * u;
    const int r = idx >> 5, c = idx & 31;
    // Y(r, c) = sum_l T(r, l) V1(c, l): T is zero left of its diagonal and V1
    // (staged with its unit diagonal and zeros) right of its own
    float y = 0.0f;
#pragma unroll
    for (int l = 0; l < 32; ++l) y = fmaf(Ts[r][l], V1s[c][l], y);
    Yo[idx] = y;
  }
}

// The panel's own columns: thread = row r of [k0, n); reads its row of V,
// writes its row of Q (in place: no other thread touches that row).
__global__ void __launch_bounds__(256) orgqr_panel_kernel(float* __restrict__ Q, int64_t qs0, int ldq, int n, int p,
                                                          int64_t batch, const float* __restrict__ Yws) {
  const int64_t b = blockIdx.y;
  const int k0 = 32 * p;
  const int nb = min(32, n - k0);
  __shared__ float Ys[32][33];
  const float* Yp = Yws + (((int64_t)(p / kMaxSlots) * batch + b) * kMaxSlots + (p % kMaxSlots)) * 1024;
  for (int idx = threadIdx.x; idx < 1024; idx += 256) Ys[idx >> 5][idx & 31] = Yp[idx];
  __syncthreads();
  const int rr = blockIdx.x * 256 + threadIdx.x;  // row within the panel
  if (rr >= n - k0) return;
  float* Qc = Q + b * qs0 + (int64_t)k0 * ldq + k0 + rr;
  float v[32];
#pragma unroll
  for (int l = 0; l < 32; ++l) {
    float x = 0.0f;
    if (l < nb) x = (l == rr) ? 1.0f : (l > rr ? 0.0f : Qc[(int64_t)l * ldq]);
    v[l] = x;
  }
#pragma unroll
  for (int c = 0; c < 32; ++c) {
    float s = 0.0f;
#pragma unroll
    for (int l = 0; l < 32; ++l) s = fmaf(v[l], Ys[l][c], s);
    if (c < nb) Qc[(int64_t)c * ldq] = (c == rr ? 1.0f : 0.0f) - s;
  }
}

// Small batches of tall matrices: the narrow updates inside a panel group run
// on the row-split kernels, spread over row blocks (as geqrf's narrow updates).
static bool orgqr_narrow_rowsplit(int64_t batch, int n) { return batch <= 16 && n > 1024; }

// n <= 32 (a single panel): one workgroup of four waves per matrix does the
// whole product in LDS, V read straight from H (any strides): G = V^T V, T (row i in lane i's
// registers), Y = T V^T, Q = I - V Y.  Every read of H precedes the first
// barrier and every write of Q follows it, so Q may be H itself.
__global__ void __launch_bounds__(256) orgqr_small_kernel(const float* __restrict__ H, int64_t hs0, int64_t hs1,
                                                         int64_t hs2, const float* __restrict__ tau, int64_t ts0,
                                                         int64_t ts1, float* __restrict__ Q, int64_t qs0, int64_t ldq,
                                                         int n) {
  const int64_t b = blockIdx.x;
  const int t = threadIdx.x;
  __shared__ float Vs[32][33];
  __shared__ float Gs[32][33];
  __shared__ float Ts[32][33];
  __shared__ float taus[32];
  const float* Hb = H + b * hs0;
  for (int e = t; e < 1024; e += 256) {
    const int r = e & 31, c = e >> 5;
    float x = 0.0f;
    if (r < n && c < n) x = (r == c) ? 1.0f : (r < c ? 0.0f : Hb[r * hs1 + c * hs2]);
    Vs[r][c] = x;
  }
  if (t < 32) taus[t] = (t < n) ? tau[b * ts0 + t * ts1] : 0.0f;
  __syncthreads();
  for (int e = t; e < 1024; e += 256) {
    const int i = e >> 5, j = e & 31;
    float g = 0.0f;
#pragma unroll
    for (int r = 0; r < 32; ++r) g = fmaf(Vs[r][i], Vs[r][j], g);
    Gs[i][j] = g;
  }
  __syncthreads();
  if (t < 32) {
    const int i = t;
    float trow[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      float acc_s = 0.0f;
#pragma unroll
      for (int l = 0; l < j; ++l) acc_s = fmaf(trow[l], Gs[j][l], acc_s);  // G symmetric
      const float tj = taus[j];
      trow[j] = (i == j) ? tj : (i < j ? -tj * acc_s : 0.0f);
    }
#pragma unroll
    for (int j = 0; j < 32; ++j) Ts[i][j] = trow[j];
  }
  __syncthreads();
  for (int e = t; e < 1024; e += 256) {  // Y into Gs: Y(i, c) = sum_l T(i, l) V(c, l)
    const int i = e >> 5, c = e & 31;
    float y = 0.0f;
#pragma unroll
    for (int l = 0; l < 32; ++l) y = fmaf(Ts[i][l], Vs[c][l], y);
    Gs[i][c] = y;
  }
  __syncthreads();
  float* Qb = Q + b * qs0;
  for (int e = t; e < 1024; e += 256) {
    const int r = e & 31, c = e >> 5;
    float s = 0.0f;
#pragma unroll
    for (int l = 0; l < 32; ++l) s = fmaf(Vs[r][l], Gs[l][c], s);
    if (r < n && c < n) Qb[c * ldq + r] = (r == c ? 1.0f : 0.0f) - s;
  }
}

size_t orgqr_workspace_floats(int64_t batch, int n) {
  if (n <= 32) return 0;  // orgqr_small_kernel: no scratch
  const int64_t npan = (n + 31) / 32;
  const int64_t nchunk = (npan + kMaxSlots - 1) / kMaxSlots;
  size_t f = 2 * (size_t)(nchunk * batch * kMaxSlots * 1024);
  if (n > kOrgqrRowSplitMinN || orgqr_narrow_rowsplit(batch, n)) f += wyr_workspace_floats(batch, n);
  return f;
}

hipError_t launch_orgqr(const float* H, int64_t batch, int n, int64_t hs0, int64_t hs1, int64_t hs2, const float* tau,
                        int64_t ts0, int64_t ts1, float* Q, int64_t qs0, int64_t ldq, float* ws, bool vec,
                        hipStream_t stream) {
  if (n <= 32) {
    hipLaunchKernelGGL(orgqr_small_kernel, dim3((unsigned)batch), dim3(256), 0, stream, H, hs0, hs1, hs2, tau, ts0, ts1,
                       Q, qs0, ldq, n);
    return hipGetLastError();
  }
  const int npan = (n + 31) / 32;
  const int64_t nchunk = (npan + kMaxSlots - 1) / kMaxSlots;
  float* Tws = ws;
  float* Yws = ws + nchunk * batch * kMaxSlots * 1024;
  float* scratch = Yws + nchunk * batch * kMaxSlots * 1024;

  hipLaunchKernelGGL(orgqr_init_kernel, dim3((unsigned)n, (unsigned)batch), dim3(256), 0, stream, H, hs0, hs1, hs2, Q,
                     qs0, ldq, n);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(orgqr_larft_kernel, dim3((unsigned)npan, (unsigned)batch), dim3(256), 0, stream, Q, qs0,
                     (int)ldq, n, n, tau, ts0, ts1, batch, Tws, Yws, 1, 0);
  if ((e = hipGetLastError()) != hipSuccess) return e;

  auto panel_q = [&](int p) -> hipError_t {
    hipLaunchKernelGGL(orgqr_panel_kernel, dim3((unsigned)((n - 32 * p + 255) / 256), (unsigned)batch), dim3(256), 0,
                       stream, Q, qs0, (int)ldq, n, p, batch, Yws);
    return hipGetLastError();
  };
  auto t_chunk = [&](int p) { return Tws + (int64_t)(p / kMaxSlots) * batch * kMaxSlots * 1024; };

  if (n > kOrgqrRowSplitMinN) {
    // tall matrices: one panel per row-split update
    for (int p = npan - 1; p >= 0; --p) {
      const int k0 = 32 * p;
      const int c0 = k0 + 32;
      if (c0 < n) {
        WyrCall wc{};
        wc.H = Q;
        wc.hs0 = qs0;
        wc.ldh = (int)ldq;
        wc.n = n;
        wc.batch = batch;
        wc.kv = k0;
        wc.k = 32;
        wc.c_begin = c0;
        wc.c_end = n;
        wc.Tws = t_chunk(p);
        wc.Tslot = t_chunk(p) + (p % kMaxSlots) * 1024;
        wc.scratch = scratch;
        wc.rows_per_blk = wyr_rows_per_block(n - k0, batch, n - c0);
        wc.vec = vec;
        wc.hi_prio = true;
        if ((e = launch_wyr(wc, stream)) != hipSuccess) return e;
      }
      if ((e = panel_q(p)) != hipSuccess) return e;
    }
    return hipSuccess;
  }

  // Groups of kMaxWY panels (the T chunks hold a whole number of groups).
  // The group's transforms reach the columns right of it in one update, last
  // panel first; inside the group, panel p's own columns are formed after its
  // transform has been applied to the group's columns right of p.  The group
  // costs kMaxWY - 1 more (narrow) launches than one update per panel and
  // saves re-reading the trailing matrix: it pays for large batches (measured
  // on MI355X: 640 x 512 17% and 60 x 1024 24% faster, 8 x 2048 and 40 x 352
  // 4-6% slower), so small batches keep one update per panel -- except tall
  // matrices in small batches, grouped with their narrow updates on the
  // row-split kernels (8 x 2048: 3.46 ms per panel, 3.45 ms grouped).
  static_assert(kMaxSlots % kMaxWY == 0, "a panel group must not straddle two T chunks");
  const bool narrow_rs = orgqr_narrow_rowsplit(batch, n);
  const int gw = (batch >= kOrgqrGroupMinBatch || narrow_rs) ? kMaxWY : 1;
  const int ngroups = (npan + gw - 1) / gw;
  for (int g = ngroups - 1; g >= 0; --g) {
    const int p0 = gw * g;
    const int p1 = min(p0 + gw, npan);
    const int g_end = min(32 * p1, n);
    if (g_end < n) {
      e = launch_wy_update(Q, batch, qs0, ldq, t_chunk(p0), n, 32 * p0, 32, p0 % kMaxSlots, p1 - p0, g_end, n, vec,
                           false, 0, stream, /*reverse=*/true);
      if (e != hipSuccess) return e;
    }
    if (batch >= kOrgqrLeftLookingMinBatch) {
      // Left-looking inside the group: once panel p's columns are formed they
      // receive the group's earlier transforms p0 .. p-1 in one launch, last
      // first, so each column block is loaded once for all of them.  Panel p'
      // < p still holds its reflectors then (its own columns are formed
      // later), as the update reads them.  A launch then covers one 32-column
      // block per matrix, too few workgroups below one per CU (measured on
      // MI355X: 640 x 512 3.5% faster, 60 x 1024 7% slower), so smaller
      // batches apply one transform at a time to the group's formed columns.
      for (int p = p1 - 1; p >= p0; --p) {
        if ((e = panel_q(p)) != hipSuccess) return e;
        if (p > p0) {
          e = launch_wy_update(Q, batch, qs0, ldq, t_chunk(p0), n, 32 * p0, 32, p0 % kMaxSlots, p - p0, 32 * p,
                               min(32 * p + 32, n), vec, false, 0, stream, /*reverse=*/true);
          if (e != hipSuccess) return e;
        }
      }
      continue;
    }
    for (int p = p1 - 1; p >= p0; --p) {
      if (32 * p + 32 < g_end) {
        if (narrow_rs) {
          WyrCall wc{};
          wc.H = Q;
          wc.hs0 = qs0;
          wc.ldh = (int)ldq;
          wc.n = n;
          wc.batch = batch;
          wc.kv = 32 * p;
          wc.k = 32;
          wc.c_begin = 32 * p + 32;
          wc.c_end = g_end;
          wc.Tws = t_chunk(p);
          wc.Tslot = t_chunk(p) + (p % kMaxSlots) * 1024;
          wc.scratch = scratch;
          wc.rows_per_blk = wyr_rows_per_block(n - 32 * p, batch, g_end - 32 * p - 32);
          wc.vec = vec;
          wc.hi_prio = true;
          e = launch_wyr(wc, stream);
        } else {
          e = launch_wy_update(Q, batch, qs0, ldq, t_chunk(p), n, 32 * p, 32, p % kMaxSlots, 1, 32 * p + 32, g_end,
                               vec, false, 0, stream);
        }
        if (e != hipSuccess) return e;
      }
      if ((e = panel_q(p)) != hipSuccess) return e;
    }
  }
  return hipSuccess;
}

// Rows a strip-resident update holds in registers (8 waves x 8 tiles of 32);
// taller groups of reflectors go to the row-split kernels with a group T.
constexpr int kOrmqrResidentRows = 2048;
// C columns per row-split call (bounds its partial-product scratch)
constexpr int kOrmqrChunkCols = 4096;

// Panel groups (kMaxWY panels each) before the first whose rows fit a strip.
static int ormqr_tall_groups(int m, int r) {
  const int npan = (r + 31) / 32;
  const int ngroups = (npan + kMaxWY - 1) / kMaxWY;
  int g = 0;
  while (g < ngroups && m - 32 * kMaxWY * g > kOrmqrResidentRows) ++g;
  return g;
}

size_t ormqr_workspace_floats(int64_t batch, int m, int r, int k) {
  const int64_t npan = (r + 31) / 32;
  const int64_t nchunk = (npan + kMaxSlots - 1) / kMaxSlots;
  size_t f = (size_t)(nchunk * batch * kMaxSlots * 1024);
  if (ormqr_tall_groups(m, r) > 0) {
    const int cols = k < kOrmqrChunkCols ? k : kOrmqrChunkCols;
    f += (size_t)batch * kWyrTgStride + wyr_workspace_floats(batch, m > cols ? m : cols);
  }
  return f;
}

// LAPACK sormqr (SIDE = 'L') in compact-WY form, as the blocked geqrf applies
// a panel group: T of every 32-column panel by orgqr_larft_kernel (stored as
// T for Q^T C, whose blocks B_p^T = I - V T^T V^T are what the update kernels
// apply with a stored T, and as T^T for Q C, whose blocks are
// B_p = I - V T V^T), then one strip-resident update of every column of C per
// group of kMaxWY panels: C is loaded and stored once per group.  Groups of
// more than kOrmqrResidentRows rows are applied by the row-split kernels with
// the group's T (its Gram matrix and panel T's joined, as geqrf's tall
// path), read transposed for Q C; their panels' T stay untransposed for the join.
hipError_t launch_ormqr(const float* H, int64_t batch, int m, int r, int64_t hs0, int64_t ldh, const float* tau,
                        int64_t ts0, int64_t ts1, float* C, int64_t cs0, int64_t ldc, int k, bool transpose, float* ws,
                        bool vec, hipStream_t stream) {
  if (r <= 0 || k <= 0) return hipSuccess;
  const int npan = (r + 31) / 32;
  const int ngroups = (npan + kMaxWY - 1) / kMaxWY;
  const int g_tall = ormqr_tall_groups(m, r);
  const int p_tall = g_tall * kMaxWY < npan ? g_tall * kMaxWY : npan;
  hipError_t e = hipSuccess;
  if (p_tall > 0) {
    hipLaunchKernelGGL(orgqr_larft_kernel, dim3((unsigned)p_tall, (unsigned)batch), dim3(256), 0, stream, H, hs0,
                       (int)ldh, m, r, tau, ts0, ts1, batch, ws, nullptr, 0, 0);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  if (npan > p_tall) {
    hipLaunchKernelGGL(orgqr_larft_kernel, dim3((unsigned)(npan - p_tall), (unsigned)batch), dim3(256), 0, stream, H,
                       hs0, (int)ldh, m, r, tau, ts0, ts1, batch, ws, nullptr, transpose ? 0 : 1, p_tall);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  const int64_t nchunk = (npan + kMaxSlots - 1) / kMaxSlots;
  float* Tg = ws + nchunk * batch * kMaxSlots * 1024;
  float* scratch = Tg + batch * kWyrTgStride;
  static_assert(kMaxSlots % kMaxWY == 0, "a panel group must not straddle two T chunks");
  for (int s = 0; s < ngroups; ++s) {
    const int g = transpose ? s : ngroups - 1 - s;  // Q^T C: H_0 first; Q C: H_{r-1} first
    const int p0 = kMaxWY * g;
    const int p1 = min(p0 + kMaxWY, npan);
    const int k0 = 32 * p0;
    const float* Tchunk = ws + (int64_t)(p0 / kMaxSlots) * batch * kMaxSlots * 1024;
    if (g >= g_tall) {
      e = launch_wy_apply(H, batch, hs0, ldh, r, C, cs0, ldc, k, Tchunk, m, k0, 32, p0 % kMaxSlots, p1 - p0, vec,
                          stream, /*reverse=*/!transpose);
      if (e != hipSuccess) return e;
      continue;
    }
    const int kg = min(32 * (p1 - p0), r - k0);  // the group's reflectors
    WyrCall gc{};  // group T: Gram matrix of the group's reflectors, panel T's joined
    gc.H = const_cast<float*>(H);
    gc.hs0 = hs0;
    gc.ldh = (int)ldh;
    gc.n = m;
    gc.batch = batch;
    gc.kv = k0;
    gc.k = kg;
    gc.c_begin = k0;
    gc.c_end = k0 + kg;
    gc.gram = true;
    gc.use_tg = true;
    gc.q = p1 - p0;
    gc.nb = 32;
    gc.slot0 = p0 % kMaxSlots;
    gc.Tws = Tchunk;
    gc.Tg = Tg;
    gc.scratch = scratch;
    gc.rows_per_blk = wyr_rows_per_block(m - k0, batch, kg);
    gc.vec = vec;
    gc.vcols = r;
    if ((e = launch_wyr(gc, stream)) != hipSuccess) return e;
    for (int c0 = 0; c0 < k; c0 += kOrmqrChunkCols) {
      const int c1 = (k - c0 < kOrmqrChunkCols) ? k : c0 + kOrmqrChunkCols;
      WyrCall ac{};
      ac.H = const_cast<float*>(H);
      ac.hs0 = hs0;
      ac.ldh = (int)ldh;
      ac.n = m;
      ac.batch = batch;
      ac.kv = k0;
      ac.k = kg;
      ac.c_begin = c0;
      ac.c_end = c1;
      ac.use_tg = true;
      ac.Tg = Tg;
      ac.Tws = Tchunk;
      ac.scratch = scratch;
      ac.rows_per_blk = wyr_rows_per_block(m - k0, batch, c1 - c0);
      ac.vec = vec;
      ac.X = C;
      ac.xs0 = cs0;
      ac.ldx = (int)ldc;
      ac.xcols = k;
      ac.vcols = r;
      ac.t_trans = !transpose;
      if ((e = launch_wyr(ac, stream)) != hipSuccess) return e;
    }
  }
  return hipSuccess;
}

}  // namespace fastqr
