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
// (the next chunk's loads in flight while the current one is summed); thread
// (i, j0) accumulates G(i, j0..j0+3) = sum_r V(r, i) V(r, j0..j0+3).  The
// slarft recurrence T(i, j) = -tau_j sum_{i <= l < j} T(i, l) G(l, j) needs
// only row i of T, so lane i runs it alone.
__global__ void __launch_bounds__(256) orgqr_larft_kernel(const float* __restrict__ Q, int64_t qs0, int ldq, int n,
                                                          const float* __restrict__ tau, int64_t ts0, int64_t ts1,
                                                          int64_t batch, float* __restrict__ Tws,
                                                          float* __restrict__ Yws) {
  const int p = blockIdx.x;
  const int64_t b = blockIdx.y;
  const int k0 = 32 * p;
  const int nb = min(32, n - k0);
  const int m = n - k0;
  const float* Qb = Q + b * qs0;
  const int t = threadIdx.x;
  const int gi = t >> 3, gj = 4 * (t & 7);

  __shared__ __attribute__((aligned(16))) float Vs[64][36];
  __shared__ float V1s[32][33];
  __shared__ float Gs[32][33];
  __shared__ float Ts[32][33];
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
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
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
    const int rows = min(64, m - r0);
    for (int rr = 0; rr < rows; ++rr) {
      const float a = Vs[rr][gi];
      const f32x4 w = *reinterpret_cast<const f32x4*>(&Vs[rr][gj]);
      acc[0] = fmaf(a, w[0], acc[0]);
      acc[1] = fmaf(a, w[1], acc[1]);
      acc[2] = fmaf(a, w[2], acc[2]);
      acc[3] = fmaf(a, w[3], acc[3]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) Gs[gi][gj + q] = acc[q];
  __syncthreads();

  if (t < 32) {
    const int i = t;
    for (int j = 0; j < 32; ++j) {
      float v = 0.0f;
      if (j < nb) {
        if (i == j) {
          v = taus[j];
        } else if (i < j) {
          float s = 0.0f;
          for (int l = i; l < j; ++l) s = fmaf(Ts[i][l], Gs[l][j], s);
          v = -taus[j] * s;
        }
      }
      Ts[i][j] = v;
    }
  }
  __syncthreads();

  float* To = Tws + (((int64_t)(p / kMaxSlots) * batch + b) * kMaxSlots + (p % kMaxSlots)) * 1024;
  float* Yo = Yws + (((int64_t)(p / kMaxSlots) * batch + b) * kMaxSlots + (p % kMaxSlots)) * 1024;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int idx = t + 256 * u;
    const int r = idx >> 5, c = idx & 31;
    To[idx] = Ts[c][r];
    float y = 0.0f;
    for (int l = r; l <= c; ++l) y = fmaf(Ts[r][l], V1s[c][l], y);  // T upper, V1 unit lower
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
    if (c >= nb) break;
    float s = 0.0f;
#pragma unroll
    for (int l = 0; l < 32; ++l) s = fmaf(v[l], Ys[l][c], s);
    Qc[(int64_t)c * ldq] = (c == rr ? 1.0f : 0.0f) - s;
  }
}

size_t orgqr_workspace_floats(int64_t batch, int n) {
  const int64_t npan = (n + 31) / 32;
  const int64_t nchunk = (npan + kMaxSlots - 1) / kMaxSlots;
  size_t f = 2 * (size_t)(nchunk * batch * kMaxSlots * 1024);
  if (n > kOrgqrRowSplitMinN) f += wyr_workspace_floats(batch, n);
  return f;
}

hipError_t launch_orgqr(const float* H, int64_t batch, int n, int64_t hs0, int64_t hs1, int64_t hs2, const float* tau,
                        int64_t ts0, int64_t ts1, float* Q, int64_t qs0, int64_t ldq, float* ws, bool vec,
                        hipStream_t stream) {
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
                     (int)ldq, n, tau, ts0, ts1, batch, Tws, Yws);
  if ((e = hipGetLastError()) != hipSuccess) return e;

  for (int p = npan - 1; p >= 0; --p) {
    const int k0 = 32 * p;
    const int c0 = k0 + 32;
    float* Tchunk = Tws + (int64_t)(p / kMaxSlots) * batch * kMaxSlots * 1024;
    if (c0 < n) {
      if (n > kOrgqrRowSplitMinN) {
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
        wc.Tws = Tchunk;
        wc.Tslot = Tchunk + (p % kMaxSlots) * 1024;
        wc.scratch = scratch;
        wc.rows_per_blk = wyr_rows_per_block(n - k0, batch, n - c0);
        wc.vec = vec;
        wc.hi_prio = true;
        e = launch_wyr(wc, stream);
      } else {
        e = launch_wy_update(Q, batch, qs0, ldq, Tchunk, n, k0, 32, p % kMaxSlots, 1, c0, n, vec, false, 0, stream);
      }
      if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(orgqr_panel_kernel, dim3((unsigned)((n - k0 + 255) / 256), (unsigned)batch), dim3(256), 0,
                       stream, Q, qs0, (int)ldq, n, p, batch, Yws);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace fastqr
