// h_states of the SSD prefill: hs[b, t, n] = mean over (h, p) of the state h_t[h, p, n]
// (mamformer/layers/mamba2.py:114-116).  The channel sum of the state obeys a recurrence of its own,
//     Z_t[h, n] = sum_p h_t[h, p, n] = e^{A_h dt_t,h} Z_{t-1}[h, n] + dt_t,h xs_t[h] B_t[g(h), n],
//     xs_t[h] = sum_p x_t[h, p],        hs_t[n] = sum_h Z_t[h, n] / (H P),
// so h_states needs one scalar input per (token, head) instead of P of them.  Three passes over 32-token
// segments, all in fp32:
//   ssd_hs_local_kernel  (segment, batch): dt processed as the prefill does it, c = in-segment inclusive cumsum
//                        of A dt, xs per (token, head) into the workspace, u = dt xs, and the segment's own
//                        contribution Zloc[h][n] = sum_s e^{c_end - c_s} u_s[h] B_s[g(h)][n] with the decay
//                        e^{c_end} of each head.
//   ssd_hs_carry_kernel  (batch, head, n): Zin of every segment, Zin_0 = sum_p h0[h, p, n] (or 0),
//                        Zin_{k+1} = e^{c_end,k} Zin_k + Zloc_k (in place over Zloc).
//   ssd_hs_out_kernel    (segment, batch): hs_t[n] = (sum_h e^{c_t,h} Zin[h][n]
//                        + sum_g sum_{s <= t} W_g[t][s] B_s[g][n]) / (H P),  W_g[t][s] = sum_{h in g} e^{c_t,h - c_s,h} u_s[h],
//                        W formed as a product over heads of E[t][h] = e^{c_t,h - m_h} and F[s][h] = e^{m_h - c_s,h} u_s[h]
//                        (m_h the midpoint of the head's range in the segment); a head whose range exceeds PR
//                        adds its terms with one exponential each instead, so no factor exceeds e^{PR / 2}.
// The other exponents are <= 0 (A <= 0, dt >= 0): no factor can overflow whatever the decay.
#include "common.h"
#include "launch.h"
#include "ssd_shared.h"

namespace mh {

namespace {

constexpr int HS_SEG = 32;       // tokens per segment
constexpr int HS_MAXH = 128;     // heads held in LDS
constexpr int HS_MAXN = 256;
constexpr int HS_ZH = 32;        // heads of entering sums staged in LDS at a time
constexpr float PR = 80.f;       // largest in-segment range of c factorised as E F

__device__ __forceinline__ float hs_dt(const SsdParams& p, float d, int h) {
  if (p.dt_bias) d += p.dt_bias[h];
  if (p.dt_softplus) d = softplus_f(d);
  if (p.has_dt_limit) d = fminf(fmaxf(d, p.dt_min), p.dt_max);
  return d;
}

struct HsSmem {
  float c[HS_SEG][HS_MAXH];      // raw dt, then the in-segment inclusive cumsum of A dt (flat past the end)
  float u[HS_SEG][HS_MAXH];      // dt xs (0 past the end); local pass: e^{c_end - c_s} dt xs
  float E[HS_SEG][HS_MAXH];      // out pass: e^{c_t - m}
  float F[HS_SEG][HS_MAXH];      // out pass: e^{m - c_s} u_s
  float Ei[HS_SEG][HS_MAXH];     // out pass: e^{c_t}
  float Bt[HS_SEG][HS_MAXN];     // B of one group
  float Zs[HS_ZH][HS_MAXN];      // out pass: entering state sums of HS_ZH heads
  float W[HS_SEG][HS_SEG + 4];   // W_g[t][s]
  float cend[HS_MAXH], mid[HS_MAXH];
  int wide[HS_MAXH];
  int anywide;
};

// dt, c and u = dt xs of segment si into LDS, xs = sum_p x computed from x (local pass, and written to the
// workspace) or read from it (out pass).
template <typename T, bool FROM_WS>
__device__ void hs_prologue(const SsdParams& p, const HsParams& q, HsSmem& sm, int b, int si, int len) {
  const int H = p.nheads, tid = threadIdx.x;
  const int64_t tok0 = (int64_t)si * HS_SEG;
  float* uws = q.u + ((int64_t)b * p.seqlen + tok0) * H;
  // raw dt of the segment into LDS (all loads in flight together; the per-head cumsum below reads LDS)
  const float* dtb = p.dt + (int64_t)b * p.dt_sb;
  for (int e = tid; e < HS_SEG * H; e += blockDim.x) {
    const int t = e / H, h = e % H;
    sm.c[t][h] = t < len ? dtb[(tok0 + t) * p.dt_sl + h] : 0.f;
  }
  if (!FROM_WS) {
    // xs[t][h] = sum_p x[t][h][p] (P = 64): one (token, head) row per thread pass, its 16 loads issued together
    const T* xb = reinterpret_cast<const T*>(p.x) + (int64_t)b * p.x_sb;
    for (int e = tid; e < HS_SEG * H; e += blockDim.x) {
      const int t = e / H, h = e % H;
      float xs = 0.f;
      if (t < len) {
        const T* row = xb + (tok0 + t) * p.x_sl + (int64_t)h * p.x_sh;
        float part[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) {
          if constexpr (sizeof(T) == 2) {
            const bf16x4 v = *reinterpret_cast<const bf16x4*>(row + 4 * k);
            part[k] = ((float)v[0] + (float)v[1]) + ((float)v[2] + (float)v[3]);
          } else {
            const f32x4 v = *reinterpret_cast<const f32x4*>(row + 4 * k);
            part[k] = (v[0] + v[1]) + (v[2] + v[3]);
          }
        }
#pragma unroll
        for (int k = 0; k < 16; ++k) xs += part[k];
      }
      sm.u[t][h] = xs;                 // xs for now; times dt below
    }
  } else {
    for (int e = tid; e < HS_SEG * H; e += blockDim.x) {
      const int t = e / H, h = e % H;
      sm.u[t][h] = t < len ? uws[(int64_t)t * H + h] : 0.f;
    }
  }
  __syncthreads();
  // per head: processed dt, cumsum c, u = dt xs (local pass)
  for (int h = tid; h < H; h += blockDim.x) {
    const float A = p.A[h];
    float c = 0.f;
    for (int t = 0; t < HS_SEG; ++t) {
      if (t < len) {
        const float d = hs_dt(p, sm.c[t][h], h);
        c += A * d;
        const float xs = sm.u[t][h];
        if (!FROM_WS) uws[(int64_t)t * H + h] = xs;
        sm.u[t][h] = d * xs;
      } else {
        sm.u[t][h] = 0.f;
      }
      sm.c[t][h] = c;
    }
    sm.cend[h] = c;
    sm.mid[h] = 0.5f * (sm.c[0][h] + c);
    sm.wide[h] = sm.c[0][h] - c > PR;
  }
}

// B of group g for the segment's tokens (0 past the end) into LDS as fp32.
template <typename T>
__device__ void hs_load_b(const SsdParams& p, HsSmem& sm, int b, int si, int len, int g) {
  const int N = p.dstate, tid = threadIdx.x;
  const T* Bb = reinterpret_cast<const T*>(p.B) + (int64_t)b * p.B_sb + (int64_t)g * N;
  const int64_t tok0 = (int64_t)si * HS_SEG;
  for (int e = tid; e < HS_SEG * N / 4; e += blockDim.x) {
    const int t = e / (N / 4), n = 4 * (e % (N / 4));
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    if (t < len) {
      const T* src = Bb + (tok0 + t) * p.B_sl + n;
      if constexpr (sizeof(T) == 2) {
        const bf16x4 w = *reinterpret_cast<const bf16x4*>(src);
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = (float)w[j];
      } else {
        v = *reinterpret_cast<const f32x4*>(src);
      }
    }
    *reinterpret_cast<f32x4*>(&sm.Bt[t][n]) = v;
  }
}

// 8 consecutive columns of an LDS row
__device__ __forceinline__ void ld8f(const float* p, float (&v)[8]) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(p), b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
  for (int j = 0; j < 4; ++j) { v[j] = a[j]; v[4 + j] = b[j]; }
}

template <typename T>
__global__ __launch_bounds__(256) void ssd_hs_local_kernel(SsdParams p, HsParams q) {
  __shared__ HsSmem sm;
  const int si = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int H = p.nheads, N = p.dstate, hpg = H / p.ngroups, N8 = N / 8;
  const int len = min(HS_SEG, p.seqlen - si * HS_SEG);
  hs_prologue<T, false>(p, q, sm, b, si, len);
  __syncthreads();
  // w[s][h] = e^{c_end - c_s} u_s[h] (<= u: the exponent is <= 0), in place over u
  for (int e = tid; e < HS_SEG * H; e += blockDim.x) {
    const int s = e / H, h = e % H;
    sm.u[s][h] *= __expf(sm.cend[h] - sm.c[s][h]);
  }
  float* zl = q.z + (((int64_t)b * p.nseg + si) * H) * N;
  for (int g = 0; g < p.ngroups; ++g) {
    __syncthreads();                   // w complete; the previous group's B no longer read
    hs_load_b<T>(p, sm, b, si, len, g);
    __syncthreads();
    // Zloc[h][n0 .. n0 + 8) = sum_s w[s][h] B[s][n]
    for (int e = tid; e < hpg * N8; e += blockDim.x) {
      const int h = g * hpg + e / N8, n0 = 8 * (e % N8);
      float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
      for (int s = 0; s < HS_SEG; ++s) {
        float bv[8];
        ld8f(&sm.Bt[s][n0], bv);
        const float w = sm.u[s][h];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] += w * bv[j];
      }
      float* o = zl + (int64_t)h * N + n0;
      *reinterpret_cast<f32x4*>(o) = f32x4{acc[0], acc[1], acc[2], acc[3]};
      *reinterpret_cast<f32x4*>(o + 4) = f32x4{acc[4], acc[5], acc[6], acc[7]};
    }
  }
  if (tid < H) q.dec[((int64_t)b * p.nseg + si) * H + tid] = __expf(sm.cend[tid]);
}

__global__ __launch_bounds__(256) void ssd_hs_carry_kernel(SsdParams p, HsParams q) {
  const int H = p.nheads, N = p.dstate, P = p.headdim;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)p.batch * H * N) return;
  const int n = (int)(i % N), h = (int)((i / N) % H), b = (int)(i / ((int64_t)N * H));
  float Z = 0.f;
  if (p.init_state) {
    const float* s0 = p.init_state + (((int64_t)b * H + h) * P) * N + n;
    for (int k = 0; k < P; ++k) Z += s0[(int64_t)k * N];
  }
  float* zp = q.z + ((int64_t)b * p.nseg * H + h) * N + n;
  const float* dp = q.dec + (int64_t)b * p.nseg * H + h;
  const int64_t zs = (int64_t)H * N;
  // 16 segments' loads issued together, then the 16 steps of the chain: the load latency is paid once per 16
  for (int s0 = 0; s0 < p.nseg; s0 += 16) {
    float zl[16], d[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const bool in = s0 + k < p.nseg;
      zl[k] = in ? zp[(s0 + k) * zs] : 0.f;
      d[k] = in ? dp[(int64_t)(s0 + k) * H] : 1.f;
    }
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (s0 + k < p.nseg) zp[(s0 + k) * zs] = Z;    // the state sum entering segment s0 + k
      Z = d[k] * Z + zl[k];
    }
  }
}

template <typename T>
__global__ __launch_bounds__(256) void ssd_hs_out_kernel(SsdParams p, HsParams q) {
  __shared__ HsSmem sm;
  const int si = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int H = p.nheads, N = p.dstate, hpg = H / p.ngroups, N8 = N / 8;
  const int len = min(HS_SEG, p.seqlen - si * HS_SEG);
  if (tid == 0) sm.anywide = 0;
  hs_prologue<T, true>(p, q, sm, b, si, len);
  __syncthreads();
  if (tid < H && sm.wide[tid]) sm.anywide = 1;       // benign race: every writer stores 1
  for (int e = tid; e < HS_SEG * H; e += blockDim.x) {
    const int t = e / H, h = e % H;
    const float c = sm.c[t][h], m = sm.mid[h];
    const bool wide = sm.wide[h];
    sm.E[t][h] = wide ? 0.f : __expf(c - m);
    sm.F[t][h] = wide ? 0.f : __expf(m - c) * sm.u[t][h];
    sm.Ei[t][h] = __expf(c);
  }
  // output blocks (row t, 8 columns n0 ..): thread tid owns blocks tid, tid + 256, ... (at most 4)
  constexpr int MB = HS_SEG * (HS_MAXN / 8) / 256;
  const int nblk = HS_SEG * N8;
  float acc[MB][8];
#pragma unroll
  for (int k = 0; k < MB; ++k)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[k][j] = 0.f;
  // inter-segment part: sum_h e^{c_t,h} Zin[h][n], HS_ZH heads of Zin staged in LDS at a time
  const float* zin = q.z + (((int64_t)b * p.nseg + si) * H) * N;
  for (int h0 = 0; h0 < H; h0 += HS_ZH) {
    const int nh = min(HS_ZH, H - h0);
    __syncthreads();                   // E / F / Ei formed; the previous heads' Zs no longer read
    for (int e = tid; e < nh * N / 4; e += blockDim.x) {
      const int hh = e / (N / 4), n = 4 * (e % (N / 4));
      *reinterpret_cast<f32x4*>(&sm.Zs[hh][n]) = *reinterpret_cast<const f32x4*>(zin + (int64_t)(h0 + hh) * N + n);
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < MB; ++k) {
      const int e = tid + 256 * k;
      if (e < nblk) {
        const int t = e / N8, n0 = 8 * (e % N8);
        for (int hh = 0; hh < nh; ++hh) {
          float zv[8];
          ld8f(&sm.Zs[hh][n0], zv);
          const float ei = sm.Ei[t][h0 + hh];
#pragma unroll
          for (int j = 0; j < 8; ++j) acc[k][j] += ei * zv[j];
        }
      }
    }
  }
  for (int g = 0; g < p.ngroups; ++g) {
    __syncthreads();                   // the previous group's W and B no longer read
    hs_load_b<T>(p, sm, b, si, len, g);
    // W_g[t][s] = sum_{h in g} E[t][h] F[s][h] (+ the wide heads' terms directly), s <= t
    for (int e = tid; e < HS_SEG * HS_SEG; e += blockDim.x) {
      const int t = e / HS_SEG, s = e % HS_SEG;
      float w = 0.f;
      if (s <= t) {
        float w4[4] = {0.f, 0.f, 0.f, 0.f};
        int h = g * hpg;
        for (; h + 4 <= (g + 1) * hpg; h += 4)
#pragma unroll
          for (int k = 0; k < 4; ++k) w4[k] += sm.E[t][h + k] * sm.F[s][h + k];
        for (; h < (g + 1) * hpg; ++h) w4[0] += sm.E[t][h] * sm.F[s][h];
        w = (w4[0] + w4[1]) + (w4[2] + w4[3]);
        if (sm.anywide)
          for (h = g * hpg; h < (g + 1) * hpg; ++h)
            if (sm.wide[h]) w += __expf(sm.c[t][h] - sm.c[s][h]) * sm.u[s][h];
      }
      sm.W[t][s] = w;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < MB; ++k) {
      const int e = tid + 256 * k;
      if (e < nblk) {
        const int t = e / N8, n0 = 8 * (e % N8);
        for (int s = 0; s <= t; ++s) {
          float bv[8];
          ld8f(&sm.Bt[s][n0], bv);
          const float w = sm.W[t][s];
#pragma unroll
          for (int j = 0; j < 8; ++j) acc[k][j] += w * bv[j];
        }
      }
    }
  }
  T* out = reinterpret_cast<T*>(q.hs) + ((int64_t)b * p.seqlen + (int64_t)si * HS_SEG) * N;
  const float scale = 1.f / ((float)H * (float)p.headdim);
#pragma unroll
  for (int k = 0; k < MB; ++k) {
    const int e = tid + 256 * k;
    if (e < nblk) {
      const int t = e / N8, n0 = 8 * (e % N8);
      if (t < len) {
#pragma unroll
        for (int j = 0; j < 8; ++j) out[(int64_t)t * N + n0 + j] = from_f32<T>(acc[k][j] * scale);
      }
    }
  }
}

// ---------------------------------------------------------------- backward
// Gradients of <ghs, hs> for ghs the gradient of h_states.  With g_t = ghs_t / (H P) (the same for every head),
// the adjoint of Z^h_t is lambda^h_t = g_t + a^h_{t+1} lambda^h_{t+1}.  Per 32-token segment, with c the in-segment
// cumsum of A dt, a_t = e^{A dt_t}, Zin the state sum entering the segment and Lam the adjoint handed in from the
// right (a lambda of the next segment's first token):
//   lambda_t = sum_{t' >= t} e^{c_t' - c_t} g_t' + e^{c_31 - c_t} Lam,
//   Z_{t-1}  = e^{c_{t-1}} Zin + sum_{s < t} e^{c_{t-1} - c_s} u_s B_s,
//   du_t = lambda_t . B_t = Y[t][t] + e^{c_31 - c_t} R[t]          (M[t'][s] = g_t' . B_s, R[s] = Lam . B_s),
//   q_t  = lambda_t . Z_{t-1} = e^{c_31 - c_t + c_{t-1}} Zin . Lam + e^{c_{t-1}} Y2[t]
//          + e^{c_31 - c_t} sum_{s<t} e^{c_{t-1} - c_s} u_s R[s] + sum_{s<t} e^{c_{t-1} - c_s} u_s Y[t][s],
//   Y[t][s] = sum_{t' >= t} e^{c_t' - c_t} M[t'][s] = M[t][s] + a_{t+1} Y[t+1][s]   (Y2 likewise from P[t'] = Zin . g_t'),
//   dB_t = sum_h u^h_t lambda^h_t = sum_{t' >= t} V[t][t'] g_t' + sum_h u^h_t e^{c_31 - c_t} Lam^h,
//          V[t][t'] = sum_h u^h_t e^{c_t' - c_t},
// then d dt_t = A a_t q_t + xs_t du_t (through bias, softplus and clamp), d xs_t = dt_t du_t (dx[t][h][p] for every
// p), dA = sum dt a q and d h0[h][p][n] = the adjoint before the first token.  Every exponent is <= 0.
//   ssd_hsb_local_kernel (segment, batch): GL[h][n] = sum_t e^{c_t} g_t[n] (the segment's part of the adjoint
//                        handed to the left).
//   ssd_hsb_carry_kernel (batch, head, n): Lam of every segment, right to left (in place over GL), and d h0.
//   ssd_hsb_main_kernel  (segment, batch): du, q, dB, dx, ddt and per-segment dA / d_dt_bias partials.
//   ssd_hsb_reduce_kernel: dA and d_dt_bias summed over (batch, segment) in a fixed order.
constexpr int HSB_MAXH = 128, HSB_MAXN = 128;

struct HsbSmem {
  float c[HS_SEG][HSB_MAXH];     // raw dt, then the in-segment cumsum of A dt
  float d[HS_SEG][HSB_MAXH];     // processed dt (0 past the end)
  float xs[HS_SEG][HSB_MAXH];    // sum_p x (0 past the end)
  float g[HS_SEG][HSB_MAXN];     // ghs / (H P)
  float Bt[HS_SEG][HSB_MAXN];    // B of one group
  float M[HS_SEG][HS_SEG + 1];   // g_t' . B_s
  float V[HS_SEG][HS_SEG + 1];   // sum_h u_t e^{c_t' - c_t}  (t' >= t)
  float q[HS_SEG][HSB_MAXH];     // q_t, then d xs_t
  float du[HS_SEG][HSB_MAXH];
  float R[HSB_MAXH][HS_SEG + 1]; // Lam . B_s
  float P[HSB_MAXH][HS_SEG + 1]; // Zin . g_t'
  float S1[HSB_MAXH], cend[HSB_MAXH];
};

__device__ __forceinline__ float hsb_dt_chain(const SsdParams& p, float raw, float bias) {
  const float u = raw + bias;
  float g = 1.f, v = u;
  if (p.dt_softplus) {
    if (u <= 20.f) g = 1.f / (1.f + __expf(-u));
    v = softplus_f(u);
  }
  if (p.has_dt_limit && !(v >= p.dt_min && v <= p.dt_max)) g = 0.f;
  return g;
}

// g of the segment (0 past the end) into g[t][n]
template <typename T, int W>
__device__ void hsb_load_g(const SsdParams& p, const HsParams& q, float (*g)[W], int b, int si, int len) {
  const int N = p.dstate;
  const float scale = 1.f / ((float)p.nheads * (float)p.headdim);
  const T* src = reinterpret_cast<const T*>(q.dhs) + ((int64_t)b * p.seqlen + (int64_t)si * HS_SEG) * N;
  for (int e = threadIdx.x; e < HS_SEG * N; e += blockDim.x) {
    const int t = e / N, n = e % N;
    g[t][n] = t < len ? to_f32(src[(int64_t)t * N + n]) * scale : 0.f;
  }
}

template <typename T>
__global__ __launch_bounds__(256) void ssd_hsb_local_kernel(SsdParams p, HsParams q) {
  __shared__ HsSmem sm;
  const int si = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int H = p.nheads, N = p.dstate, N8 = N / 8;
  const int len = min(HS_SEG, p.seqlen - si * HS_SEG);
  hs_prologue<T, true>(p, q, sm, b, si, len);
  hsb_load_g<T, HS_MAXN>(p, q, sm.Bt, b, si, len);           // g in the B buffer
  __syncthreads();
  for (int e = tid; e < HS_SEG * H; e += blockDim.x) {
    const int t = e / H, h = e % H;
    sm.Ei[t][h] = __expf(sm.c[t][h]);
  }
  __syncthreads();
  float* gl = q.lam + (((int64_t)b * p.nseg + si) * H) * N;
  for (int e = tid; e < H * N8; e += blockDim.x) {
    const int h = e / N8, n0 = 8 * (e % N8);
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
    for (int t = 0; t < HS_SEG; ++t) {
      float gv[8];
      ld8f(&sm.Bt[t][n0], gv);
      const float w = sm.Ei[t][h];
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] += w * gv[j];
    }
    float* o = gl + (int64_t)h * N + n0;
    *reinterpret_cast<f32x4*>(o) = f32x4{acc[0], acc[1], acc[2], acc[3]};
    *reinterpret_cast<f32x4*>(o + 4) = f32x4{acc[4], acc[5], acc[6], acc[7]};
  }
}

__global__ __launch_bounds__(256) void ssd_hsb_carry_kernel(SsdParams p, HsParams q, float* dh0) {
  const int H = p.nheads, N = p.dstate, P = p.headdim;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)p.batch * H * N) return;
  const int n = (int)(i % N), h = (int)((i / N) % H), b = (int)(i / ((int64_t)N * H));
  float* lp = q.lam + ((int64_t)b * p.nseg * H + h) * N + n;
  const float* dp = q.dec + (int64_t)b * p.nseg * H + h;
  const int64_t ls = (int64_t)H * N;
  float L = 0.f;
  // right to left, 16 segments' loads issued together per batch of steps
  for (int k1 = p.nseg - 1; k1 >= 0; k1 -= 16) {
    float gl[16], d[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int si = k1 - k;
      gl[k] = si >= 0 ? lp[si * ls] : 0.f;
      d[k] = si >= 0 ? dp[(int64_t)si * H] : 1.f;
    }
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int si = k1 - k;
      if (si >= 0) lp[si * ls] = L;                  // the adjoint handed into segment si from the right
      L = d[k] * L + gl[k];
    }
  }
  if (dh0) {
    float* o = dh0 + (((int64_t)b * H + h) * P) * N + n;
    for (int k = 0; k < P; ++k) o[(int64_t)k * N] = L;
  }
}

template <typename T>
__global__ __launch_bounds__(256) void ssd_hsb_main_kernel(SsdParams p, HsParams q) {
  __shared__ HsbSmem sm;
  const int si = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int w = wave_id(), l = lane_id();
  const int H = p.nheads, N = p.dstate, N8 = N / 8, G = p.ngroups, hpg = H / G;
  const int64_t tok0 = (int64_t)si * HS_SEG;
  const int len = min(HS_SEG, p.seqlen - (int)tok0);
  const float* zin = q.z + (((int64_t)b * p.nseg + si) * H) * N;
  const float* lam = q.lam + (((int64_t)b * p.nseg + si) * H) * N;
  // ---- dt (processed), c, xs
  const float* dtb = p.dt + (int64_t)b * p.dt_sb;
  const float* xsw = q.u + ((int64_t)b * p.seqlen + tok0) * H;
  for (int e = tid; e < HS_SEG * H; e += blockDim.x) {
    const int t = e / H, h = e % H;
    sm.c[t][h] = t < len ? dtb[(tok0 + t) * p.dt_sl + h] : 0.f;
    sm.xs[t][h] = t < len ? xsw[(int64_t)t * H + h] : 0.f;
  }
  hsb_load_g<T, HSB_MAXN>(p, q, sm.g, b, si, len);
  __syncthreads();
  for (int h = tid; h < H; h += blockDim.x) {
    const float A = p.A[h];
    float c = 0.f;
    for (int t = 0; t < HS_SEG; ++t) {
      const float d = t < len ? hs_dt(p, sm.c[t][h], h) : 0.f;
      c += A * d;
      sm.d[t][h] = d;
      sm.c[t][h] = c;
    }
    sm.cend[h] = c;
  }
  // ---- P[h][t'] = Zin^h . g_t',  S1[h] = Zin^h . Lam^h
  for (int e = tid; e < H * HS_SEG; e += blockDim.x) {
    const int h = e / HS_SEG, t = e % HS_SEG;
    const float* zr = zin + (int64_t)h * N;
    float a = 0.f;
    for (int n = 0; n < N; n += 4) {
      const f32x4 z4 = *reinterpret_cast<const f32x4*>(zr + n);
      a += z4[0] * sm.g[t][n] + z4[1] * sm.g[t][n + 1] + z4[2] * sm.g[t][n + 2] + z4[3] * sm.g[t][n + 3];
    }
    sm.P[h][t] = a;
  }
  for (int h = tid; h < H; h += blockDim.x) {
    const float* zr = zin + (int64_t)h * N;
    const float* lr = lam + (int64_t)h * N;
    float a = 0.f;
    for (int n = 0; n < N; n += 4) {
      const f32x4 z4 = *reinterpret_cast<const f32x4*>(zr + n), l4 = *reinterpret_cast<const f32x4*>(lr + n);
      a += z4[0] * l4[0] + z4[1] * l4[1] + z4[2] * l4[2] + z4[3] * l4[3];
    }
    sm.S1[h] = a;
  }
  for (int gi = 0; gi < G; ++gi) {
    __syncthreads();                   // c, d, g ready; the previous group's B, M, V no longer read
    {
      const T* Bb = reinterpret_cast<const T*>(p.B) + (int64_t)b * p.B_sb + (int64_t)gi * N;
      for (int e = tid; e < HS_SEG * N; e += blockDim.x) {
        const int t = e / N, n = e % N;
        sm.Bt[t][n] = t < len ? to_f32(Bb[(tok0 + t) * p.B_sl + n]) : 0.f;
      }
    }
    __syncthreads();
    // M[t'][s] = g_t' . B_s;  R[h][s] = Lam^h . B_s;  V[t][t'] = sum_{h in group} u_t e^{c_t' - c_t} (t' >= t)
    for (int e = tid; e < HS_SEG * HS_SEG; e += blockDim.x) {
      const int tp = e / HS_SEG, s_ = e % HS_SEG;
      float a = 0.f;
      for (int n = 0; n < N; ++n) a += sm.g[tp][n] * sm.Bt[s_][n];
      sm.M[tp][s_] = a;
      float v = 0.f;
      const int t = tp, t2 = s_;        // V[t][t2], t2 >= t
      if (t2 >= t)
        for (int h = gi * hpg; h < (gi + 1) * hpg; ++h)
          v += sm.d[t][h] * sm.xs[t][h] * __expf(sm.c[t2][h] - sm.c[t][h]);
      sm.V[t][t2] = v;
    }
    for (int e = tid; e < hpg * HS_SEG; e += blockDim.x) {
      const int h = gi * hpg + e / HS_SEG, s_ = e % HS_SEG;
      const float* lr = lam + (int64_t)h * N;
      float a = 0.f;
      for (int n = 0; n < N; n += 4) {
        const f32x4 l4 = *reinterpret_cast<const f32x4*>(lr + n);
        a += l4[0] * sm.Bt[s_][n] + l4[1] * sm.Bt[s_][n + 1] + l4[2] * sm.Bt[s_][n + 2] + l4[3] * sm.Bt[s_][n + 3];
      }
      sm.R[h][s_] = a;
    }
    __syncthreads();
    // Y columns, two heads per wave (lane half = head, lane % 32 = s), walking t from the segment end
    for (int h0 = gi * hpg + 2 * w; h0 < (gi + 1) * hpg; h0 += 8) {
      const int h = h0 + (l >> 5), s_ = l & 31;
      const bool hv = h < (gi + 1) * hpg;
      const int hh = hv ? h : h0;
      const float cs = sm.c[s_][hh], us = sm.d[s_][hh] * sm.xs[s_][hh];
      float y = 0.f;
      for (int t = HS_SEG - 1; t >= 0; --t) {
        const float an = t + 1 < HS_SEG ? __expf(sm.c[t + 1][hh] - sm.c[t][hh]) : 0.f;
        y = sm.M[t][s_] + an * y;
        const float cm1 = t > 0 ? sm.c[t - 1][hh] : 0.f;
        float term = s_ < t ? __expf(cm1 - cs) * us * y : 0.f;
#pragma unroll
        for (int o = 16; o >= 1; o >>= 1) term += __shfl_xor(term, o, 64);
        if (hv) {
          if (s_ == t) sm.du[t][hh] = y + __expf(sm.cend[hh] - sm.c[t][hh]) * sm.R[hh][t];
          if (s_ == 0) sm.q[t][hh] = term;
        }
      }
    }
    // dB_t[n] = sum_{t' >= t} V[t][t'] g_t'[n] + sum_{h in group} u_t e^{c_31 - c_t} Lam^h[n]
    T* dB = reinterpret_cast<T*>(q.dB) + ((int64_t)b * p.seqlen + tok0) * G * N + (int64_t)gi * N;
    for (int e = tid; e < HS_SEG * N8; e += blockDim.x) {
      const int t = e / N8, n0 = 8 * (e % N8);
      float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      for (int tp = t; tp < HS_SEG; ++tp) {
        float gv[8];
        ld8f(&sm.g[tp][n0], gv);
        const float v = sm.V[t][tp];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] += v * gv[j];
      }
      for (int h = gi * hpg; h < (gi + 1) * hpg; ++h) {
        const float e2 = sm.d[t][h] * sm.xs[t][h] * __expf(sm.cend[h] - sm.c[t][h]);
        const float* lr = lam + (int64_t)h * N + n0;
        const f32x4 a4 = *reinterpret_cast<const f32x4*>(lr), b4 = *reinterpret_cast<const f32x4*>(lr + 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          acc[j] += e2 * a4[j];
          acc[4 + j] += e2 * b4[j];
        }
      }
      if (t < len) {
#pragma unroll
        for (int j = 0; j < 8; ++j) dB[(int64_t)t * G * N + n0 + j] = from_f32<T>(acc[j]);
      }
    }
  }
  __syncthreads();
  // ---- per head: the remaining terms of q, then d dt, d xs and the dA / d_dt_bias partials
  float* part = q.part + (((int64_t)b * p.nseg + si) * H) * 2;
  for (int h = tid; h < H; h += blockDim.x) {
    const float A = p.A[h], S1 = sm.S1[h], ce = sm.cend[h];
    const float bias = p.dt_bias ? p.dt_bias[h] : 0.f;
    float y2 = 0.f;
    for (int t = HS_SEG - 1; t >= 0; --t) {
      const float an = t + 1 < HS_SEG ? __expf(sm.c[t + 1][h] - sm.c[t][h]) : 0.f;
      y2 = sm.P[h][t] + an * y2;
      const float cm1 = t > 0 ? sm.c[t - 1][h] : 0.f;
      sm.q[t][h] += __expf(cm1) * y2;
    }
    float acc = 0.f, dA = 0.f, db = 0.f;
    for (int t = 0; t < HS_SEG; ++t) {
      const float cm1 = t > 0 ? sm.c[t - 1][h] : 0.f;
      const float ec = __expf(ce - sm.c[t][h]);
      const float qv = sm.q[t][h] + ec * (__expf(cm1) * S1 + acc);
      const float at = __expf(sm.c[t][h] - cm1);
      const float d = sm.d[t][h], xs = sm.xs[t][h], du = sm.du[t][h];
      acc = at * acc + d * xs * sm.R[h][t];
      if (t < len) {
        const float raw = dtb[(tok0 + t) * p.dt_sl + h];
        const float ddr = (A * at * qv + xs * du) * hsb_dt_chain(p, raw, bias);
        q.ddt[((int64_t)b * p.seqlen + tok0 + t) * H + h] = ddr;
        dA += d * at * qv;
        db += ddr;
      }
      sm.q[t][h] = d * du;               // d xs
    }
    part[2 * h] = dA;
    part[2 * h + 1] = db;
  }
  __syncthreads();
  // ---- dx[t][h][p] = d xs_t^h for every p
  T* dx = reinterpret_cast<T*>(q.dx) + ((int64_t)b * p.seqlen + tok0) * H * HD;
  for (int e = tid; e < len * H; e += blockDim.x) {
    const int t = e / H, h = e % H;
    const float v = sm.q[t][h];
    T* o = dx + ((int64_t)t * H + h) * HD;
    if constexpr (sizeof(T) == 2) {
      bf16x8 v8;
#pragma unroll
      for (int j = 0; j < 8; ++j) v8[j] = (bf16)v;
#pragma unroll
      for (int k = 0; k < HD / 8; ++k) *reinterpret_cast<bf16x8*>(o + 8 * k) = v8;
    } else {
#pragma unroll
      for (int k = 0; k < HD / 4; ++k) *reinterpret_cast<f32x4*>(o + 4 * k) = f32x4{v, v, v, v};
    }
  }
}

// dA[h], d_dt_bias[h]: one wave per head, the (batch, segment) partials summed in a fixed order.
__global__ __launch_bounds__(256) void ssd_hsb_reduce_kernel(SsdParams p, HsParams q) {
  const int h = blockIdx.x * 4 + wave_id(), l = lane_id();
  const int H = p.nheads, nbs = p.batch * p.nseg;
  if (h >= H) return;
  float a = 0.f, bb = 0.f;
  for (int k = l; k < nbs; k += 64) {
    a += q.part[((int64_t)k * H + h) * 2];
    bb += q.part[((int64_t)k * H + h) * 2 + 1];
  }
  a = wave_sum(a);
  bb = wave_sum(bb);
  if (l == 0) {
    if (q.dA) q.dA[h] = a;
    if (q.d_dt_bias) q.d_dt_bias[h] = bb;
  }
}

}  // namespace

bool ssd_hs_supported(int nheads, int dstate) { return nheads <= HS_MAXH && dstate <= HS_MAXN; }
bool ssd_hs_bwd_supported(int nheads, int dstate) { return nheads <= HSB_MAXH && dstate <= HSB_MAXN; }

size_t ssd_hs_workspace_bytes(int batch, int seqlen, int nheads, int dstate, bool backward) {
  const size_t nseg = (seqlen + HS_SEG - 1) / HS_SEG;
  const size_t st = align256((size_t)batch * nseg * nheads * dstate * sizeof(float));
  return st + align256((size_t)batch * nseg * nheads * sizeof(float)) +
         align256((size_t)batch * seqlen * nheads * sizeof(float)) +
         (backward ? st + align256((size_t)batch * nseg * nheads * 2 * sizeof(float)) : 0);
}

void ssd_hs_workspace_layout(SsdParams& p, HsParams& q, void* workspace, bool backward) {
  p.nseg = (p.seqlen + HS_SEG - 1) / HS_SEG;     // this pass's segments
  char* c = reinterpret_cast<char*>(workspace);
  const size_t st = align256((size_t)p.batch * p.nseg * p.nheads * p.dstate * sizeof(float));
  q.z = reinterpret_cast<float*>(c);
  c += st;
  q.dec = reinterpret_cast<float*>(c);
  c += align256((size_t)p.batch * p.nseg * p.nheads * sizeof(float));
  q.u = reinterpret_cast<float*>(c);
  c += align256((size_t)p.batch * p.seqlen * p.nheads * sizeof(float));
  q.lam = backward ? reinterpret_cast<float*>(c) : nullptr;
  c += backward ? st : 0;
  q.part = backward ? reinterpret_cast<float*>(c) : nullptr;
}

hipError_t launch_ssd_hs_bwd(const SsdParams& p, const HsParams& q, float* dh0, hipStream_t st) {
  const dim3 grid((unsigned)p.nseg, (unsigned)p.batch);
  const int64_t nc = (int64_t)p.batch * p.nheads * p.dstate;
  const bool bf = p.dtype == DT_BF16;
  if (p.seqlen == 0) {                 // d h0 = 0 (the carry over no segments), dA = d_dt_bias = 0
    hipLaunchKernelGGL(ssd_hsb_carry_kernel, dim3((unsigned)((nc + 255) / 256)), dim3(256), 0, st, p, q, dh0);
    hipLaunchKernelGGL(ssd_hsb_reduce_kernel, dim3((unsigned)((p.nheads + 3) / 4)), dim3(256), 0, st, p, q);
    return hipGetLastError();
  }
  // the forward's local contributions and entering sums, then the adjoint's
  if (bf) hipLaunchKernelGGL(ssd_hs_local_kernel<bf16>, grid, dim3(256), 0, st, p, q);
  else hipLaunchKernelGGL(ssd_hs_local_kernel<float>, grid, dim3(256), 0, st, p, q);
  hipLaunchKernelGGL(ssd_hs_carry_kernel, dim3((unsigned)((nc + 255) / 256)), dim3(256), 0, st, p, q);
  if (bf) hipLaunchKernelGGL(ssd_hsb_local_kernel<bf16>, grid, dim3(256), 0, st, p, q);
  else hipLaunchKernelGGL(ssd_hsb_local_kernel<float>, grid, dim3(256), 0, st, p, q);
  hipLaunchKernelGGL(ssd_hsb_carry_kernel, dim3((unsigned)((nc + 255) / 256)), dim3(256), 0, st, p, q, dh0);
  if (bf) hipLaunchKernelGGL(ssd_hsb_main_kernel<bf16>, grid, dim3(256), 0, st, p, q);
  else hipLaunchKernelGGL(ssd_hsb_main_kernel<float>, grid, dim3(256), 0, st, p, q);
  hipLaunchKernelGGL(ssd_hsb_reduce_kernel, dim3((unsigned)((p.nheads + 3) / 4)), dim3(256), 0, st, p, q);
  return hipGetLastError();
}

hipError_t launch_ssd_hs(const SsdParams& p, const HsParams& q, hipStream_t st) {
  if (p.seqlen == 0) return hipSuccess;
  const dim3 grid((unsigned)p.nseg, (unsigned)p.batch);
  if (p.dtype == DT_BF16)
    hipLaunchKernelGGL(ssd_hs_local_kernel<bf16>, grid, dim3(256), 0, st, p, q);
  else
    hipLaunchKernelGGL(ssd_hs_local_kernel<float>, grid, dim3(256), 0, st, p, q);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t nc = (int64_t)p.batch * p.nheads * p.dstate;
  hipLaunchKernelGGL(ssd_hs_carry_kernel, dim3((unsigned)((nc + 255) / 256)), dim3(256), 0, st, p, q);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (p.dtype == DT_BF16)
    hipLaunchKernelGGL(ssd_hs_out_kernel<bf16>, grid, dim3(256), 0, st, p, q);
  else
    hipLaunchKernelGGL(ssd_hs_out_kernel<float>, grid, dim3(256), 0, st, p, q);
  return hipGetLastError();
}

}  // namespace mh
