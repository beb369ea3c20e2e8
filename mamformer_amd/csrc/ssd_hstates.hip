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
constexpr int HS_HP = HS_MAXH + 1;   // row pitch of the per-(token, head) arrays: a column (one head, 32 tokens)
                                     // then spans 32 banks
constexpr float PR = 80.f;       // largest in-segment range of c factorised as E F

__device__ __forceinline__ float hs_dt(const SsdParams& p, float d, int h) {
  if (p.dt_bias) d += p.dt_bias[h];
  if (p.dt_softplus) d = softplus_f(d);
  if (p.has_dt_limit) d = fminf(fmaxf(d, p.dt_min), p.dt_max);
  return d;
}

struct HsSmem {
  float c[HS_SEG][HS_HP];        // raw dt, then the in-segment inclusive cumsum of A dt (flat past the end)
  float u[HS_SEG][HS_HP];        // dt xs (0 past the end); local pass: e^{c_end - c_s} dt xs
  float E[HS_SEG][HS_HP];        // out pass: e^{c_t - m}
  float F[HS_SEG][HS_HP];        // out pass: e^{m - c_s} u_s
  float Ei[HS_SEG][HS_HP];       // out pass: e^{c_t}
  float Bt[HS_SEG][HS_MAXN];     // B of one group
  float Zs[HS_ZH][HS_MAXN];      // out pass: entering state sums of HS_ZH heads
  float W[HS_SEG][HS_SEG + 4];   // W_g[t][s]
  float cend[HS_MAXH], mid[HS_MAXH];
  int wide[HS_MAXH];
  int anywide;
};

// dt, c and u = dt xs of segment si into LDS, xs = sum_p x computed from x (local pass, and written to the
// workspace) or read from it (out pass).
template <typename T, bool FROM_WS, typename Smem>
__device__ void hs_prologue(const SsdParams& p, const HsParams& q, Smem& sm, int b, int si, int len) {
  const int H = p.nheads, tid = threadIdx.x;
  const int64_t tok0 = (int64_t)si * HS_SEG;
  float* uws = q.u + ((int64_t)b * p.seqlen + tok0) * H;
  // raw dt of the segment into LDS (all loads in flight together; the per-head cumsum below reads LDS)
  const float* dtb = p.dt + (int64_t)b * p.dt_sb;
  for (int e = tid; e < HS_SEG * H; e += blockDim.x) {
    const int t = e / H, h = e % H;
    sm.c[t][h] = t < len ? dtb[(tok0 + t) * p.dt_sl + h] : 0.f;
  }
  if (!FROM_WS && p.xsum) {
    // xs[t][h] from the sums of x over each half of the head that the prefill wrote (x is not read)
    const float* xsb = p.xsum + ((int64_t)b * p.seqlen + tok0) * H * 2;
    for (int e = tid; e < HS_SEG * H; e += blockDim.x) {
      const int t = e / H, h = e % H;
      float xs = 0.f;
      if (t < len) {
        const f32x2 v = *reinterpret_cast<const f32x2*>(xsb + ((int64_t)t * H + h) * 2);
        xs = v[0] + v[1];
      }
      sm.u[t][h] = xs;                 // xs for now; times dt below
    }
  } else if (!FROM_WS) {
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
  // 16 segments' loads issued together, the next 16's while the chain runs through these (two buffers)
  auto ld = [&](int s0, float (&zl)[16], float (&d)[16]) {
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const bool in = s0 + k < p.nseg;
      zl[k] = in ? zp[(s0 + k) * zs] : 0.f;
      d[k] = in ? dp[(int64_t)(s0 + k) * H] : 1.f;
    }
  };
  auto step = [&](int s0, const float (&zl)[16], const float (&d)[16]) {
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (s0 + k < p.nseg) zp[(s0 + k) * zs] = Z;    // the state sum entering segment s0 + k
      Z = d[k] * Z + zl[k];
    }
  };
  float za[16], da[16], zb[16], dbf[16];
  if (p.nseg > 0) ld(0, za, da);
  for (int s0 = 0; s0 < p.nseg; s0 += 32) {
    if (s0 + 16 < p.nseg) ld(s0 + 16, zb, dbf);
    step(s0, za, da);
    if (s0 + 16 < p.nseg) {
      if (s0 + 32 < p.nseg) ld(s0 + 32, za, da);
      step(s0 + 16, zb, dbf);
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
// the adjoint of Z^h_t is lambda^h_t = g_t + a^h_{t+1} lambda^h_{t+1}, a_t = e^{A dt_t}, and
//   du_t = lambda_t . B_t,   q_t = lambda_t . Z_{t-1},   dB_t = sum_h u^h_t lambda^h_t,
//   d dt_t = A a_t q_t + xs_t du_t (through bias, softplus and clamp),   d xs_t = dt_t du_t (dx[t][h][p], every p),
//   dA = sum_t dt_t a_t q_t,   d h0[h][p][n] = a_0 lambda_0 (the adjoint of the state sum before the first token).
// Per 32-token segment with Zin the state sum entering it and Lam = a lambda of the next segment's first token:
//   ssd_hsb_local_kernel (segment, batch): the forward's local pass (xs, Zloc, segment decay) and
//                        GL[h][n] = sum_t e^{c_t} g_t[n] (c the in-segment inclusive cumsum of A dt), the
//                        segment's part of the adjoint handed to the left.
//   ssd_hsb_carry_kernel (batch, head, n): Zin of every segment left to right (in place over Zloc) and Lam of
//                        every segment right to left (in place over GL), then d h0.
//   ssd_hsb_main_kernel  (segment, batch): one head per wave at a time, lanes over the state columns: the two
//                        recurrences inside the segment run directly (Z forward from Zin, lambda backward from
//                        Lam; every factor a <= 1), du and q as lane partials reduced across the wave, dB summed
//                        over the waves in a fixed order, dx, ddt and per-segment dA / d_dt_bias partials.
//   ssd_hsb_reduce_kernel: dA and d_dt_bias summed over (batch, segment) in a fixed order.
constexpr int HSB_MAXH = 128, HSB_MAXN = 128;   // state columns: two per lane
constexpr int HSB_WAVES = 4, HSB_WAVES_LOC = 8;

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

__device__ __forceinline__ float hsb_readlane(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// g of the segment into g[t][n] (0 past the end and for n >= N, so whole rows of W columns can be read)
template <typename T, int W>
__device__ void hsb_load_g(const SsdParams& p, const HsParams& q, float (*g)[W], int b, int si, int len) {
  const int N = p.dstate;
  const float scale = 1.f / ((float)p.nheads * (float)p.headdim);
  const T* src = reinterpret_cast<const T*>(q.dhs) + ((int64_t)b * p.seqlen + (int64_t)si * HS_SEG) * N;
  for (int e = threadIdx.x; e < HS_SEG * W; e += blockDim.x) {
    const int t = e / W, n = e % W;
    g[t][n] = (t < len && n < N) ? to_f32(src[(int64_t)t * N + n]) * scale : 0.f;
  }
}

struct HsbLocSmem {
  float c[HS_SEG][HS_HP];        // as in HsSmem
  float u[HS_SEG][HS_HP];
  float g[HS_SEG][HSB_MAXN];     // ghs / (H P) (0 past the end and beyond N)
  float B[HS_SEG][HSB_MAXN];     // B of one group (likewise)
  float cend[HSB_MAXH], mid[HSB_MAXH];
  int wide[HSB_MAXH];
};

// One head per wave at a time, lanes over pairs of state columns, the per-token weights broadcast from lane t:
// GL[h][n] = sum_t e^{c_t} g_t[n] and Zloc[h][n] = sum_s e^{c_end - c_s} u_s B_s[n].
template <typename T>
__global__ __launch_bounds__(64 * HSB_WAVES_LOC) void ssd_hsb_local_kernel(SsdParams p, HsParams q) {
  __shared__ HsbLocSmem sm;
  const int si = blockIdx.x, b = blockIdx.y, tid = threadIdx.x, w = wave_id(), l = lane_id();
  const int H = p.nheads, N = p.dstate, G = p.ngroups, hpg = H / G;
  const int64_t tok0 = (int64_t)si * HS_SEG;
  const int len = min(HS_SEG, p.seqlen - (int)tok0);
  const int n0 = 2 * l, t = l & 31;
  hs_prologue<T, false>(p, q, sm, b, si, len);
  hsb_load_g<T, HSB_MAXN>(p, q, sm.g, b, si, len);
  float* gl = q.lam + (((int64_t)b * p.nseg + si) * H) * N;
  float* zl = q.z + (((int64_t)b * p.nseg + si) * H) * N;
  for (int gi = 0; gi < G; ++gi) {
    __syncthreads();                   // c, u, g stored; the previous group's B no longer read
    {
      const T* Bb = reinterpret_cast<const T*>(p.B) + (int64_t)b * p.B_sb + (int64_t)gi * N;
      for (int e = tid; e < HS_SEG * HSB_MAXN; e += blockDim.x) {
        const int s = e / HSB_MAXN, n = e % HSB_MAXN;
        sm.B[s][n] = (s < len && n < N) ? to_f32(Bb[(tok0 + s) * p.B_sl + n]) : 0.f;
      }
    }
    __syncthreads();
    for (int h = gi * hpg + w; h < (gi + 1) * hpg; h += HSB_WAVES_LOC) {
      const float c = sm.c[t][h];
      const float ei = __expf(c), wt = __expf(sm.cend[h] - c) * sm.u[t][h];   // both exponents <= 0
      float g0 = 0.f, g1 = 0.f, z0 = 0.f, z1 = 0.f;
#pragma unroll
      for (int s = 0; s < HS_SEG; ++s) {
        const float es = hsb_readlane(ei, s), ws = hsb_readlane(wt, s);
        const float2 gv = *reinterpret_cast<const float2*>(&sm.g[s][n0]);
        const float2 bv = *reinterpret_cast<const float2*>(&sm.B[s][n0]);
        g0 += es * gv.x;
        g1 += es * gv.y;
        z0 += ws * bv.x;
        z1 += ws * bv.y;
      }
      if (n0 < N) {
        *reinterpret_cast<float2*>(gl + (int64_t)h * N + n0) = float2{g0, g1};
        *reinterpret_cast<float2*>(zl + (int64_t)h * N + n0) = float2{z0, z1};
      }
    }
  }
  if (tid < H) q.dec[((int64_t)b * p.nseg + si) * H + tid] = __expf(sm.cend[tid]);
}

// Both carries of one (batch, head, column): forward Zin_{k+1} = dec_k Zin_k + Zloc_k from the summed initial
// state, backward Lam_{k-1} = dec_k Lam_k + GL_k from Lam_last = 0; 16 segments of each chain loaded together.
__global__ __launch_bounds__(256) void ssd_hsb_carry_kernel(SsdParams p, HsParams q, float* dh0) {
  const int H = p.nheads, N = p.dstate, P = p.headdim, ns = p.nseg;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)p.batch * H * N) return;
  const int n = (int)(i % N), h = (int)((i / N) % H), b = (int)(i / ((int64_t)N * H));
  float Z = 0.f;
  if (p.init_state) {
    const float* s0 = p.init_state + (((int64_t)b * H + h) * P) * N + n;
    for (int k = 0; k < P; ++k) Z += s0[(int64_t)k * N];
  }
  float* zp = q.z + ((int64_t)b * ns * H + h) * N + n;
  float* lp = q.lam + ((int64_t)b * ns * H + h) * N + n;
  const float* dp = q.dec + (int64_t)b * ns * H + h;
  const int64_t zs = (int64_t)H * N;
  float L = 0.f;
  // 16 segments of each chain loaded together, the next 16's while the chains run through these (two buffers;
  // the loads read segments neither chain has written yet)
  struct Batch { float zl[16], df[16], gl[16], db[16]; };
  auto ld = [&](int s0, Batch& t) {
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int sf = s0 + k, sb = ns - 1 - s0 - k;
      t.zl[k] = sf < ns ? zp[sf * zs] : 0.f;
      t.df[k] = sf < ns ? dp[(int64_t)sf * H] : 1.f;
      t.gl[k] = sb >= 0 ? lp[sb * zs] : 0.f;
      t.db[k] = sb >= 0 ? dp[(int64_t)sb * H] : 1.f;
    }
  };
  auto step = [&](int s0, const Batch& t) {
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int sf = s0 + k, sb = ns - 1 - s0 - k;
      if (sf < ns) zp[sf * zs] = Z;      // the state sum entering segment sf
      Z = t.df[k] * Z + t.zl[k];
      if (sb >= 0) lp[sb * zs] = L;      // the adjoint handed into segment sb from the right
      L = t.db[k] * L + t.gl[k];
    }
  };
  Batch ba, bb;
  if (ns > 0) ld(0, ba);
  for (int s0 = 0; s0 < ns; s0 += 32) {
    if (s0 + 16 < ns) ld(s0 + 16, bb);
    step(s0, ba);
    if (s0 + 16 < ns) {
      if (s0 + 32 < ns) ld(s0 + 32, ba);
      step(s0 + 16, bb);
    }
  }
  if (dh0) {
    float* o = dh0 + (((int64_t)b * H + h) * P) * N + n;
    for (int k = 0; k < P; ++k) o[(int64_t)k * N] = L;
  }
}

// One step of the reduction below for lane mask M over the first K values.
template <int M, int K, int NV>
__device__ __forceinline__ void hsb_rs_step(float (&v)[NV], int l) {
  const bool up = (l & M) != 0;
#pragma unroll
  for (int k = 0; k < K / 2; ++k) {
    const float keep = up ? v[k + K / 2] : v[k], send = up ? v[k] : v[k + K / 2];
    v[k] = keep + __shfl_xor(send, M, 64);
  }
}

// Sum over the 64 lanes of v[k] for every k, lanes 2k and 2k + 1 ending with the sum of v[k]: at each step the
// lanes whose mask bit is set keep the upper half of their values and trade the lower half with the partner.
__device__ __forceinline__ float hsb_reduce_scatter(float (&v)[32]) {
  const int l = lane_id();
  // mask 32: v_permlane32_swap hands the lower lanes the partner's first half and the upper ones its second
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[k]), __float_as_uint(v[k + 16]), false, false);
    v[k] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  // mask 16: v_permlane16_swap, the same within each half
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[k]), __float_as_uint(v[k + 8]), false, false);
    v[k] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  hsb_rs_step<8, 8>(v, l);
  hsb_rs_step<4, 4>(v, l);
  hsb_rs_step<2, 2>(v, l);
  return v[0] + __shfl_xor(v[0], 1, 64);
}

struct HsbSmem {
  float g[HS_SEG][HSB_MAXN];     // ghs / (H P) (0 past the end and beyond N)
  float B[HS_SEG][HSB_MAXN];     // B of one group (likewise)
  float dB[HS_SEG][HSB_MAXN];    // the group's dB, summed over the waves in wave order
};

template <typename T>
__global__ __launch_bounds__(64 * HSB_WAVES) void ssd_hsb_main_kernel(SsdParams p, HsParams q) {
  __shared__ HsbSmem sm;
  const int si = blockIdx.x, b = blockIdx.y, tid = threadIdx.x, w = wave_id(), l = lane_id();
  const int H = p.nheads, N = p.dstate, G = p.ngroups, hpg = H / G;
  const int64_t tok0 = (int64_t)si * HS_SEG;
  const int len = min(HS_SEG, p.seqlen - (int)tok0);
  const int n0 = 2 * l;                // this lane's two state columns (zero rows beyond N)
  const int t = l & 31;                // this lane's token in the per-token steps (both halves hold it)
  const bool tv = t < len;
  const float* dtb = p.dt + (int64_t)b * p.dt_sb + tok0 * p.dt_sl;
  const float* xsw = q.u + ((int64_t)b * p.seqlen + tok0) * H;
  const float* zin = q.z + (((int64_t)b * p.nseg + si) * H) * N;
  const float* lam = q.lam + (((int64_t)b * p.nseg + si) * H) * N;
  float* part = q.part + (((int64_t)b * p.nseg + si) * H) * 2;
  T* dxb = reinterpret_cast<T*>(q.dx) + ((int64_t)b * p.seqlen + tok0) * H * HD;
  float* ddtb = q.ddt + ((int64_t)b * p.seqlen + tok0) * H;
  hsb_load_g<T, HSB_MAXN>(p, q, sm.g, b, si, len);
  for (int gi = 0; gi < G; ++gi) {
    __syncthreads();                   // g stored; the previous group's B and dB no longer read
    {
      const T* Bb = reinterpret_cast<const T*>(p.B) + (int64_t)b * p.B_sb + (int64_t)gi * N;
      for (int e = tid; e < HS_SEG * HSB_MAXN; e += blockDim.x) {
        const int s = e / HSB_MAXN, n = e % HSB_MAXN;
        sm.B[s][n] = (s < len && n < N) ? to_f32(Bb[(tok0 + s) * p.B_sl + n]) : 0.f;
      }
    }
    __syncthreads();
    float acc[HS_SEG][2];              // this wave's part of dB for the group's heads it handles
#pragma unroll
    for (int s = 0; s < HS_SEG; ++s) acc[s][0] = acc[s][1] = 0.f;
    // the global inputs of a head (raw dt and xs of token t, Zin and Lam of the lane's columns), loaded one
    // head ahead so that their latency overlaps the previous head's work
    const int hend = (gi + 1) * hpg;
    float nraw = 0.f, nxs = 0.f;
    float2 nz = {0.f, 0.f}, nl = {0.f, 0.f};
    auto fetch = [&](int hh) {
      nraw = tv ? dtb[(int64_t)t * p.dt_sl + hh] : 0.f;
      nxs = tv ? xsw[(int64_t)t * H + hh] : 0.f;
      if (n0 < N) {
        nz = *reinterpret_cast<const float2*>(zin + (int64_t)hh * N + n0);
        nl = *reinterpret_cast<const float2*>(lam + (int64_t)hh * N + n0);
      }
    };
    if (gi * hpg + w < hend) fetch(gi * hpg + w);
    for (int h = gi * hpg + w; h < hend; h += HSB_WAVES) {
      // per-token scalars, token t in lanes t and t + 32
      const float raw = nraw, xs = nxs;
      float Z0 = nz.x, Z1 = nz.y, L0 = nl.x, L1 = nl.y;
      if (h + HSB_WAVES < hend) fetch(h + HSB_WAVES);
      const float A = p.A[h];
      const float d = tv ? hs_dt(p, raw, h) : 0.f;
      const float a = __expf(A * d);   // 1 past the end
      const float u = d * xs;
      // The segment in two halves of 16 tokens (Z_{s-1} kept for one half at a time): forward to Z_15, then
      // for s = 16 .. 31 and again from Zin for s = 0 .. 15, Z_{s-1} of every token (Z_s = a_s Z_{s-1} + u_s B_s),
      // and backward lambda_s = g_s + a_{s+1} lambda_{s+1} (lambda_31 = g_31 + Lam) with the lane partials of
      // du_s = lambda_s . B_s and q_s = lambda_s . Z_{s-1}, and u_s lambda_s into dB.
      const float Zi0 = Z0, Zi1 = Z1;
#pragma unroll
      for (int s = 0; s < HS_SEG / 2; ++s) {
        const float as = hsb_readlane(a, s), us = hsb_readlane(u, s);
        const float2 bv = *reinterpret_cast<const float2*>(&sm.B[s][n0]);
        Z0 = as * Z0 + us * bv.x;
        Z1 = as * Z1 + us * bv.y;
      }
      float r[2];
#pragma unroll
      for (int hf = 1; hf >= 0; --hf) {
        const int s0 = 16 * hf;
        if (hf == 0) {
          Z0 = Zi0;
          Z1 = Zi1;
        }
        float zp[16][2];
#pragma unroll
        for (int k = 0; k < 16; ++k) {
          const int s = s0 + k;
          zp[k][0] = Z0;
          zp[k][1] = Z1;
          if (k < 15) {
            const float as = hsb_readlane(a, s), us = hsb_readlane(u, s);
            const float2 bv = *reinterpret_cast<const float2*>(&sm.B[s][n0]);
            Z0 = as * Z0 + us * bv.x;
            Z1 = as * Z1 + us * bv.y;
          }
        }
        float v[32];
#pragma unroll
        for (int k = 15; k >= 0; --k) {
          const int s = s0 + k;
          const float2 gv = *reinterpret_cast<const float2*>(&sm.g[s][n0]);
          const float an = s == HS_SEG - 1 ? 1.f : hsb_readlane(a, s + 1);
          L0 = gv.x + an * L0;
          L1 = gv.y + an * L1;
          const float2 bv = *reinterpret_cast<const float2*>(&sm.B[s][n0]);
          v[k] = L0 * bv.x + L1 * bv.y;
          v[16 + k] = L0 * zp[k][0] + L1 * zp[k][1];
          const float us = hsb_readlane(u, s);
          acc[s][0] += us * L0;
          acc[s][1] += us * L1;
        }
        r[hf] = hsb_reduce_scatter(v);   // lanes 2k, 2k + 1: du_{s0 + k} (k < 16), q_{s0 + k - 16} (k >= 16)
      }
      const int src = (2 * t) & 31;
      const float du0 = __shfl(r[0], src, 64), du1 = __shfl(r[1], src, 64);
      const float q0 = __shfl(r[0], 32 + src, 64), q1 = __shfl(r[1], 32 + src, 64);
      const float du = t < 16 ? du0 : du1, qv = t < 16 ? q0 : q1;
      float dA = 0.f, db = 0.f;
      if (l < 32 && tv) {
        const float bias = p.dt_bias ? p.dt_bias[h] : 0.f;
        const float ddr = (A * a * qv + xs * du) * hsb_dt_chain(p, raw, bias);
        ddtb[(int64_t)t * H + h] = ddr;
        dA = d * a * qv;
        db = ddr;
      }
      dA = wave_sum(dA);
      db = wave_sum(db);
      if (l == 0) {
        part[2 * h] = dA;
        part[2 * h + 1] = db;
      }
      // dx[t][h][p] = dt_t du_t for every p: lane t writes the first half of the row, lane t + 32 the second
      if (tv) {
        const float dxs = d * du;
        T* o = dxb + ((int64_t)t * H + h) * HD + (l >> 5) * (HD / 2);
        if constexpr (sizeof(T) == 2) {
          bf16x8 v8;
#pragma unroll
          for (int j = 0; j < 8; ++j) v8[j] = (bf16)dxs;
#pragma unroll
          for (int k = 0; k < HD / 16; ++k) *reinterpret_cast<bf16x8*>(o + 8 * k) = v8;
        } else {
#pragma unroll
          for (int k = 0; k < HD / 8; ++k) *reinterpret_cast<f32x4*>(o + 4 * k) = f32x4{dxs, dxs, dxs, dxs};
        }
      }
    }
    // dB of the group: the waves' parts added in wave order
    for (int k = 0; k < HSB_WAVES; ++k) {
      if (w == k) {
#pragma unroll
        for (int s = 0; s < HS_SEG; ++s) {
          float2* o = reinterpret_cast<float2*>(&sm.dB[s][n0]);
          const float2 prev = k == 0 ? float2{0.f, 0.f} : *o;
          *o = float2{prev.x + acc[s][0], prev.y + acc[s][1]};
        }
      }
      __syncthreads();
    }
    T* dB = reinterpret_cast<T*>(q.dB) + ((int64_t)b * p.seqlen + tok0) * G * N + (int64_t)gi * N;
    for (int e = tid; e < len * N; e += blockDim.x) {
      const int s = e / N, n = e % N;
      dB[(int64_t)s * G * N + n] = from_f32<T>(sm.dB[s][n]);
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
  // the segments' local sums of the state and of the adjoint, both carries, then the gradients
  if (bf) hipLaunchKernelGGL(ssd_hsb_local_kernel<bf16>, grid, dim3(64 * HSB_WAVES_LOC), 0, st, p, q);
  else hipLaunchKernelGGL(ssd_hsb_local_kernel<float>, grid, dim3(64 * HSB_WAVES_LOC), 0, st, p, q);
  hipLaunchKernelGGL(ssd_hsb_carry_kernel, dim3((unsigned)((nc + 255) / 256)), dim3(256), 0, st, p, q, dh0);
  if (bf) hipLaunchKernelGGL(ssd_hsb_main_kernel<bf16>, grid, dim3(64 * HSB_WAVES), 0, st, p, q);
  else hipLaunchKernelGGL(ssd_hsb_main_kernel<float>, grid, dim3(64 * HSB_WAVES), 0, st, p, q);
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
