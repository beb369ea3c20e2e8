// h_states of the SSD prefill: hs[b, t, n] = mean over (h, p) of the state h_t[h, p, n]
// (mamformer/layers/mamba2.py:114-116).  The channel sum of the state obeys a recurrence of its own,
//     Z_t[h, n] = sum_p h_t[h, p, n] = e^{A_h dt_t,h} Z_{t-1}[h, n] + dt_t,h xs_t[h] B_t[g(h), n],
//     xs_t[h] = sum_p x_t[h, p],        hs_t[n] = sum_h Z_t[h, n] / (H P),
// so h_states needs one scalar input per (token, head) instead of P of them.  Three passes over 32-token
// segments, all in fp32:
//   ssd_hs_local_kernel  (segment, batch): dt processed as the prefill does it, c = in-segment inclusive cumsum
//                        of A dt, xs and u = dt xs per (token, head) into the workspace, and the segment's own
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

// dt, c and (from x) u of segment si into LDS; u also to the workspace (local pass) or from it (out pass).
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
        if (!FROM_WS) {
          const float uv = d * sm.u[t][h];
          sm.u[t][h] = uv;
          uws[(int64_t)t * H + h] = uv;
        }
      } else if (!FROM_WS) {
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

}  // namespace

bool ssd_hs_supported(int nheads, int dstate) { return nheads <= HS_MAXH && dstate <= HS_MAXN; }

size_t ssd_hs_workspace_bytes(int batch, int seqlen, int nheads, int dstate) {
  const size_t nseg = (seqlen + HS_SEG - 1) / HS_SEG;
  return align256((size_t)batch * nseg * nheads * dstate * sizeof(float)) +
         align256((size_t)batch * nseg * nheads * sizeof(float)) +
         align256((size_t)batch * seqlen * nheads * sizeof(float));
}

void ssd_hs_workspace_layout(SsdParams& p, HsParams& q, void* workspace) {
  p.nseg = (p.seqlen + HS_SEG - 1) / HS_SEG;     // this pass's segments
  char* c = reinterpret_cast<char*>(workspace);
  q.z = reinterpret_cast<float*>(c);
  c += align256((size_t)p.batch * p.nseg * p.nheads * p.dstate * sizeof(float));
  q.dec = reinterpret_cast<float*>(c);
  c += align256((size_t)p.batch * p.nseg * p.nheads * sizeof(float));
  q.u = reinterpret_cast<float*>(c);
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
