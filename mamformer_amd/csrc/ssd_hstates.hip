// h_states of the SSD prefill: hs[b, t, n] = mean over (h, p) of the state h_t[h, p, n]
// (mamformer/layers/mamba2.py:114-116).  The channel sum of the state obeys a recurrence of its own,
//     Z_t[h, n] = sum_p h_t[h, p, n] = e^{A_h dt_t,h} Z_{t-1}[h, n] + dt_t,h xs_t[h] B_t[g(h), n],
//     xs_t[h] = sum_p x_t[h, p],        hs_t[n] = sum_h Z_t[h, n] / (H P),
// so h_states needs one scalar input per (token, head) instead of P of them.  Three passes over 32-token
// segments, all in fp32, the state columns in blocks of HS_NB:
//   ssd_hs_local_kernel  (segment, batch, column block): dt processed as the prefill does it, c = in-segment
//                        inclusive cumsum of A dt, u = dt xs (xs from the prefill's per-head sums of x, or from x),
//                        the segment's own contribution Zloc[h][n] = sum_s e^{c_end - c_s} u_s[h] B_s[g(h)][n] for
//                        the block's columns (fp32 MFMAs), and its share of the segment's factors
//                        Ei[h][t] = e^{c_t,h} and W_g[t][s] = sum_{h in g} e^{c_t,h - c_s,h} u_s[h] (s <= t).
//   ssd_hs_carry_kernel  (batch, head, n): Zin of every segment, Zin_0 = sum_p h0[h, p, n] (or 0),
//                        Zin_{k+1} = e^{c_end,k} Zin_k + Zloc_k (in place over Zloc), a two-level scan.
//   ssd_hs_out_kernel    (segment, batch, column block), one wave of fp32 MFMAs:
//                        hs_t[n] = (sum_h Ei[h][t] Zin[h][n] + sum_g sum_{s <= t} W_g[t][s] B_s[g][n]) / (H P).
// Every exponent is <= 0 (A <= 0, dt >= 0, c falls along the segment): no factor can overflow whatever the decay.
#include "common.h"
#include "launch.h"
#include "ssd_shared.h"

namespace mh {

namespace {

constexpr int HS_SEG = 32;       // tokens per segment
constexpr int HS_MAXH = 128;     // heads held in LDS
constexpr int HS_MAXN = 256;
constexpr int HS_NB = 32;        // state columns per forward workgroup
constexpr int HS_HP = HS_MAXH + 1;   // row pitch of the per-(token, head) arrays: a column (one head, 32 tokens)
                                     // then spans 32 banks
constexpr int HS_LP = HS_MAXH + 4;   // the same in the forward local pass: 16-byte reads of 4 heads, and 16
                                     // consecutive rows read together fall on distinct banks

__device__ __forceinline__ float hs_dt(const SsdParams& p, float d, int h) {
  if (p.dt_bias) d += p.dt_bias[h];
  if (p.dt_softplus) d = softplus_f(d);
  if (p.has_dt_limit) d = fminf(fmaxf(d, p.dt_min), p.dt_max);
  return d;
}

// dt, c and u = dt xs of segment si into LDS (sm.c, sm.u, sm.cend).  xs = sum_p x is taken from the prefill's
// per-half sums (p.xsum) when given, else summed from x; xs_out (or null) receives xs per (token, head).  dt is
// processed element-parallel (bias, softplus, clamp) as it arrives; only the cumsum of A dt runs per head.
// The element loads are unconditional at clamped (valid) addresses, so that each thread's KB loads of a pass are
// in flight together: an element past the end of the segment is zeroed by a factor 0 (its dt finite), and a thread
// past the last element repeats the last one (the same value written twice).
template <bool XS, int KB, typename Smem>
__device__ void hs_prologue_elems(const SsdParams& p, Smem& sm, int b, int si, int len, float* uws) {
  const int H = p.nheads, tid = threadIdx.x, tot = HS_SEG * H, nt = blockDim.x;
  const int64_t tok0 = (int64_t)si * HS_SEG;
  const float* dtb = p.dt + (int64_t)b * p.dt_sb;
  const float* xsb = XS ? p.xsum + ((int64_t)b * p.seqlen + tok0) * H * 2 : nullptr;
  const float* bias = p.dt_bias ? p.dt_bias : p.A;       // any valid per-head array when there is no bias
  const float bmul = p.dt_bias ? 1.f : 0.f;
  // element e = tid + nt i is (t, h) = (e / H, e % H), stepped by (nt / H, nt % H) without a division per element
  const int dq = nt / H, dr = nt % H;
  int te = tid / H, he = tid % H;
  for (int base = 0; base < tot; base += KB * nt) {
    float d[KB], av[KB], bv[KB];
    f32x2 xv[KB];
    int tk[KB], hk[KB];
#pragma unroll
    for (int k = 0; k < KB; ++k) {
      const bool past = te >= HS_SEG;                     // e >= tot: repeat the last element
      tk[k] = past ? HS_SEG - 1 : te;
      hk[k] = past ? H - 1 : he;
      he += dr;
      te += dq;
      if (he >= H) {
        he -= H;
        ++te;
      }
      const int t = tk[k], h = hk[k], tc = min(t, len - 1);
      d[k] = dtb[(tok0 + tc) * p.dt_sl + h];
      av[k] = p.A[h];
      bv[k] = bias[h];
      if constexpr (XS) xv[k] = *reinterpret_cast<const f32x2*>(xsb + ((int64_t)tc * H + h) * 2);
    }
    __builtin_amdgcn_sched_barrier(0);  // every load of the pass issued before the first use
#pragma unroll
    for (int k = 0; k < KB; ++k) {
      const int t = tk[k], h = hk[k];
      float x = d[k] + bv[k] * bmul;
      if (p.dt_softplus) x = softplus_f(x);
      if (p.has_dt_limit) x = fminf(fmaxf(x, p.dt_min), p.dt_max);
      const float dd = x * (t < len ? 1.f : 0.f);          // 0 past the end: c flat, u = 0
      sm.c[t][h] = av[k] * dd;                               // the cumsum below makes it c
      if constexpr (XS) {
        const float xs = xv[k][0] + xv[k][1];
        if (uws && t < len) uws[(int64_t)t * H + h] = xs;
        sm.u[t][h] = dd * xs;
      } else {
        sm.u[t][h] = dd;                                     // times xs below
      }
    }
  }
}

// KB: elements per thread and pass (KB x the workgroup's threads = 2048 covers a segment of 64 heads in one pass).
template <typename T, int KB, typename Smem>
__device__ void hs_prologue(const SsdParams& p, Smem& sm, int b, int si, int len, float* xs_out) {
  const int H = p.nheads, tid = threadIdx.x, tot = HS_SEG * H, nt = blockDim.x;
  const int64_t tok0 = (int64_t)si * HS_SEG;
  float* uws = xs_out ? xs_out + ((int64_t)b * p.seqlen + tok0) * H : nullptr;
  const bool xsb = p.xsum != nullptr;
  if (xsb) hs_prologue_elems<true, KB>(p, sm, b, si, len, uws);
  else hs_prologue_elems<false, KB>(p, sm, b, si, len, uws);
  if (!xsb) {
    __syncthreads();                   // the element pass's repeated writes of the last element are done
    // xs[t][h] = sum_p x[t][h][p] (P = 64): one (token, head) row per thread pass, its 16 loads issued together
    const T* xb = reinterpret_cast<const T*>(p.x) + (int64_t)b * p.x_sb;
    for (int e = tid; e < tot; e += nt) {
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
        if (uws) uws[(int64_t)t * H + h] = xs;
      }
      sm.u[t][h] *= xs;
    }
  }
  __syncthreads();
  // per head: the inclusive cumsum of A dt over the segment
  for (int h = tid; h < H; h += nt) {
    float a[HS_SEG];
#pragma unroll
    for (int t = 0; t < HS_SEG; ++t) a[t] = sm.c[t][h];
    float c = 0.f;
#pragma unroll
    for (int t = 0; t < HS_SEG; ++t) {
      c += a[t];
      sm.c[t][h] = c;
    }
    sm.cend[h] = c;
  }
}

struct __align__(16) HsLocSmem {
  float c[HS_SEG][HS_LP];        // raw dt, then the in-segment inclusive cumsum of A dt
  float u[HS_SEG][HS_LP];        // dt xs
  float cend[HS_MAXH];
};

// W_g[t][s] = sum_{h in g} e^{c_t,h - c_s,h} u_s[h] for s <= t (every exponent c_t - c_s <= 0).
__device__ __forceinline__ float hs_weight(const HsLocSmem& sm, int g, int hpg, int t, int s) {
  float w = 0.f;
  if (hpg % 4 == 0) {
    for (int h = g * hpg; h < (g + 1) * hpg; h += 4) {
      const f32x4 ct = *reinterpret_cast<const f32x4*>(&sm.c[t][h]);
      const f32x4 cs = *reinterpret_cast<const f32x4*>(&sm.c[s][h]);
      const f32x4 us = *reinterpret_cast<const f32x4*>(&sm.u[s][h]);
#pragma unroll
      for (int j = 0; j < 4; ++j) w += __expf(ct[j] - cs[j]) * us[j];
    }
  } else {
    for (int h = g * hpg; h < (g + 1) * hpg; ++h) w += __expf(sm.c[t][h] - sm.c[s][h]) * sm.u[s][h];
  }
  return w;
}

// Forward: HS_FS workgroups of HS_LOC_FWD threads per (segment, batch), each over every block of HS_NB state
// columns, so that the prologue runs HS_FS times per segment instead of once per column block: the prologue,
// then its share of
//  - the output pass's factors: W_g[t][s] for the pairs s <= t (one pair per thread; the entries s > t are never
//    written: the output pass masks them), stored s-major (row s of WT holds W_g[.][s] over the 32 tokens), and
//    Ei[h][t] = e^{c_t,h} (0 past the end);
//  - Zloc[h][n] = sum_s e^{c_end - c_s} u_s[h] B_s[n], one (column block, group, 32 heads) tile of fp32 MFMAs per
//    wave at a time (32 heads x 32 columns, k over pairs of tokens, B read from global memory);
//  - the segment's decays.
// BWD: the backward's local pass, one workgroup of 256 threads per (segment, batch, column block zb): no W or
// Ei, xs per (token, head) written to q.u (column block 0), and besides Zloc the segment's part of the adjoint
// handed left, GL[h][n] = sum_t e^{c_t} g_t[n] with g = dhs / (H P), into q.lam (MFMA tiles like Zloc's,
// A = e^{c_t} (0 past the end), B = the block's columns of dhs).
// Forward workgroups per segment and their threads: 2 x 256 (b2 L4096 H64 N128 on one box, the three h_states
// passes: 29.4 us, against 30.8 us with one workgroup per (segment, column block) and 29.9 / 32.4 us with
// 1 x 512 / 4 x 128).
constexpr int HS_FS = 2;
constexpr int HS_LOC_FWD = 512 / HS_FS;
template <typename T, bool BWD>
__global__ __launch_bounds__(BWD ? 256 : HS_LOC_FWD) void ssd_hs_local_kernel(SsdParams p, HsParams q) {
  __shared__ HsLocSmem sm;
  const int si = blockIdx.x, b = blockIdx.y, zb = blockIdx.z;
  // forward: workgroup zb of the segment's HS_FS takes, of each list (W pairs, Ei entries), the items
  // fs0 + tid + k fstep, and of the Zloc tiles the units zb nw + wave + k ustep
  const int fs0 = BWD ? 0 : zb * blockDim.x, fstep = BWD ? blockDim.x : HS_FS * blockDim.x;
  const int tid = threadIdx.x, H = p.nheads, N = p.dstate, G = p.ngroups, hpg = H / G;
  const int len = min(HS_SEG, p.seqlen - si * HS_SEG);
  const int64_t tok0 = (int64_t)si * HS_SEG;
  const int l = lane_id(), i = l & 31, hf = l >> 5, tiles = (hpg + 31) / 32;
  // B operands of this wave's tile (k = token pairs), loaded before the prologue so that they arrive meanwhile;
  // unmasked at clamped addresses: a token past the end meets a zero A operand, a lane past the last column feeds
  // an output column that is not stored.  Units of a column block: [0, G tiles) Zloc of (group, 32 heads), B of
  // the group's columns; BWD [G tiles, 2 G tiles): GL, the columns of dhs.  The forward's unit u is unit u % per
  // of column block u / per.
  const int nz = G * tiles, per = BWD ? 2 * nz : nz, nunit = BWD ? per : per * ((N + HS_NB - 1) / HS_NB);
  auto unit_n0 = [&](int unit) { return HS_NB * (BWD ? zb : unit / per); };
  const int nw = blockDim.x / 64, ustep = BWD ? nw : HS_FS * nw;
  T bv[HS_SEG / 2];                    // converted at their use, so that nothing waits for them before
  auto load_b = [&](int unit) {
    const int n0 = unit_n0(unit), uu = unit % per;
    const T* Bg = uu < nz
        ? reinterpret_cast<const T*>(p.B) + (int64_t)b * p.B_sb + (int64_t)(uu / tiles) * N
        : reinterpret_cast<const T*>(q.dhs) + (int64_t)b * p.seqlen * N;
    const int64_t ld = uu < nz ? p.B_sl : N;
    Bg += n0 + min(i, N - 1 - n0);
#pragma unroll
    for (int m = 0; m < HS_SEG / 2; ++m) bv[m] = Bg[(tok0 + min(2 * m + hf, len - 1)) * ld];
  };
  int unit = (BWD ? 0 : zb * nw) + wave_id();
  if (unit < nunit) load_b(unit);
  hs_prologue<T, BWD ? 8 : HS_SEG * 64 / HS_LOC_FWD>(p, sm, b, si, len, (BWD && zb == 0) ? q.u : nullptr);
  __syncthreads();
  if constexpr (!BWD) {
    // pair r = t (t + 1) / 2 + s of group g (s <= t), t from the inverse triangular number (float estimate,
    // corrected by one either way)
    constexpr int NPAIR = HS_SEG * (HS_SEG + 1) / 2;
    float* wt = q.w + ((int64_t)b * p.nseg + si) * G * (HS_SEG * HS_SEG);
    for (int e = fs0 + tid; e < G * NPAIR; e += fstep) {
      const int g = e / NPAIR, r = e - g * NPAIR;
      int t = (int)((sqrtf(8.f * (float)r + 1.f) - 1.f) * 0.5f);
      if ((t + 1) * (t + 2) / 2 <= r) ++t;
      if (t * (t + 1) / 2 > r) --t;
      const int s = r - t * (t + 1) / 2;
      wt[((int64_t)g * HS_SEG + s) * HS_SEG + t] = hs_weight(sm, g, hpg, t, s);
    }
    float* eit = q.u + ((int64_t)b * p.nseg + si) * H * HS_SEG;
    for (int e = fs0 + tid; e < H * HS_SEG; e += fstep) {
      const int t = e % HS_SEG, h = e / HS_SEG;
      eit[(int64_t)h * HS_SEG + t] = t < len ? __expf(sm.c[t][h]) : 0.f;
    }
  }
  // Zloc (and GL): tiles of (group, 32 heads), one per wave at a time
  const float gscale = 1.f / ((float)H * (float)p.headdim);
  for (; unit < nunit; unit += ustep) {
    const int n0 = unit_n0(unit), uu = unit % per;
    const bool col = n0 + i < N;
    const bool gl = BWD && uu >= nz;
    const int uz = gl ? uu - nz : uu;
    const int g = uz / tiles, hl = (uz % tiles) * 32;
    const int h = g * hpg + min(hl + i, hpg - 1);            // A row (clamped; rows past hpg are not stored)
    const float ce = sm.cend[h];
    float a[HS_SEG / 2];
#pragma unroll
    for (int m = 0; m < HS_SEG / 2; ++m) {
      const int sk = 2 * m + hf;
      if (gl) a[m] = sk < len ? __expf(sm.c[sk][h]) : 0.f;
      else a[m] = sm.u[sk][h] * __expf(ce - sm.c[sk][h]);      // u is 0 past the end
    }
    f32x16 acc = zero16();
#pragma unroll
    for (int m = 0; m < HS_SEG / 2; ++m)
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[m], to_f32(bv[m]), acc, 0, 0, 0);
    if (unit + ustep < nunit) load_b(unit + ustep);
    if (col) {
      float* zl = (gl ? q.lam : q.z) + (((int64_t)b * p.nseg + si) * H + g * hpg + hl) * N + n0 + i;
      const float sc = gl ? gscale : 1.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int hr = acc_row(hf, r);
        if (hl + hr < hpg) zl[(int64_t)hr * N] = acc[r] * sc;
      }
    }
  }
  if (zb == 0)
    for (int h = tid; h < H; h += blockDim.x) q.dec[((int64_t)b * p.nseg + si) * H + h] = __expf(sm.cend[h]);
}

// The carry over segments as a two-level scan.  The segments of a chain (b, h, n) are cut into NP parts of
// consecutive segments; within a wave, lane j * CW + i holds part j of the wave's chain i (CW = 64 / NP chains per
// wave, consecutive in n, so a load of one part covers CW consecutive floats).  Each lane reduces its part to
// (decay product, sum entering from zero), forms the sum entering its part from the parts before it, read across
// the wave, starting at sum_p h0 (summed by all parts, rows p = j, j + NP, ...), then walks its part again writing
// every segment's entering sum in place over Zloc.  A part of at most KB segments stays in registers between the
// two walks; a longer one is loaded KB segments at a time, twice.
template <int NP>
__global__ __launch_bounds__(256) void ssd_hs_carry_kernel(SsdParams p, HsParams q) {
  constexpr int CW = 64 / NP, KB = 16;
  const int H = p.nheads, N = p.dstate, P = p.headdim, l = lane_id();
  const int part = l / CW, ci = l % CW;
  const int64_t chain = ((int64_t)blockIdx.x * 4 + wave_id()) * CW + ci;
  const bool on = chain < (int64_t)p.batch * H * N;
  const int64_t ch = on ? chain : 0;
  const int n = (int)(ch % N), h = (int)((ch / N) % H), b = (int)(ch / ((int64_t)N * H));
  const int pl = (p.nseg + NP - 1) / NP, k0 = min(p.nseg, part * pl), k1 = min(p.nseg, k0 + pl);
  float* zp = q.z + ((int64_t)b * p.nseg * H + h) * N + n;
  const float* dp = q.dec + (int64_t)b * p.nseg * H + h;
  const int64_t zs = (int64_t)H * N;
  float d[KB], z[KB];
  auto load = [&](int k) {
#pragma unroll
    for (int j = 0; j < KB; ++j) {
      const bool in = on && k + j < k1;
      d[j] = in ? dp[(int64_t)(k + j) * H] : 1.f;
      z[j] = in ? zp[(int64_t)(k + j) * zs] : 0.f;
    }
  };
  float Z0 = 0.f;
  if (on && p.init_state) {
    const float* s0 = p.init_state + (((int64_t)b * H + h) * P) * N + n;
    for (int k = part; k < P; k += NP) Z0 += s0[(int64_t)k * N];
  }
  float Zp = 0.f, Dp = 1.f;
  for (int k = k0; k < k1 || k == k0; k += KB) {     // at least once: the registers hold the first KB segments
    load(k);
#pragma unroll
    for (int j = 0; j < KB; ++j) {
      Zp = d[j] * Zp + z[j];
      Dp *= d[j];
    }
  }
  float Z = 0.f;
#pragma unroll
  for (int j = 0; j < NP; ++j) Z += __shfl(Z0, j * CW + ci, 64);
#pragma unroll
  for (int j = 0; j < NP - 1; ++j) {
    const float dj = __shfl(Dp, j * CW + ci, 64), zj = __shfl(Zp, j * CW + ci, 64);
    if (j < part) Z = dj * Z + zj;
  }
  if (on)
    for (int k = k0; k < k1; k += KB) {
      if (pl > KB) load(k);              // else the registers still hold the part
#pragma unroll
      for (int j = 0; j < KB; ++j)
        if (k + j < k1) {
          zp[(int64_t)(k + j) * zs] = Z;   // the state sum entering segment k + j
          Z = d[j] * Z + z[j];
        }
    }
}

// One wave per (segment, batch, column block), operands straight from global memory into fp32 MFMAs
// (32 tokens x 32 columns):
//   hs_t[n] = (sum_h Ei[h][t] Zin[h][n] + sum_g sum_s WT_g[s][t] B_s[g][n]) / (H P),
// k-steps over pairs of heads, then over pairs of tokens of each group (WT_g[s][t] = 0 for s > t and past the end).
// Loads are unconditional at clamped (valid) addresses, so that a batch of them is in flight together: group 0's
// in-segment operands and the first heads' go out first, the next heads' before the current ones' MFMAs.  No B
// operand is masked: a lane past the last column only feeds an output column that is not stored, and a token
// past the end meets WT_g[s][t] = 0 (u = 0 there); a head past H (odd H) has its Ei operand multiplied by 0.
template <typename T>
__global__ __launch_bounds__(64) void ssd_hs_out_kernel(SsdParams p, HsParams q) {
  const int si = blockIdx.x, b = blockIdx.y, n0 = HS_NB * blockIdx.z, l = lane_id(), i = l & 31, hf = l >> 5;
  const int H = p.nheads, N = p.dstate, G = p.ngroups;
  const int len = min(HS_SEG, p.seqlen - si * HS_SEG);
  const int64_t tok0 = (int64_t)si * HS_SEG;
  const bool col = n0 + i < N;
  const int ic = min(i, N - 1 - n0);                                             // a valid column for every lane
  const float* eit = q.u + ((int64_t)b * p.nseg + si) * H * HS_SEG + i;        // [h][t], this lane's t
  const float* zin = q.z + (((int64_t)b * p.nseg + si) * H) * N + n0 + ic;     // [h][n], this lane's n
  const float* wseg = q.w + ((int64_t)b * p.nseg + si) * G * (HS_SEG * HS_SEG) + i;   // [g][s][t]
  const T* Bb = reinterpret_cast<const T*>(p.B) + (int64_t)b * p.B_sb + n0 + ic;
  constexpr int KU = 16, KS = HS_SEG / 2;
  f32x16 acc = zero16();
  auto mm = [&](const float (&a)[KU], const float (&bq)[KU]) {
#pragma unroll
    for (int j = 0; j < KU; ++j) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[j], bq[j], acc, 0, 0, 0);
  };
  // in-segment operands of group g: step m = tokens (2m, 2m + 1), lane half hf takes token 2m + hf
  auto ldw = [&](int g, float (&a)[KS], float (&bq)[KS]) {
#pragma unroll
    for (int m = 0; m < KS; ++m) {
      const int sk = 2 * m + hf, skc = min(sk, len - 1);
      a[m] = sk <= i ? wseg[((int64_t)g * HS_SEG + sk) * HS_SEG] : 0.f;   // W_g[t][s] = 0 for s > t
      bq[m] = to_f32(Bb[(tok0 + skc) * p.B_sl + (int64_t)g * N]);
    }
  };
  // inter-segment operands: step k = heads (2k, 2k + 1), lane half hf takes head 2k + hf
  auto ldz = [&](int k0, float (&a)[KU], float (&bq)[KU]) {
#pragma unroll
    for (int j = 0; j < KU; ++j) {
      const int h = 2 * (k0 + j) + hf, hc = min(h, H - 1);
      a[j] = eit[(int64_t)hc * HS_SEG] * (h < H ? 1.f : 0.f);     // Ei in [0, 1]
      bq[j] = zin[(int64_t)hc * N];
    }
  };
  const int nz = (H + 1) / 2;
  float aw[KS], bw[KS], a0[KU], b0[KU], a1[KU], b1[KU];
  ldw(0, aw, bw);
  ldz(0, a0, b0);
  for (int k0 = 0; k0 < nz; k0 += 2 * KU) {
    const bool more = k0 + KU < nz, more2 = k0 + 2 * KU < nz;
    if (more) ldz(k0 + KU, a1, b1);
    mm(a0, b0);
    if (more2) ldz(k0 + 2 * KU, a0, b0);
    if (more) mm(a1, b1);
  }
  mm(aw, bw);
  for (int g = 1; g < G; ++g) {
    ldw(g, aw, bw);
    mm(aw, bw);
  }
  if (col) {
    const float scale = 1.f / ((float)H * (float)p.headdim);
    T* out = reinterpret_cast<T*>(q.hs) + ((int64_t)b * p.seqlen + tok0) * N + n0 + i;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int t = acc_row(hf, r);
      if (t < len) out[(int64_t)t * N] = from_f32<T>(acc[r] * scale);
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
//   ssd_hs_local_kernel<T, true> (segment, batch, column block): the forward's local pass (xs, Zloc, segment
//                        decay) and GL[h][n] = sum_t e^{c_t} g_t[n] (c the in-segment inclusive cumsum of A dt),
//                        the segment's part of the adjoint handed to the left, both as fp32 MFMA tiles.
//   ssd_hsb_carry_kernel (batch, head, n): Zin of every segment left to right (in place over Zloc) and Lam of
//                        every segment right to left (in place over GL), then d h0.
//   ssd_hsb_main_kernel  (segment, batch): one head per wave at a time, lanes over the state columns: the two
//                        recurrences inside the segment run directly (Z forward from Zin, lambda backward from
//                        Lam; every factor a <= 1), du and q as lane partials reduced across the wave, dB summed
//                        over the waves in a fixed order, dx, ddt and per-segment dA / d_dt_bias partials.
//   ssd_hsb_reduce_kernel: dA and d_dt_bias summed over (batch, segment) in a fixed order.
constexpr int HSB_MAXH = 128, HSB_MAXN = 128;   // state columns: two per lane
constexpr int HSB_WAVES = 4;

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

// Both carries of the chains (batch, head, column), as two-level scans like the forward's: the forward
// Zin_{k+1} = dec_k Zin_k + Zloc_k from the summed initial state, written over Zloc, and the adjoint handed into
// each segment from the right, Lam_{k-1} = dec_k Lam_k + GL_k from Lam = 0 past the last segment, written over GL;
// finally d h0 = the adjoint left of segment 0 in every row p.  Lane j * CW + i holds part j (NP parts of
// consecutive segments) of the wave's chain i; each part is reduced in both directions from registers, the parts
// before it (forward) and after it (adjoint) are folded across the wave, and the part is walked again.
template <int NP>
__global__ __launch_bounds__(256) void ssd_hsb_carry_kernel(SsdParams p, HsParams q, float* dh0) {
  constexpr int CW = 64 / NP, KB = 16;
  const int H = p.nheads, N = p.dstate, P = p.headdim, ns = p.nseg, l = lane_id();
  const int part = l / CW, ci = l % CW;
  const int64_t chain = ((int64_t)blockIdx.x * 4 + wave_id()) * CW + ci;
  const bool on = chain < (int64_t)p.batch * H * N;
  const int64_t ch = on ? chain : 0;
  const int n = (int)(ch % N), h = (int)((ch / N) % H), b = (int)(ch / ((int64_t)N * H));
  const int pl = (ns + NP - 1) / NP, k0 = min(ns, part * pl), k1 = min(ns, k0 + pl);
  float* zp = q.z + ((int64_t)b * ns * H + h) * N + n;
  float* lp = q.lam + ((int64_t)b * ns * H + h) * N + n;
  const float* dp = q.dec + (int64_t)b * ns * H + h;
  const int64_t zs = (int64_t)H * N;
  float d[KB], z[KB], gl[KB];
  auto load = [&](int k) {
#pragma unroll
    for (int j = 0; j < KB; ++j) {
      const bool in = on && k + j < k1;
      d[j] = in ? dp[(int64_t)(k + j) * H] : 1.f;
      z[j] = in ? zp[(int64_t)(k + j) * zs] : 0.f;
      gl[j] = in ? lp[(int64_t)(k + j) * zs] : 0.f;
    }
  };
  float Z0 = 0.f;
  if (on && p.init_state) {
    const float* s0 = p.init_state + (((int64_t)b * H + h) * P) * N + n;
    for (int k = part; k < P; k += NP) Z0 += s0[(int64_t)k * N];
  }
  // the part's reductions: forward (decay product, sum from zero, in order) and adjoint (sum from zero, right to
  // left: the chunks of KB segments from the last back); a part of one chunk stays in registers throughout
  float Zp = 0.f, Dp = 1.f, Lp = 0.f;
  for (int k = k0; k < k1 || k == k0; k += KB) {
    load(k);
#pragma unroll
    for (int j = 0; j < KB; ++j) {
      Zp = d[j] * Zp + z[j];
      Dp *= d[j];
    }
  }
  const int nck = max(1, (k1 - k0 + KB - 1) / KB);
  for (int c = nck - 1; c >= 0; --c) {
    if (pl > KB) load(k0 + c * KB);
#pragma unroll
    for (int j = KB - 1; j >= 0; --j) Lp = d[j] * Lp + gl[j];
  }
  float Z = 0.f, L = 0.f, Lall = 0.f;
#pragma unroll
  for (int j = 0; j < NP; ++j) Z += __shfl(Z0, j * CW + ci, 64);
#pragma unroll
  for (int j = 0; j < NP - 1; ++j) {
    const float dj = __shfl(Dp, j * CW + ci, 64), zj = __shfl(Zp, j * CW + ci, 64);
    if (j < part) Z = dj * Z + zj;
  }
#pragma unroll
  for (int j = NP - 1; j >= 0; --j) {
    const float dj = __shfl(Dp, j * CW + ci, 64), lj = __shfl(Lp, j * CW + ci, 64);
    if (j > part) L = dj * L + lj;
    Lall = dj * Lall + lj;
  }
  if (on) {
    // forward walk in order, adjoint walk right to left (from registers when the part is one chunk)
    for (int k = k0; k < k1; k += KB) {
      if (pl > KB) load(k);
#pragma unroll
      for (int j = 0; j < KB; ++j)
        if (k + j < k1) {
          zp[(int64_t)(k + j) * zs] = Z;   // the state sum entering segment k + j
          Z = d[j] * Z + z[j];
        }
    }
    for (int c = nck - 1; c >= 0; --c) {
      const int k = k0 + c * KB;
      if (pl > KB) load(k);
#pragma unroll
      for (int j = KB - 1; j >= 0; --j)
        if (k + j < k1) {
          lp[(int64_t)(k + j) * zs] = L;   // the adjoint handed into segment k + j from the right
          L = d[j] * L + gl[j];
        }
    }
    if (dh0) {
      float* o = dh0 + (((int64_t)b * H + h) * P) * N + n;
      for (int k = part; k < P; k += NP) o[(int64_t)k * N] = Lall;
    }
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
      // dx[t][h][p] = dt_t du_t for every p: lane t writes the first half of the row, lane t + 32 the second (or
      // lane t the row's one value into dx_rows)
      if (tv && q.dx_rows) {
        if (l < 32) q.dx_rows[((int64_t)b * p.seqlen + tok0 + t) * H + h] = d * du;
      } else if (tv) {
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

size_t ssd_hs_workspace_bytes(int batch, int seqlen, int nheads, int dstate, int ngroups, bool backward) {
  const size_t nseg = (seqlen + HS_SEG - 1) / HS_SEG;
  const size_t st = align256((size_t)batch * nseg * nheads * dstate * sizeof(float));
  return st + align256((size_t)batch * nseg * nheads * sizeof(float)) +
         align256((size_t)batch * nseg * HS_SEG * nheads * sizeof(float)) +
         (backward ? st + align256((size_t)batch * nseg * nheads * 2 * sizeof(float))
                   : align256((size_t)batch * nseg * ngroups * HS_SEG * HS_SEG * sizeof(float)));
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
  c += align256((size_t)p.batch * p.nseg * HS_SEG * p.nheads * sizeof(float));
  q.lam = backward ? reinterpret_cast<float*>(c) : nullptr;
  q.w = backward ? nullptr : reinterpret_cast<float*>(c);
  c += backward ? st : 0;
  q.part = backward ? reinterpret_cast<float*>(c) : nullptr;
}

hipError_t launch_ssd_hs_bwd(const SsdParams& p, const HsParams& q, float* dh0, hipStream_t st) {
  const dim3 grid((unsigned)p.nseg, (unsigned)p.batch);
  const int64_t nc = (int64_t)p.batch * p.nheads * p.dstate;
  const bool bf = p.dtype == DT_BF16;
  auto carry = [&]() {
    const int np = p.nseg >= 128 ? 8 : p.nseg >= 64 ? 4 : p.nseg >= 32 ? 2 : 1;
    const dim3 cg((unsigned)(((nc * np + 63) / 64 + 3) / 4));
    switch (np) {
      case 8: hipLaunchKernelGGL(ssd_hsb_carry_kernel<8>, cg, dim3(256), 0, st, p, q, dh0); break;
      case 4: hipLaunchKernelGGL(ssd_hsb_carry_kernel<4>, cg, dim3(256), 0, st, p, q, dh0); break;
      case 2: hipLaunchKernelGGL(ssd_hsb_carry_kernel<2>, cg, dim3(256), 0, st, p, q, dh0); break;
      default: hipLaunchKernelGGL(ssd_hsb_carry_kernel<1>, cg, dim3(256), 0, st, p, q, dh0); break;
    }
  };
  if (p.seqlen == 0) {                 // d h0 = 0 (the carry over no segments), dA = d_dt_bias = 0
    carry();
    hipLaunchKernelGGL(ssd_hsb_reduce_kernel, dim3((unsigned)((p.nheads + 3) / 4)), dim3(256), 0, st, p, q);
    return hipGetLastError();
  }
  // the segments' local sums of the state and of the adjoint, both carries, then the gradients
  const dim3 lgrid((unsigned)p.nseg, (unsigned)p.batch, (unsigned)((p.dstate + HS_NB - 1) / HS_NB));
  if (bf) hipLaunchKernelGGL((ssd_hs_local_kernel<bf16, true>), lgrid, dim3(256), 0, st, p, q);
  else hipLaunchKernelGGL((ssd_hs_local_kernel<float, true>), lgrid, dim3(256), 0, st, p, q);
  carry();
  if (bf) hipLaunchKernelGGL(ssd_hsb_main_kernel<bf16>, grid, dim3(64 * HSB_WAVES), 0, st, p, q);
  else hipLaunchKernelGGL(ssd_hsb_main_kernel<float>, grid, dim3(64 * HSB_WAVES), 0, st, p, q);
  hipLaunchKernelGGL(ssd_hsb_reduce_kernel, dim3((unsigned)((p.nheads + 3) / 4)), dim3(256), 0, st, p, q);
  return hipGetLastError();
}

hipError_t launch_ssd_hs(const SsdParams& p, const HsParams& q, hipStream_t st) {
  if (p.seqlen == 0) return hipSuccess;
  const dim3 grid((unsigned)p.nseg, (unsigned)p.batch, (unsigned)((p.dstate + HS_NB - 1) / HS_NB));
  const dim3 lgrid((unsigned)p.nseg, (unsigned)p.batch, (unsigned)HS_FS);
  if (p.dtype == DT_BF16)
    hipLaunchKernelGGL((ssd_hs_local_kernel<bf16, false>), lgrid, dim3(HS_LOC_FWD), 0, st, p, q);
  else
    hipLaunchKernelGGL((ssd_hs_local_kernel<float, false>), lgrid, dim3(HS_LOC_FWD), 0, st, p, q);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  // parts per chain: about 16 segments each, at most 8 (a part's load then covers 8 consecutive columns)
  const int np = p.nseg >= 128 ? 8 : p.nseg >= 64 ? 4 : p.nseg >= 32 ? 2 : 1;
  const int64_t nc = (int64_t)p.batch * p.nheads * p.dstate;
  const int64_t waves = (nc * np + 63) / 64;
  const dim3 cg((unsigned)((waves + 3) / 4));
  switch (np) {
    case 8: hipLaunchKernelGGL(ssd_hs_carry_kernel<8>, cg, dim3(256), 0, st, p, q); break;
    case 4: hipLaunchKernelGGL(ssd_hs_carry_kernel<4>, cg, dim3(256), 0, st, p, q); break;
    case 2: hipLaunchKernelGGL(ssd_hs_carry_kernel<2>, cg, dim3(256), 0, st, p, q); break;
    default: hipLaunchKernelGGL(ssd_hs_carry_kernel<1>, cg, dim3(256), 0, st, p, q); break;
  }
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (p.dtype == DT_BF16)
    hipLaunchKernelGGL(ssd_hs_out_kernel<bf16>, grid, dim3(64), 0, st, p, q);
  else
    hipLaunchKernelGGL(ssd_hs_out_kernel<float>, grid, dim3(64), 0, st, p, q);
  return hipGetLastError();
}

}  // namespace mh
