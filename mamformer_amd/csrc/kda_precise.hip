// KDA chunked scans in fp32 arithmetic (fp32 MFMA, v_mfma_f32_32x32x2f32) for the sizes and types the
// bf16 kernels (kda_scan.hip, kda_backward.hip: bf16 I/O, dk = dv = 128) do not cover: fp32 or bf16 I/O
// with dk, dv in {64, 128}.  Same operators and results as those kernels, to fp32 rounding:
//   gated      S_t = diag(exp(g_t)) S_{t-1} + k_t^T v_t,  o_t = (q1_t - lam q2_t) S_t
//   reference  phi = elu + 1 on the first kernel_dim channels, S_t = S_{t-1} + phi(k_t)^T v_t,
//              z_t = z_{t-1} + phi(k_t),  o_i,t = phi(q_i,t) S_t / (phi(q_i,t) . z_t + 1e-8)
//              (mamformer/layers/kda_diff.py:357-478, mamformer/kernels/triton_ssd.py:121-181, 260-350),
//              and its backward (the gradient autograd forms through kda_diff.py:357-478).
// Every operand lives in LDS as a row-major fp32 matrix (row pitch W + 4 floats) and each product is a
// 32x32 output tile read from LDS along rows or down columns, so one routine serves every contraction.
// The walks use 32-token chunks; the gated operator is factorised per window as in kda_gated_kernel,
//   A[t][s] = sum_k (q_t e^{G_t - m})[k] (k_s e^{m - G_s})[k],  m the midpoint of the window's G range,
// with windows cut so that the range stays within PRANGE (every factor below e^{PRANGE / 2} in fp32).
//
// Backward (reference mode), per 32-token chunk, with dnum_t = coef do_t / n_t, dn_t = -coef do_t . num_t / n_t^2
// (coef = 1, or c and -lam c for the two queries of the differential output, c = 1 / (1 - lam + 1e-8)):
//   dphi(q_t) = sum_{s<=t} G[t][s] phi(k_s) + S_prev dnum_t + dn_t z_prev,   G[t][s] = dnum_t . v_s + dn_t
//   dv_s      = sum_i sum_{t>=s} A_i[t][s] dnum_i,t + phi(k_s) DS,   A_i[t][s] = phi(q_i,t) . phi(k_s)
//   dphi(k_s) = sum_i sum_{t>=s} G_i[t][s] phi(q_i,t) + DS v_s + Dz
//   DS += sum_i phi(q_i)^T dnum_i,  Dz += sum_i phi(q_i)^T dn_i        (walking backwards)
// with dq = dphi(q) phi'(q), phi'(x) = min(phi(x), 1); kda_precise_bwd_q_kernel walks forwards (dq, and
// n_t, dn_t and sum_t do . o_i into the workspace), kda_precise_bwd_kv_kernel backwards (dk, dv, dS0, dz0).
#include "common.h"
#include "launch.h"

namespace mh {

namespace {

constexpr int CT = 32;            // tokens per chunk
constexpr float PRANGE = 80.f;    // max spread of G per channel within a factorisation window

// ---------------------------------------------------------------- fp32 LDS operand fragments
// Row read: the 8 values M[idx][k0 + KSET(half, j)] (contraction along row idx).
template <int P>
__device__ __forceinline__ Frag<float> frow(const float* M, int idx, int k0, int half) {
  const float* p = M + idx * P + k0 + 4 * half;
  const f32x4 lo = *reinterpret_cast<const f32x4*>(p);
  const f32x4 hi = *reinterpret_cast<const f32x4*>(p + 8);
  Frag<float> f;
#pragma unroll
  for (int j = 0; j < 4; ++j) { f.v[j] = lo[j]; f.v[4 + j] = hi[j]; }
  return f;
}
// Column read: the 8 values M[k0 + KSET(half, j)][idx] (contraction down column idx).
template <int P>
__device__ __forceinline__ Frag<float> fcol(const float* M, int idx, int k0, int half) {
  Frag<float> f;
#pragma unroll
  for (int j = 0; j < 8; ++j) f.v[j] = M[(k0 + kset(half, j)) * P + idx];
  return f;
}

// acc[i][j] += sum_{k < K} A(i0 + i, k) * B(k, j0 + j) for one 32x32 tile.  A is stored as M[i][k]
// (AT = false) or M[k][i] (AT = true); B as M[k][j] (BT = false) or M[j][k] (BT = true).  `ascale` scales
// the lane's A row (i0 + l32); `bk`, when given, scales B per k.  Accumulator element r of lane (half, l32)
// is (row i0 + acc_row(half, r), column j0 + l32).
template <bool AT, bool BT, int PA, int PB, int K>
__device__ __forceinline__ f32x16 tile_mma(f32x16 acc, const float* A, int i0, const float* B, int j0, int half,
                                           int l32, float ascale = 1.f, const float* bk = nullptr) {
#pragma unroll 2
  for (int k0 = 0; k0 < K; k0 += 16) {
    Frag<float> a = AT ? fcol<PA>(A, i0 + l32, k0, half) : frow<PA>(A, i0 + l32, k0, half);
    Frag<float> b = BT ? frow<PB>(B, j0 + l32, k0, half) : fcol<PB>(B, j0 + l32, k0, half);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      a.v[j] *= ascale;
      if (bk) b.v[j] *= bk[k0 + kset(half, j)];
    }
    acc = mma(a, b, acc);
  }
  return acc;
}

__device__ __forceinline__ float phi_p(float x) { return x > 0.f ? x + 1.f : __expf(x); }

// 4 consecutive elements of an I/O tensor as fp32.
__device__ __forceinline__ f32x4 ld4(const float* p) { return *reinterpret_cast<const f32x4*>(p); }
__device__ __forceinline__ f32x4 ld4(const bf16* p) {
  const bf16x4 v = *reinterpret_cast<const bf16x4*>(p);
  f32x4 r;
#pragma unroll
  for (int j = 0; j < 4; ++j) r[j] = (float)v[j];
  return r;
}
__device__ __forceinline__ void st1(float* p, float v) { *p = v; }
__device__ __forceinline__ void st1(bf16* p, float v) { *p = (bf16)v; }

// Rows [0, CT) x DW columns of a (rows, row_stride) tensor from row `row0` into LDS (pitch P, fp32), rows
// at or past `len` zero; f is applied to each value with its column index.
template <typename T, int DW, int P, int NTH, typename F>
__device__ __forceinline__ void load_rows(float* dst, const T* src, int64_t row0, int64_t row_stride, int len,
                                          int col0, F f) {
  const int tid = threadIdx.x;
  for (int e = tid; e < CT * DW / 4; e += NTH) {
    const int r = e / (DW / 4), c = 4 * (e % (DW / 4));
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    if (r < len) v = ld4(src + (row0 + r) * row_stride + col0 + c);
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = r < len ? f(v[j], c + j) : 0.f;
    *reinterpret_cast<f32x4*>(dst + r * P + c) = v;
  }
}

// ---------------------------------------------------------------- forward
constexpr int FW = 4;             // waves per forward workgroup

template <int DK, int VB, int NQ, bool GATED>
struct PFwdSmem {
  static constexpr int PK = DK + 4, PV = VB + 4, PC = CT + 4;
  float Q[NQ][CT * PK];                  // operand q (gated: q_e e^{G - m}; reference: phi(q_i))
  float K[CT * PK];                      // operand k (gated: k e^{m - G}; reference: phi(k))
  float Qr[GATED ? CT * PK : 1];         // gated: raw q_e = q1 - lam q2
  float Kr[GATED ? CT * PK : 1];         // gated: raw k
  float G[GATED ? CT * DK : 1];          // gated: raw g, then its in-chunk inclusive cumsum
  float V[CT * PV];                      // v[:, v0 .. v0 + VB)
  float A[NQ][CT * PC];                  // masked A[t][s]
  float S[DK * PV];                      // state S[k][v0 + v]
  float O[NQ][CT * PV];                  // output rows (normalised in reference mode)
  float z[DK];                           // reference: running sum of phi(k)
  float nrm[NQ][CT];                     // reference: n_t
  float mm[DK], em[DK], ek[DK], eg[DK];  // gated window factors: m, e^{m - base}, e^{end - m}, e^{end - base}
  int wend, cut;
};

template <typename T, int DK, int DV, int NQ, bool GATED>
__global__ __launch_bounds__(64 * FW) void kda_precise_fwd_kernel(KdaParams p) {
  constexpr int VB = DV < 64 ? DV : 64;
  using SM = PFwdSmem<DK, VB, NQ, GATED>;
  constexpr int PK = SM::PK, PV = SM::PV, PC = SM::PC;
  __shared__ SM sm;
  const int nvb = DV / VB;
  const int bh = blockIdx.x / nvb, v0 = (blockIdx.x % nvb) * VB;
  const int h = bh % p.nheads;
  const int w = wave_id(), l = lane_id(), half = l >> 5, l32 = l & 31;
  const int tid = threadIdx.x;
  const int S = p.seqlen, kd = GATED ? DK : p.kernel_dim;
  const float lam = p.lam_h ? p.lam_h[h] : p.lam;
  const int64_t rowbase = (int64_t)bh * S;
  const T* q1 = reinterpret_cast<const T*>(p.q1);
  const T* q2 = reinterpret_cast<const T*>(p.q2);
  const T* kk = reinterpret_cast<const T*>(p.k);
  const T* vv = reinterpret_cast<const T*>(p.v);
  const bool fuse_diff = !GATED && NQ == 2 && p.o2 == nullptr;

  for (int e = tid; e < DK * VB; e += 64 * FW) {
    const int k = e / VB, c = e % VB;
    sm.S[k * PV + c] = p.init_state ? p.init_state[((int64_t)bh * DK + k) * DV + v0 + c] : 0.f;
  }
  if (!GATED && tid < DK) sm.z[tid] = p.init_z ? p.init_z[(int64_t)bh * DK + tid] : 0.f;
  if (tid < DK) sm.mm[tid] = 0.f, sm.em[tid] = sm.ek[tid] = sm.eg[tid] = 1.f;
  __syncthreads();

  for (int pos = 0; pos < S; pos += CT) {
    const int len = min(CT, S - pos);
    // ---- rows of the chunk
    if constexpr (GATED) {
      const bool has_q2 = q2 != nullptr;
      load_rows<T, DK, PK, 64 * FW>(sm.Qr, q1, rowbase + pos, DK, len, 0, [](float x, int) { return x; });
      load_rows<T, DK, PK, 64 * FW>(sm.Kr, kk, rowbase + pos, DK, len, 0, [](float x, int) { return x; });
      if (p.g) load_rows<float, DK, DK, 64 * FW>(sm.G, p.g, rowbase + pos, DK, len, 0, [](float x, int) { return x; });
      else for (int e = tid; e < CT * DK; e += 64 * FW) sm.G[e] = 0.f;
      __syncthreads();
      if (has_q2) {                      // q_e = q1 - lam q2 (the rows of q2 added in place)
        for (int e = tid; e < CT * DK / 4; e += 64 * FW) {
          const int r = e / (DK / 4), c = 4 * (e % (DK / 4));
          if (r < len) {
            const f32x4 b = ld4(q2 + (rowbase + pos + r) * DK + c);
#pragma unroll
            for (int j = 0; j < 4; ++j) sm.Qr[r * PK + c + j] -= lam * b[j];
          }
        }
      }
      // in-chunk inclusive cumsum of g per channel (g = 0 past the end keeps G flat)
      if (tid < DK) {
        float run = 0.f, gmin = INFINITY, gmax = -INFINITY;
        for (int t = 0; t < CT; ++t) {
          run += t < len ? sm.G[t * DK + tid] : 0.f;
          sm.G[t * DK + tid] = run;
          if (t < len) { gmin = fminf(gmin, run); gmax = fmaxf(gmax, run); }
        }
        if (tid == 0) sm.cut = 0;
        const float m = 0.5f * (gmin + gmax);
        sm.mm[tid] = m;
        sm.em[tid] = __expf(m);
        sm.ek[tid] = __expf(run - m);
        sm.eg[tid] = __expf(run);
      }
      __syncthreads();
      if (tid < DK) {
        float gmin = INFINITY, gmax = -INFINITY;
        for (int t = 0; t < len; ++t) { gmin = fminf(gmin, sm.G[t * DK + tid]); gmax = fmaxf(gmax, sm.G[t * DK + tid]); }
        if (gmax - gmin > PRANGE) sm.cut = 1;            // benign race: every writer stores 1
      }
    } else {
      const auto phik = [kd](float x, int c) { return c < kd ? phi_p(x) : 0.f; };
      load_rows<T, DK, PK, 64 * FW>(sm.Q[0], q1, rowbase + pos, DK, len, 0, phik);
      if (NQ == 2) load_rows<T, DK, PK, 64 * FW>(sm.Q[NQ - 1], q2, rowbase + pos, DK, len, 0, phik);
      load_rows<T, DK, PK, 64 * FW>(sm.K, kk, rowbase + pos, DK, len, 0, phik);
    }
    load_rows<T, VB, PV, 64 * FW>(sm.V, vv, rowbase + pos, DV, len, v0, [](float x, int) { return x; });
    __syncthreads();

    // ---- factorisation windows [a, b) (the whole chunk in reference mode)
    for (int a = 0; a < len;) {
      int b = len;
      if constexpr (GATED) {
        if (sm.cut) {
          if (tid == 0) sm.wend = len;
          __syncthreads();
          if (tid < DK) {
            float mn = INFINITY, mx = -INFINITY;
            int bad = len;
            for (int t = a; t < len; ++t) {
              const float gv = sm.G[t * DK + tid];
              mn = fminf(mn, gv);
              mx = fmaxf(mx, gv);
              if (mx - mn > PRANGE) { bad = t; break; }
            }
            atomicMin(&sm.wend, bad);
          }
          __syncthreads();
          b = max(sm.wend, a + 1);
          if (tid < DK) {
            float mn = INFINITY, mx = -INFINITY;
            for (int t = a; t < b; ++t) { mn = fminf(mn, sm.G[t * DK + tid]); mx = fmaxf(mx, sm.G[t * DK + tid]); }
            const float base = a ? sm.G[(a - 1) * DK + tid] : 0.f, end = sm.G[(b - 1) * DK + tid];
            const float m = 0.5f * (mn + mx);
            sm.mm[tid] = m;
            sm.em[tid] = __expf(m - base);
            sm.ek[tid] = __expf(end - m);
            sm.eg[tid] = __expf(end - base);
          }
          __syncthreads();
        }
        // operands on rows [a, b), zero elsewhere
        for (int e = tid; e < CT * DK; e += 64 * FW) {
          const int r = e / DK, c = e % DK;
          const bool in = r >= a && r < b;
          const float d = sm.G[r * DK + c] - sm.mm[c];
          sm.Q[0][r * PK + c] = in ? sm.Qr[r * PK + c] * __expf(d) : 0.f;
          sm.K[r * PK + c] = in ? sm.Kr[r * PK + c] * __expf(-d) : 0.f;
        }
        __syncthreads();
      }

      // ---- masked A[t][s] = Q_t . K_s (s <= t) per query; reference mode: n_t = rowsum + phi(q_t) . z + 1e-8
      if (w < NQ) {
        f32x16 acc = tile_mma<false, true, PK, PK, DK>(zero16(), sm.Q[w], 0, sm.K, 0, half, l32);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int t = acc_row(half, r);
          sm.A[w][t * PC + l32] = l32 <= t ? acc[r] : 0.f;
        }
      }
      __syncthreads();
      if constexpr (!GATED) {
        if (tid < NQ * CT) {
          const int qi = tid / CT, t = tid % CT;
          float n = 0.f;
          for (int s = 0; s < CT; ++s) n += sm.A[qi][t * PC + s];
          float qz = 0.f;
          for (int k = 0; k < DK; ++k) qz += sm.Q[qi][t * PK + k] * sm.z[k];
          sm.nrm[qi][t] = n + qz + 1e-8f;
        }
        __syncthreads();
      }

      // ---- output tiles (query, v-tile): sum_s A[t][s] v_s + sum_k Q_t[k] (S[k][v] e^{m - base})
      for (int ti = w; ti < NQ * (VB / 32); ti += FW) {
        const int qi = ti / (VB / 32), vt = ti % (VB / 32);
        f32x16 acc = tile_mma<false, false, PC, PV, CT>(zero16(), sm.A[qi], 0, sm.V, 32 * vt, half, l32);
        acc = tile_mma<false, false, PK, PV, DK>(acc, sm.Q[qi], 0, sm.S, 32 * vt, half, l32, 1.f,
                                                 GATED ? sm.em : nullptr);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int t = acc_row(half, r);
          sm.O[qi][t * PV + 32 * vt + l32] = GATED ? acc[r] : acc[r] / sm.nrm[qi][t];
        }
      }
      __syncthreads();

      // ---- state update: S[k][v] <- e^{end - base} S[k][v] + sum_s (K_s e^{end - m})[k] v_s[v]; z += sum_s phi(k_s)
      for (int ti = w; ti < (DK / 32) * (VB / 32); ti += FW) {
        const int kt = ti / (VB / 32), vt = ti % (VB / 32);
        f32x16 acc;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int k = 32 * kt + acc_row(half, r);
          acc[r] = sm.S[k * PV + 32 * vt + l32] * (GATED ? sm.eg[k] : 1.f);
        }
        acc = tile_mma<true, false, PK, PV, CT>(acc, sm.K, 32 * kt, sm.V, 32 * vt, half, l32,
                                                GATED ? sm.ek[32 * kt + l32] : 1.f);
#pragma unroll
        for (int r = 0; r < 16; ++r) sm.S[(32 * kt + acc_row(half, r)) * PV + 32 * vt + l32] = acc[r];
      }
      if (!GATED && tid < DK) {
        float zs = 0.f;
        for (int s = 0; s < CT; ++s) zs += sm.K[s * PK + tid];
        sm.z[tid] += zs;
      }

      // ---- outputs of rows [a, b)
      {
        T* o1 = reinterpret_cast<T*>(p.o);
        T* o2 = reinterpret_cast<T*>(p.o2);
        const float inv_1ml = 1.f / (1.f - lam + 1e-8f);
        for (int e = tid; e < CT * VB; e += 64 * FW) {
          const int t = e / VB, c = e % VB;
          if (t < a || t >= b) continue;
          const int64_t off = (rowbase + pos + t) * DV + v0 + c;
          if (fuse_diff) {
            st1(o1 + off, (sm.O[0][t * PV + c] - lam * sm.O[NQ - 1][t * PV + c]) * inv_1ml);
          } else {
            st1(o1 + off, sm.O[0][t * PV + c]);
            if (NQ == 2 && o2) st1(o2 + off, sm.O[NQ - 1][t * PV + c]);
          }
        }
      }
      __syncthreads();
      a = b;
    }
  }

  if (p.final_state)
    for (int e = tid; e < DK * VB; e += 64 * FW) {
      const int k = e / VB, c = e % VB;
      p.final_state[((int64_t)bh * DK + k) * DV + v0 + c] = sm.S[k * PV + c];
    }
  if (!GATED && p.final_z && v0 == 0 && tid < DK) p.final_z[(int64_t)bh * DK + tid] = sm.z[tid];
}

// ---------------------------------------------------------------- backward (reference mode)
constexpr int BW = 8;             // waves per backward workgroup

template <int DK, int DV>
struct PBwdSmem {
  static constexpr int PK = DK + 4, PV = DV + 4, PC = CT + 4;
  float M[DK * PV];                // q-walk: S before the chunk;  kv-walk: the adjoint DS
  float Q[CT * PK];                // phi(q_i)
  float K[CT * PK];                // phi(k)
  float V[CT * PV];
  float D[CT * PV];                // raw output gradient, then dnum
  float A[CT * PC];                // q-walk: A[t][s] (s <= t);   kv-walk: A_i[t][s] (t >= s)
  float G[CT * PC];                // q-walk: G^T[s][t] (s <= t); kv-walk: G_i[t][s] (t >= s)
  float z[DK];                     // q-walk: z before the chunk;  kv-walk: Dz
  float n[CT], dn[CT], dot[CT];
  float dotp[DV / 32][CT];
  float lam[BW];
  float dov[CT];                   // q-walk: do_t . Vsum_t (Vsum_t = sum of v over the tokens up to t)
  float vsum[DV];                  // q-walk: sum of v over the chunks before this one
};

// Output-gradient pointer and coefficient of query stream qi (see KdaBwdParams).
__device__ __forceinline__ float stream_coef(const KdaBwdParams& q, int h, int qi) {
  if (!q.diff) return 1.f;
  const float lam = q.f.lam_h ? q.f.lam_h[h] : q.f.lam;
  const float c = 1.f / (1.f - lam + 1e-8f);
  return qi == 0 ? c : -lam * c;
}

template <typename T, int DK, int DV>
__global__ __launch_bounds__(64 * BW) void kda_precise_bwd_q_kernel(KdaBwdParams q) {
  using SM = PBwdSmem<DK, DV>;
  constexpr int PK = SM::PK, PV = SM::PV, PC = SM::PC;
  __shared__ SM sm;
  const KdaParams& p = q.f;
  const int nbh = p.batch * p.nheads;
  const int bh = blockIdx.x, qi = blockIdx.y;
  const int h = bh % p.nheads;
  const int w = wave_id(), l = lane_id(), half = l >> 5, l32 = l & 31;
  const int tid = threadIdx.x;
  const int S = p.seqlen, kd = p.kernel_dim;
  const int64_t rowbase = (int64_t)bh * S;
  const T* qp = reinterpret_cast<const T*>(qi == 0 ? p.q1 : p.q2);
  const T* kp = reinterpret_cast<const T*>(p.k);
  const T* vp = reinterpret_cast<const T*>(p.v);
  const T* dop = reinterpret_cast<const T*>(q.diff ? q.do1 : (qi == 0 ? q.do1 : q.do2));   // null: zero
  T* dqp = reinterpret_cast<T*>(qi == 0 ? q.dq1 : q.dq2);
  float* nbuf = q.nbuf + ((int64_t)qi * nbh + bh) * S;
  float* dnbuf = q.dnbuf + ((int64_t)qi * nbh + bh) * S;
  const float coef = stream_coef(q, h, qi);
  const auto phik = [kd](float x, int c) { return c < kd ? phi_p(x) : 0.f; };
  const auto same = [](float x, int) { return x; };

  for (int e = tid; e < DK * DV; e += 64 * BW)
    sm.M[(e / DV) * PV + e % DV] = p.init_state ? p.init_state[(int64_t)bh * DK * DV + e] : 0.f;
  if (tid < DK) sm.z[tid] = p.init_z ? p.init_z[(int64_t)bh * DK + tid] : 0.f;
  // lambda gradient pieces (threads t < CT): sum_t do_t . (o_t - Vsum_t / cnt_t) and, once, sum_t do_t . Vsum_t /
  // cnt_t.  In reference mode o1 ~ o2 ~ Vsum / cnt (phi ~ 1), so the two queries' centred sums keep the digits
  // that d lambda (their difference) needs.
  float lam_acc = 0.f, base_acc = 0.f;
  if (tid < DV) sm.vsum[tid] = 0.f;
  __syncthreads();

  for (int pos = 0; pos < S; pos += CT) {
    const int len = min(CT, S - pos);
    load_rows<T, DK, PK, 64 * BW>(sm.Q, qp, rowbase + pos, DK, len, 0, phik);
    load_rows<T, DK, PK, 64 * BW>(sm.K, kp, rowbase + pos, DK, len, 0, phik);
    load_rows<T, DV, PV, 64 * BW>(sm.V, vp, rowbase + pos, DV, len, 0, same);
    if (dop) load_rows<T, DV, PV, 64 * BW>(sm.D, dop, rowbase + pos, DV, len, 0, same);
    else for (int e = tid; e < CT * PV; e += 64 * BW) sm.D[e] = 0.f;
    __syncthreads();
    // A[t][s] (s <= t); n_t = rowsum + phi(q_t) . z + 1e-8
    if (w == 0) {
      const f32x16 acc = tile_mma<false, true, PK, PK, DK>(zero16(), sm.Q, 0, sm.K, 0, half, l32);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int t = acc_row(half, r);
        sm.A[t * PC + l32] = l32 <= t ? acc[r] : 0.f;
      }
    }
    __syncthreads();
    if (tid < CT) {
      float n = 0.f, qz = 0.f;
      for (int s = 0; s < CT; ++s) n += sm.A[tid * PC + s];
      for (int k = 0; k < DK; ++k) qz += sm.Q[tid * PK + k] * sm.z[k];
      sm.n[tid] = n + qz + 1e-8f;
    }
    __syncthreads();
    // num tiles (rows t, v-tile): sum_s A[t][s] v_s + phi(q_t) S; per row the partial of do_t . num_t.
    // Wave DV / 32: do_t . Vsum_t = do_t . vsum + sum_{s <= t} v_s . do_t (masked column sums of V do^T).
    if (w == DV / 32) {
      const f32x16 acc = tile_mma<false, true, PV, PV, DV>(zero16(), sm.V, 0, sm.D, 0, half, l32);
      float d = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) d += acc_row(half, r) <= l32 ? acc[r] : 0.f;
      for (int c = half * (DV / 2); c < (half + 1) * (DV / 2); ++c) d += sm.D[l32 * PV + c] * sm.vsum[c];
      d += __shfl_xor(d, 32, 64);
      if (half == 0) sm.dov[l32] = d;
    }
    if (w < DV / 32) {
      f32x16 acc = tile_mma<false, false, PC, PV, CT>(zero16(), sm.A, 0, sm.V, 32 * w, half, l32);
      acc = tile_mma<false, false, PK, PV, DK>(acc, sm.Q, 0, sm.M, 32 * w, half, l32);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float d = acc[r] * sm.D[acc_row(half, r) * PV + 32 * w + l32];
#pragma unroll
        for (int o = 16; o >= 1; o >>= 1) d += __shfl_xor(d, o, 64);
        if (l32 == 0) sm.dotp[w][acc_row(half, r)] = d;
      }
    }
    __syncthreads();
    if (tid < CT) {
      float d = 0.f;
      for (int i = 0; i < DV / 32; ++i) d += sm.dotp[i][tid];
      const float n = sm.n[tid];
      sm.dn[tid] = tid < len ? -coef * d / (n * n) : 0.f;
      if (tid < len) {
        const float base = sm.dov[tid] / (float)(pos + tid + 1);
        lam_acc += d / n - base;
        base_acc += base;
        nbuf[pos + tid] = n;
        dnbuf[pos + tid] = -coef * d / (n * n);
      }
    }
    for (int e = tid; e < CT * DV; e += 64 * BW) {          // dnum = coef do / n
      const int t = e / DV, c = e % DV;
      sm.D[t * PV + c] *= coef / sm.n[t];
    }
    __syncthreads();
    // G^T[s][t] = v_s . dnum_t + dn_t (s <= t)
    if (w == 0) {
      const f32x16 acc = tile_mma<false, true, PV, PV, DV>(zero16(), sm.V, 0, sm.D, 0, half, l32);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int s = acc_row(half, r);
        sm.G[s * PC + l32] = s <= l32 ? acc[r] + sm.dn[l32] : 0.f;
      }
    }
    __syncthreads();
    // dq tiles (rows t, k-tile): sum_s G^T[s][t] phi(k_s) + S dnum_t + dn_t z, times phi'(q)
    if (w < DK / 32) {
      f32x16 acc = tile_mma<true, false, PC, PK, CT>(zero16(), sm.G, 0, sm.K, 32 * w, half, l32);
      acc = tile_mma<false, true, PV, PV, DV>(acc, sm.D, 0, sm.M, 32 * w, half, l32);
      const int k = 32 * w + l32;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int t = acc_row(half, r);
        if (t < len) {
          const float dphi = acc[r] + sm.dn[t] * sm.z[k];
          st1(dqp + (rowbase + pos + t) * DK + k, dphi * fminf(sm.Q[t * PK + k], 1.f));
        }
      }
    }
    __syncthreads();
    // S += phi(k)^T v,  z += sum_s phi(k_s)
    for (int ti = w; ti < (DK / 32) * (DV / 32); ti += BW) {
      const int kt = ti / (DV / 32), vt = ti % (DV / 32);
      f32x16 acc;
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] = sm.M[(32 * kt + acc_row(half, r)) * PV + 32 * vt + l32];
      acc = tile_mma<true, false, PK, PV, CT>(acc, sm.K, 32 * kt, sm.V, 32 * vt, half, l32);
#pragma unroll
      for (int r = 0; r < 16; ++r) sm.M[(32 * kt + acc_row(half, r)) * PV + 32 * vt + l32] = acc[r];
    }
    if (tid < DK) {
      float zs = 0.f;
      for (int s = 0; s < CT; ++s) zs += sm.K[s * PK + tid];
      sm.z[tid] += zs;
    }
    if (tid < DV) {                                        // rows past len are zero
      float vs = 0.f;
      for (int s = 0; s < CT; ++s) vs += sm.V[s * PV + tid];
      sm.vsum[tid] += vs;
    }
    __syncthreads();
  }
  // P_i = sum do . (o_i - Vsum / cnt) in slot qi and, from the first query, B = sum do . Vsum / cnt in slot nq
  if (tid < 64) {
    const float v = wave_sum(tid < CT ? lam_acc : 0.f);
    const float b = wave_sum(tid < CT ? base_acc : 0.f);
    if (tid == 0) {
      q.lam_part[(int64_t)qi * nbh + bh] = v;
      if (qi == 0) q.lam_part[(int64_t)q.nq * nbh + bh] = b;
    }
  }
}

template <typename T, int DK, int DV>
__global__ __launch_bounds__(64 * BW) void kda_precise_bwd_kv_kernel(KdaBwdParams q) {
  using SM = PBwdSmem<DK, DV>;
  constexpr int PK = SM::PK, PV = SM::PV, PC = SM::PC;
  constexpr int NDV = DV / 32, NDK = DK / 32;
  __shared__ SM sm;
  const KdaParams& p = q.f;
  const int nbh = p.batch * p.nheads;
  const int bh = blockIdx.x;
  const int h = bh % p.nheads;
  const int w = wave_id(), l = lane_id(), half = l >> 5, l32 = l & 31;
  const int tid = threadIdx.x;
  const int S = p.seqlen, kd = p.kernel_dim;
  const int64_t rowbase = (int64_t)bh * S;
  const T* kp = reinterpret_cast<const T*>(p.k);
  const T* vp = reinterpret_cast<const T*>(p.v);
  T* dkp = reinterpret_cast<T*>(q.dk);
  T* dvp = reinterpret_cast<T*>(q.dv);
  const auto phik = [kd](float x, int c) { return c < kd ? phi_p(x) : 0.f; };
  const auto same = [](float x, int) { return x; };

  for (int e = tid; e < DK * DV; e += 64 * BW)
    sm.M[(e / DV) * PV + e % DV] = q.d_final ? q.d_final[(int64_t)bh * DK * DV + e] : 0.f;
  if (tid < DK) sm.z[tid] = q.d_final_z ? q.d_final_z[(int64_t)bh * DK + tid] : 0.f;
  __syncthreads();

  const int nch = (S + CT - 1) / CT;
  for (int c = nch - 1; c >= 0; --c) {
    const int pos = c * CT, len = min(CT, S - pos);
    load_rows<T, DK, PK, 64 * BW>(sm.K, kp, rowbase + pos, DK, len, 0, phik);
    load_rows<T, DV, PV, 64 * BW>(sm.V, vp, rowbase + pos, DV, len, 0, same);
    __syncthreads();
    // the state terms, with DS and Dz of the later chunks: dv_s = phi(k_s) DS, dphi(k_s) = DS v_s + Dz
    f32x16 acc = zero16();
    if (w < NDV) {
      acc = tile_mma<false, false, PK, PV, DK>(acc, sm.K, 0, sm.M, 32 * w, half, l32);
    } else if (w < NDV + NDK) {
      const int kt = w - NDV;
      acc = tile_mma<false, true, PV, PV, DV>(acc, sm.V, 0, sm.M, 32 * kt, half, l32);
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] += sm.z[32 * kt + l32];
    }
    for (int qi = 0; qi < q.nq; ++qi) {
      const T* qp = reinterpret_cast<const T*>(qi == 0 ? p.q1 : p.q2);
      const T* dop = reinterpret_cast<const T*>(q.diff ? q.do1 : (qi == 0 ? q.do1 : q.do2));
      const float coef = stream_coef(q, h, qi);
      const float* nb = q.nbuf + ((int64_t)qi * nbh + bh) * S + pos;
      const float* dnb = q.dnbuf + ((int64_t)qi * nbh + bh) * S + pos;
      __syncthreads();                                     // the previous stream's Q, D, A, G are consumed
      load_rows<T, DK, PK, 64 * BW>(sm.Q, qp, rowbase + pos, DK, len, 0, phik);
      if (dop) load_rows<T, DV, PV, 64 * BW>(sm.D, dop, rowbase + pos, DV, len, 0, same);
      else for (int e = tid; e < CT * PV; e += 64 * BW) sm.D[e] = 0.f;
      if (tid < CT) {
        sm.n[tid] = tid < len ? nb[tid] : 1.f;
        sm.dn[tid] = tid < len ? dnb[tid] : 0.f;
      }
      __syncthreads();
      for (int e = tid; e < CT * DV; e += 64 * BW) {      // dnum = coef do / n
        const int t = e / DV, cc = e % DV;
        sm.D[t * PV + cc] *= coef / sm.n[t];
      }
      __syncthreads();
      // A_i[t][s] = phi(q_t) . phi(k_s) and G_i[t][s] = dnum_t . v_s + dn_t, both for t >= s
      if (w == 0) {
        const f32x16 a = tile_mma<false, true, PK, PK, DK>(zero16(), sm.Q, 0, sm.K, 0, half, l32);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int t = acc_row(half, r);
          sm.A[t * PC + l32] = t >= l32 ? a[r] : 0.f;
        }
      } else if (w == 1) {
        const f32x16 g = tile_mma<false, true, PV, PV, DV>(zero16(), sm.D, 0, sm.V, 0, half, l32);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int t = acc_row(half, r);
          sm.G[t * PC + l32] = t >= l32 ? g[r] + sm.dn[t] : 0.f;
        }
      }
      __syncthreads();
      // dv_s += sum_t A_i[t][s] dnum_t;  dphi(k_s) += sum_t G_i[t][s] phi(q_t)
      if (w < NDV) {
        acc = tile_mma<true, false, PC, PV, CT>(acc, sm.A, 0, sm.D, 32 * w, half, l32);
      } else if (w < NDV + NDK) {
        acc = tile_mma<true, false, PC, PK, CT>(acc, sm.G, 0, sm.Q, 32 * (w - NDV), half, l32);
      }
      // DS += phi(q_i)^T dnum_i (every read of DS this chunk came before the stream loop), Dz += phi(q_i)^T dn_i
      for (int ti = w; ti < NDK * NDV; ti += BW) {
        const int kt = ti / NDV, vt = ti % NDV;
        f32x16 s;
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] = sm.M[(32 * kt + acc_row(half, r)) * PV + 32 * vt + l32];
        s = tile_mma<true, false, PK, PV, CT>(s, sm.Q, 32 * kt, sm.D, 32 * vt, half, l32);
#pragma unroll
        for (int r = 0; r < 16; ++r) sm.M[(32 * kt + acc_row(half, r)) * PV + 32 * vt + l32] = s[r];
      }
      if (tid < DK) {
        float zs = 0.f;
        for (int t = 0; t < CT; ++t) zs += sm.Q[t * PK + tid] * sm.dn[t];
        sm.z[tid] += zs;
      }
    }
    // dv and dk rows of the chunk
    if (w < NDV) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int s = acc_row(half, r);
        if (s < len) st1(dvp + (rowbase + pos + s) * DV + 32 * w + l32, acc[r]);
      }
    } else if (w < NDV + NDK) {
      const int k = 32 * (w - NDV) + l32;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int s = acc_row(half, r);
        if (s < len) st1(dkp + (rowbase + pos + s) * DK + k, acc[r] * fminf(sm.K[s * PK + k], 1.f));
      }
    }
    __syncthreads();
  }
  if (q.dS0)
    for (int e = tid; e < DK * DV; e += 64 * BW) q.dS0[(int64_t)bh * DK * DV + e] = sm.M[(e / DV) * PV + e % DV];
  if (q.dz0 && tid < DK) q.dz0[(int64_t)bh * DK + tid] = sm.z[tid];
}

template <typename T, int DK, int DV>
hipError_t launch_fwd_t(const KdaParams& p, hipStream_t st) {
  constexpr int VB = DV < 64 ? DV : 64;
  const dim3 grid((unsigned)(p.batch * p.nheads * (DV / VB)));
  if (p.mode == 0)
    hipLaunchKernelGGL((kda_precise_fwd_kernel<T, DK, DV, 1, true>), grid, dim3(64 * FW), 0, st, p);
  else if (p.q2)
    hipLaunchKernelGGL((kda_precise_fwd_kernel<T, DK, DV, 2, false>), grid, dim3(64 * FW), 0, st, p);
  else
    hipLaunchKernelGGL((kda_precise_fwd_kernel<T, DK, DV, 1, false>), grid, dim3(64 * FW), 0, st, p);
  return hipGetLastError();
}

template <typename T, int DK, int DV>
hipError_t launch_bwd_t(const KdaBwdParams& q, hipStream_t st) {
  const unsigned nbh = (unsigned)(q.f.batch * q.f.nheads);
  hipLaunchKernelGGL((kda_precise_bwd_q_kernel<T, DK, DV>), dim3(nbh, (unsigned)q.nq), dim3(64 * BW), 0, st, q);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((kda_precise_bwd_kv_kernel<T, DK, DV>), dim3(nbh), dim3(64 * BW), 0, st, q);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_fwd_dt(const KdaParams& p, hipStream_t st) {
  if (p.dk == 128 && p.dv == 128) return launch_fwd_t<T, 128, 128>(p, st);
  if (p.dk == 128 && p.dv == 64) return launch_fwd_t<T, 128, 64>(p, st);
  if (p.dk == 64 && p.dv == 128) return launch_fwd_t<T, 64, 128>(p, st);
  if (p.dk == 64 && p.dv == 64) return launch_fwd_t<T, 64, 64>(p, st);
  return hipErrorInvalidValue;
}

template <typename T>
hipError_t launch_bwd_dt(const KdaBwdParams& q, hipStream_t st) {
  const KdaParams& p = q.f;
  if (p.dk == 128 && p.dv == 128) return launch_bwd_t<T, 128, 128>(q, st);
  if (p.dk == 128 && p.dv == 64) return launch_bwd_t<T, 128, 64>(q, st);
  if (p.dk == 64 && p.dv == 128) return launch_bwd_t<T, 64, 128>(q, st);
  if (p.dk == 64 && p.dv == 64) return launch_bwd_t<T, 64, 64>(q, st);
  return hipErrorInvalidValue;
}

}  // namespace

bool kda_precise_path(const KdaParams& p) { return !(p.dtype == DT_BF16 && p.dk == 128 && p.dv == 128); }

hipError_t launch_kda_precise(const KdaParams& p, hipStream_t st) {
  return p.dtype == DT_F32 ? launch_fwd_dt<float>(p, st) : launch_fwd_dt<bf16>(p, st);
}

hipError_t launch_kda_bwd_precise(const KdaBwdParams& q, hipStream_t st) {
  return q.f.dtype == DT_F32 ? launch_bwd_dt<float>(q, st) : launch_bwd_dt<bf16>(q, st);
}

}  // namespace mh
