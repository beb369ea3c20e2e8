// Backward of the Mamba-2 SSD chunked-scan prefill for gfx950: gradients of
//     L = <dy, y> + <d_final, h_L>,   y, h_L = scan(x, dt, A, B, C, D, h0)
// with respect to x, the raw dt (through bias / softplus / clamp), A, B, C, D, dt_bias and h0 -- what
// PyTorch autograd computes through the reference's selective_scan (mamformer/layers/mamba2.py:70-130,
// trained through in tests/test_mamba2.py:56-71), in the per-head SSD parameterisation.
//
// Per head, with a_t = exp(A dt_t), the adjoint of the state h_t is
//     lam_t = a_{t+1} lam_{t+1} + dy_t C_t^T,        lam_{L-1} = dy_{L-1} C_{L-1}^T + d_final
// and, per 64-token segment with in-segment inclusive log-decay c_t (c_t <= 0, non-increasing), entering
// state h_in and lam_out the adjoint of the state leaving the segment (the next segment's entering adjoint):
//     dx_s  = dt_s [ sum_{t>=s} M[t][s] dy_t + e^{c_end - c_s} lam_out B_s ] + D dy_s
//     dB_s  = sum_h dt_s [ sum_{t>=s} C_t L[t][s] XD[t][s] + e^{c_end - c_s} lam_out^T x_s ]
//     dC_t  = sum_h [ sum_{s<=t} B_s L[t][s] XD[t][s] dt_s + e^{c_t} h_in^T dy_t ]
// where L[t][s] = e^{c_t - c_s} (s <= t), CB[t][s] = C_t.B_s, M = L o CB, XD[t][s] = dy_t.x_s.
// The decay gradient per token comes from per-token sums: with
//     colG_s = sum_t (M o XD)[t][s],             bint_s = B_s . (dB_s inter part / dt_s),
//     rowG_t = sum_s (M o XD)[t][s] dt_s,        u_t = C_t . (dC_t inter part),
// dL/dc_t = rowG_t - dt_t colG_t + u_t inside the segment, and the state terms give
//     da_tau = sum_{t>=tau} dL/dc_t + e^{c_end} <lam_out, h_in> + sum_{s<tau} dt_s bint_s
//     ddt_tau = colG_tau + bint_tau + A da_tau,    dA = sum_tau dt_tau da_tau,    dD = sum dy . x.
//
// Launches (caller's stream):
//   0. ssd_bwd_zero      clears dA, dD, d_dt_bias (a kernel, not a memset node).
//   1. ssd_bwd_sweep     grid (2 directions, H, b): the forward direction walks the segments
//      first to last and stores the entering state h_in of every 64-token segment; the adjoint direction walks
//      them last to first, stores lam_out of every segment and finally dh0
//      (lam <- e^{c_end} lam + sum_t e^{c_t} C_t^T dy_t).  Both into the workspace, fragment-native order.
//   2. ssd_bwd_grad      grid (nseg, H / HB, b): one workgroup per (segment, block of HB heads of a group),
//      fully parallel; dx and ddt stored directly, dB / dC summed over the block's heads in registers and
//      stored as one fp32 partial per head block; dA / dD / dt_bias as per-segment partials.
//   3. ssd_bwd_reduce    partials -> dB, dC (fixed summation order) in the I/O dtype and the caller's strides.
// Token-contracted products take their transposed operands from the MFMA unit (identity products), as in
// the forward; all accumulation is fp32.
#include <type_traits>

#include "common.h"
#include "launch.h"
#include "ssd_shared.h"
#include "tiles.h"

namespace mh {

// ------------------------------------------------------------------ helpers

// KSET-ordered identity B operand for k-step c: element j of lane (column l32) is 1 where
// 16 c + kset(half, j) == l32.
template <typename TM>
__device__ __forceinline__ Frag<TM> ident_kset(int c, int half, int l32) {
  Frag<TM> f;
#pragma unroll
  for (int j = 0; j < 8; ++j) f.set(j, (16 * c + kset(half, j) == l32) ? 1.f : 0.f);
  return f;
}

// One 32x32 block of a state in fragment-native order (16 values per lane, element i = row acc_row(half, i)
// of column l32).
template <typename T> struct StateBlk;
template <> struct StateBlk<bf16> {
  bf16x8 v[2];
  __device__ __forceinline__ float at(int i) const { return (float)v[i >> 3][i & 7]; }
  __device__ __forceinline__ Frag<bf16> frag(int c) const { Frag<bf16> f; f.v = v[c]; return f; }
};
template <> struct StateBlk<float> {
  f32x4 v[4];
  __device__ __forceinline__ float at(int i) const { return v[i >> 2][i & 3]; }
  __device__ __forceinline__ Frag<float> frag(int c) const {
    Frag<float> f;
#pragma unroll
    for (int j = 0; j < 8; ++j) f.v[j] = v[2 * c + (j >> 2)][j & 3];
    return f;
  }
};
template <typename T>
__device__ __forceinline__ StateBlk<T> load_state_blk(const T* base, int nt, int pt, int l) {
  StateBlk<T> s;
  if constexpr (sizeof(T) == 2) {
    s.v[0] = *reinterpret_cast<const bf16x8*>(base + frag_off_bf(nt, pt, l, 0));
    s.v[1] = *reinterpret_cast<const bf16x8*>(base + frag_off_bf(nt, pt, l, 1));
  } else {
    const T* q = base + frag_off(nt, pt, l);
#pragma unroll
    for (int i = 0; i < 4; ++i) s.v[i] = *reinterpret_cast<const f32x4*>(q + 4 * i);
  }
  return s;
}
template <typename T>
__device__ __forceinline__ void store_state_blk(T* base, int nt, int pt, int l, const f32x16& a) {
  if constexpr (sizeof(T) == 2) {
    bf16x8 lo, hi;
#pragma unroll
    for (int i = 0; i < 8; ++i) { lo[i] = (bf16)a[i]; hi[i] = (bf16)a[8 + i]; }
    *reinterpret_cast<bf16x8*>(base + frag_off_bf(nt, pt, l, 0)) = lo;
    *reinterpret_cast<bf16x8*>(base + frag_off_bf(nt, pt, l, 1)) = hi;
  } else {
    T* q = base + frag_off(nt, pt, l);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f32x4 v;
#pragma unroll
      for (int k = 0; k < 4; ++k) v[k] = a[4 * i + k];
      *reinterpret_cast<f32x4*>(q + 4 * i) = v;
    }
  }
}

// Transposed fragments of a state block X (rows n, columns p): out[c] has lane = row n, k = p = 16 c + KSET --
// two products with the KSET identity turn the column-per-lane block into a row-per-lane accumulator.
template <typename T>
__device__ __forceinline__ void blk_transpose(const StateBlk<T>& s, const Frag<T> (&idk)[2], Frag<T> (&out)[2]) {
  f32x16 e = zero16();
  e = mma(s.frag(0), idk[0], e);
  e = mma(s.frag(1), idk[1], e);
  out[0] = acc_to_frag<T>(e, 0);
  out[1] = acc_to_frag<T>(e, 1);
}

// Row `row` of a swizzled Tile<T, W> at the 16 columns col0 + acc_row(half, i) -- the values an
// accumulator tile whose lane column is `row` holds (col0 % 32 == 0).
template <typename T, int W>
__device__ __forceinline__ void acc_cols(const T* tile, int row, int col0, int half, float (&v)[16]) {
  using TL = Tile<T, W>;
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) {
    const int c = col0 + 8 * jj + 4 * half;
    if constexpr (sizeof(T) == 2) {
      const bf16x4 q = *reinterpret_cast<const bf16x4*>(tile + TL::chunk(row, c / 8) + (c & 7));
#pragma unroll
      for (int k = 0; k < 4; ++k) v[4 * jj + k] = (float)q[k];
    } else {
      const f32x4 q = *reinterpret_cast<const f32x4*>(tile + TL::chunk(row, c / 4));
#pragma unroll
      for (int k = 0; k < 4; ++k) v[4 * jj + k] = q[k];
    }
  }
}

// 16 values of a per-token LDS array at the rows r0 + acc_row(half, i).
__device__ __forceinline__ void acc_rows(const float* a, int r0, int half, float (&v)[16]) {
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) {
    const f32x4 q = *reinterpret_cast<const f32x4*>(a + r0 + 8 * jj + 4 * half);
#pragma unroll
    for (int k = 0; k < 4; ++k) v[4 * jj + k] = q[k];
  }
}

template <typename T>
__device__ __forceinline__ Frag<T> scaled(Frag<T> f, float s) {
#pragma unroll
  for (int j = 0; j < 8; ++j) f.set(j, f.get(j) * s);
  return f;
}

// Operand fragments f[c] of the transposed 32x32 block of a Tile<T, W> at rows r0.., columns q0..: lane = column
// q0 + lane % 32, k = row r0 + 16 c + KSET.  bf16: two transposing LDS reads each; fp32: the identity product.
template <typename T, int W>
__device__ __forceinline__ void tr_frags(const T* tile, int r0, int q0, const Frag<T> (&id)[2], int half, int l32,
                                         Frag<T> (&f)[2]) {
  if constexpr (sizeof(T) == 2) {
    f[0] = col_frag_tr_tile<W>(tile, q0, r0);
    f[1] = col_frag_tr_tile<W>(tile, q0, r0 + 16);
  } else {
    const f32x16 d = mfma_transpose<T, T, W>(tile, r0, q0, id, half, l32);
    f[0] = acc_to_frag<T>(d, 0);
    f[1] = acc_to_frag<T>(d, 1);
  }
}

// x^T-style transpose of a 32-column half tile (XHalf layout): D[r][q] = tile[r0 + r][q], lane = column q.
template <typename T>
__device__ __forceinline__ f32x16 xhalf_transpose(const T* tile, int r0, const Frag<T> (&id)[2], int half, int l32) {
  f32x16 acc = zero16();
#pragma unroll
  for (int c = 0; c < 2; ++c) acc = mma(xrow_frag<T, T>(tile, r0 + l32, 16 * c + 8 * half), id[c], acc);
  return acc;
}

// d(processed dt) / d(raw dt): sigmoid below softplus' threshold (identity above), times the clamp's pass mask.
__device__ __forceinline__ float dt_chain(const SsdParams& p, float raw, float bias) {
  const float u = raw + bias;
  float g = 1.f, v = u;
  if (p.dt_softplus) {
    if (u <= 20.f) g = 1.f / (1.f + __expf(-u));
    v = softplus_f(u);
  }
  if (p.has_dt_limit && !(v >= p.dt_min && v <= p.dt_max)) g = 0.f;
  return g;
}

// ------------------------------------------------------------------ kernel 0: clear accumulators

struct ZeroRanges {
  float* p[5];
  int64_t n[5];
};
// (an empty sequence's dA, dD and d_dt_bias; otherwise the partial sums' reduction writes them)
__global__ __launch_bounds__(256) void ssd_bwd_zero_kernel(ZeroRanges z) {
  const int r = blockIdx.y;
  float* p = z.p[r];
  if (!p) return;
  const int64_t n = z.n[r];
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) p[i] = 0.f;
}

// dh0 of an empty sequence: d_final itself (or zero).
__global__ __launch_bounds__(256) void ssd_bwd_copy_kernel(const float* __restrict__ src, float* __restrict__ dst,
                                                           size_t n) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) dst[i] = src ? src[i] : 0.f;
}

// ------------------------------------------------------------------ kernel 1: state sweeps

template <typename T, int N>
struct SweepStage {
  T M[SEG * N];             // Tile<T, N>: B (forward sweep) or C (adjoint sweep)
  T V[SEG * HD];            // Tile<T, HD>: x (forward) or dy (adjoint)
  float dtraw[SEG];
};
template <typename T, int N, int NST>
struct SweepSmem {
  SweepStage<T, N> st[NST];
  float w[2 * (N / 32)][SEG];   // per compute wave: per-token weight of the segment
};
// Two loader waves split each stage's loads (M blocks, V blocks; the first also dt) and wait for the oldest of up
// to NST - 1 stages in flight with vmcnt(later stages' loads), which counts to 63: as many stages as both that and
// the LDS allow.
template <typename T, int N>
constexpr int sweep_dps = Tile<T, N>::NBLK / 2 + Tile<T, HD>::NBLK / 2 + 1;   // loads per stage of loader 0
template <typename T, int N, int K>
constexpr bool sweep_fits = (K - 2) * sweep_dps<T, N> <= 63 && sizeof(SweepSmem<T, N, K>) <= 160 * 1024;
template <typename T, int N>
constexpr int sweep_nst = sweep_fits<T, N, 6> ? 6 : (sweep_fits<T, N, 5> ? 5 : (sweep_fits<T, N, 4> ? 4 : 3));

// Wait until at most `later` stages of DPS loads each remain in flight (a smaller count than needed only waits
// longer).
template <int DPS>
__device__ __forceinline__ void wait_stages(int later) {
  switch (later) {
    case 0: wait_vmem_n<0>(); break;
    case 1: wait_vmem_n<DPS>(); break;
    case 2: if constexpr (2 * DPS <= 63) wait_vmem_n<2 * DPS>(); else wait_vmem_n<DPS>(); break;
    case 3: if constexpr (3 * DPS <= 63) wait_vmem_n<3 * DPS>(); else wait_vmem_n<DPS>(); break;
    default: if constexpr (4 * DPS <= 63) wait_vmem_n<4 * DPS>(); else wait_vmem_n<DPS>(); break;
  }
}

// One workgroup per (direction, head, batch): compute wave w owns state tile (nt, pt) = (w % (N/32), w / (N/32)),
// and two more waves only fetch: they keep up to NST - 1 segments in flight (global -> LDS) and wait for them
// with exact counts, which the compute waves, whose state stores share the same counter, could not.
//   forward (dir 0): S = h, segments first to last, weights w_s = e^{c_end - c_s} dt_s on B^T x:
//       stores the entering state of every segment, S <- e^{c_end} S + sum_s B_s^T w_s x_s
//   adjoint (dir 1): S = lam, segments last to first, weights w_t = e^{c_t} on C^T dy:
//       stores lam_out of every segment, S <- e^{c_end} S + sum_t C_t^T w_t dy_t, finally dh0 = S.
// Both directions run in one launch (independent workgroups).
template <typename T, int N>
__global__ __launch_bounds__(64 * (2 * (N / 32) + 2)) void ssd_bwd_sweep_kernel(SsdBwdParams q) {
  constexpr int NB = N / 32, NW = 2 * NB;
  constexpr int NST = sweep_nst<T, N>;
  constexpr int DPS = sweep_dps<T, N>;
  __shared__ SweepSmem<T, N, NST> sm;
  const SsdParams& p = q.f;
  const int dir = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int g = h / (p.nheads / p.ngroups);
  const int w = wave_id(), l = lane_id(), half = l >> 5, l32 = l & 31;
  const int nseg = p.nseg;
  auto seg_of = [&](int i) { return dir ? nseg - 1 - i : i; };
  if (w >= NW) {
    // ---- loader waves (lw = 0, 1: halves of the M and V blocks; lw 0 also dt)
    const int lw = w - NW;
    const T* Mb = reinterpret_cast<const T*>(dir ? p.C : p.B) + (int64_t)b * (dir ? p.C_sb : p.B_sb) + g * N;
    const int64_t M_sl = dir ? p.C_sl : p.B_sl;
    const T* Vb = dir ? reinterpret_cast<const T*>(q.dy) + (int64_t)b * q.dy_sb + (int64_t)h * q.dy_sh
                      : reinterpret_cast<const T*>(p.x) + (int64_t)b * p.x_sb + (int64_t)h * p.x_sh;
    const int64_t V_sl = dir ? q.dy_sl : p.x_sl;
    const float* dtb = p.dt + (int64_t)b * p.dt_sb + h;
    auto issue = [&](int i) {
      const int k = seg_of(i), s = i % NST;
      const int t0 = k * SEG, lst = min(t0 + SEG, p.seqlen) - 1;
      constexpr int mb = Tile<T, N>::NBLK / 2, vb = Tile<T, HD>::NBLK / 2;
      fetch_tile<T, N>(sm.st[s].M, Mb, M_sl, t0, lst, lw * mb, mb, l);
      fetch_tile<T, HD>(sm.st[s].V, Vb, V_sl, t0, lst, lw * vb, vb, l);
      if (lw == 0) fetch_dt(sm.st[s].dtraw, dtb, p.dt_sl, t0, lst, l);
    };
    for (int i = 0; i < NST - 1 && i < nseg; ++i) issue(i);
    for (int i = 0; i < nseg; ++i) {
      const int later = min(NST - 2, nseg - 1 - i);      // stages issued after stage i
      if (lw == 0) wait_stages<DPS>(later);                          // loader 0: M, V halves and dt
      else wait_stages<DPS - 1>(later);                               // loader 1: M, V halves
      lds_barrier();                                     // publish stage i; iteration i - 1 is done everywhere
      if (i + NST - 1 < nseg) issue(i + NST - 1);        // into the stage iteration i - 1 read
    }
    return;
  }
  // ---- compute waves
  const int nt = w % NB, pt = w / NB;
  const float Ah = p.A[h], bias = p.dt_bias ? p.dt_bias[h] : 0.f;
  Frag<T> id[2];
#pragma unroll
  for (int c = 0; c < 2; ++c) id[c] = ident_frag<T>(c, half, l32);
  const int64_t per = (int64_t)HD * N;
  // initial state, canonical (p, n) -> block (nt, pt): h0 (forward) or d_final (adjoint)
  const float* s0 = dir ? q.d_final : p.init_state;
  f32x16 S = zero16();
  if (s0) {
    const float* src = s0 + ((int64_t)b * p.nheads + h) * per + (32 * pt + l32) * N + 32 * nt;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(src + 8 * jj + 4 * half);
#pragma unroll
      for (int k = 0; k < 4; ++k) S[4 * jj + k] = v[k];
    }
  }
  T* out = reinterpret_cast<T*>(dir ? q.lam : q.hin);
  for (int i = 0; i < nseg; ++i) {
    const int k = seg_of(i), s = i % NST;
    // the state entering segment k (forward) / leaving it (adjoint), stored before the update
    store_state_blk<T>(out + (((int64_t)b * nseg + k) * p.nheads + h) * per, nt, pt, l, S);
    lds_barrier();
    const int len = min(SEG, p.seqlen - k * SEG);
    float dtv;
    const float cs = seg_decay(p, sm.st[s].dtraw[l], bias, Ah, l, len, dtv);
    const float cend = lane_val(cs, 63);
    sm.w[w][l] = dir ? ((l < len) ? __expf(cs) : 0.f) : __expf(cend - cs) * dtv;
    f32x16 acc = zero16();
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
      Frag<T> mf[2], vf[2];
      tr_frags<T, N>(sm.st[s].M, 32 * tb, 32 * nt, id, half, l32, mf);    // lane n, k = t
      tr_frags<T, HD>(sm.st[s].V, 32 * tb, 32 * pt, id, half, l32, vf);   // lane p, k = t
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        float e[8];
        kset_vals(sm.w[w], 2 * tb + c, half, e);
        Frag<T> a;
#pragma unroll
        for (int j = 0; j < 8; ++j) a.set(j, mf[c].get(j) * e[j]);
        acc = mma(a, vf[c], acc);                        // [n][p] += sum_t M[t][n] w_t V[t][p]
      }
    }
    const float dec = __expf(cend);
#pragma unroll
    for (int j = 0; j < 16; ++j) S[j] = dec * S[j] + acc[j];
  }
  if (dir && q.dh0) {
    float* dst = q.dh0 + ((int64_t)b * p.nheads + h) * per + (32 * pt + l32) * N + 32 * nt;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      f32x4 v;
#pragma unroll
      for (int k = 0; k < 4; ++k) v[k] = S[4 * jj + k];
      *reinterpret_cast<f32x4*>(dst + 8 * jj + 4 * half) = v;
    }
  }
}

// ------------------------------------------------------------------ kernel 2: gradients per segment

template <typename T, int N>
struct GradStage {
  T X[SEG * HD];            // Tile<T, HD> of the head
  T DY[SEG * HD];
  float dtraw[SEG];
};
template <typename T, int N, bool SL> struct GradStates {};
template <typename T, int N> struct GradStates<T, N, true> {
  T Lam[HD * N];            // lam_out and h_in of the head, fragment-native order (as in the workspaces)
  T Hin[HD * N];
};
// With 8 waves the dx^T tiles' state contraction is split over the two halves of the workgroup; the first half
// leaves its partial tile here.
template <int NW> struct DxPartial { float v[NW == 8 ? 4 : 1][64 * 16]; };
// The six distinct masked/decayed dy.x^T tiles of a head as B-operand fragments: L o XD (t-block, s-block) =
// (0,0), (1,0), (1,1) and (L o XD o dt)^T (s-block, t-block) = (0,0), (0,1), (1,1).  Shared through LDS for bf16
// (one wave forms each); fp32 fragments are twice the size and do not fit, so each wave forms its own.
template <typename T>
struct XdTiles {
  Frag<T> xd[3][2][64];
  Frag<T> xt[3][2][64];
};
template <>
struct XdTiles<float> {};

template <typename T, int N, int NST, bool SL>
struct GradSmem {
  GradStage<T, N> st[NST];
  GradStates<T, N, SL> sts;
  DxPartial<2 * (N / 32)> dxp;
  T B[SEG * N];             // Tile<T, N>
  T C[SEG * N];
  float cs[2 * (N / 32)][SEG];   // per wave: c_t of the current head
  float dtp[2 * (N / 32)][SEG];  // per wave: processed dt
  float red[2][N / 32][SEG];     // per n-block partial dots: bint, u
  XdTiles<T> xds;                // bf16: the head's XD tiles, formed once and shared (fp32: per wave, none here)
  float colg[3][32];             // per XD tile (t-block, s-block) = (0,0), (1,0), (1,1): sum_t (M o XD)[t][s]
  float rowg[3][32];             // per XD^T tile (s-block, t-block) = (0,0), (0,1), (1,1): sum_s (M o XD)[t][s] dt_s
  float lh[N / 32];              // <lam_out, h_in> per n-block
  float dd[2];                   // trace of dy x^T per diagonal 32-block
  alignas(16) float cb[3][64 * 16];   // CB[t][s] tiles (t-block, s-block) = (0,0), (1,0), (1,1), accumulator
                                      // order (16-byte aligned: read and written as f32x4)
  float cbt[3][64 * 16];         // CB^T[s][t] tiles (s-block, t-block) = (0,0), (0,1), (1,1)
};
constexpr size_t GRAD_LDS = 160 * 1024;
// The per-head tiles are double-buffered (the next head's fetch overlaps this head's work) and the head's states
// staged in LDS (else read from HBM where used), as far as the LDS allows, in that order of preference.
template <typename T, int N, int NST, bool SL>
constexpr bool grad_fits = sizeof(GradSmem<T, N, NST, SL>) <= GRAD_LDS;
template <typename T, int N>
constexpr int grad_nst = (grad_fits<T, N, 2, true> || grad_fits<T, N, 2, false>) ? 2 : 1;
template <typename T, int N>
constexpr bool grad_sl = grad_fits<T, N, grad_nst<T, N>, true>;

// Work split (NW = 2 N/32 waves): wave w owns n-block nb = w % (N/32) and token block r = w / (N/32) of the
// dB^T [n][s] and dC^T [n][t] tiles; waves 0-3 also own the dx^T [p][s] tile (p-block w & 1, s-block w >> 1).
template <typename T, int N>
__global__ __launch_bounds__(128 * (N / 32)) void ssd_bwd_grad_kernel(SsdBwdParams q) {
  constexpr int NB = N / 32, NW = 2 * NB;
  using TB = Tile<T, N>;
  using TX = Tile<T, HD>;
  constexpr bool SL = grad_sl<T, N>;
  constexpr int NST = grad_nst<T, N>;
  __shared__ GradSmem<T, N, NST, SL> sm;
  const SsdParams& p = q.f;
  const int si = blockIdx.x, b = blockIdx.z;
  const int HB = q.heads_per_wg;
  const int hfirst = blockIdx.y * HB;
  const int hpg = p.nheads / p.ngroups;
  const int g = hfirst / hpg;
  const int w = wave_id(), l = lane_id(), half = l >> 5, l32 = l & 31;
  const int nb = w % NB, r = w / NB;
  const bool dxw = w < 4;                   // first dx half (all of dx with 4 waves)
  constexpr bool SPLIT = NW == 8;           // the second half (waves 4-7) takes half of the state contraction
  const int pb = w & 1, sbx = (w >> 1) & 1;
  const int tok0 = si * SEG;
  const int len = min(SEG, p.seqlen - tok0);
  const int last = tok0 + len - 1;
  const int s_l = 32 * r + l32;             // token column of this lane in the dB / dC tiles
  const int s_x = 32 * sbx + l32;           // token column of this lane in the dx tile
  const int64_t per = (int64_t)HD * N;

  const T* xb = reinterpret_cast<const T*>(p.x) + (int64_t)b * p.x_sb;
  const T* dyb = reinterpret_cast<const T*>(q.dy) + (int64_t)b * q.dy_sb;
  const float* dtb = p.dt + (int64_t)b * p.dt_sb;
  {
    constexpr int nblk = TB::NBLK / NW;
    fetch_tile<T, N>(sm.B, reinterpret_cast<const T*>(p.B) + (int64_t)b * p.B_sb + g * N, p.B_sl, tok0, last,
                     w * nblk, nblk, l);
    fetch_tile<T, N>(sm.C, reinterpret_cast<const T*>(p.C) + (int64_t)b * p.C_sb + g * N, p.C_sl, tok0, last,
                     w * nblk, nblk, l);
  }
  const char* hin_ws = reinterpret_cast<const char*>(q.hin);
  const char* lam_ws = reinterpret_cast<const char*>(q.lam);
  // one head's tiles, dt and both states (contiguous HD x N blocks of the workspaces) into stage st
  auto fetch_head = [&](int h, auto stc) {
    constexpr int st = decltype(stc)::value;
    // lane offsets computed here from a laundered lane id: hoisted out of the head loop, the per-lane
    // addresses would be spilled, and reloading them drains the vector-memory counter before every fetch
    int l = lane_id();
    asm volatile("" : "+v"(l));
    constexpr int nblk = TX::NBLK / NW;
    fetch_tile<T, HD>(sm.st[st].X, xb + (int64_t)h * p.x_sh, p.x_sl, tok0, last, w * nblk, nblk, l);
    fetch_tile<T, HD>(sm.st[st].DY, dyb + (int64_t)h * q.dy_sh, q.dy_sl, tok0, last, w * nblk, nblk, l);
    if (w == 0) fetch_dt(sm.st[st].dtraw, dtb + h, p.dt_sl, tok0, last, l);
  };
  auto fetch_states = [&](int h) {
    if constexpr (SL) {
      int l = lane_id();
      asm volatile("" : "+v"(l));
      constexpr int sblk = HD * N * (int)sizeof(T) / 1024 / NW;
      const int64_t soff = (((int64_t)b * p.nseg + si) * p.nheads + h) * per * (int64_t)sizeof(T);
      fetch_blocks(reinterpret_cast<char*>(sm.sts.Lam), lam_ws + soff, w * sblk, sblk, l);
      fetch_blocks(reinterpret_cast<char*>(sm.sts.Hin), hin_ws + soff, w * sblk, sblk, l);
    }
  };
  fetch_head(hfirst, std::integral_constant<int, 0>());
  fetch_states(hfirst);
  f32x16 dBacc = zero16(), dCacc = zero16();

  wait_vmem();                      // B / C tiles (and the first head's tiles) in LDS
  lds_barrier();
  if (dxw && pb == 1) {
    // CB^T[s][t] = B_s . C_t for the tiles (sb, sbx), sb <= sbx (t-block sbx)
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      if (sb <= sbx) {
        f32x16 a = zero16();
#pragma unroll
        for (int k = 0; k < N / 16; ++k)
          a = mma(row_frag<T, T, N>(sm.B, 32 * sb + l32, 16 * k + 8 * half),
                  row_frag<T, T, N>(sm.C, s_x, 16 * k + 8 * half), a);
        float* o = sm.cbt[sb + sbx] + 16 * l;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          f32x4 v;
#pragma unroll
          for (int k = 0; k < 4; ++k) v[k] = a[4 * i + k];
          *reinterpret_cast<f32x4*>(o + 4 * i) = v;
        }
      }
    }
  }
  if (dxw && pb == 0) {
    // CB[t][s] = C_t . B_s for the tiles (tb, sbx), tb >= sbx, parked in LDS for every head of the block
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
      if (tb >= sbx) {
        f32x16 a = zero16();
#pragma unroll
        for (int k = 0; k < N / 16; ++k)
          a = mma(row_frag<T, T, N>(sm.C, 32 * tb + l32, 16 * k + 8 * half),
                  row_frag<T, T, N>(sm.B, s_x, 16 * k + 8 * half), a);
        float* o = sm.cb[tb + sbx] + 16 * l;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          f32x4 v;
#pragma unroll
          for (int k = 0; k < 4; ++k) v[k] = a[4 * i + k];
          *reinterpret_cast<f32x4*>(o + 4 * i) = v;
        }
      }
    }
  }
  lds_barrier();                    // CB tiles visible
  // One head: its stage index is a compile-time constant (the loop below is unrolled by two), so the compiler
  // sees that the next head's fetch and this head's LDS reads touch different bytes (with a run-time index it
  // orders every LDS access after the pending fetch).
  auto head = [&](const int j, auto stc) {
    constexpr int st = decltype(stc)::value;
    // Lane-derived values are recomputed per head from a laundered lane id (and length): otherwise the
    // compiler keeps dozens of loop-invariant row indices and masks in registers across the head loop.
    int lq = l, lenq = len;
    asm volatile("" : "+v"(lq), "+s"(lenq));
    const int l = lq, len = lenq;
    const int half = l >> 5, l32 = l & 31;
    const int s_l = 32 * r + l32, s_x = 32 * sbx + l32;
    Frag<T> id[2], idk[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      id[c] = ident_frag<T>(c, half, l32);
      idk[c] = ident_kset<T>(c, half, l32);
    }
    const int h = hfirst + j;
    auto& sg = sm.st[st];
    const int64_t sidx = (((int64_t)b * p.nseg + si) * p.nheads + h) * per;
    auto lam_src = [&]() -> const T* {
      if constexpr (SL) return sm.sts.Lam;
      else return reinterpret_cast<const T*>(lam_ws) + sidx;
    };
    auto hin_src = [&]() -> const T* {
      if constexpr (SL) return sm.sts.Hin;
      else return reinterpret_cast<const T*>(hin_ws) + sidx;
    };
    StateBlk<T> Lb[2], Hb[2];
#pragma unroll
    for (int pt = 0; pt < 2; ++pt) {
      Lb[pt] = load_state_blk<T>(lam_src(), nb, pt, l);
      Hb[pt] = load_state_blk<T>(hin_src(), nb, pt, l);
    }
    // ---- decay of this head (lane = token), wave-private copies for per-row reads
    const float Ah = p.A[h];
    const float bias = p.dt_bias ? p.dt_bias[h] : 0.f;
    const float raw = sg.dtraw[l];
    float dtv;
    const float cs = seg_decay(p, raw, bias, Ah, l, len, dtv);
    const float cend = lane_val(cs, 63);
    sm.cs[w][l] = cs;
    sm.dtp[w][l] = dtv;
    const float cs_l = from_half(cs, r), dt_l = from_half(dtv, r);

    constexpr bool SHARE = sizeof(T) == 2;
    Frag<T> XDf[2][2], XTf[2][2];        // per-wave tiles (fp32 only)
    if constexpr (SHARE) {
      // the six distinct XD tiles of the head, wave w forming tiles w, w + NW, ... (same masks, decays and sums
      // as the per-wave path below; each wave reads its own copies of the decays)
      for (int tix = w; tix < 6; tix += NW) {
      if (tix < 3) {
        const int tb = tix == 0 ? 0 : 1, rr = tix == 2 ? 1 : 0;
        const int s_p = 32 * rr + l32;
        const float cs_p = from_half(cs, rr);
        f32x16 a = zero16();
#pragma unroll
        for (int k = 0; k < HD / 16; ++k)
          a = mma(row_frag<T, T, HD>(sg.DY, 32 * tb + l32, 16 * k + 8 * half),
                  row_frag<T, T, HD>(sg.X, s_p, 16 * k + 8 * half), a);
        float ct[16];
        acc_rows(sm.cs[w], 32 * tb, half, ct);
        float d = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int t = 32 * tb + acc_row(half, i);
          a[i] = (t < len && t >= s_p) ? a[i] * __expf(ct[i] - cs_p) : 0.f;
          d += (t == s_p) ? a[i] : 0.f;
        }
        if (tb == rr) {
          d = wave_sum(d);
          if (l == 0) sm.dd[rr] = d;
        }
        float cg = 0.f;
        const float* cbp = sm.cb[tix] + 16 * l;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const f32x4 v = *reinterpret_cast<const f32x4*>(cbp + 4 * i);
#pragma unroll
          for (int k = 0; k < 4; ++k) cg += v[k] * a[4 * i + k];
        }
        cg = sum_halves(cg);
        if (half == 0) sm.colg[tix][l32] = cg;
#pragma unroll
        for (int c = 0; c < 2; ++c) sm.xds.xd[tix][c][l] = acc_to_frag<T>(a, c);
      } else {
        const int ti = tix - 3, sb = ti == 2 ? 1 : 0, rr = ti == 0 ? 0 : 1;
        const int t_p = 32 * rr + l32;
        const float cs_p = from_half(cs, rr);
        f32x16 a = zero16();
#pragma unroll
        for (int k = 0; k < HD / 16; ++k)
          a = mma(row_frag<T, T, HD>(sg.X, 32 * sb + l32, 16 * k + 8 * half),
                  row_frag<T, T, HD>(sg.DY, t_p, 16 * k + 8 * half), a);
        float cr[16], dr[16];
        acc_rows(sm.cs[w], 32 * sb, half, cr);
        acc_rows(sm.dtp[w], 32 * sb, half, dr);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int s_ = 32 * sb + acc_row(half, i);
          a[i] = (t_p < len && s_ <= t_p) ? a[i] * __expf(cs_p - cr[i]) * dr[i] : 0.f;
        }
        float rg = 0.f;
        const float* cbp = sm.cbt[ti] + 16 * l;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const f32x4 v = *reinterpret_cast<const f32x4*>(cbp + 4 * i);
#pragma unroll
          for (int k = 0; k < 4; ++k) rg += v[k] * a[4 * i + k];
        }
        rg = sum_halves(rg);
        if (half == 0) sm.rowg[ti][l32] = rg;
#pragma unroll
        for (int c = 0; c < 2; ++c) sm.xds.xt[ti][c][l] = acc_to_frag<T>(a, c);
      }
      }
      lds_barrier();                     // the shared XD tiles are in LDS
    } else {
      // ---- XD[t][s] = dy_t . x_s (tiles tb >= r, column block r), masked and decayed (L o XD), as
      //      B-operand fragments (column s, k = t)
      // The per-token sums of M o XD that the decay gradient needs (colG here, rowG below) are taken from
      // these fp32 tiles, not from the bf16-operand products: the two sums cancel pairwise in da, and only
      // identically rounded copies cancel.
      float colg = 0.f;
  #pragma unroll
      for (int tb = 0; tb < 2; ++tb) {
        f32x16 a = zero16();
        if (tb >= r) {
  #pragma unroll
          for (int k = 0; k < HD / 16; ++k)
            a = mma(row_frag<T, T, HD>(sg.DY, 32 * tb + l32, 16 * k + 8 * half),
                    row_frag<T, T, HD>(sg.X, s_l, 16 * k + 8 * half), a);
          float ct[16];
          acc_rows(sm.cs[w], 32 * tb, half, ct);
          float d = 0.f;
  #pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int t = 32 * tb + acc_row(half, i);
            a[i] = (t < len && t >= s_l) ? a[i] * __expf(ct[i] - cs_l) : 0.f;
            d += (t == s_l) ? a[i] : 0.f;
          }
          if (nb == 0) {
            // trace of dy x^T (per-head D): the diagonal block (r, r)
            if (tb == r) {
              d = wave_sum(d);
              if (l == 0) sm.dd[r] = d;
            }
            const float* cbp = sm.cb[tb + r] + 16 * l;
  #pragma unroll
            for (int i = 0; i < 4; ++i) {
              const f32x4 v = *reinterpret_cast<const f32x4*>(cbp + 4 * i);
  #pragma unroll
              for (int k = 0; k < 4; ++k) colg += v[k] * a[4 * i + k];
            }
          }
        }
  #pragma unroll
        for (int c = 0; c < 2; ++c) XDf[tb][c] = acc_to_frag<T>(a, c);
      }
      if (nb == 0) {
        colg = sum_halves(colg);
        if (half == 0) {
          sm.colg[r == 0 ? 0 : 2][l32] = colg;      // the s-block's sum over its t-blocks
          if (r == 0) sm.colg[1][l32] = 0.f;
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);   // keep the phases apart: bounded register lifetimes
    // ---- dB^T tile (n-block nb, s-block r): inter part from lam_out, intra part from C^T (L o XD)
    {
      Frag<T> lamT[2][2];
#pragma unroll
      for (int pt = 0; pt < 2; ++pt) blk_transpose<T>(Lb[pt], idk, lamT[pt]);
      const float wend_l = __expf(cend - cs_l);
      f32x16 ai = zero16(), aa = zero16();
#pragma unroll
      for (int pt = 0; pt < 2; ++pt)
#pragma unroll
        for (int c = 0; c < 2; ++c)
          ai = mma(lamT[pt][c], scaled<T>(kset_frag<T, T, HD>(sg.X, s_l, 32 * pt + 16 * c, half), wend_l), ai);
#pragma unroll
      for (int tb = 0; tb < 2; ++tb) {
        if (tb >= r) {
          Frag<T> ct[2];
          tr_frags<T, N>(sm.C, 32 * tb, 32 * nb, id, half, l32, ct);   // lane n, k = t
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            if constexpr (SHARE) aa = mma(ct[c], sm.xds.xd[r == 0 ? tb : 2][c][l], aa);
            else aa = mma(ct[c], XDf[tb][c], aa);
          }
        }
      }
      float Bv[16];
      acc_cols<T, N>(sm.B, s_l, 32 * nb, half, Bv);
      float sI = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        sI += ai[i] * Bv[i];
        dBacc[i] += dt_l * (ai[i] + aa[i]);
      }
      sI = sum_halves(sI);
      if (half == 0) sm.red[0][nb][s_l] = sI;
    }
    __builtin_amdgcn_sched_barrier(0);   // keep the phases apart: bounded register lifetimes
    if constexpr (!SHARE) {
      // ---- XD^T[s][t] (tiles sb <= r, column block r), masked, decayed, scaled by dt_s: (column t, k = s)
      float rowg = 0.f;
  #pragma unroll
      for (int sb = 0; sb < 2; ++sb) {
        f32x16 a = zero16();
        if (sb <= r) {
  #pragma unroll
          for (int k = 0; k < HD / 16; ++k)
            a = mma(row_frag<T, T, HD>(sg.X, 32 * sb + l32, 16 * k + 8 * half),
                    row_frag<T, T, HD>(sg.DY, s_l, 16 * k + 8 * half), a);
          float cr[16], dr[16];
          acc_rows(sm.cs[w], 32 * sb, half, cr);
          acc_rows(sm.dtp[w], 32 * sb, half, dr);
  #pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int s = 32 * sb + acc_row(half, i);
            a[i] = (s_l < len && s <= s_l) ? a[i] * __expf(cs_l - cr[i]) * dr[i] : 0.f;
          }
          if (nb == 0) {
            const float* cbp = sm.cbt[sb + r] + 16 * l;
  #pragma unroll
            for (int i = 0; i < 4; ++i) {
              const f32x4 v = *reinterpret_cast<const f32x4*>(cbp + 4 * i);
  #pragma unroll
              for (int k = 0; k < 4; ++k) rowg += v[k] * a[4 * i + k];
            }
          }
        }
  #pragma unroll
        for (int c = 0; c < 2; ++c) XTf[sb][c] = acc_to_frag<T>(a, c);
      }
      if (nb == 0) {
        rowg = sum_halves(rowg);
        if (half == 0) {
          sm.rowg[r == 0 ? 0 : 1][l32] = rowg;      // the t-block's sum over its s-blocks
          if (r == 1) sm.rowg[2][l32] = 0.f;
        }
      }

    }

    // <lam_out, h_in> over the blocks of n-block nb (one wave per n-block)
    if (r == 0) {
      float d = 0.f;
#pragma unroll
      for (int pt = 0; pt < 2; ++pt)
#pragma unroll
        for (int i = 0; i < 16; ++i) d += Lb[pt].at(i) * Hb[pt].at(i);
      d = wave_sum(d);
      if (l == 0) sm.lh[nb] = d;
    }

    // ---- dC^T tile (n-block nb, t-block r): inter part from h_in, intra part from B^T (L o XD o dt)^T
    {
      Frag<T> hT[2][2];
#pragma unroll
      for (int pt = 0; pt < 2; ++pt) blk_transpose<T>(Hb[pt], idk, hT[pt]);
      const float ec_l = __expf(cs_l);
      f32x16 ah = zero16(), ac = zero16();
#pragma unroll
      for (int pt = 0; pt < 2; ++pt)
#pragma unroll
        for (int c = 0; c < 2; ++c)
          ah = mma(hT[pt][c], scaled<T>(kset_frag<T, T, HD>(sg.DY, s_l, 32 * pt + 16 * c, half), ec_l), ah);
#pragma unroll
      for (int sb = 0; sb < 2; ++sb) {
        if (sb <= r) {
          Frag<T> bt[2];
          tr_frags<T, N>(sm.B, 32 * sb, 32 * nb, id, half, l32, bt);   // lane n, k = s
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            if constexpr (SHARE) ac = mma(bt[c], sm.xds.xt[r == 0 ? 0 : (sb == 0 ? 1 : 2)][c][l], ac);
            else ac = mma(bt[c], XTf[sb][c], ac);
          }
        }
      }
      float Cv[16];
      acc_cols<T, N>(sm.C, s_l, 32 * nb, half, Cv);
      float sU = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        sU += ah[i] * Cv[i];
        dCacc[i] += ah[i] + ac[i];
      }
      sU = sum_halves(sU);
      if (half == 0) sm.red[1][nb][s_l] = sU;
    }

    __builtin_amdgcn_sched_barrier(0);   // keep the phases apart: bounded register lifetimes
    // ---- dx^T tile (p-block pb, s-block sbx).  dx = dt_s (intra + e^{c_end - c_s} lam_out B_s) + D dy: the first
    // half owns intra and, with the split, the state blocks nt < NB/2; the second half the others and the store.
    float dyv[16], Dv[16];
    f32x16 ax = zero16();
    const bool dxB = SPLIT && w >= 4;
    if (dxw || dxB) {
      const float csx = from_half(cs, sbx), wx = __expf(cend - csx);
      if (dxw) {
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
          if (tb >= sbx) {
            f32x16 m;
            const float* cbp = sm.cb[tb + sbx] + 16 * l;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const f32x4 v = *reinterpret_cast<const f32x4*>(cbp + 4 * i);
#pragma unroll
              for (int k = 0; k < 4; ++k) m[4 * i + k] = v[k];
            }
            float ct[16];
            acc_rows(sm.cs[w], 32 * tb, half, ct);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
              const int t = 32 * tb + acc_row(half, i);
              m[i] = (t < len && t >= s_x) ? m[i] * __expf(ct[i] - csx) : 0.f;
            }
            Frag<T> dyt[2];
            tr_frags<T, HD>(sg.DY, 32 * tb, 32 * pb, id, half, l32, dyt);   // lane p, k = t
#pragma unroll
            for (int c = 0; c < 2; ++c) ax = mma(dyt[c], acc_to_frag<T>(m, c), ax);
          }
        }
      }
      constexpr int NT0 = SPLIT ? NB / 2 : NB;
      const int nt0 = dxB ? NT0 : 0;
#pragma unroll
      for (int k = 0; k < NT0; ++k) {
        const int nt = nt0 + k;
        const StateBlk<T> lx = load_state_blk<T>(lam_src(), nt, pb, l);
#pragma unroll
        for (int c = 0; c < 2; ++c)
          ax = mma(lx.frag(c), scaled<T>(kset_frag<T, T, N>(sm.B, s_x, 32 * nt + 16 * c, half), wx), ax);
      }
      if (!SPLIT || dxB) {
        acc_cols<T, HD>(sg.DY, s_x, 32 * pb, half, dyv);
#pragma unroll
        for (int i = 0; i < 16; ++i)
          Dv[i] = p.D ? (p.D_per_channel ? p.D[h * HD + 32 * pb + acc_row(half, i)] : p.D[h]) : 0.f;
        if (p.D_per_channel && q.dD) {
          // per-channel dD of this token half: sum over the lane-half's 32 tokens in a fixed shuffle order,
          // one partial per (segment, head, token half) in the workspace, summed in order by the reduce kernel
          float xv[16];
          acc_cols<T, HD>(sg.X, s_x, 32 * pb, half, xv);
          float* dst = q.part_dc + ((((int64_t)b * p.nseg + si) * p.nheads + h) * 2 + sbx) * HD + 32 * pb;
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            float v = s_x < len ? xv[i] * dyv[i] : 0.f;
#pragma unroll
            for (int o = 16; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
            if (l32 == 0) dst[acc_row(half, i)] = v;
          }
        }
      } else {
        float* o = sm.dxp.v[w & 3] + 16 * l;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          f32x4 v;
#pragma unroll
          for (int k = 0; k < 4; ++k) v[k] = ax[4 * i + k];
          *reinterpret_cast<f32x4*>(o + 4 * i) = v;
        }
      }
    }
    // dx = dt_s * ax + D dy, stored by the owner of the finished tile
    auto store_dx = [&]() {
      const float dtx = from_half(dtv, sbx);
      if (s_x < len) {
        const float xr = q.dx_rows ? q.dx_rows[((int64_t)b * q.f.seqlen + tok0 + s_x) * q.f.nheads + h] : 0.f;
        T* o = reinterpret_cast<T*>(q.dx) + (int64_t)b * q.dx_sb + (int64_t)(tok0 + s_x) * q.dx_sl +
               (int64_t)h * q.dx_sh + 32 * pb + 4 * half;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          if constexpr (sizeof(T) == 2) {
            bf16x4 v;
#pragma unroll
            for (int k = 0; k < 4; ++k) v[k] = (bf16)(dtx * ax[4 * jj + k] + Dv[4 * jj + k] * dyv[4 * jj + k] + xr);
            *reinterpret_cast<bf16x4*>(o + 8 * jj) = v;
          } else {
            f32x4 v;
#pragma unroll
            for (int k = 0; k < 4; ++k) v[k] = dtx * ax[4 * jj + k] + Dv[4 * jj + k] * dyv[4 * jj + k] + xr;
            *reinterpret_cast<f32x4*>(o + 8 * jj) = v;
          }
        }
      }
    };
    if (!SPLIT && dxw) store_dx();

    // The next head's fetch: into the other stage (head j - 1's, read by nobody since the last barrier) before
    // the barrier, or, with one stage, after it.  It is issued late on purpose: a spill reload in the work above
    // would wait for it (the vector-memory counter is shared).
    if (NST == 2 && j + 1 < HB) fetch_head(h + 1, std::integral_constant<int, st ^ 1>());
    lds_barrier();                     // partial dots and dx partials complete; this head's states no longer read
    if (j + 1 < HB) {
      if (NST == 1) fetch_head(h + 1, std::integral_constant<int, 0>());
      fetch_states(h + 1);
    }
    if (dxB) {
      const float* ip = sm.dxp.v[w & 3] + 16 * l;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(ip + 4 * i);
#pragma unroll
        for (int k = 0; k < 4; ++k) ax[4 * i + k] += v[k];
      }
      store_dx();
    }
    if (w == 0) {
      const float colG = l < 32 ? sm.colg[0][l] + sm.colg[1][l] : sm.colg[2][l - 32];
      const float rowG = l < 32 ? sm.rowg[0][l] : sm.rowg[1][l - 32] + sm.rowg[2][l - 32];
      float bint = 0.f, u = 0.f, lh = 0.f;
#pragma unroll
      for (int k = 0; k < NB; ++k) {
        bint += sm.red[0][k][l];
        u += sm.red[1][k][l];
        lh += sm.lh[k];
      }
      const bool valid = l < len;
      const float qv = valid ? rowG - dtv * colG + u : 0.f;
      const float vv = dtv * bint;
      const float qi = wave_incl_scan_dpp(qv);
      const float qtot = lane_val(qi, 63);
      const float vi = wave_incl_scan_dpp(vv);
      const float da = (qtot - qi + qv) + __expf(cend) * lh + (vi - vv);
      const float ddr = valid ? (colG + bint + Ah * da) * dt_chain(p, raw, bias) : 0.f;
      if (valid) q.ddt[(int64_t)b * q.ddt_sb + (int64_t)(tok0 + l) * q.ddt_sl + h] = ddr;
      const float sdA = wave_sum(valid ? dtv * da : 0.f);
      const float sdb = wave_sum(ddr);
      if (l == 0) {                    // this segment's partials, summed in a fixed order by the reduce kernel
        float* ps = q.part_s + (((int64_t)b * p.nseg + si) * p.nheads + h) * 3;
        ps[0] = sdA;
        ps[1] = sdb;
        ps[2] = sm.dd[0] + sm.dd[1];
      }
    }
    if (j + 1 < HB) {
      wait_vmem();                     // the next head's stage (and this head's stores)
      lds_barrier();
    }
  };
  for (int j = 0; j < HB; j += NST) {
    head(j, std::integral_constant<int, 0>());
    if constexpr (NST == 2) {
      if (j + 1 < HB) head(j + 1, std::integral_constant<int, 1>());
    }
  }

  // sums over this block's heads -> partial kb of the group: fp32 (b, L, G, N), plain stores (the partials of a
  // group's head blocks are added in a fixed order afterwards: no atomics, run-to-run identical results)
  if (s_l < len) {
    const int kb = (hfirst % hpg) / HB;
    const int64_t row = ((((int64_t)kb * p.batch + b) * p.seqlen + tok0 + s_l) * p.ngroups + g) * N + 32 * nb;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      f32x4 vb, vc;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        vb[k] = dBacc[4 * jj + k];
        vc[k] = dCacc[4 * jj + k];
      }
      *reinterpret_cast<f32x4*>(q.dB_part + row + 8 * jj + 4 * half) = vb;
      *reinterpret_cast<f32x4*>(q.dC_part + row + 8 * jj + 4 * half) = vc;
    }
  }
}

// ------------------------------------------------------------------ kernel 3: partials -> dB, dC

// out[b, t, g, n] = sum over the nparts head-block partials (fixed order), in the I/O dtype and the caller's strides.
template <typename T>
__global__ __launch_bounds__(256) void ssd_bwd_reduce_kernel(const float* __restrict__ part, int nparts,
                                                             void* out, int64_t sb, int64_t sl, int L, int GN,
                                                             int64_t n4) {
  const int64_t i4 = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i4 >= n4) return;
  const int64_t e = i4 * 4;
  f32x4 v = *reinterpret_cast<const f32x4*>(part + e);
  for (int k = 1; k < nparts; ++k) {
    const f32x4 u = *reinterpret_cast<const f32x4*>(part + (int64_t)k * n4 * 4 + e);
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] += u[j];
  }
  const int64_t row = e / GN;
  const int col = (int)(e - row * GN);
  const int64_t bb = row / L, t = row - bb * L;
  T* o = reinterpret_cast<T*>(out) + bb * sb + t * sl + col;
  if constexpr (sizeof(T) == 2) {
    bf16x4 u;
#pragma unroll
    for (int k = 0; k < 4; ++k) u[k] = (bf16)v[k];
    *reinterpret_cast<bf16x4*>(o) = u;
  } else {
    *reinterpret_cast<f32x4*>(o) = v;
  }
}

// dA, d_dt_bias and dD from the per-(batch, segment, head) partials, summed in a fixed order (deterministic):
// one wave per output, lane k taking partials k, k + 64, ... in order, then a fixed shuffle tree.  Output o < H:
// dA, d_dt_bias, dD (per head) of head o; o = H + h * P + c: dD[h, c] (per channel, both token halves).
__global__ __launch_bounds__(256) void ssd_bwd_param_reduce_kernel(SsdBwdParams q) {
  const SsdParams& p = q.f;
  const int o = blockIdx.x * 4 + wave_id(), l = lane_id();
  const int H = p.nheads, nbs = p.batch * p.nseg;
  if (o < H) {
    float a = 0.f, bi = 0.f, d = 0.f;
    for (int k = l; k < nbs; k += 64) {
      const float* ps = q.part_s + ((int64_t)k * H + o) * 3;
      a += ps[0];
      bi += ps[1];
      d += ps[2];
    }
    a = wave_sum(a);
    bi = wave_sum(bi);
    d = wave_sum(d);
    if (l == 0) {
      q.dA[o] = a;
      if (q.dbias) q.dbias[o] = bi;
      if (q.dD && !p.D_per_channel) q.dD[o] = d;
    }
  } else if (q.dD && p.D_per_channel && o < H + H * HD) {
    const int h = (o - H) / HD, c = (o - H) % HD;
    float d = 0.f;
    for (int k = l; k < 2 * nbs; k += 64) d += q.part_dc[(((int64_t)(k >> 1) * H + h) * 2 + (k & 1)) * HD + c];
    d = wave_sum(d);
    if (l == 0) q.dD[h * HD + c] = d;
  }
}

// ------------------------------------------------------------------ host side

struct BwdWorkspace {
  size_t states, part, ps, pc;
  size_t total() const { return 2 * align256(states) + 2 * align256(part) + align256(ps) + align256(pc); }
};
static BwdWorkspace bwd_workspace(int batch, int seqlen, int nheads, int dstate, int ngroups, int dtype,
                                  int heads_per_wg, int d_per_channel) {
  const int nseg = (seqlen + SEG - 1) / SEG;
  const int nparts = (nheads / ngroups) / heads_per_wg;
  BwdWorkspace w;
  w.states = (size_t)batch * nseg * nheads * HD * dstate * (dtype == DT_BF16 ? sizeof(bf16) : sizeof(float));
  w.part = (size_t)nparts * batch * seqlen * ngroups * dstate * sizeof(float);
  w.ps = (size_t)batch * nseg * nheads * 3 * sizeof(float);
  w.pc = d_per_channel ? (size_t)batch * nseg * nheads * 2 * HD * sizeof(float) : 0;
  return w;
}

size_t ssd_bwd_workspace_bytes(int batch, int seqlen, int nheads, int dstate, int ngroups, int dtype,
                               int heads_per_wg, int d_per_channel) {
  return bwd_workspace(batch, seqlen, nheads, dstate, ngroups, dtype, heads_per_wg, d_per_channel).total();
}

void ssd_bwd_workspace_layout(SsdBwdParams& q, void* workspace) {
  const SsdParams& p = q.f;
  const BwdWorkspace w = bwd_workspace(p.batch, p.seqlen, p.nheads, p.dstate, p.ngroups, p.dtype, q.heads_per_wg,
                                       p.D_per_channel);
  char* c = reinterpret_cast<char*>(workspace);
  q.hin = c;
  c += align256(w.states);
  q.lam = c;
  c += align256(w.states);
  q.dB_part = reinterpret_cast<float*>(c);
  c += align256(w.part);
  q.dC_part = reinterpret_cast<float*>(c);
  c += align256(w.part);
  q.part_s = reinterpret_cast<float*>(c);
  c += align256(w.ps);
  q.part_dc = w.pc ? reinterpret_cast<float*>(c) : nullptr;
}

template <typename T, int N>
static hipError_t launch_bwd_t(const SsdBwdParams& q, hipStream_t st) {
  const SsdParams& p = q.f;
  constexpr int NB = N / 32;
  hipLaunchKernelGGL((ssd_bwd_sweep_kernel<T, N>), dim3(2, (unsigned)p.nheads, (unsigned)p.batch),
                     dim3(64 * (2 * NB + 2)), 0, st, q);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((ssd_bwd_grad_kernel<T, N>),
                     dim3((unsigned)p.nseg, (unsigned)(p.nheads / q.heads_per_wg), (unsigned)p.batch),
                     dim3(128 * NB), 0, st, q);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int GN = p.ngroups * N;
  const int nparts = (p.nheads / p.ngroups) / q.heads_per_wg;
  const int64_t n4 = (int64_t)p.batch * p.seqlen * GN / 4;
  const unsigned nblk = (unsigned)((n4 + 255) / 256);
  hipLaunchKernelGGL((ssd_bwd_reduce_kernel<T>), dim3(nblk), dim3(256), 0, st, q.dB_part, nparts, q.dB, q.dB_sb,
                     q.dB_sl, p.seqlen, GN, n4);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((ssd_bwd_reduce_kernel<T>), dim3(nblk), dim3(256), 0, st, q.dC_part, nparts, q.dC, q.dC_sb,
                     q.dC_sl, p.seqlen, GN, n4);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int nout = p.nheads * (1 + (p.D_per_channel && q.dD ? HD : 0));
  hipLaunchKernelGGL(ssd_bwd_param_reduce_kernel, dim3((unsigned)((nout + 3) / 4)), dim3(256), 0, st, q);
  return hipGetLastError();
}

hipError_t launch_ssd_bwd(const SsdBwdParams& q, hipStream_t st) {
  const SsdParams& p = q.f;
  ZeroRanges z;
  for (int i = 0; i < 5; ++i) { z.p[i] = nullptr; z.n[i] = 0; }
  z.p[0] = q.dA;      z.n[0] = p.nheads;
  z.p[1] = q.dD;      z.n[1] = p.D_per_channel ? (int64_t)p.nheads * HD : p.nheads;
  z.p[2] = q.dbias;   z.n[2] = p.nheads;
  hipLaunchKernelGGL(ssd_bwd_zero_kernel, dim3(1, 3), dim3(256), 0, st, z);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (p.nseg == 0) {
    if (!q.dh0) return hipSuccess;
    const size_t n = (size_t)p.batch * p.nheads * HD * p.dstate;
    hipLaunchKernelGGL(ssd_bwd_copy_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, q.d_final, q.dh0, n);
    return hipGetLastError();
  }
  if (p.dtype == DT_BF16) {
    if (p.dstate == 128) return launch_bwd_t<bf16, 128>(q, st);
    if (p.dstate == 64) return launch_bwd_t<bf16, 64>(q, st);
  } else {
    if (p.dstate == 128) return launch_bwd_t<float, 128>(q, st);
    if (p.dstate == 64) return launch_bwd_t<float, 64>(q, st);
  }
  return hipErrorInvalidValue;
}

}  // namespace mh
