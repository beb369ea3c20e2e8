// Mamba-2 SSD chunked-scan prefill for gfx950.
//
// Recurrence (per batch b, head h with group g = h / (H/G), channel p, state n):
//     h_t = exp(A_h dt_t) h_{t-1} + dt_t x_t[p] B_t[g, n]
//     y_t[p] = sum_n C_t[g, n] h_t[p, n] + D x_t[p]
// i.e. the reference's selective_scan (mamformer/layers/mamba2.py:84-126) in the
// per-head SSD parameterisation, with an optional initial state (prefill of a
// cached sequence) and the final state returned for the decode cache.
//
// Decomposition (three launches on the caller's stream):
//   1. ssd_chunk_state  grid (nchunks, H/HG, b): for each state chunk of
//      `chunk_len` tokens the chunk-local final state
//          S_k[p, n] = sum_{s in k} exp(sum_{s<tau in k} A dt_tau) dt_s x_s[p] B_s[n]
//      as an MFMA reduction over tokens, plus the chunk's total log-decay.
//   2. ssd_state_pass   elementwise over (b, h, P*N): H_0 = h0, H_{k+1} = e^{T_k} H_k + S_k.
//      Writes the *entering* state H_k over S_k and the final state.
//   3. ssd_chunk_scan   grid (nchunks, H/HG, b): one wave per head walks its
//      state chunk in segments of <= 64 tokens, keeping the running state
//      H (P x N fp32) in MFMA accumulator registers:
//          Y  = [C B^T o mask] (e^{m - cs} dt x)          intra-segment (factored decay)
//             + C (e^{m} H)^T                              carried state
//          y  = e^{cs_t - m} Y + D x
//          H <- e^{cs_end} H + B^T (e^{cs_end - cs} dt x)
//      cs is the in-segment inclusive cumsum of A*dt and m the midpoint of its
//      range.  The factorisation exp(cs_t - cs_s) = e^{cs_t - m} e^{m - cs_s} is
//      exact; segments are cut short whenever the range of cs would exceed
//      RANGE so no factor leaves [e^-RANGE/2, e^RANGE/2] (a single token always
//      qualifies), which keeps the fast form valid for any decay.
// C B^T is computed once per segment and shared by the HG heads of a group.
// All contractions are 32x32x16 bf16 MFMAs (bf16 I/O) or 32x32x2 fp32 MFMAs
// (fp32 I/O); accumulation is fp32 everywhere.
#include "common.h"
#include "launch.h"

namespace mh {

constexpr int SEG = 64;         // tokens per segment (max)
constexpr int HD = 64;          // headdim handled by these kernels
constexpr float RANGE = 80.f;   // max spread of in-segment cumsum for the factored form

// ------------------------------------------------------------------ helpers

// Reverse inclusive prefix sum over the 64 lanes: r_l = sum_{i >= l} v_i.
__device__ __forceinline__ float wave_incl_rscan(float v) {
  const int l = lane_id();
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    float o = __shfl_down(v, off, 64);
    if (l + off < 64) v += o;
  }
  return v;
}
__device__ __forceinline__ float wave_prefix_max(float v) {
  const int l = lane_id();
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    float o = __shfl_up(v, off, 64);
    if (l >= off) v = fmaxf(v, o);
  }
  return v;
}
__device__ __forceinline__ float wave_prefix_min(float v) {
  const int l = lane_id();
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    float o = __shfl_up(v, off, 64);
    if (l >= off) v = fminf(v, o);
  }
  return v;
}

__device__ __forceinline__ float process_dt(const SsdParams& p, float dt, int h) {
  if (p.dt_bias) dt += p.dt_bias[h];
  if (p.dt_softplus) dt = softplus_f(dt);
  if (p.has_dt_limit) dt = fminf(fmaxf(dt, p.dt_min), p.dt_max);
  return dt;
}

// Copy `rows` rows of `W` elements (16-byte vectors) from global into LDS with
// a padded pitch; rows whose token index is >= lim are zero-filled.
template <typename T, int W, int PITCH>
__device__ __forceinline__ void load_rows(T* dst, const T* src, int64_t row_stride, int tok0, int lim,
                                          int tid, int nthreads) {
  constexpr int VPR = W * (int)sizeof(T) / 16;   // 16-byte vectors per row
  for (int e = tid; e < SEG * VPR; e += nthreads) {
    const int r = e / VPR, v = e - r * VPR;
    uint4 val = make_uint4(0, 0, 0, 0);
    if (tok0 + r < lim)
      val = *reinterpret_cast<const uint4*>(src + (int64_t)(tok0 + r) * row_stride + v * (16 / (int)sizeof(T)));
    *reinterpret_cast<uint4*>(dst + r * PITCH + v * (16 / (int)sizeof(T))) = val;
  }
}

// Fragment of 8 consecutive elements of an LDS row (canonical k mapping).
template <typename TM, typename T>
__device__ __forceinline__ Frag<TM> row_frag(const T* row) {
  Frag<TM> f;
#pragma unroll
  for (int j = 0; j < 8; ++j) f.set(j, to_f32(row[j]));
  return f;
}
// Fragment with the KSET mapping: elements base+4*half+{0..3} and base+8+4*half+{0..3}.
template <typename TM, typename T>
__device__ __forceinline__ Frag<TM> kset_frag(const T* row, int half) {
  Frag<TM> f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    f.set(j, to_f32(row[4 * half + j]));
    f.set(4 + j, to_f32(row[8 + 4 * half + j]));
  }
  return f;
}

template <typename T, typename TM, int N, int HG>
struct ScanSmem {
  static constexpr int PB = N + 16 / (int)sizeof(T);     // padded pitch of B/C rows
  static constexpr int PX = HD + 16 / (int)sizeof(T);    // padded pitch of x rows
  T B[SEG * PB];
  T C[SEG * PB];
  T X[HG][SEG * PX];
  Frag<TM> CB[3][2][64];        // masked (C B^T)^T as MFMA B-operand fragments: tile, k-step, lane
  Frag<TM> Bt[N / 32][4][64];   // B^T as MFMA A-operand fragments: n-tile, s-step, lane
  float cs[HG][SEG];
  float sa[HG][SEG];            // e^{m - cs_s} dt_s   (intra operand scale)
  float ss[HG][SEG];            // e^{cs_end - cs_s} dt_s (state operand scale)
  int len[HG];
};

template <typename T, typename TM, int N, int HG>
struct StateSmem {
  static constexpr int PB = N + 16 / (int)sizeof(T);
  static constexpr int PX = HD + 16 / (int)sizeof(T);
  T B[SEG * PB];
  T X[HG][SEG * PX];
  Frag<TM> Bt[N / 32][4][64];
  float w[HG][SEG];
};

// Build B^T A-operand fragments (row n, k = s with the KSET mapping) from the B tile.
template <typename T, typename TM, int N, int PB>
__device__ __forceinline__ void build_bt(Frag<TM> (*Bt)[4][64], const T* Bs, int tid, int nthreads) {
  for (int e = tid; e < (N / 32) * 4 * 64; e += nthreads) {
    const int ln = e & 63, c = (e >> 6) & 3, nt = e >> 8;
    const int n = 32 * nt + (ln & 31), hf = ln >> 5;
    Frag<TM> f;
#pragma unroll
    for (int j = 0; j < 8; ++j) f.set(j, to_f32(Bs[(16 * c + kset(hf, j)) * PB + n]));
    Bt[nt][c][ln] = f;
  }
}

// ------------------------------------------------------------------ kernel 1

template <typename T, typename TM, int N, int HG>
__global__ __launch_bounds__(64 * HG) void ssd_chunk_state_kernel(SsdParams p) {
  using SM = StateSmem<T, TM, N, HG>;
  __shared__ SM sm;
  constexpr int NT = N / 32;
  const int k = blockIdx.x, b = blockIdx.z;
  const int w = wave_id(), l = lane_id(), half = l >> 5, l32 = l & 31;
  const int h = blockIdx.y * HG + w;
  const int g = h / (p.nheads / p.ngroups);
  const int c0 = k * p.chunk_len;
  const int c1 = min(p.seqlen, c0 + p.chunk_len);
  const float Ah = p.A[h];
  const T* xg = reinterpret_cast<const T*>(p.x) + (int64_t)b * p.x_sb + (int64_t)h * p.x_sh;
  const T* Bg = reinterpret_cast<const T*>(p.B) + (int64_t)b * p.B_sb + (int64_t)g * N;
  const float* dtg = p.dt + (int64_t)b * p.dt_sb + h;

  f32x16 acc[NT][2];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) { acc[nt][0] = zero16(); acc[nt][1] = zero16(); }

  // Walk the chunk backwards so the decay to the chunk end is a running suffix sum.
  float suffix = 0.f;
  const int nseg = (c1 - c0 + SEG - 1) / SEG;
  for (int si = nseg - 1; si >= 0; --si) {
    const int pos = c0 + si * SEG;
    const int t = pos + l;
    float dtv = 0.f;
    if (t < c1) dtv = process_dt(p, dtg[(int64_t)t * p.dt_sl], h);
    const float a = Ah * dtv;
    const float rs = wave_incl_rscan(a);                 // sum_{i >= l} a_i within segment
    float ex = __shfl_down(rs, 1, 64);                    // sum_{i > l}
    if (l == 63) ex = 0.f;
    sm.w[w][l] = __expf(ex + suffix) * dtv;
    suffix += __shfl(rs, 0, 64);

    load_rows<T, N, SM::PB>(sm.B, Bg, p.B_sl, pos, c1, threadIdx.x, 64 * HG);
    load_rows<T, HD, SM::PX>(sm.X[w], xg, p.x_sl, pos, c1, l, 64);
    __syncthreads();
    build_bt<T, TM, N, SM::PB>(sm.Bt, sm.B, threadIdx.x, 64 * HG);
    // x~'[s][p] = w_s x[s][p] as B-operand fragments (col p, k = s via KSET)
    Frag<TM> xs[2][4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int s = 16 * c + kset(half, j);
        const float ws = sm.w[w][s];
#pragma unroll
        for (int pt = 0; pt < 2; ++pt) xs[pt][c].set(j, ws * to_f32(sm.X[w][s * SM::PX + 32 * pt + l32]));
      }
    }
    __syncthreads();
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const Frag<TM> bt = sm.Bt[nt][c][l];
        acc[nt][0] = mma(bt, xs[0][c], acc[nt][0]);
        acc[nt][1] = mma(bt, xs[1][c], acc[nt][1]);
      }
    __syncthreads();
  }

  float* out = p.chunk_states + (((int64_t)b * p.nchunks + k) * p.nheads + h) * (HD * N);
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int pt = 0; pt < 2; ++pt)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = 32 * nt + 8 * q + 4 * half, pc = 32 * pt + l32;
        float4 v = make_float4(acc[nt][pt][4 * q], acc[nt][pt][4 * q + 1], acc[nt][pt][4 * q + 2],
                               acc[nt][pt][4 * q + 3]);
        *reinterpret_cast<float4*>(out + pc * N + n) = v;
      }
  if (l == 0) p.chunk_decay[((int64_t)b * p.nheads + h) * p.nchunks + k] = suffix;
}

// ------------------------------------------------------------------ kernel 2

__global__ __launch_bounds__(256) void ssd_state_pass_kernel(SsdParams p) {
  const int bh = blockIdx.y;
  const int b = bh / p.nheads, h = bh - b * p.nheads;
  const int per = HD * p.dstate;                  // state elements per (b, h)
  const int e4 = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (e4 >= per) return;
  float4 H = make_float4(0.f, 0.f, 0.f, 0.f);
  if (p.init_state) H = *reinterpret_cast<const float4*>(p.init_state + (int64_t)bh * per + e4);
  const float* dec = p.chunk_decay + (int64_t)bh * p.nchunks;
  for (int k = 0; k < p.nchunks; ++k) {
    float* sp = p.chunk_states + (((int64_t)b * p.nchunks + k) * p.nheads + h) * per + e4;
    const float4 S = *reinterpret_cast<const float4*>(sp);
    *reinterpret_cast<float4*>(sp) = H;
    const float a = __expf(dec[k]);
    H.x = a * H.x + S.x;
    H.y = a * H.y + S.y;
    H.z = a * H.z + S.z;
    H.w = a * H.w + S.w;
  }
  if (p.final_state) *reinterpret_cast<float4*>(p.final_state + (int64_t)bh * per + e4) = H;
}

// ------------------------------------------------------------------ kernel 3

template <typename T, typename TM, int N, int HG>
__global__ __launch_bounds__(64 * HG) void ssd_chunk_scan_kernel(SsdParams p) {
  using SM = ScanSmem<T, TM, N, HG>;
  __shared__ SM sm;
  constexpr int NT = N / 32;
  const int k = blockIdx.x, b = blockIdx.z;
  const int w = wave_id(), l = lane_id(), half = l >> 5, l32 = l & 31;
  const int h = blockIdx.y * HG + w;
  const int g = h / (p.nheads / p.ngroups);
  const int c0 = k * p.chunk_len;
  const int c1 = min(p.seqlen, c0 + p.chunk_len);
  const float Ah = p.A[h];
  const T* xg = reinterpret_cast<const T*>(p.x) + (int64_t)b * p.x_sb + (int64_t)h * p.x_sh;
  const T* Bg = reinterpret_cast<const T*>(p.B) + (int64_t)b * p.B_sb + (int64_t)g * N;
  const T* Cg = reinterpret_cast<const T*>(p.C) + (int64_t)b * p.C_sb + (int64_t)g * N;
  const float* dtg = p.dt + (int64_t)b * p.dt_sb + h;
  T* yg = reinterpret_cast<T*>(p.y) + (int64_t)b * p.y_sb + (int64_t)h * p.y_sh;
  const float Dh = (p.D && !p.D_per_channel) ? p.D[h] : 0.f;

  // Entering state H_k in accumulator layout: tile (nt, pt) of H^T[n][p].
  f32x16 H[NT][2];
  {
    const float* hk = p.chunk_states + (((int64_t)b * p.nchunks + k) * p.nheads + h) * (HD * N);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int pt = 0; pt < 2; ++pt)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int n = 32 * nt + 8 * q + 4 * half, pc = 32 * pt + l32;
          const float4 v = *reinterpret_cast<const float4*>(hk + pc * N + n);
          H[nt][pt][4 * q] = v.x;
          H[nt][pt][4 * q + 1] = v.y;
          H[nt][pt][4 * q + 2] = v.z;
          H[nt][pt][4 * q + 3] = v.w;
        }
  }

  for (int pos = c0; pos < c1;) {
    // ---- per wave: dt, in-segment cumsum, longest admissible prefix
    const int t = pos + l;
    float dtv = 0.f;
    if (t < c1) dtv = process_dt(p, dtg[(int64_t)t * p.dt_sl], h);
    const float cs = wave_incl_scan(Ah * dtv);
    const float pmax = wave_prefix_max(cs), pmin = wave_prefix_min(cs);
    const bool ok = (pmax - pmin <= RANGE) && (t < c1);
    const uint64_t bal = __ballot(ok);
    const int len_w = (~bal == 0ull) ? 64 : __builtin_ctzll(~bal);
    sm.cs[w][l] = cs;
    if (l == 0) sm.len[w] = len_w;

    // ---- tiles: B, C (shared by the group), x (per head)
    load_rows<T, N, SM::PB>(sm.B, Bg, p.B_sl, pos, p.seqlen, threadIdx.x, 64 * HG);
    load_rows<T, N, SM::PB>(sm.C, Cg, p.C_sl, pos, p.seqlen, threadIdx.x, 64 * HG);
    load_rows<T, HD, SM::PX>(sm.X[w], xg, p.x_sl, pos, p.seqlen, l, 64);
    __syncthreads();

    int len = sm.len[0];
#pragma unroll
    for (int i = 1; i < HG; ++i) len = min(len, sm.len[i]);
    const float mx = __shfl(pmax, len - 1, 64), mn = __shfl(pmin, len - 1, 64);
    const float m = 0.5f * (mx + mn);
    const float cs_end = __shfl(cs, len - 1, 64);
    sm.sa[w][l] = (l < len) ? __expf(m - cs) * dtv : 0.f;
    sm.ss[w][l] = (l < len) ? __expf(cs_end - cs) * dtv : 0.f;

    // ---- masked (C B^T)^T tiles (s-tile, t-tile) in {(0,0), (0,1), (1,1)}, shared by the heads
    for (int ti = w; ti < 3; ti += HG) {
      const int st = (ti == 2) ? 1 : 0, tt = (ti == 0) ? 0 : 1;
      f32x16 acc = zero16();
#pragma unroll
      for (int c = 0; c < N / 16; ++c) {
        const Frag<TM> a = row_frag<TM>(sm.B + (32 * st + l32) * SM::PB + 16 * c + 8 * half);
        const Frag<TM> bb = row_frag<TM>(sm.C + (32 * tt + l32) * SM::PB + 16 * c + 8 * half);
        acc = mma(a, bb, acc);
      }
      const int tl = 32 * tt + l32;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int s = 32 * st + acc_row(half, r);
        if (!(s <= tl && s < len)) acc[r] = 0.f;
      }
      sm.CB[ti][0][l] = acc_to_frag<TM>(acc, 0);
      sm.CB[ti][1][l] = acc_to_frag<TM>(acc, 1);
    }
    build_bt<T, TM, N, SM::PB>(sm.Bt, sm.B, threadIdx.x, 64 * HG);
    __syncthreads();

    // ---- per wave (head): operand fragments of x~ = e^{m-cs} dt x and x~' = e^{cs_end-cs} dt x
    Frag<TM> xa[2][4], xs[2][4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int s = 16 * c + kset(half, j);
        const float fa = sm.sa[w][s], fs = sm.ss[w][s];
#pragma unroll
        for (int pt = 0; pt < 2; ++pt) {
          const float xv = to_f32(sm.X[w][s * SM::PX + 32 * pt + l32]);
          xa[pt][c].set(j, fa * xv);
          xs[pt][c].set(j, fs * xv);
        }
      }
    }

    // ---- Y^T[p][t]: intra-segment part
    f32x16 Y[2][2];
#pragma unroll
    for (int pt = 0; pt < 2; ++pt) {
      f32x16 y0 = zero16(), y1 = zero16();
      y0 = mma(xa[pt][0], sm.CB[0][0][l], y0);
      y0 = mma(xa[pt][1], sm.CB[0][1][l], y0);
      y1 = mma(xa[pt][0], sm.CB[1][0][l], y1);
      y1 = mma(xa[pt][1], sm.CB[1][1][l], y1);
      y1 = mma(xa[pt][2], sm.CB[2][0][l], y1);
      y1 = mma(xa[pt][3], sm.CB[2][1][l], y1);
      Y[pt][0] = y0;
      Y[pt][1] = y1;
    }
    // ---- carried state: Y^T += (e^m H) C^T
    const float em = __expf(m);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const Frag<TM> h0 = acc_to_frag_scaled<TM>(H[nt][0], c, em);
        const Frag<TM> h1 = acc_to_frag_scaled<TM>(H[nt][1], c, em);
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
          const Frag<TM> cf = kset_frag<TM>(sm.C + (32 * tt + l32) * SM::PB + 32 * nt + 16 * c, half);
          Y[0][tt] = mma(h0, cf, Y[0][tt]);
          Y[1][tt] = mma(h1, cf, Y[1][tt]);
        }
      }
    // ---- output y[t][p] = e^{cs_t - m} Y + D x
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int tl = 32 * tt + l32;
      if (tl < len) {
        const float rsc = __expf(sm.cs[w][tl] - m);
        T* yrow = yg + (int64_t)(pos + tl) * p.y_sl;
        const T* xrow = sm.X[w] + tl * SM::PX;
#pragma unroll
        for (int pt = 0; pt < 2; ++pt)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int p0 = 32 * pt + 8 * q + 4 * half;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const float dd = p.D ? (p.D_per_channel ? p.D[h * HD + p0 + i] : Dh) : 0.f;
              yrow[p0 + i] = from_f32<T>(rsc * Y[pt][tt][4 * q + i] + dd * to_f32(xrow[p0 + i]));
            }
          }
      }
    }
    // ---- state update: H <- e^{cs_end} H + B^T x~'
    const float ae = __expf(cs_end);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int pt = 0; pt < 2; ++pt) {
        f32x16 acc = H[nt][pt] * ae;
#pragma unroll
        for (int c = 0; c < 4; ++c) acc = mma(sm.Bt[nt][c][l], xs[pt][c], acc);
        H[nt][pt] = acc;
      }
    __syncthreads();
    pos += len;
  }
}

// ------------------------------------------------------------------ launch

size_t ssd_workspace_bytes(int batch, int nchunks, int nheads, int headdim, int dstate) {
  const size_t states = (size_t)batch * nchunks * nheads * headdim * dstate * sizeof(float);
  const size_t decay = (size_t)batch * nheads * nchunks * sizeof(float);
  return ((states + 255) / 256) * 256 + ((decay + 255) / 256) * 256;
}

template <typename T, typename TM, int N, int HG>
static hipError_t launch_ssd_t(const SsdParams& p, hipStream_t st) {
  dim3 grid((unsigned)p.nchunks, (unsigned)(p.nheads / HG), (unsigned)p.batch);
  hipLaunchKernelGGL((ssd_chunk_state_kernel<T, TM, N, HG>), grid, dim3(64 * HG), 0, st, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int per4 = HD * N / 4;
  dim3 g2((unsigned)((per4 + 255) / 256), (unsigned)(p.batch * p.nheads));
  hipLaunchKernelGGL(ssd_state_pass_kernel, g2, dim3(256), 0, st, p);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((ssd_chunk_scan_kernel<T, TM, N, HG>), grid, dim3(64 * HG), 0, st, p);
  return hipGetLastError();
}

template <typename T, typename TM, int N>
static hipError_t launch_ssd_n(const SsdParams& p, hipStream_t st) {
  switch (p.heads_per_wg) {
    case 4:
      if constexpr (sizeof(T) == 4 && N == 128) return hipErrorInvalidValue;  // exceeds LDS
      else return launch_ssd_t<T, TM, N, 4>(p, st);
    case 2: return launch_ssd_t<T, TM, N, 2>(p, st);
    case 1: return launch_ssd_t<T, TM, N, 1>(p, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_ssd(const SsdParams& p, hipStream_t st) {
  if (p.nchunks == 0) {
    // Empty sequence: the final state is the initial state.
    if (!p.final_state) return hipSuccess;
    const size_t bytes = (size_t)p.batch * p.nheads * HD * p.dstate * sizeof(float);
    if (p.init_state) return hipMemcpyAsync(p.final_state, p.init_state, bytes, hipMemcpyDeviceToDevice, st);
    return hipMemsetAsync(p.final_state, 0, bytes, st);
  }
  if (p.dtype == DT_BF16) {
    if (p.dstate == 128) return launch_ssd_n<bf16, bf16, 128>(p, st);
    if (p.dstate == 64) return launch_ssd_n<bf16, bf16, 64>(p, st);
  } else {
    if (p.dstate == 128) return launch_ssd_n<float, float, 128>(p, st);
    if (p.dstate == 64) return launch_ssd_n<float, float, 64>(p, st);
  }
  return hipErrorInvalidValue;
}

}  // namespace mh
