// Causal depthwise conv1d (+ optional SiLU) over channels-last (b, L, D) input
// for gfx950: the Mamba layer prologue in front of the SSD scan.
//
//   y[b, t, d] = act( bias[d] + sum_{j<K} w[d, j] * xin[b, t - (K-1) + j, d] )
//   xin[b, t', d] = x[b, t', d]                      for t' >= 0
//                 = conv_state[b, S_c + t', d]       for -S_c <= t' < 0
//                 = 0                                otherwise
// which is the reference's _causal_conv1d (mamformer/layers/mamba2.py:370-405):
// left zero padding of K-1, cross-correlation with the (D, 1, K) depthwise
// weight, and the cached raw inputs (S_c <= K-1 rows) prepended on the
// incremental path.
//
// Bandwidth-bound: each thread owns 8 consecutive channels (one 16-byte bf16
// vector) and a run of TT tokens, keeping the K-row window in registers, so x
// is read once (plus a K-1 row halo per run) and y written once.
#include "common.h"
#include "launch.h"

namespace mh {

namespace {

constexpr int CV = 8;      // channels per thread
constexpr int TT = 32;     // tokens per thread in the backward (one dweight/dbias partial per run)
constexpr int TTF = 32;    // tokens per thread in the forward (four row groups; 16 and 8 measured slower)
constexpr int KMAX = 8;

template <typename T>
__device__ __forceinline__ void load8(const T* p, float (&v)[CV]) {
  if constexpr (sizeof(T) == 2) {
    const bf16x8 r = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
    for (int i = 0; i < CV; ++i) v[i] = (float)r[i];
  } else {
    const f32x4 a = *reinterpret_cast<const f32x4*>(p);
    const f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) { v[i] = a[i]; v[4 + i] = b[i]; }
  }
}
template <typename T>
__device__ __forceinline__ void store8(T* p, const float (&v)[CV]) {
  if constexpr (sizeof(T) == 2) {
    bf16x8 r;
#pragma unroll
    for (int i = 0; i < CV; ++i) r[i] = (bf16)v[i];
    *reinterpret_cast<bf16x8*>(p) = r;
  } else {
    f32x4 a, b;
#pragma unroll
    for (int i = 0; i < 4; ++i) { a[i] = v[i]; b[i] = v[4 + i]; }
    *reinterpret_cast<f32x4*>(p) = a;
    *reinterpret_cast<f32x4*>(p + 4) = b;
  }
}

// A row of 8 channels as loaded (converted to fp32 when used), so that a group of rows can be in flight at once:
// a run walks its tokens in order, and one load per step would put the full memory latency on every token.
template <typename T> struct Raw8;
template <> struct Raw8<bf16> { bf16x8 v; };
template <> struct Raw8<float> { f32x4 a, b; };
template <typename T>
__device__ __forceinline__ Raw8<T> ldraw(const T* p) {
  Raw8<T> r;
  if constexpr (sizeof(T) == 2) {
    r.v = *reinterpret_cast<const bf16x8*>(p);
  } else {
    r.a = *reinterpret_cast<const f32x4*>(p);
    r.b = *reinterpret_cast<const f32x4*>(p + 4);
  }
  return r;
}
template <typename T>
__device__ __forceinline__ void cvt8(const Raw8<T>& r, float (&v)[CV]) {
  if constexpr (sizeof(T) == 2) {
#pragma unroll
    for (int i = 0; i < CV; ++i) v[i] = (float)r.v[i];
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) { v[i] = r.a[i]; v[4 + i] = r.b[i]; }
  }
}

// The K-1 window rows before t0 (rows of x, the cached rows before the sequence, or 0), loaded together: each row's
// source is chosen by address and the row masked by a factor afterwards, so that no load waits behind a branch.
template <typename T, int K>
__device__ __forceinline__ void load_halo(const Conv1dParams& p, const T* xb, const T* sb, int t0,
                                          float (&win)[K][CV]) {
  constexpr int NH = K > 1 ? K - 1 : 1;
  Raw8<T> hr[NH];
  float hm[NH];
#pragma unroll
  for (int j = 0; j < K - 1; ++j) {
    const int tp = t0 - (K - 1) + j;
    const bool inx = tp >= 0, ins = !inx && sb && tp >= -p.cs_len;
    const T* src = inx ? xb + (int64_t)tp * p.x_sl : ins ? sb + (int64_t)(p.cs_len + tp) * p.cs_sl : xb;
    hm[j] = (inx || ins) ? 1.f : 0.f;
    hr[j] = ldraw<T>(src);
  }
#pragma unroll
  for (int j = 0; j < K - 1; ++j) {
    cvt8<T>(hr[j], win[j]);
#pragma unroll
    for (int i = 0; i < CV; ++i) win[j][i] *= hm[j];
  }
}
constexpr int RG = 8;      // rows loaded together

template <typename T, int K>
__global__ __launch_bounds__(256) void conv1d_kernel(Conv1dParams p) {
  const int c8 = blockIdx.x * 256 + threadIdx.x;
  const int d0 = c8 * CV;
  if (d0 >= p.dim) return;
  const int b = blockIdx.z;
  const int t0 = blockIdx.y * TTF;
  const T* xb = reinterpret_cast<const T*>(p.x) + (int64_t)b * p.x_sb + d0;
  const T* sb = p.conv_state ? reinterpret_cast<const T*>(p.conv_state) + (int64_t)b * p.cs_sb + d0 : nullptr;
  T* yb = reinterpret_cast<T*>(p.y) + (int64_t)b * p.y_sb + d0;

  float w[K][CV];
#pragma unroll
  for (int i = 0; i < CV; ++i)
#pragma unroll
    for (int j = 0; j < K; ++j) w[j][i] = p.weight[(int64_t)(d0 + i) * K + j];
  float bias[CV];
#pragma unroll
  for (int i = 0; i < CV; ++i) bias[i] = p.bias ? p.bias[d0 + i] : 0.f;

  // window rows t0-K+1 .. t0-1 (win[j] holds xin[t - (K-1) + j] for the next output t)
  float win[K][CV];
  load_halo<T, K>(p, xb, sb, t0, win);
  const int t1 = min(p.seqlen, t0 + TTF);
  auto emit = [&](int t) {               // win[K-1] holds row t
    float o[CV];
#pragma unroll
    for (int i = 0; i < CV; ++i) {
      float acc = bias[i];
#pragma unroll
      for (int j = 0; j < K; ++j) acc += w[j][i] * win[j][i];
      o[i] = p.silu ? silu_f(acc) : acc;
    }
    store8<T>(yb + (int64_t)t * p.y_sl, o);
#pragma unroll
    for (int j = 0; j < K - 1; ++j)
#pragma unroll
      for (int i = 0; i < CV; ++i) win[j][i] = win[j + 1][i];
  };
  int t = t0;
  for (; t + RG <= t1; t += RG) {
    Raw8<T> rx[RG];
#pragma unroll
    for (int r = 0; r < RG; ++r) rx[r] = ldraw<T>(xb + (int64_t)(t + r) * p.x_sl);
#pragma unroll
    for (int r = 0; r < RG; ++r) {
      cvt8<T>(rx[r], win[K - 1]);
      emit(t + r);
    }
  }
  for (; t < t1; ++t) {
    load8<T>(xb + (int64_t)t * p.x_sl, win[K - 1]);
    emit(t);
  }
}

// Backward: with u = bias + sum_j w_j xin[t - (K-1) + j] (recomputed) and du = dy * act'(u),
//   dx[s] = sum_j w_j du[s + (K-1) - j],   dw_j += du[t] xin[t - (K-1) + j],   dbias += du[t].
// A thread owns 8 channels and the TT tokens of its run for dx, dw and dbias, and recomputes du on the K-1
// tokens after the run (the halo dx needs); the threads of run 0 also write the cached rows' gradient
//   d_conv_state[S_c + s] = sum_j w_j du[s + (K-1) - j]  (s = -S_c .. -1)  when it is asked for.
// dw / dbias leave as one fp32 partial per (batch, run), summed in a fixed order by conv1d_reduce_kernel.
template <typename T, int K>
__global__ __launch_bounds__(256) void conv1d_bwd_kernel(Conv1dBwdParams q) {
  const Conv1dParams& p = q.f;
  const int c8 = blockIdx.x * 256 + threadIdx.x;
  const int d0 = c8 * CV;
  if (d0 >= p.dim) return;
  const int b = blockIdx.z;
  const int t0 = blockIdx.y * TT;
  const T* xb = reinterpret_cast<const T*>(p.x) + (int64_t)b * p.x_sb + d0;
  const T* sb = p.conv_state ? reinterpret_cast<const T*>(p.conv_state) + (int64_t)b * p.cs_sb + d0 : nullptr;
  const T* dyb = reinterpret_cast<const T*>(q.dy) + (int64_t)b * q.dy_sb + d0;
  T* dxb = reinterpret_cast<T*>(q.dx) + (int64_t)b * q.dx_sb + d0;

  float w[K][CV];
#pragma unroll
  for (int i = 0; i < CV; ++i)
#pragma unroll
    for (int j = 0; j < K; ++j) w[j][i] = p.weight[(int64_t)(d0 + i) * K + j];
  float bias[CV];
#pragma unroll
  for (int i = 0; i < CV; ++i) bias[i] = p.bias ? p.bias[d0 + i] : 0.f;

  float win[K][CV];       // win[j] = xin[t - (K-1) + j] for the current t
  load_halo<T, K>(p, xb, sb, t0, win);
  float duw[K][CV];       // duw[K-1-j] = du[t - j]
#pragma unroll
  for (int j = 0; j < K; ++j)
#pragma unroll
    for (int i = 0; i < CV; ++i) duw[j][i] = 0.f;
  float dw[K][CV], db[CV];
#pragma unroll
  for (int i = 0; i < CV; ++i) {
    db[i] = 0.f;
#pragma unroll
    for (int j = 0; j < K; ++j) dw[j][i] = 0.f;
  }
  const int tend = min(p.seqlen, t0 + TT);          // this run's tokens: [t0, tend)
  const int tlast = min(p.seqlen, tend + K - 1);    // du needed up to tlast - 1
  // gradient rows this thread stores: [slo, tend); run 0 also owns the cached rows -cs_len .. -1
  const int slo = (t0 == 0 && q.dcs) ? -p.cs_len : t0;
  T* dcsb = q.dcs ? reinterpret_cast<T*>(q.dcs) + (int64_t)b * q.dcs_sb + d0 : nullptr;
  auto row = [&](int s) { return s >= 0 ? dxb + (int64_t)s * q.dx_sl : dcsb + (int64_t)(p.cs_len + s) * q.dcs_sl; };
  auto step = [&](int t, const float (&g)[CV]) {   // win[K-1] holds x row t, g the output gradient of row t
    float du[CV];
#pragma unroll
    for (int i = 0; i < CV; ++i) {
      float u = bias[i];
#pragma unroll
      for (int j = 0; j < K; ++j) u += w[j][i] * win[j][i];
      if (p.silu) {
        const float sg = sigmoid_f(u);
        du[i] = g[i] * sg * (1.f + u * (1.f - sg));
      } else {
        du[i] = g[i];
      }
    }
    if (t < tend) {
#pragma unroll
      for (int i = 0; i < CV; ++i) {
        db[i] += du[i];
#pragma unroll
        for (int j = 0; j < K; ++j) dw[j][i] += du[i] * win[j][i];
      }
    }
#pragma unroll
    for (int j = 0; j < K - 1; ++j)
#pragma unroll
      for (int i = 0; i < CV; ++i) {
        duw[j][i] = duw[j + 1][i];
        win[j][i] = win[j + 1][i];
      }
#pragma unroll
    for (int i = 0; i < CV; ++i) duw[K - 1][i] = du[i];
    const int s = t - (K - 1);
    if (s >= slo) {
      float o[CV];
#pragma unroll
      for (int i = 0; i < CV; ++i) {
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < K; ++j) acc += w[j][i] * duw[K - 1 - j][i];
        o[i] = acc;
      }
      store8<T>(row(s), o);
    }
  };
  int t = t0;
  for (; t + RG <= tlast; t += RG) {
    Raw8<T> rx[RG], rg[RG];
#pragma unroll
    for (int r = 0; r < RG; ++r) {
      rx[r] = ldraw<T>(xb + (int64_t)(t + r) * p.x_sl);
      rg[r] = ldraw<T>(dyb + (int64_t)(t + r) * q.dy_sl);
    }
#pragma unroll
    for (int r = 0; r < RG; ++r) {
      float g[CV];
      cvt8<T>(rx[r], win[K - 1]);
      cvt8<T>(rg[r], g);
      step(t + r, g);
    }
  }
  for (; t < tlast; ++t) {
    float g[CV];
    load8<T>(xb + (int64_t)t * p.x_sl, win[K - 1]);
    load8<T>(dyb + (int64_t)t * q.dy_sl, g);
    step(t, g);
  }
  // rows whose du window runs past the sequence end (du = 0 there).  The window advances one zero per s
  // from s = tlast - (K-1) (the first s the main loop did not emit), so its last slot is du[s + K - 1]
  // even when that s lies before slo (runs shorter than K - 1 tokens).
  for (int s = tlast - (K - 1); s < tend; ++s) {
#pragma unroll
    for (int j = 0; j < K - 1; ++j)
#pragma unroll
      for (int i = 0; i < CV; ++i) duw[j][i] = duw[j + 1][i];
#pragma unroll
    for (int i = 0; i < CV; ++i) duw[K - 1][i] = 0.f;
    if (s < slo) continue;
    float o[CV];
#pragma unroll
    for (int i = 0; i < CV; ++i) {
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < K; ++j) acc += w[j][i] * duw[K - 1 - j][i];
      o[i] = acc;
    }
    store8<T>(row(s), o);
  }
  const int64_t part = (int64_t)b * gridDim.y + blockIdx.y;
#pragma unroll
  for (int i = 0; i < CV; ++i) {
    q.db_part[part * p.dim + d0 + i] = db[i];
#pragma unroll
    for (int j = 0; j < K; ++j) q.dw_part[(part * p.dim + d0 + i) * K + j] = dw[j][i];
  }
}

// dweight (D, K) and dbias (D,) = sums over the nparts partials, in a fixed order: 64 outputs per workgroup, each
// output's partials split over 4 slices of the workgroup (partial k to slice k % 4), the slices added in order.
__global__ __launch_bounds__(256) void conv1d_reduce_kernel(const float* __restrict__ dw_part,
                                                            const float* __restrict__ db_part, int nparts, int dim,
                                                            int K, float* __restrict__ dw, float* __restrict__ db) {
  __shared__ float red[4][64];
  const int lo = threadIdx.x & 63, sl = threadIdx.x >> 6;
  const int e = blockIdx.x * 64 + lo;
  const int nw = dim * K, n = nw + (db ? dim : 0);
  float acc = 0.f;
  if (e < n) {
    const float* src = e < nw ? dw_part + e : db_part + (e - nw);
    const int64_t stride = e < nw ? nw : dim;
#pragma unroll 8
    for (int k = sl; k < nparts; k += 4) acc += src[(int64_t)k * stride];
  }
  red[sl][lo] = acc;
  __syncthreads();
  if (sl == 0 && e < n) {
    const float v = ((red[0][lo] + red[1][lo]) + red[2][lo]) + red[3][lo];
    if (e < nw) dw[e] = v;
    else db[e - nw] = v;
  }
}

template <typename T>
hipError_t launch_bwd_t(const Conv1dBwdParams& q, hipStream_t st) {
  const Conv1dParams& p = q.f;
  const int nrun = (p.seqlen + TT - 1) / TT;
  dim3 grid((unsigned)((p.dim / CV + 255) / 256), (unsigned)nrun, (unsigned)p.batch);
  switch (p.width) {
#define CASE(K) case K: hipLaunchKernelGGL((conv1d_bwd_kernel<T, K>), grid, dim3(256), 0, st, q); break;
    CASE(1) CASE(2) CASE(3) CASE(4) CASE(5) CASE(6) CASE(7) CASE(8)
#undef CASE
    default: return hipErrorInvalidValue;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int n = p.dim * p.width + p.dim;
  hipLaunchKernelGGL(conv1d_reduce_kernel, dim3((unsigned)((n + 63) / 64)), dim3(256), 0, st, q.dw_part, q.db_part,
                     p.batch * nrun, p.dim, p.width, q.dweight, q.dbias);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_t(const Conv1dParams& p, hipStream_t st) {
  dim3 grid((unsigned)((p.dim / CV + 255) / 256), (unsigned)((p.seqlen + TTF - 1) / TTF), (unsigned)p.batch);
  switch (p.width) {
#define CASE(K) case K: hipLaunchKernelGGL((conv1d_kernel<T, K>), grid, dim3(256), 0, st, p); break;
    CASE(1) CASE(2) CASE(3) CASE(4) CASE(5) CASE(6) CASE(7) CASE(8)
#undef CASE
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_conv1d(const Conv1dParams& p, hipStream_t st) {
  if (p.seqlen == 0) return hipSuccess;
  return p.dtype == DT_BF16 ? launch_t<bf16>(p, st) : launch_t<float>(p, st);
}

// Empty sequence: zero weight, bias and cached-row gradients (kernels, not memset nodes).
template <typename T>
__global__ __launch_bounds__(256) void conv1d_zero_rows_kernel(T* __restrict__ d, int64_t sb, int64_t sl, int dim) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c < dim) d[(int64_t)blockIdx.z * sb + (int64_t)blockIdx.y * sl + c] = (T)0.f;
}

__global__ __launch_bounds__(256) void conv1d_zero_kernel(float* __restrict__ dw, float* __restrict__ db, int nw,
                                                          int nd) {
  const int e = blockIdx.x * 256 + threadIdx.x;
  if (e < nw) dw[e] = 0.f;
  else if (e < nw + nd && db) db[e - nw] = 0.f;
}

size_t conv1d_bwd_workspace_bytes(int batch, int seqlen, int dim, int width) {
  const size_t nparts = (size_t)batch * ((seqlen + TT - 1) / TT);
  return nparts * dim * (width + 1) * sizeof(float);
}

void conv1d_bwd_workspace_layout(Conv1dBwdParams& q, void* workspace) {
  const Conv1dParams& p = q.f;
  const size_t nparts = (size_t)p.batch * ((p.seqlen + TT - 1) / TT);
  q.dw_part = reinterpret_cast<float*>(workspace);
  q.db_part = q.dw_part + nparts * p.dim * p.width;
}

hipError_t launch_conv1d_bwd(const Conv1dBwdParams& q, hipStream_t st) {
  const Conv1dParams& p = q.f;
  if (p.seqlen == 0) {
    const int n = p.dim * p.width + p.dim;
    hipLaunchKernelGGL(conv1d_zero_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, q.dweight, q.dbias,
                       p.dim * p.width, p.dim);
    if (q.dcs && p.cs_len > 0) {
      const dim3 g((unsigned)((p.dim + 255) / 256), (unsigned)p.cs_len, (unsigned)p.batch);
      if (p.dtype == DT_BF16)
        hipLaunchKernelGGL(conv1d_zero_rows_kernel<bf16>, g, dim3(256), 0, st, reinterpret_cast<bf16*>(q.dcs),
                           q.dcs_sb, q.dcs_sl, p.dim);
      else
        hipLaunchKernelGGL(conv1d_zero_rows_kernel<float>, g, dim3(256), 0, st, reinterpret_cast<float*>(q.dcs),
                           q.dcs_sb, q.dcs_sl, p.dim);
    }
    return hipGetLastError();
  }
  return p.dtype == DT_BF16 ? launch_bwd_t<bf16>(q, st) : launch_bwd_t<float>(q, st);
}

}  // namespace mh
