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
constexpr int TT = 32;     // tokens per thread
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

template <typename T, int K>
__global__ __launch_bounds__(256) void conv1d_kernel(Conv1dParams p) {
  const int c8 = blockIdx.x * 256 + threadIdx.x;
  const int d0 = c8 * CV;
  if (d0 >= p.dim) return;
  const int b = blockIdx.z;
  const int t0 = blockIdx.y * TT;
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
#pragma unroll
  for (int j = 0; j < K - 1; ++j) {
    const int tp = t0 - (K - 1) + j;
    if (tp >= 0) {
      load8<T>(xb + (int64_t)tp * p.x_sl, win[j]);
    } else if (sb && tp >= -p.cs_len) {
      load8<T>(sb + (int64_t)(p.cs_len + tp) * p.cs_sl, win[j]);
    } else {
#pragma unroll
      for (int i = 0; i < CV; ++i) win[j][i] = 0.f;
    }
  }
  const int t1 = min(p.seqlen, t0 + TT);
  for (int t = t0; t < t1; ++t) {
    load8<T>(xb + (int64_t)t * p.x_sl, win[K - 1]);
    float o[CV];
#pragma unroll
    for (int i = 0; i < CV; ++i) {
      float acc = bias[i];
#pragma unroll
      for (int j = 0; j < K; ++j) acc += w[j][i] * win[j][i];
      o[i] = p.silu ? acc / (1.f + __expf(-acc)) : acc;
    }
    store8<T>(yb + (int64_t)t * p.y_sl, o);
#pragma unroll
    for (int j = 0; j < K - 1; ++j)
#pragma unroll
      for (int i = 0; i < CV; ++i) win[j][i] = win[j + 1][i];
  }
}

template <typename T>
hipError_t launch_t(const Conv1dParams& p, hipStream_t st) {
  dim3 grid((unsigned)((p.dim / CV + 255) / 256), (unsigned)((p.seqlen + TT - 1) / TT), (unsigned)p.batch);
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

}  // namespace mh
