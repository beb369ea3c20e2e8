// Single-token selective state update (the decode step of a Mamba-2 layer).
//
// Per (b, h):  dt' = clamp(softplus(dt + dt_bias)),  a = exp(A_h dt')
//              s[p, n] <- a * s[p, n] + dt' * x[p] * B[g, n]          (fp32, read-modify-write)
//              y[p]     = sum_n C[g, n] * s[p, n] + D * x[p]     (times silu(z[p]) when a gate is given)
// Reference semantics: Mamba2Block._recurrent_step, mamformer/layers/mamba2.py:431-458, and the
// z-gate applied after it (:337-338), in the per-head SSD convention (see the oracle's bridge), or,
// with the general form (A per state column, dt per channel), in the reference's own parameterisation
//              a[p, n] = exp(A[n] dt'[p]),  s[p, n] <- a[p, n] s[p, n] + dt'[p] x[p] B[n]   (mamba2.py:440-449).
//
// Bandwidth-bound: the fp32 state is read once and written once; everything
// else is a few KB.  One workgroup per (b, h) of up to 1024 threads: each
// thread owns a 16-byte column slice (4 states) of ROWS state rows spaced
// blockDim/(N/4) rows apart.  The state loads are issued first (nontemporal:
// the state is touched once per step), the small per-head operands (dt, B, C,
// x) after them so their latency hides under the state traffic.  The dot
// product over N is a shuffle reduction inside the N/4 lanes that share a row.
#include "common.h"
#include "launch.h"

namespace mh {

constexpr int SSU_ROWS = 2;   // state rows per thread per pass

// GEN: the general form, with the decay rate per state column (p.A_per_state) and/or the step per channel
// (p.dt_per_channel); without it one decay factor per head.  GATE: p.z is given (its rows are loaded with x's,
// not under a branch of their own, which would wait for them alone).
template <int N, typename T, bool GEN, bool GATE>
__global__ __launch_bounds__(1024) void ssu_kernel(SsuParams p) {
  constexpr int TPR = N / 4;        // threads per state row
  const int rp = blockDim.x / TPR;  // rows per pass
  const int bh = blockIdx.x;
  const int b = bh / p.nheads;
  const int h = bh - b * p.nheads;
  const int g = h / (p.nheads / p.ngroups);
  const int ln = threadIdx.x % TPR;
  const int row0 = threadIdx.x / TPR;
  const int P = p.headdim;

  const int64_t sbase = ((int64_t)b * p.nheads + h) * P * N;
  const f32x4* sin = reinterpret_cast<const f32x4*>(p.state_in + sbase);
  f32x4* sout = reinterpret_cast<f32x4*>(p.state_out + sbase);
  const T* xp = reinterpret_cast<const T*>(p.x) + (int64_t)b * p.x_stride_b + (int64_t)h * P;
  T* yp = reinterpret_cast<T*>(p.y) + (int64_t)b * p.y_stride_b + (int64_t)h * P;
  const T* zp = GATE ? reinterpret_cast<const T*>(p.z) + (int64_t)b * p.z_stride_b + (int64_t)h * P : nullptr;

  // Loads use row indices clamped into [0, P) so they are straight-line code
  // (no per-row branches, hence no early waits); only the stores are guarded.
  f32x4 s[SSU_ROWS];
  float xv[SSU_ROWS], dv[SSU_ROWS], zv[SSU_ROWS], tv[SSU_ROWS];
  const float* Dc = (p.D && p.D_per_channel) ? p.D + (int64_t)h * P : nullptr;
  const bool dtc = GEN && p.dt_per_channel;
  const float* dtrow = p.dt + (int64_t)b * p.dt_stride_b + (int64_t)h * P;   // per-channel dt of this head
  auto load = [&](int pbase) {
#pragma unroll
    for (int i = 0; i < SSU_ROWS; ++i) s[i] = __builtin_nontemporal_load(&sin[min(pbase + i * rp, P - 1) * TPR + ln]);
#pragma unroll
    for (int i = 0; i < SSU_ROWS; ++i) {
      xv[i] = to_f32(xp[min(pbase + i * rp, P - 1)]);
      if constexpr (GATE) zv[i] = to_f32(zp[min(pbase + i * rp, P - 1)]);
    }
    if (Dc) {
#pragma unroll
      for (int i = 0; i < SSU_ROWS; ++i) dv[i] = Dc[min(pbase + i * rp, P - 1)];
    }
    if (dtc) {
#pragma unroll
      for (int i = 0; i < SSU_ROWS; ++i) {
        const int pr = min(pbase + i * rp, P - 1);
        float d = dtrow[pr];
        if (p.dt_bias) d += p.dt_bias[(int64_t)h * P + pr];
        if (p.dt_softplus) d = softplus_f(d);
        if (p.has_dt_limit) d = fminf(fmaxf(d, p.dt_min), p.dt_max);
        tv[i] = d;
      }
    }
  };
  load(row0);

  float dt = dtc ? 0.f : p.dt[(int64_t)b * p.dt_stride_b + h];
  const T* Bp = reinterpret_cast<const T*>(p.B) + (int64_t)b * p.B_stride_b + (int64_t)g * N + ln * 4;
  const T* Cp = reinterpret_cast<const T*>(p.C) + (int64_t)b * p.C_stride_b + (int64_t)g * N + ln * 4;
  float Bv[4], Cv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    Bv[i] = to_f32(Bp[i]);
    Cv[i] = to_f32(Cp[i]);
  }
  if (!dtc) {
    if (p.dt_bias) dt += p.dt_bias[h];
    if (p.dt_softplus) dt = softplus_f(dt);
    if (p.has_dt_limit) dt = fminf(fmaxf(dt, p.dt_min), p.dt_max);
  }
  const float a = GEN ? 0.f : __expf(p.A[h] * dt);
  float Av[4];                                       // general form: the decay rate of each state column
#pragma unroll
  for (int i = 0; i < 4; ++i) Av[i] = (GEN && p.A_per_state) ? p.A[ln * 4 + i] : p.A[h];
  if (!GEN) {
#pragma unroll
    for (int i = 0; i < 4; ++i) Bv[i] *= dt;
  }
  const float Dh = (p.D && !p.D_per_channel) ? p.D[h] : 0.f;

  for (int pbase = row0; pbase < P; pbase += rp * SSU_ROWS) {
    if (pbase != row0) load(pbase);
#pragma unroll
    for (int i = 0; i < SSU_ROWS; ++i) {
      const int pr = pbase + i * rp;
      if (pr < P) {  // uniform within a row group
        f32x4 v = s[i];
        if constexpr (GEN) {
          const float d = dtc ? tv[i] : dt;
#pragma unroll
          for (int c = 0; c < 4; ++c) v[c] = __expf(Av[c] * d) * v[c] + d * xv[i] * Bv[c];
        } else {
#pragma unroll
          for (int c = 0; c < 4; ++c) v[c] = a * v[c] + xv[i] * Bv[c];
        }
        __builtin_nontemporal_store(v, &sout[pr * TPR + ln]);
        float part = v[0] * Cv[0] + v[1] * Cv[1] + v[2] * Cv[2] + v[3] * Cv[3];
#pragma unroll
        for (int off = TPR / 2; off > 0; off >>= 1) part += __shfl_xor(part, off, TPR);
        if (ln == 0) {
          float yv = part + (Dc ? dv[i] : Dh) * xv[i];
          if constexpr (GATE) yv *= silu_f(zv[i]);     // z-gate of mamba2.py:337-338
          yp[pr] = from_f32<T>(yv);
        }
      }
    }
  }
}

template <int N>
static hipError_t launch_ssu_n(const SsuParams& p, hipStream_t st) {
  constexpr int TPR = N / 4;
  // rows per pass: enough to cover P in SSU_ROWS rows per thread, capped at 1024 threads
  int rows = (p.headdim + SSU_ROWS - 1) / SSU_ROWS;
  if (rows * TPR > 1024) rows = 1024 / TPR;
  const int threads = ((rows * TPR + 63) / 64) * 64;   // whole waves; extra lanes fall past P
  dim3 grid((unsigned)(p.batch * p.nheads)), block((unsigned)threads);
  const bool gen = p.A_per_state || p.dt_per_channel, gate = p.z != nullptr;
#define SSU_LAUNCH(T)                                                                              \
  do {                                                                                             \
    if (gen) {                                                                                     \
      if (gate) hipLaunchKernelGGL((ssu_kernel<N, T, true, true>), grid, block, 0, st, p);         \
      else hipLaunchKernelGGL((ssu_kernel<N, T, true, false>), grid, block, 0, st, p);             \
    } else {                                                                                       \
      if (gate) hipLaunchKernelGGL((ssu_kernel<N, T, false, true>), grid, block, 0, st, p);        \
      else hipLaunchKernelGGL((ssu_kernel<N, T, false, false>), grid, block, 0, st, p);            \
    }                                                                                              \
  } while (0)
  if (p.dtype == DT_BF16) SSU_LAUNCH(bf16);
  else SSU_LAUNCH(float);
#undef SSU_LAUNCH
  return hipGetLastError();
}

hipError_t launch_ssu(const SsuParams& p, hipStream_t st) {
  switch (p.dstate) {
    case 8: return launch_ssu_n<8>(p, st);
    case 16: return launch_ssu_n<16>(p, st);
    case 32: return launch_ssu_n<32>(p, st);
    case 64: return launch_ssu_n<64>(p, st);
    case 128: return launch_ssu_n<128>(p, st);
    case 256: return launch_ssu_n<256>(p, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace mh
