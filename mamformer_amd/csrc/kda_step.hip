// One-token step of the reference's normalised linear attention (KDA decode).
//
// Per (b, h), with phi(x) = elu(x) + 1 on the first kernel_dim channels and 0
// beyond (kda_diff.py:67-89; applied here when MH_KDA_PHI is set, otherwise
// q/k arrive already feature-mapped as in the reference's call, kda_diff.py:302-304):
//     S <- S + phi(k)^T v            (dk x dv, fp32, in place)
//     z <- z + phi(k)                (dk, fp32, in place)
//     o_i = phi(q_i) S / (phi(q_i) z + 1e-8),   i = 1, 2
//     o   = (o_1 - lam o_2) / (1 - lam + 1e-8)  (or o_1, o_2 separately; or o_1 alone)
// Semantics of LinearDiffAttention._linear_attention_recurrent
// (R/mamformer/layers/kda_diff.py:564-605) and of the cache update of a
// one-token forward (kda_diff.py:329-338).
//
// Bandwidth-bound read-modify-write of the fp32 state like the SSD decode
// step: one workgroup per (b, h); each thread owns a 16-byte column slice of
// up to KSTEP_ROWS rows, issues every state load first (straight-line, rows
// clamped into range), then the small operands.  The numerators are reduced
// over rows through LDS; wave 0 updates z and forms the denominators.
#include "common.h"
#include "launch.h"

namespace mh {

constexpr int KSTEP_ROWS = 4;      // state rows per thread
constexpr int KSTEP_MAXDK = 256;

__device__ __forceinline__ float phi_step(float x) { return x > 0.f ? x + 1.f : __expf(x); }

template <int DV, typename T>
__global__ __launch_bounds__(1024) void kda_step_kernel(KdaStepParams p) {
  constexpr int TPC = DV / 4;                 // threads per state row
  __shared__ f32x4 part[2][1024 / TPC][TPC];  // per-row-group numerator partials
  __shared__ float fq[2][KSTEP_MAXDK];        // phi(q_i)
  __shared__ float fk[KSTEP_MAXDK];           // phi(k)
  __shared__ float den[2];
  const int bh = blockIdx.x;
  const int h = bh % p.nheads;
  const int tid = threadIdx.x;
  const int c = tid % TPC, r0 = tid / TPC;
  const int rg = blockDim.x / TPC;            // row groups
  const int dk = p.dk;
  const int nq = p.q2 ? 2 : 1;

  float* Sb = p.state + (int64_t)bh * dk * DV;
  f32x4* S4 = reinterpret_cast<f32x4*>(Sb);
  f32x4 s[KSTEP_ROWS];
#pragma unroll
  for (int i = 0; i < KSTEP_ROWS; ++i) s[i] = __builtin_nontemporal_load(&S4[min(r0 + i * rg, dk - 1) * TPC + c]);

  const T* vrow = reinterpret_cast<const T*>(p.v) + (int64_t)bh * DV;
  float vv[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) vv[j] = to_f32(vrow[4 * c + j]);
  // feature-mapped q_i, k into LDS
  for (int k = tid; k < dk; k += blockDim.x) {
    const bool on = k < p.kernel_dim;
    float kv = to_f32(reinterpret_cast<const T*>(p.k)[(int64_t)bh * dk + k]);
    float q1 = to_f32(reinterpret_cast<const T*>(p.q1)[(int64_t)bh * dk + k]);
    float q2 = p.q2 ? to_f32(reinterpret_cast<const T*>(p.q2)[(int64_t)bh * dk + k]) : 0.f;
    if (p.apply_phi) {
      kv = on ? phi_step(kv) : 0.f;
      q1 = on ? phi_step(q1) : 0.f;
      q2 = on ? phi_step(q2) : 0.f;
    }
    fk[k] = kv;
    fq[0][k] = q1;
    fq[1][k] = q2;
  }
  __syncthreads();

  // z update and denominators (wave 0)
  if (tid < 64) {
    float d0 = 0.f, d1 = 0.f;
    for (int k = tid; k < dk; k += 64) {
      const float zn = p.z[(int64_t)bh * dk + k] + fk[k];
      p.z[(int64_t)bh * dk + k] = zn;
      d0 += fq[0][k] * zn;
      d1 += fq[1][k] * zn;
    }
    d0 = wave_sum(d0);
    d1 = wave_sum(d1);
    if (tid == 0) {
      den[0] = d0 + 1e-8f;
      den[1] = d1 + 1e-8f;
    }
  }

  // state update and numerator partials
  f32x4 n0 = {0.f, 0.f, 0.f, 0.f}, n1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < KSTEP_ROWS; ++i) {
    const int r = r0 + i * rg;
    if (r < dk) {
      f32x4 v = s[i];
      const float kr = fk[r];
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] += kr * vv[j];
      __builtin_nontemporal_store(v, &S4[r * TPC + c]);
      const float a0 = fq[0][r], a1 = fq[1][r];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        n0[j] += a0 * v[j];
        n1[j] += a1 * v[j];
      }
    }
  }
  part[0][r0][c] = n0;
  part[1][r0][c] = n1;
  __syncthreads();

  // reduce over row groups: one thread per output column
  if (tid < DV) {
    const int cc = tid >> 2, j = tid & 3;
    float o[2] = {0.f, 0.f};
    for (int g = 0; g < rg; ++g) {
      o[0] += part[0][g][cc][j];
      o[1] += part[1][g][cc][j];
    }
    o[0] /= den[0];
    o[1] /= den[1];
    T* o1p = reinterpret_cast<T*>(p.o) + (int64_t)bh * DV;
    if (nq == 2 && !p.o2) {
      const float lam = p.lam_h ? p.lam_h[h] : p.lam;
      o1p[tid] = from_f32<T>((o[0] - lam * o[1]) / (1.f - lam + 1e-8f));
    } else {
      o1p[tid] = from_f32<T>(o[0]);
      if (p.o2) reinterpret_cast<T*>(p.o2)[(int64_t)bh * DV + tid] = from_f32<T>(o[1]);
    }
  }
}

template <int DV>
static hipError_t launch_kda_step_dv(const KdaStepParams& p, hipStream_t st) {
  constexpr int TPC = DV / 4;
  int groups = (p.dk + KSTEP_ROWS - 1) / KSTEP_ROWS;     // row groups needed
  if (groups * TPC > 1024) groups = 1024 / TPC;
  int threads = ((groups * TPC + 63) / 64) * 64;
  if (threads < DV) threads = DV;                      // the column reduction uses one thread per column
  if ((threads / TPC) * KSTEP_ROWS < p.dk) return hipErrorInvalidValue;
  dim3 grid((unsigned)(p.batch * p.nheads)), block((unsigned)threads);
  if (p.dtype == DT_BF16)
    hipLaunchKernelGGL((kda_step_kernel<DV, bf16>), grid, block, 0, st, p);
  else
    hipLaunchKernelGGL((kda_step_kernel<DV, float>), grid, block, 0, st, p);
  return hipGetLastError();
}

hipError_t launch_kda_step(const KdaStepParams& p, hipStream_t st) {
  switch (p.dv) {
    case 64: return launch_kda_step_dv<64>(p, st);
    case 128: return launch_kda_step_dv<128>(p, st);
    case 256: return launch_kda_step_dv<256>(p, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace mh
